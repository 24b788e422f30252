// serialize.hpp -- checkpoints in the reference's weight format (the
// reference's include/engine/serialize.hpp): an 8-byte "CPPAIENG" magic, a
// u32 version (1), a u32 tensor count, then per tensor a u32 name length, the
// name, a u32 rank, u64 dims and the fp32 values, all little-endian. Files are
// interchangeable with the reference's: the names come from the same
// named_parameters() scheme.
//
// Values move between HBM and the file through the ABI's copies (one D2H or
// H2D transfer per tensor); a device-resident parameter never grows a host
// mirror because of a save.
#ifndef ENGINE_SERIALIZE_HPP
#define ENGINE_SERIALIZE_HPP

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "engine/nn.hpp"
#include "engine/optim.hpp"

namespace engine {

constexpr uint32_t kSerializationVersion = 1;

using NamedTensors = std::vector<std::pair<std::string, Tensor>>;

void save_parameters(nn::Module& model, const std::string& path);
void save_parameters(const NamedTensors& params, const std::string& path);

// Copies the file's values into the parameters of the same names; a shape
// mismatch throws. strict: every parameter must be in the file and every
// tensor in the file must belong to a parameter. Returns how many loaded.
size_t load_parameters(nn::Module& model, const std::string& path, bool strict = true);
size_t load_parameters(NamedTensors& params, const std::string& path, bool strict = true);

std::vector<std::pair<std::string, std::vector<size_t>>> inspect_parameters(
    const std::string& path);
NamedTensors load_tensors(const std::string& path);

// Adam's state for an exact resume (not in the reference's format, which has
// no optimizer state; same container): "adam.t" (the step count as two floats,
// t mod 2^24 and t / 2^24, both exact), then "adam.m.<i>" and "adam.v.<i>" per
// parameter in the optimizer's order.
void save_optimizer(const optim::Adam& opt, const std::string& path);
void load_optimizer(optim::Adam& opt, const std::string& path);

}  // namespace engine

#endif  // ENGINE_SERIALIZE_HPP
