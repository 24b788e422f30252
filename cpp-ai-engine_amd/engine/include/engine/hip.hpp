// hip.hpp -- the runtime control API of the device backend, under the
// engine's namespace (the reference's include/engine/cuda.hpp:23-218, renamed:
// engine::hip instead of engine::cuda). Thin wrappers over include/ehip.h.
#ifndef ENGINE_HIP_HPP
#define ENGINE_HIP_HPP

#include <cstddef>
#include <optional>
#include <string>

namespace engine {
namespace hip {

bool available();

struct DeviceInfo {
    std::string name;
    std::string arch;
    int compute_units = 0;
    size_t total_memory = 0;
};
std::optional<DeviceInfo> device_info();

void synchronize();
size_t kernels_launched();
size_t kernels_failed();
void reset_kernel_counters();
double peak_fp32_gflops();
double peak_bandwidth_gbs();

struct TransferStats {
    size_t to_device_bytes = 0;
    size_t to_host_bytes = 0;
    size_t to_device_count = 0;
    size_t to_host_count = 0;
    double to_device_seconds = 0.0;
    double to_host_seconds = 0.0;
};
TransferStats transfer_stats();
void reset_transfer_stats();

// Throws std::runtime_error carrying ehip_last_error() when rc != 0.
void check(int rc, const char* what);

}  // namespace hip
}  // namespace engine

#endif  // ENGINE_HIP_HPP
