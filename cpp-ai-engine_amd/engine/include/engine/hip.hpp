// hip.hpp -- the runtime control API of the device backend, under the
// engine's namespace (the reference's include/engine/cuda.hpp:23-218, renamed:
// engine::hip instead of engine::cuda). Thin wrappers over include/ehip.h.
#ifndef ENGINE_HIP_HPP
#define ENGINE_HIP_HPP

#include <cstddef>
#include <functional>
#include <optional>
#include <string>
#include <vector>

namespace engine {
namespace hip {

bool available();

// Runtime switch (the reference's cuda::enabled / set_enabled). It starts on,
// or off with ENGINE_HIP=0 in the environment. This engine computes on the
// device only: with the backend switched off every operation that would launch
// a kernel throws (std::runtime_error, "switched off"), where the reference
// would run its CPU loops.
bool enabled();
void set_enabled(bool on);

// The HIP versions in play, in HIP's encoding (major * 10000000 + minor *
// 100000 + patch): the headers the backend was compiled with, and the runtime
// and driver it runs on; 0 where the runtime cannot tell.
int compiled_version();
int runtime_version();
int driver_version();

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

// What each of the backend's main kernels costs the scheduler on this device:
// the block size it is launched with, VGPRs per lane, static LDS per block,
// the blocks that fit on one CU at once, the resident waves that makes as a
// fraction of the CU's maximum, and what runs out first ("registers", "lds" or
// "waves"). The static ceiling, not the achieved occupancy. Empty without a
// device.
struct KernelOccupancy {
    std::string name;
    int block_threads = 0;
    int registers = 0;
    size_t shared_bytes = 0;
    int blocks_per_cu = 0;
    double occupancy = 0.0;
    std::string limiter;
};
std::vector<KernelOccupancy> kernel_occupancy();

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

// A sequence of engine calls captured once and replayed with one launch (the
// ehip_graph_* calls; no counterpart in the reference, whose steps are host
// loops of launches). capture() runs `body` with every launch of this thread
// recorded instead of run; if body throws, the capture is dropped and the
// exception passed on. Kernel arguments are fixed by the capture: each
// launch() reads and writes the buffers the capture saw, and the device
// allocator keeps them reserved until reset() or destruction. Values that
// change between replays must be read from device memory (Adam's
// set_device_scalars). Host transfers and synchronisation are refused inside
// body.
class Graph {
public:
    Graph() = default;
    ~Graph();
    Graph(const Graph&) = delete;
    Graph& operator=(const Graph&) = delete;
    void capture(const std::function<void()>& body);
    void launch();
    void reset();
    bool ready() const noexcept { return handle_ != nullptr; }

private:
    void* handle_ = nullptr;
};

}  // namespace hip
}  // namespace engine

#endif  // ENGINE_HIP_HPP
