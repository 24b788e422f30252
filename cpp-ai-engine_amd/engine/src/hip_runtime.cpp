// hip_runtime.cpp -- engine::hip, the control API over include/ehip.h.
#include "engine/hip.hpp"

#include <stdexcept>
#include <string>

#include "ehip.h"

namespace engine {
namespace hip {

void check(int rc, const char* what) {
    if (rc != EHIP_OK)
        throw std::runtime_error(std::string(what) + ": " + ehip_last_error() + " (status " +
                                 std::to_string(rc) + ")");
}

bool available() { return ehip_available() != 0; }

bool enabled() { return ehip_enabled() != 0; }

void set_enabled(bool on) { ehip_set_enabled(on ? 1 : 0); }

namespace {
struct Versions {
    int compiled = 0, runtime = 0, driver = 0;
};
Versions versions() {
    Versions v;
    (void)ehip_version_info(&v.compiled, &v.runtime, &v.driver);
    return v;
}
}  // namespace

int compiled_version() { return versions().compiled; }
int runtime_version() { return versions().runtime; }
int driver_version() { return versions().driver; }

std::vector<KernelOccupancy> kernel_occupancy() {
    int count = 0;
    if (ehip_kernel_occupancy(nullptr, 0, &count) != EHIP_OK || count <= 0) return {};
    std::vector<ehip_kernel_occupancy_t> raw(static_cast<size_t>(count));
    if (ehip_kernel_occupancy(raw.data(), count, &count) != EHIP_OK) return {};
    std::vector<KernelOccupancy> out;
    out.reserve(raw.size());
    for (const ehip_kernel_occupancy_t& r : raw) {
        KernelOccupancy k;
        k.name = r.name;
        k.block_threads = r.block_threads;
        k.registers = r.registers;
        k.shared_bytes = size_t(r.lds_bytes);
        k.blocks_per_cu = r.blocks_per_cu;
        k.occupancy = r.occupancy;
        k.limiter = r.limiter;
        out.push_back(std::move(k));
    }
    return out;
}

std::optional<DeviceInfo> device_info() {
    ehip_device_info_t info;
    if (ehip_device_info(&info) != EHIP_OK) return std::nullopt;
    DeviceInfo d;
    d.name = info.name;
    d.arch = info.arch;
    d.compute_units = info.compute_units;
    d.total_memory = info.total_memory;
    return d;
}

void synchronize() { check(ehip_synchronize(), "synchronize"); }

Graph::~Graph() { (void)ehip_graph_destroy(handle_); }

void Graph::capture(const std::function<void()>& body) {
    reset();
    check(ehip_graph_begin(), "graph capture");
    try {
        body();
    } catch (...) {
        (void)ehip_graph_abort();
        throw;
    }
    check(ehip_graph_end(&handle_), "graph capture");
}

void Graph::launch() {
    if (handle_ == nullptr) throw std::logic_error("Graph::launch: nothing captured");
    check(ehip_graph_launch(handle_, nullptr), "graph launch");
}

void Graph::reset() {
    void* h = handle_;
    handle_ = nullptr;
    check(ehip_graph_destroy(h), "graph destroy");
}
size_t kernels_launched() { return size_t(ehip_kernels_launched()); }
size_t kernels_failed() { return size_t(ehip_kernels_failed()); }
void reset_kernel_counters() { ehip_reset_counters(); }

double peak_fp32_gflops() {
    ehip_device_info_t info;
    return ehip_device_info(&info) == EHIP_OK ? info.peak_fp32_mfma_gflops : 0.0;
}

double peak_bandwidth_gbs() {
    ehip_device_info_t info;
    return ehip_device_info(&info) == EHIP_OK ? info.peak_hbm_gbs : 0.0;
}

TransferStats transfer_stats() {
    ehip_transfer_stats_t s;
    ehip_transfer_stats(&s);
    TransferStats t;
    t.to_device_bytes = size_t(s.to_device_bytes);
    t.to_host_bytes = size_t(s.to_host_bytes);
    t.to_device_count = size_t(s.to_device_count);
    t.to_host_count = size_t(s.to_host_count);
    t.to_device_seconds = s.to_device_seconds;
    t.to_host_seconds = s.to_host_seconds;
    return t;
}

void reset_transfer_stats() { ehip_reset_transfer_stats(); }

}  // namespace hip
}  // namespace engine
