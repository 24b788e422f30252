// storage.cpp -- device-first buffers over the HBM arena of libehip.
#include "engine/detail/storage.hpp"

#include <cstring>
#include <stdexcept>

#include "ehip.h"
#include "engine/hip.hpp"

namespace engine {

struct Storage::Buffer {
    size_t n = 0;
    float* dev = nullptr;
    std::vector<float> host;
    bool host_valid = false;
    bool device_valid = false;
    bool pending = false;  // every element equals fill_value; neither side materialised
    float fill_value = 0.0f;
    uint64_t version = 0;  // advanced by every accessor that may change the values

    ~Buffer() {
        if (dev != nullptr) ehip_arena_free(dev);
    }
    void ensure_alloc() {
        if (dev == nullptr && n > 0) {
            void* p = nullptr;
            hip::check(ehip_arena_alloc(n * sizeof(float), &p), "device allocation");
            dev = static_cast<float*>(p);
        }
    }
    void to_device() {
        ensure_alloc();
        if (device_valid || n == 0) {
            device_valid = true;
            return;
        }
        if (pending) {
            hip::check(ehip_fill_f32(dev, int64_t(n), fill_value, nullptr), "fill");
        } else if (host_valid) {
            hip::check(ehip_memcpy_h2d(dev, host.data(), n * sizeof(float), nullptr), "upload");
        } else {
            throw std::logic_error("Storage: neither side holds the values");
        }
        device_valid = true;
    }
    void to_host() {
        if (host_valid) return;
        if (pending) {
            host.assign(n, fill_value);
        } else if (device_valid) {
            host.resize(n);
            if (n > 0)
                hip::check(ehip_memcpy_d2h(host.data(), dev, n * sizeof(float), nullptr),
                           "download");
        } else {
            throw std::logic_error("Storage: neither side holds the values");
        }
        host_valid = true;
    }
};

Storage::Storage(size_t n, float fill) : buf_(std::make_shared<Buffer>()) {
    buf_->n = n;
    buf_->pending = true;
    buf_->fill_value = fill;
}

Storage::Storage(const std::vector<float>& values) : buf_(std::make_shared<Buffer>()) {
    buf_->n = values.size();
    buf_->host = values;
    buf_->host_valid = true;
}

size_t Storage::size() const noexcept { return buf_ ? buf_->n : 0; }

const float* Storage::device() const {
    if (!buf_) return nullptr;
    buf_->to_device();
    return buf_->dev;
}

float* Storage::device_mut() {
    if (!buf_) return nullptr;
    ++buf_->version;
    buf_->to_device();
    buf_->host_valid = false;
    buf_->pending = false;
    return buf_->dev;
}

float* Storage::device_write() {
    if (!buf_) return nullptr;
    ++buf_->version;
    buf_->ensure_alloc();
    buf_->device_valid = true;
    buf_->host_valid = false;
    buf_->pending = false;
    return buf_->dev;
}

const std::vector<float>& Storage::host() const {
    if (!buf_) throw std::logic_error("Storage: empty");
    buf_->to_host();
    return buf_->host;
}

std::vector<float>& Storage::host_mut() {
    if (!buf_) throw std::logic_error("Storage: empty");
    ++buf_->version;
    buf_->to_host();
    buf_->device_valid = false;
    buf_->pending = false;
    return buf_->host;
}

bool Storage::resident_on_device() const noexcept { return buf_ && buf_->device_valid; }

uint64_t Storage::version() const noexcept { return buf_ ? buf_->version : 0; }

bool Storage::exclusive() const noexcept { return buf_ && buf_.use_count() == 1; }

bool Storage::pending_constant(float* value) const noexcept {
    if (!buf_ || !buf_->pending || buf_->device_valid || buf_->host_valid) return false;
    if (value != nullptr) *value = buf_->fill_value;
    return true;
}

bool Storage::pending_zero() const noexcept {
    return buf_ && buf_->pending && buf_->fill_value == 0.0f &&
           !buf_->device_valid && !buf_->host_valid;
}

void Storage::assign(float value) {
    if (!buf_) return;
    ++buf_->version;
    buf_->pending = true;
    buf_->fill_value = value;
    buf_->device_valid = false;
    buf_->host_valid = false;
}

Storage Storage::share() const {
    Storage s;
    s.buf_ = buf_;
    return s;
}

Storage Storage::clone() const {
    Storage s;
    s.buf_ = std::make_shared<Buffer>();
    if (!buf_) return s;
    Buffer& src = *buf_;
    Buffer& dst = *s.buf_;
    dst.n = src.n;
    if (src.pending && !src.device_valid && !src.host_valid) {
        dst.pending = true;
        dst.fill_value = src.fill_value;
    } else if (src.device_valid) {
        dst.ensure_alloc();
        if (dst.n > 0)
            hip::check(ehip_memcpy_d2d(dst.dev, src.dev, dst.n * sizeof(float), nullptr),
                       "device copy");
        dst.device_valid = true;
    } else {
        dst.host = src.host;
        dst.host_valid = true;
    }
    return s;
}

BufferPoolStats buffer_pool_stats() {
    ehip_arena_stats_t a{};
    ehip_arena_stats(&a);
    BufferPoolStats b;
    b.fresh = size_t(a.driver_allocations);
    b.recycled = size_t(a.allocations - a.driver_allocations);
    b.bytes_held = size_t(a.bytes_cached);
    return b;
}

// ------------------------------------------------------------------ ints

struct DeviceInts::Block {
    size_t n = 0;
    int32_t* dev = nullptr;
    ~Block() {
        if (dev != nullptr) ehip_arena_free(dev);
    }
};

DeviceInts::DeviceInts(size_t n) : blk_(std::make_shared<Block>()) {
    blk_->n = n;
    if (n > 0) {
        void* p = nullptr;
        hip::check(ehip_arena_alloc(n * sizeof(int32_t), &p), "device allocation");
        blk_->dev = static_cast<int32_t*>(p);
    }
}

DeviceInts::DeviceInts(const std::vector<int32_t>& values) : DeviceInts(values.size()) {
    if (!values.empty())
        hip::check(ehip_memcpy_h2d(blk_->dev, values.data(), values.size() * sizeof(int32_t),
                                   nullptr),
                   "upload");
}

const int32_t* DeviceInts::get() const noexcept { return blk_ ? blk_->dev : nullptr; }
int32_t* DeviceInts::get() noexcept { return blk_ ? blk_->dev : nullptr; }
size_t DeviceInts::size() const noexcept { return blk_ ? blk_->n : 0; }

std::vector<int32_t> DeviceInts::to_host() const {
    std::vector<int32_t> out(size());
    if (!out.empty())
        hip::check(ehip_memcpy_d2h(out.data(), blk_->dev, out.size() * sizeof(int32_t), nullptr),
                   "download");
    return out;
}

}  // namespace engine
