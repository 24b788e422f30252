// storage.hpp -- the element buffer behind a Tensor: an fp32 block in the HBM
// arena plus a lazily synchronised host mirror.
//
// The reference keeps the host copy authoritative and mirrors it to the device
// on demand (include/engine/detail/storage.hpp:10-157 of the reference). Here
// the device copy is where the work happens and the host copy is made only
// when host code reads the values; the invariant is the same: at least one
// side is valid (or the buffer is a pending fill, which neither side holds
// yet). Storages made by share() are views of one buffer, so the validity
// flags live in the shared buffer.
#ifndef ENGINE_DETAIL_STORAGE_HPP
#define ENGINE_DETAIL_STORAGE_HPP

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

namespace engine {

// Reuse statistics of the device buffer pool (the HBM arena), under the
// reference's names (include/engine/detail/storage.hpp:36-46): `fresh` counts
// allocations the pool could not serve from its free lists, `recycled` those
// it could, `bytes_held` the cached free bytes.
struct BufferPoolStats {
    size_t fresh = 0;
    size_t recycled = 0;
    size_t bytes_held = 0;
};

BufferPoolStats buffer_pool_stats();

class Storage {
public:
    Storage() = default;
    // n elements, all equal to `fill` (materialised lazily, on the side that is
    // first asked for).
    explicit Storage(size_t n, float fill = 0.0f);
    // n elements copied from host memory (uploaded on first device use).
    explicit Storage(const std::vector<float>& values);

    size_t size() const noexcept;

    // Device side. device() uploads (or fills) if the device copy is stale;
    // device_mut() does the same and marks the host copy stale; device_write()
    // hands out the block for a kernel to overwrite completely, without
    // uploading anything.
    const float* device() const;
    float* device_mut();
    float* device_write();

    // Host side. host() downloads if the host copy is stale; host_mut() does
    // the same and marks the device copy stale.
    const std::vector<float>& host() const;
    std::vector<float>& host_mut();

    bool resident_on_device() const noexcept;
    // True when no other Storage shares this buffer. The engine mutates a
    // buffer in place only when it is exclusive (gradient buffers may be
    // shared after add_grad adopts a temporary).
    bool exclusive() const noexcept;
    // True while the buffer is a pending fill of zeros: add_grad uses it to
    // initialise a zeroed gradient without materialising the zeros first.
    bool pending_zero() const noexcept;
    // True while the buffer is a pending fill of one value (stored in *value):
    // a kernel that only needs that constant can take it from the host.
    bool pending_constant(float* value) const noexcept;

    // Sets every element to `value` lazily (the reference's assign,
    // src/storage.cpp:253-269): nothing is copied or launched now.
    void assign(float value);

    Storage share() const;  // a view of the same buffer
    Storage clone() const;  // a new buffer with the same values (device copy if resident)
    // True when both are views of one buffer.
    bool same_buffer(const Storage& other) const noexcept { return buf_ && buf_ == other.buf_; }
    // A counter of the buffer's mutable accesses (device_mut, device_write,
    // host_mut, assign): equal values mean the contents have not been handed
    // out for writing in between.
    uint64_t version() const noexcept;

private:
    struct Buffer;
    std::shared_ptr<Buffer> buf_;
};

// A device array of int32 (argmax, labels, gather indices), owned by the arena.
class DeviceInts {
public:
    DeviceInts() = default;
    explicit DeviceInts(const std::vector<int32_t>& values);
    explicit DeviceInts(size_t n);  // uninitialised, for kernels to write
    const int32_t* get() const noexcept;
    int32_t* get() noexcept;
    size_t size() const noexcept;
    std::vector<int32_t> to_host() const;

private:
    struct Block;
    std::shared_ptr<Block> blk_;
};

}  // namespace engine

#endif  // ENGINE_DETAIL_STORAGE_HPP
