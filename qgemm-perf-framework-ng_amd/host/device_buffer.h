// Owning device allocation for the host harness (hipMalloc / hipFree).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <string>
#include <utility>

namespace pfng::bench {

class DeviceBuffer {
  public:
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    DeviceBuffer(DeviceBuffer &&o) noexcept : ptr_(std::exchange(o.ptr_, nullptr)), bytes_(o.bytes_) {}
    ~DeviceBuffer() { reset(); }

    // Allocates `bytes` (at least one byte); returns false with `error` set.
    bool allocate(size_t bytes, std::string &error) {
        reset();
        const hipError_t e = hipMalloc(&ptr_, bytes ? bytes : 1);
        if (e != hipSuccess) {
            ptr_ = nullptr;
            error = std::string("hipMalloc(") + std::to_string(bytes) + "): " + hipGetErrorString(e);
            return false;
        }
        bytes_ = bytes;
        return true;
    }
    bool upload(const void *src, size_t bytes, std::string &error) {
        const hipError_t e = hipMemcpy(ptr_, src, bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) error = std::string("hipMemcpy H2D: ") + hipGetErrorString(e);
        return e == hipSuccess;
    }
    bool download(void *dst, size_t bytes, std::string &error) const {
        const hipError_t e = hipMemcpy(dst, ptr_, bytes, hipMemcpyDeviceToHost);
        if (e != hipSuccess) error = std::string("hipMemcpy D2H: ") + hipGetErrorString(e);
        return e == hipSuccess;
    }
    void reset() noexcept {
        if (ptr_) (void)hipFree(ptr_);
        ptr_ = nullptr;
        bytes_ = 0;
    }
    void *get() const noexcept { return ptr_; }
    size_t bytes() const noexcept { return bytes_; }

  private:
    void *ptr_ = nullptr;
    size_t bytes_ = 0;
};

}  // namespace pfng::bench
