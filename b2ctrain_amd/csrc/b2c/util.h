// Host utilities of the drop-in API: error checking, owning device buffers and pinned host buffers. The
// reference keeps these in src/gpu/util.cuh:1-65; the buffer types keep the member names its callers use
// (ptr, count, reserve, zero, upload, download, bytes). Device math lives in kernels/device_math.h.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "b2c_kernels.h"

namespace b2c {

[[noreturn]] inline void hip_fail(hipError_t e, const char* file, int line) {
  throw std::runtime_error(std::string("HIP error ") + hipGetErrorString(e) + " at " + file + ":" + std::to_string(line));
}
#define HIP_CHECK(expr)                                   \
  do {                                                    \
    const hipError_t b2c_rc_ = (expr);                    \
    if (b2c_rc_ != hipSuccess) ::b2c::hip_fail(b2c_rc_, __FILE__, __LINE__); \
  } while (0)
// The launcher layer returns hipError_t as int.
#define LAUNCH_CHECK(expr) HIP_CHECK(static_cast<hipError_t>(expr))

constexpr int TILE_W = 16;   // loss tile (util.cuh:17)
constexpr int TILE_PX = TILE_W * TILE_W;
constexpr int RT_W = 8;      // raster tile (util.cuh:19)
constexpr int RT_PX = RT_W * RT_W;
constexpr int PROJ_BLOCK = 256;
constexpr uint32_t GRAD_LANES = 13;

inline int div_up(size_t a, int b) { return (int)((a + b - 1) / b); }

// Untyped device allocation. Growth allocates the new block first, copies the old contents on the stream
// when asked to, and frees the old block only after the stream has drained (a queued kernel may still
// read it). It never shrinks.
struct DeviceBlock {
  void* base = nullptr;
  size_t size = 0;  // bytes

  void release() noexcept {
    if (base) (void)hipFree(base);
    base = nullptr;
    size = 0;
  }
  void grow_to(size_t want, bool preserve, hipStream_t stream) {
    if (want <= size) return;
    void* fresh = nullptr;
    HIP_CHECK(hipMalloc(&fresh, want));
    if (base) {
      if (preserve && size) HIP_CHECK(hipMemcpyAsync(fresh, base, size, hipMemcpyDeviceToDevice, stream));
      HIP_CHECK(hipStreamSynchronize(stream));
      (void)hipFree(base);
    }
    base = fresh;
    size = want;
  }
  // Zero `bytes` from the start with the fill kernel (capturable; a memset node is not).
  void clear(size_t bytes, hipStream_t stream) const {
    if (!base || !bytes) return;
    if (bytes % 4) HIP_CHECK(hipMemsetAsync(base, 0, bytes, stream));
    else LAUNCH_CHECK(b2c_hip_fill_u32(static_cast<uint32_t*>(base), 0u, bytes / 4, stream));
  }
};

// Typed, move-only owner of a device array (the reference's DevBuf semantics: reserve grows and discards
// the contents unless `keep`, the destructor frees).
template <typename T>
struct DevBuf {
  T* ptr = nullptr;
  size_t count = 0;

  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept { take(o); }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      free();
      take(o);
    }
    return *this;
  }
  ~DevBuf() { free(); }

  void free() noexcept {
    DeviceBlock b = block();
    b.release();
    ptr = nullptr;
    count = 0;
  }
  void reserve(size_t n, bool keep = false, hipStream_t stream = nullptr) {
    if (n <= count) return;
    DeviceBlock b = block();
    b.grow_to(n * sizeof(T), keep, stream);
    ptr = static_cast<T*>(b.base);
    count = n;
  }
  void zero(hipStream_t stream = nullptr, size_t n = (size_t)-1) { block().clear((n == (size_t)-1 ? count : n) * sizeof(T), stream); }
  void upload(const T* src, size_t n, hipStream_t stream = nullptr) {
    reserve(n);
    if (n) HIP_CHECK(hipMemcpyAsync(ptr, src, n * sizeof(T), hipMemcpyHostToDevice, stream));
  }
  void upload(const std::vector<T>& v, hipStream_t stream = nullptr) { upload(v.data(), v.size(), stream); }
  std::vector<T> download(size_t n = (size_t)-1, hipStream_t stream = nullptr) const {
    std::vector<T> host(n == (size_t)-1 ? count : n);
    if (!host.empty()) {
      HIP_CHECK(hipMemcpyAsync(host.data(), ptr, host.size() * sizeof(T), hipMemcpyDeviceToHost, stream));
      HIP_CHECK(hipStreamSynchronize(stream));
    }
    return host;
  }
  size_t bytes() const { return count * sizeof(T); }
  operator T*() const { return ptr; }

 private:
  DeviceBlock block() const { return DeviceBlock{ptr, count * sizeof(T)}; }
  void take(DevBuf& o) noexcept {
    ptr = o.ptr;
    count = o.count;
    o.ptr = nullptr;
    o.count = 0;
  }
};

// Pinned (page-locked) host array for device-to-host readbacks; grows, never shrinks.
template <typename T>
struct PinnedBuf {
  T* ptr = nullptr;
  size_t count = 0;

  PinnedBuf() = default;
  PinnedBuf(const PinnedBuf&) = delete;
  PinnedBuf& operator=(const PinnedBuf&) = delete;
  ~PinnedBuf() { drop(); }

  void reserve(size_t n) {
    if (n <= count) return;
    drop();
    void* p = nullptr;
    HIP_CHECK(hipHostMalloc(&p, n * sizeof(T), hipHostMallocDefault));
    ptr = static_cast<T*>(p);
    count = n;
  }

 private:
  void drop() noexcept {
    if (ptr) (void)hipHostFree(ptr);
    ptr = nullptr;
    count = 0;
  }
};

}  // namespace b2c
