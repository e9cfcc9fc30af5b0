// Host utilities of the drop-in API (replaces src/gpu/util.cuh:1-57 host parts): error checking, owning
// device buffers, pinned host buffers. Device math lives in kernels/device_math.h.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "b2c_kernels.h"

namespace b2c {

#define HIP_CHECK(expr)                                                                                     \
  do {                                                                                                      \
    hipError_t _e = (expr);                                                                                 \
    if (_e != hipSuccess)                                                                                   \
      throw std::runtime_error(std::string("HIP error ") + hipGetErrorString(_e) + " at " + __FILE__ + ":" + \
                               std::to_string(__LINE__));                                                   \
  } while (0)
// Launchers return hipError_t as int.
#define LAUNCH_CHECK(expr) HIP_CHECK((hipError_t)(expr))

constexpr int TILE_W = 16;   // loss tile (util.cuh:17)
constexpr int TILE_PX = TILE_W * TILE_W;
constexpr int RT_W = 8;      // raster tile (util.cuh:19)
constexpr int RT_PX = RT_W * RT_W;
constexpr int PROJ_BLOCK = 256;
constexpr uint32_t GRAD_LANES = 13;

inline int div_up(size_t a, int b) { return (int)((a + b - 1) / b); }

// Owning device buffer (util.cuh:26-57 semantics): move-only, reserve grows (contents discarded unless
// keep), freed in the destructor.
template <typename T>
struct DevBuf {
  T* ptr = nullptr;
  size_t count = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : ptr(o.ptr), count(o.count) { o.ptr = nullptr; o.count = 0; }
  DevBuf& operator=(DevBuf&& o) noexcept {
    free();
    ptr = o.ptr; count = o.count;
    o.ptr = nullptr; o.count = 0;
    return *this;
  }
  ~DevBuf() { free(); }
  void free() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    count = 0;
  }
  void reserve(size_t n, bool keep = false, hipStream_t stream = nullptr) {
    if (n <= count) return;
    T* np = nullptr;
    HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&np), n * sizeof(T)));
    if (keep && ptr && count) HIP_CHECK(hipMemcpyAsync(np, ptr, count * sizeof(T), hipMemcpyDeviceToDevice, stream));
    if (ptr) {
      HIP_CHECK(hipStreamSynchronize(stream));
      (void)hipFree(ptr);
    }
    ptr = np;
    count = n;
  }
  // Zero the first n entries with a fill kernel (safe inside captured graphs, unlike a memset node).
  void zero(hipStream_t stream = nullptr, size_t n = (size_t)-1) {
    if (!ptr) return;
    const size_t bytes = (n == (size_t)-1 ? count : n) * sizeof(T);
    if (bytes % 4 == 0)
      LAUNCH_CHECK(b2c_hip_fill_u32(reinterpret_cast<uint32_t*>(ptr), 0u, bytes / 4, stream));
    else
      HIP_CHECK(hipMemsetAsync(ptr, 0, bytes, stream));
  }
  void upload(const T* src, size_t n, hipStream_t stream = nullptr) {
    reserve(n);
    HIP_CHECK(hipMemcpyAsync(ptr, src, n * sizeof(T), hipMemcpyHostToDevice, stream));
  }
  void upload(const std::vector<T>& v, hipStream_t stream = nullptr) { upload(v.data(), v.size(), stream); }
  std::vector<T> download(size_t n = (size_t)-1, hipStream_t stream = nullptr) const {
    if (n == (size_t)-1) n = count;
    std::vector<T> v(n);
    if (n) {
      HIP_CHECK(hipMemcpyAsync(v.data(), ptr, n * sizeof(T), hipMemcpyDeviceToHost, stream));
      HIP_CHECK(hipStreamSynchronize(stream));
    }
    return v;
  }
  size_t bytes() const { return count * sizeof(T); }
  operator T*() const { return ptr; }
};

// Pinned host buffer for readbacks (util.cuh:59-65).
template <typename T>
struct PinnedBuf {
  T* ptr = nullptr;
  size_t count = 0;
  PinnedBuf() = default;
  PinnedBuf(const PinnedBuf&) = delete;
  PinnedBuf& operator=(const PinnedBuf&) = delete;
  void reserve(size_t n) {
    if (n <= count) return;
    if (ptr) (void)hipHostFree(ptr);
    ptr = nullptr;
    HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&ptr), n * sizeof(T), hipHostMallocDefault));
    count = n;
  }
  ~PinnedBuf() {
    if (ptr) (void)hipHostFree(ptr);
  }
};

}  // namespace b2c
