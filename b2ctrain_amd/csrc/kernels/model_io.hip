// Model storage on the device: scatter of an uploaded splat cloud into the Model's float4 / planar-SH
// layout, the inverse gather for downloads, and the planar re-layout when the capacity grows. The layout
// is the reference's (src/model.h:8-23) because refine / cage / evidence code reads it; the data movement
// runs here as coalesced grid-stride kernels instead of host-side re-layout loops, so an upload is five
// contiguous host-to-device copies plus one launch.
#include <hip/hip_runtime.h>

#include "b2c_kernels.h"

namespace b2c {
namespace dev {
namespace {

constexpr int IO_BLOCK = 256;

__device__ __forceinline__ size_t grid_stride() { return (size_t)gridDim.x * blockDim.x; }
__device__ __forceinline__ size_t grid_index() { return (size_t)blockIdx.x * blockDim.x + threadIdx.x; }

// One thread per splat for the float4 fields.
__global__ void __launch_bounds__(IO_BLOCK) scatter_params_kernel(b2c_cloud_dev c, b2c_model_dev m) {
  for (size_t i = grid_index(); i < (size_t)m.n; i += grid_stride()) {
    reinterpret_cast<float4*>(m.pos_op)[i] = make_float4(c.pos[3 * i], c.pos[3 * i + 1], c.pos[3 * i + 2], c.opacity[i]);
    reinterpret_cast<float4*>(m.quat)[i] = make_float4(c.quat[4 * i], c.quat[4 * i + 1], c.quat[4 * i + 2], c.quat[4 * i + 3]);
    reinterpret_cast<float4*>(m.lscale)[i] =
        make_float4(c.log_scale[3 * i], c.log_scale[3 * i + 1], c.log_scale[3 * i + 2], c.floor_ ? c.floor_[i] : 0.f);
  }
}

// One thread per (lane, splat) coefficient, lane-major so the planar writes are coalesced.
__global__ void __launch_bounds__(IO_BLOCK) scatter_sh_kernel(b2c_cloud_dev c, b2c_model_dev m) {
  const size_t total = (size_t)m.n * m.sh_lanes;
  for (size_t e = grid_index(); e < total; e += grid_stride()) {
    const size_t lane = e / (size_t)m.n, i = e - lane * (size_t)m.n;
    const float v = c.sh[i * m.sh_lanes + lane];
    if (lane < 3) {
      m.sh_dc[lane * m.cap + i] = v;
    } else {
      const size_t o = (lane - 3) * m.cap + i;
      if (m.sh_hi32) m.sh_hi32[o] = v;
      else m.sh_hi16[o] = __builtin_bit_cast(uint16_t, (_Float16)v);  // v_cvt_f16_f32: round to nearest even
    }
  }
}

__global__ void __launch_bounds__(IO_BLOCK) gather_params_kernel(b2c_model_dev m, b2c_cloud_dev c) {
  for (size_t i = grid_index(); i < (size_t)m.n; i += grid_stride()) {
    const float4 p = reinterpret_cast<const float4*>(m.pos_op)[i];
    const float4 q = reinterpret_cast<const float4*>(m.quat)[i];
    const float4 s = reinterpret_cast<const float4*>(m.lscale)[i];
    c.pos[3 * i] = p.x; c.pos[3 * i + 1] = p.y; c.pos[3 * i + 2] = p.z; c.opacity[i] = p.w;
    c.quat[4 * i] = q.x; c.quat[4 * i + 1] = q.y; c.quat[4 * i + 2] = q.z; c.quat[4 * i + 3] = q.w;
    c.log_scale[3 * i] = s.x; c.log_scale[3 * i + 1] = s.y; c.log_scale[3 * i + 2] = s.z;
    if (c.floor_) c.floor_[i] = s.w;
  }
}

__global__ void __launch_bounds__(IO_BLOCK) gather_sh_kernel(b2c_model_dev m, b2c_cloud_dev c) {
  const size_t total = (size_t)m.n * m.sh_lanes;
  for (size_t e = grid_index(); e < total; e += grid_stride()) {
    const size_t lane = e / (size_t)m.n, i = e - lane * (size_t)m.n;
    float v;
    if (lane < 3) {
      v = m.sh_dc[lane * m.cap + i];
    } else {
      const size_t o = (lane - 3) * m.cap + i;
      v = m.sh_hi32 ? m.sh_hi32[o] : (float)__builtin_bit_cast(_Float16, m.sh_hi16[o]);
    }
    c.sh[i * m.sh_lanes + lane] = v;
  }
}

template <typename T>
__global__ void __launch_bounds__(IO_BLOCK) regrow_kernel(const T* src, T* dst, int lanes, int n, int old_cap, int new_cap) {
  const size_t total = (size_t)lanes * new_cap;
  for (size_t e = grid_index(); e < total; e += grid_stride()) {
    const size_t lane = e / (size_t)new_cap, i = e - lane * (size_t)new_cap;
    dst[e] = (src && i < (size_t)n) ? src[lane * old_cap + i] : T(0);
  }
}

__global__ void __launch_bounds__(IO_BLOCK) set_floor_kernel(float* lscale, const float* floor_, int n) {
  for (size_t i = grid_index(); i < (size_t)n; i += grid_stride()) lscale[4 * i + 3] = floor_[i];
}

dim3 grid_for(size_t work) {
  const size_t blocks = (work + IO_BLOCK - 1) / IO_BLOCK;
  return dim3((unsigned)(blocks < 8192 ? (blocks ? blocks : 1) : 8192));
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" int b2c_hip_model_scatter(const b2c_cloud_dev* src, const b2c_model_dev* dst, hipStream_t stream) {
  if (dst->n < 0 || dst->n > dst->cap || dst->sh_lanes < 3) return (int)hipErrorInvalidValue;
  if (dst->n == 0) return 0;
  if (dst->sh_lanes > 3 && !dst->sh_hi32 && !dst->sh_hi16) return (int)hipErrorInvalidValue;
  scatter_params_kernel<<<grid_for((size_t)dst->n), dim3(IO_BLOCK), 0, stream>>>(*src, *dst);
  scatter_sh_kernel<<<grid_for((size_t)dst->n * dst->sh_lanes), dim3(IO_BLOCK), 0, stream>>>(*src, *dst);
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_model_gather(const b2c_model_dev* src, const b2c_cloud_dev* dst, hipStream_t stream) {
  if (src->n < 0 || src->n > src->cap || src->sh_lanes < 3) return (int)hipErrorInvalidValue;
  if (src->n == 0) return 0;
  if (src->sh_lanes > 3 && !src->sh_hi32 && !src->sh_hi16) return (int)hipErrorInvalidValue;
  gather_params_kernel<<<grid_for((size_t)src->n), dim3(IO_BLOCK), 0, stream>>>(*src, *dst);
  gather_sh_kernel<<<grid_for((size_t)src->n * src->sh_lanes), dim3(IO_BLOCK), 0, stream>>>(*src, *dst);
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_planar_regrow(const void* src, void* dst, int elem_bytes, int lanes, int n, int old_cap,
                                     int new_cap, hipStream_t stream) {
  if (lanes <= 0) return 0;
  if (!dst || n < 0 || new_cap < n || (src && old_cap < n)) return (int)hipErrorInvalidValue;
  const dim3 grid = grid_for((size_t)lanes * new_cap);
  if (elem_bytes == 4)
    regrow_kernel<uint32_t><<<grid, dim3(IO_BLOCK), 0, stream>>>(static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst),
                                                                 lanes, n, old_cap, new_cap);
  else if (elem_bytes == 2)
    regrow_kernel<uint16_t><<<grid, dim3(IO_BLOCK), 0, stream>>>(static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst),
                                                                 lanes, n, old_cap, new_cap);
  else
    return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_model_set_floor(float* lscale, const float* floor_, int n, hipStream_t stream) {
  if (n <= 0) return 0;
  set_floor_kernel<<<grid_for((size_t)n), dim3(IO_BLOCK), 0, stream>>>(lscale, floor_, n);
  return (int)hipGetLastError();
}
