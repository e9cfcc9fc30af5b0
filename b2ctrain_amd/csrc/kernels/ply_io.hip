// PLY vertex rows <-> model layout on the device (replaces the per-row decode and encode loops of
// src/ply.cpp:127-160 and 188-224). A file's binary rows are copied to the device in chunks and decoded
// straight into the model's float4 / planar-SH arrays; a save encodes the model into write_ply's row layout
// on the device and the host only writes the bytes. Both are byte work bound by HBM (and, end to end, by
// the host link and the disk): one wave per 64 rows, the rows staged through LDS with coalesced 32-bit
// loads whatever the row stride, one lane per row for the decode, one lane per output float for the
// encode.
#include <hip/hip_runtime.h>

#include "b2c_kernels.h"

namespace b2c {
namespace dev {
namespace {

constexpr int DEC_ROWS = 64;
constexpr float SH_C0F = 0.28209479177387814f;

__device__ __forceinline__ uint32_t bytes_u32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// One property value widened to double, as the reference's reader holds every value (ply.cpp:38-49).
__device__ __forceinline__ double prop_value(const uint8_t* p, int type) {
  switch (type) {
    case B2C_PLY_F32: return (double)__uint_as_float(bytes_u32(p));
    case B2C_PLY_F64: {
      const uint64_t lo = bytes_u32(p), hi = bytes_u32(p + 4);
      return __longlong_as_double((long long)(lo | (hi << 32)));
    }
    case B2C_PLY_U8: return (double)p[0];
    case B2C_PLY_I8: return (double)(int8_t)p[0];
    case B2C_PLY_U16: return (double)(uint16_t)(p[0] | (p[1] << 8));
    case B2C_PLY_I16: return (double)(int16_t)(uint16_t)(p[0] | (p[1] << 8));
    case B2C_PLY_U32: return (double)bytes_u32(p);
    default: return (double)(int32_t)bytes_u32(p);
  }
}

__global__ void __launch_bounds__(64) ply_decode_kernel(b2c_ply_decode_args a) {
  extern __shared__ uint32_t s_rows[];
  const int r0 = blockIdx.x * DEC_ROWS;
  const int rows = min(DEC_ROWS, a.count - r0);
  if (rows <= 0) return;
  const size_t byte0 = (size_t)r0 * a.row_bytes;
  const size_t w0 = byte0 >> 2, w1 = (byte0 + (size_t)rows * a.row_bytes + 3) >> 2;
  const uint32_t* words = reinterpret_cast<const uint32_t*>(a.rows);
  for (size_t w = w0 + threadIdx.x; w < w1; w += DEC_ROWS) s_rows[w - w0] = words[w];
  __syncthreads();
  const int lane = threadIdx.x;
  if (lane >= rows) return;
  const uint8_t* row = reinterpret_cast<const uint8_t*>(s_rows) + (byte0 & 3) + (size_t)lane * a.row_bytes;
  const size_t i = (size_t)a.first + (size_t)(r0 + lane);
  const auto get = [&](int t, float absent) -> float {
    return a.col[t] < 0 ? absent : (float)prop_value(row + a.col[t], a.type[t]);
  };
  const b2c_model_dev& m = a.model;
  reinterpret_cast<float4*>(m.pos_op)[i] =
      make_float4(get(B2C_PLY_T_POS, 0.f), get(B2C_PLY_T_POS + 1, 0.f), get(B2C_PLY_T_POS + 2, 0.f),
                  get(B2C_PLY_T_OPACITY, 0.f));
  reinterpret_cast<float4*>(m.quat)[i] = make_float4(get(B2C_PLY_T_ROT, 1.f), get(B2C_PLY_T_ROT + 1, 0.f),
                                                     get(B2C_PLY_T_ROT + 2, 0.f), get(B2C_PLY_T_ROT + 3, 0.f));
  reinterpret_cast<float4*>(m.lscale)[i] = make_float4(get(B2C_PLY_T_SCALE, 0.f), get(B2C_PLY_T_SCALE + 1, 0.f),
                                                       get(B2C_PLY_T_SCALE + 2, 0.f), 0.f);
  for (int ch = 0; ch < 3; ch++) {
    float dc = get(B2C_PLY_T_DC + ch, 0.f);
    if (a.rgb_dc && a.col[B2C_PLY_T_RGB + ch] >= 0) {
#pragma clang fp contract(off)
      const double v = prop_value(row + a.col[B2C_PLY_T_RGB + ch], a.type[B2C_PLY_T_RGB + ch]);
      dc = (float)((v * a.rgb_scale - 0.5) / (double)SH_C0F);
    }
    m.sh_dc[(size_t)ch * m.cap + i] = dc;
  }
  // f_rest_j with j = ch (K - 1) + (k - 1) is coefficient k of channel ch: model lane 3k + ch, planar
  // band lane 3k + ch - 3
  const int bands = m.sh_lanes / 3 - 1;
  for (int ch = 0; ch < 3; ch++)
    for (int k = 1; k <= bands; k++) {
      const float v = get(B2C_PLY_T_REST + ch * bands + (k - 1), 0.f);
      const size_t o = (size_t)(3 * k + ch - 3) * m.cap + i;
      if (m.sh_hi32) m.sh_hi32[o] = v;
      else m.sh_hi16[o] = __builtin_bit_cast(uint16_t, (_Float16)v);  // round to nearest even, as an upload
    }
}

__global__ void __launch_bounds__(256) ply_encode_kernel(b2c_ply_encode_args a) {
#pragma clang fp contract(off)
  const size_t total = (size_t)a.count * a.row_floats;
  const b2c_model_dev& m = a.model;
  const int bands = m.sh_lanes / 3 - 1;
  const int rest = 3 * bands;
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
    const size_t r = e / (size_t)a.row_floats;
    int c = (int)(e - r * (size_t)a.row_floats);
    const size_t i = (size_t)a.first + r;
    float v = 0.f;
    if (c < 7) {
      const float4 p = reinterpret_cast<const float4*>(m.pos_op)[i];
      const float4 s = reinterpret_cast<const float4*>(m.lscale)[i];
      const float f[7] = {p.x, p.y, p.z, s.x, s.y, s.z, p.w};
#pragma unroll
      for (int k = 0; k < 7; k++)
        if (c == k) v = f[k];
    } else if (c < 11) {  // the unit quaternion: the norm as ((w^2 + x^2) + y^2) + z^2, IEEE sqrt and divide
      const float4 q = reinterpret_cast<const float4*>(m.quat)[i];
      float qw = q.x, qx = q.y, qy = q.z, qz = q.w;
      float qn = sqrtf(((qw * qw + qx * qx) + qy * qy) + qz * qz);
      if (!(qn > 1e-32f)) {
        qn = 1.f;
        qw = 1.f;
        qx = qy = qz = 0.f;
      }
      const float comp = c == 7 ? qw : (c == 8 ? qx : (c == 9 ? qy : qz));
      v = comp / qn;
    } else if (c < 14) {
      v = m.sh_dc[(size_t)(c - 11) * m.cap + i];
    } else if (c < 14 + rest) {
      const int j = c - 14, ch = j / bands, k = j - ch * bands + 1;
      const size_t o = (size_t)(3 * k + ch - 3) * m.cap + i;
      v = m.sh_hi32 ? m.sh_hi32[o] : (float)__builtin_bit_cast(_Float16, m.sh_hi16[o]);
    } else {
      c -= 14 + rest;
      const float* blocks[6] = {a.evidence, a.labels, a.fill, a.gate, a.gate_s, a.open};
      const int widths[6] = {7, 2, 1, 2, 1, 4};
#pragma unroll
      for (int b = 0; b < 6; b++) {
        if (!blocks[b]) continue;
        if (c >= 0 && c < widths[b]) v = blocks[b][i * widths[b] + c];
        c -= widths[b];
      }
    }
    a.rows[e] = v;
  }
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" int b2c_hip_ply_decode(const b2c_ply_decode_args* a, hipStream_t stream) {
  if (a->count <= 0) return 0;
  if (!a->rows || a->row_bytes == 0 || a->first < 0 || a->first + a->count > a->model.n ||
      a->model.sh_lanes < 3 || a->model.sh_lanes > 75 || a->model.sh_lanes % 3)
    return (int)hipErrorInvalidValue;
  if (a->model.sh_lanes > 3 && !a->model.sh_hi32 && !a->model.sh_hi16) return (int)hipErrorInvalidValue;
  for (int t = 0; t < B2C_PLY_TARGETS; t++)
    if (a->col[t] >= 0 && ((uint32_t)a->col[t] >= a->row_bytes || a->type[t] > B2C_PLY_I32)) return (int)hipErrorInvalidValue;
  const size_t lds = ((size_t)DEC_ROWS * a->row_bytes + 8 + 3) & ~(size_t)3;
  if (lds > 64 * 1024) return (int)hipErrorInvalidValue;  // rows over 1 KiB: not a splat layout
  ply_decode_kernel<<<dim3((a->count + DEC_ROWS - 1) / DEC_ROWS), dim3(DEC_ROWS), lds, stream>>>(*a);
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_ply_encode(const b2c_ply_encode_args* a, hipStream_t stream) {
  if (a->count <= 0) return 0;
  const int rest = a->model.sh_lanes - 3;
  int want = 14 + rest;
  const float* blocks[6] = {a->evidence, a->labels, a->fill, a->gate, a->gate_s, a->open};
  const int widths[6] = {7, 2, 1, 2, 1, 4};
  for (int b = 0; b < 6; b++) want += blocks[b] ? widths[b] : 0;
  if (!a->rows || a->row_floats != want || a->first < 0 || a->first + a->count > a->model.n ||
      a->model.sh_lanes < 3 || a->model.sh_lanes > 75 || a->model.sh_lanes % 3)
    return (int)hipErrorInvalidValue;
  const size_t total = (size_t)a->count * a->row_floats;
  const int grid = (int)std::min<size_t>((total + 255) / 256, 65536);
  ply_encode_kernel<<<dim3(grid), dim3(256), 0, stream>>>(*a);
  return (int)hipGetLastError();
}
