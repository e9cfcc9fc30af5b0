// Device-side math shared by the HIP kernels (gfx950). Everything that decides which tiles a splat
// touches (projection, tile test, bounding box) is evaluated without FMA contraction, with IEEE
// division and square root, and with exp/log from the Cephes single-precision method, so that the
// tile and key lists are reproducible bit for bit on any IEEE machine that evaluates the same
// operation sequence.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace b2c {
namespace dev {

constexpr int RT_W = 8;                      // raster tile edge (src/gpu/util.cuh:19)
constexpr int RT_PX = RT_W * RT_W;
constexpr float ALPHA_CUTOFF = 1.0f / 255.0f;  // splat_math.cuh:7
constexpr float T_CUTOFF = 1e-4f;              // splat_math.cuh:8
constexpr float ALPHA_MAX = 0.999f;            // splat_math.cuh:9
constexpr int GRAD_LANES = 13;                 // splat_math.cuh:10: xy(2) conic(3) rgb(3) opac(1) refine(1) feat(3)
constexpr float SH_C0 = 0.28209479177387814f;

struct Sym2 { float c00, c01, c11; };

// The projected splat's centre, conic and cutoff power from its 64-byte raster record ((mx, my, c00 / 2,
// c01), (c11 / 2, opacity, power, .)): doubling the stored halves restores the conic exactly.
struct SplatRecGeom {
  float mx, my;
  Sym2 conic;
  float power;
};
__device__ __forceinline__ SplatRecGeom splat_rec_geom(const float* raster_rec, uint32_t i) {
  const float4* rec = reinterpret_cast<const float4*>(raster_rec) + (size_t)i * 4;
  const float4 r0 = rec[0], r1 = rec[1];
  return SplatRecGeom{r0.x, r0.y, Sym2{2.f * r0.z, r0.w, 2.f * r1.x}, r1.z};
}

// Cephes expf (S. L. Moshier, Cephes Math Library, single/expf.c): n = round(x / ln2), r = x - n ln2 with
// ln2 split in two constants (Cody-Waite), degree-6 polynomial for e^r, scaled by 2^n. Inputs below -86
// return 0 so no subnormal is produced; above 88 return +inf.
__device__ __forceinline__ float det_expf(float xx) {
#pragma clang fp contract(off)
  float x = xx;
  if (!(x <= 88.0f)) return x != x ? x : __builtin_inff();
  if (x < -86.0f) return 0.0f;
  float t = 1.44269504088896341f * x;
  t = t + 0.5f;
  float z = floorf(t);
  x = x - z * 0.693359375f;
  x = x - z * -2.12194440e-4f;
  int n = (int)z;
  z = x * x;
  float p = 1.9875691500e-4f;
  p = p * x + 1.3981999507e-3f;
  p = p * x + 8.3334519073e-3f;
  p = p * x + 4.1665795894e-2f;
  p = p * x + 1.6666665459e-1f;
  p = p * x + 5.0000001201e-1f;
  p = p * z;
  p = p + x;
  p = p + 1.0f;
  return ldexpf(p, n);
}

// Cephes logf (single/logf.c): x = m 2^e with m in [sqrt(1/2), sqrt(2)), degree-9 polynomial in m - 1.
__device__ __forceinline__ float det_logf(float xx) {
#pragma clang fp contract(off)
  float x = xx;
  if (!(x > 0.0f)) return x == 0.0f ? -__builtin_inff() : __builtin_nanf("");
  if (__builtin_isinf(x)) return x;
  int e;
  x = frexpf(x, &e);
  if (x < 0.707106781186547524f) {
    e -= 1;
    x = x + x;
    x = x - 1.0f;
  } else {
    x = x - 1.0f;
  }
  float z = x * x;
  float y = 7.0376836292e-2f;
  y = y * x - 1.1514610310e-1f;
  y = y * x + 1.1676998740e-1f;
  y = y * x - 1.2420140846e-1f;
  y = y * x + 1.4249322787e-1f;
  y = y * x - 1.6668057665e-1f;
  y = y * x + 2.0000714765e-1f;
  y = y * x - 2.4999993993e-1f;
  y = y * x + 3.3333331174e-1f;
  y = y * x;
  y = y * z;
  float fe = (float)e;
  if (e) y = y + -2.12194440e-4f * fe;
  y = y + -0.5f * z;
  z = x + y;
  if (e) z = z + 0.693359375f * fe;
  return z;
}

// Mahalanobis half-distance of pixel (px, py) to a splat (splat_math.cuh:21-24), uncontracted so the
// forward, the backward and the CPU restatement make identical `sigma <= power` decisions.
__device__ __forceinline__ float calc_sigma(float px, float py, float c00, float c01, float c11, float mx, float my) {
#pragma clang fp contract(off)
  float dx = px - mx, dy = py - my;
  return 0.5f * (c00 * dx * dx + c11 * dy * dy) + c01 * dx * dy;
}

// Ellipse-vs-rectangle test (StopThePop / brush `will_primitive_contribute`, splat_math.cuh:27-41): the
// rectangle point nearest the centre along each edge in the conic metric must satisfy sigma <= power.
__device__ __forceinline__ bool tile_hit(float rmin_x, float rmin_y, float rmax_x, float rmax_y, float mx, float my,
                                         Sym2 conic, float power) {
#pragma clang fp contract(off)
  bool x_left = mx < rmin_x, x_right = mx > rmax_x, in_x = !(x_left || x_right);
  bool y_above = my < rmin_y, y_below = my > rmax_y, in_y = !(y_above || y_below);
  if (in_x && in_y) return true;
  float corner_x = x_left ? rmin_x : rmax_x, corner_y = y_above ? rmin_y : rmax_y;
  float width = rmax_x - rmin_x, height = rmax_y - rmin_y;
  float dxf = x_left ? width : -width, dyf = y_above ? height : -height;
  float diff_x = mx - corner_x, diff_y = my - corner_y;
  float tx_raw = (dxf * conic.c00 * diff_x + dxf * conic.c01 * diff_y) / (dxf * conic.c00 * dxf);
  float ty_raw = (dyf * conic.c01 * diff_x + dyf * conic.c11 * diff_y) / (dyf * conic.c11 * dyf);
  float tx = in_y ? 0.f : fminf(fmaxf(tx_raw, 0.f), 1.f);
  float ty = in_x ? 0.f : fminf(fmaxf(ty_raw, 0.f), 1.f);
  float px = corner_x + tx * dxf, py = corner_y + ty * dyf;
  return calc_sigma(px, py, conic.c00, conic.c01, conic.c11, mx, my) <= power;
}

struct TileBox { int min_x, min_y, max_x, max_y; };

// Tile-unit bounding box of a splat's extent (splat_math.cuh:43-53).
__device__ __forceinline__ TileBox tile_bbox(float mx, float my, float ex, float ey, int tiles_x, int tiles_y) {
#pragma clang fp contract(off)
  const float tw = (float)RT_W;
  float cx = mx / tw, cy = my / tw, dx = ex / tw, dy = ey / tw;
  TileBox b;
  b.min_x = (int)fminf(fmaxf(cx - dx, 0.f), (float)tiles_x);
  b.min_y = (int)fminf(fmaxf(cy - dy, 0.f), (float)tiles_y);
  b.max_x = (int)fminf(fmaxf(cx + dx + 1.f, 0.f), (float)tiles_x);
  b.max_y = (int)fminf(fmaxf(cy + dy + 1.f, 0.f), (float)tiles_y);
  return b;
}

// Opacity-adaptive extent recomputed from the stored conic and power (binning.cu:78-84).
__device__ __forceinline__ void extent_from_conic(Sym2 conic, float power, float& ex, float& ey) {
#pragma clang fp contract(off)
  float detc = conic.c00 * conic.c11 - conic.c01 * conic.c01;
  float inv_detc = 1.f / detc;
  ex = sqrtf(2.f * power * conic.c11 * inv_detc);
  ey = sqrtf(2.f * power * conic.c00 * inv_detc);
}

// Forward-mode derivative along the three components of a direction: value v and partials (x, y, z).
// sh_basis instantiated on it yields each basis function's gradient with its value, which the projection
// VJP contracts into d(colour)/d(view direction).
struct Dual3 {
  float v, x, y, z;
};
__device__ __forceinline__ Dual3 operator+(Dual3 a, Dual3 b) { return {a.v + b.v, a.x + b.x, a.y + b.y, a.z + b.z}; }
__device__ __forceinline__ Dual3 operator-(Dual3 a, Dual3 b) { return {a.v - b.v, a.x - b.x, a.y - b.y, a.z - b.z}; }
__device__ __forceinline__ Dual3 operator+(Dual3 a, float k) { return {a.v + k, a.x, a.y, a.z}; }
__device__ __forceinline__ Dual3 operator-(Dual3 a, float k) { return {a.v - k, a.x, a.y, a.z}; }
__device__ __forceinline__ Dual3 operator*(float k, Dual3 a) { return {k * a.v, k * a.x, k * a.y, k * a.z}; }
__device__ __forceinline__ Dual3 operator*(Dual3 a, Dual3 b) {
  return {a.v * b.v, a.v * b.x + a.x * b.v, a.v * b.y + a.y * b.v, a.v * b.z + a.z * b.v};
}

// Real SH basis in Sloan order up to degree 4 (the constants and recurrences of splat_math.cuh:122-145)
// into b[0 .. (deg+1)^2). T = float gives the values; T = Dual3 the values and their gradients.
template <int DEG, typename T>
__device__ __forceinline__ void sh_basis(T vx, T vy, T vz, T* b) {
#pragma clang fp contract(off)
  b[0] = T{} + SH_C0;
  if constexpr (DEG >= 1) {
    const float f0a = 0.4886025f;
    b[1] = -f0a * vy; b[2] = f0a * vz; b[3] = -f0a * vx;
    if constexpr (DEG >= 2) {
      T z2 = vz * vz, f0b = -1.0925485f * vz;
      const float f1a = 0.54627424f;
      T fc1 = vx * vx - vy * vy, fs1 = 2.f * vx * vy;
      b[4] = f1a * fs1; b[5] = f0b * vy; b[6] = 0.9461747f * z2 - 0.31539157f; b[7] = f0b * vx; b[8] = f1a * fc1;
      if constexpr (DEG >= 3) {
        T f0c = -2.285229f * z2 + 0.4570458f, f1b = 1.4453057f * vz;
        const float f2a = -0.5900436f;
        T fc2 = vx * fc1 - vy * fs1, fs2 = vx * fs1 + vy * fc1;
        b[9] = f2a * fs2; b[10] = f1b * fs1; b[11] = f0c * vy; b[12] = vz * (1.8658817f * z2 - 1.119529f);
        b[13] = f0c * vx; b[14] = f1b * fc1; b[15] = f2a * fc2;
        if constexpr (DEG >= 4) {
          T f0d = vz * (-4.683326f * z2 + 2.0071396f), f1c = 3.3116114f * z2 - 0.47308735f;
          T f2b = -1.7701308f * vz;
          const float f3a = 0.62583575f;
          T fc3 = vx * fc2 - vy * fs2, fs3 = vx * fs2 + vy * fc2;
          b[16] = f3a * fs3; b[17] = f2b * fs2; b[18] = f1c * fs1; b[19] = f0d * vy;
          b[20] = 1.9843135f * vz * b[12] - 1.0062306f * b[6];
          b[21] = f0d * vx; b[22] = f1c * fc1; b[23] = f2b * fc2; b[24] = f3a * fc3;
        }
      }
    }
  }
}

// Planar SH storage (util.cuh:129-164): lanes 0..2 (DC) fp32 in dc[lane*stride + i]; higher lanes fp32 in
// hi32[(lane-3)*stride + i] or fp16 in hi16 (exact widening on load).
struct ShView {
  const float* dc;
  const _Float16* hi16;
  const float* hi32;
  size_t stride;
  __device__ __forceinline__ float get(int lane, int i) const {
    if (lane < 3) return dc[(size_t)lane * stride + i];
    size_t o = (size_t)(lane - 3) * stride + i;
    return hi32 ? hi32[o] : (float)hi16[o];
  }
  // All 3 (DEG + 1)^2 coefficients of splat i, issued back to back (one memory round trip); lanes beyond
  // the active degree are loaded too and weighted by zero by the caller. HALF selects the band storage
  // at compile time: with both forms behind a runtime branch, the fp16 form was compiled as one load,
  // wait and convert per coefficient. The fp16 form loads every raw half first and converts afterwards.
  template <int DEG, bool HALF>
  __device__ __forceinline__ void load_all(int i, float* c) const {
    constexpr int L = 3 * (DEG + 1) * (DEG + 1);
#pragma unroll
    for (int k = 0; k < 3; k++) c[k] = dc[(size_t)k * stride + i];
    if constexpr (HALF) {
      const uint16_t* h = reinterpret_cast<const uint16_t*>(hi16);
      uint32_t raw[L > 3 ? L - 3 : 1];
#pragma unroll
      for (int k = 3; k < L; k++) raw[k - 3] = h[(size_t)(k - 3) * stride + i];
#pragma unroll
      for (int k = 3; k < L; k++) c[k] = (float)__builtin_bit_cast(_Float16, (uint16_t)raw[k - 3]);
    } else {
#pragma unroll
      for (int k = 3; k < L; k++) c[k] = hi32[(size_t)(k - 3) * stride + i];
    }
  }
  // fp32 bands, with the storage chosen at run time (hi16 as the fallback). The projection VJP measured
  // 4 us faster with this form for fp32 bands than with load_all<DEG, false> (the compiler schedules the
  // surrounding code differently); the fp16 bands use load_all<DEG, true>.
  template <int DEG>
  __device__ __forceinline__ void load_all_either(int i, float* c) const {
    constexpr int L = 3 * (DEG + 1) * (DEG + 1);
#pragma unroll
    for (int k = 0; k < 3; k++) c[k] = dc[(size_t)k * stride + i];
    if (hi32) {
#pragma unroll
      for (int k = 3; k < L; k++) c[k] = hi32[(size_t)(k - 3) * stride + i];
    } else {
#pragma unroll
      for (int k = 3; k < L; k++) c[k] = (float)hi16[(size_t)(k - 3) * stride + i];
    }
  }
};

// Row-major 3x3 helpers and the quaternion rotation (util.cuh:218-243).
struct Mat3 { float m[9]; };

// The axis of the smallest of three log scales (the first of equal ones), as three exclusive flags, so a
// column of a matrix is picked with selects: a runtime index into a register array would move the array
// (and the struct holding it) to scratch memory.
struct AxisPick {
  bool x, y, z;
  __device__ __forceinline__ float of(float a, float b, float c) const { return x ? a : (y ? b : c); }
};
__device__ __forceinline__ AxisPick smallest_axis(float lx, float ly, float lz) {
  const bool x = lx <= ly && lx <= lz;
  const bool y = !x && ly <= lz;
  return AxisPick{x, y, !x && !y};
}

__device__ __forceinline__ Mat3 mat3_mul(const Mat3& A, const Mat3& B) {
#pragma clang fp contract(off)
  Mat3 C;
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int j = 0; j < 3; j++) C.m[i * 3 + j] = A.m[i * 3] * B.m[j] + A.m[i * 3 + 1] * B.m[3 + j] + A.m[i * 3 + 2] * B.m[6 + j];
  return C;
}

// Rotation matrix from a normalised (w, x, y, z) quaternion.
__device__ __forceinline__ Mat3 quat_to_mat(float w, float x, float y, float z) {
#pragma clang fp contract(off)
  float x2 = x * x, y2 = y * y, z2 = z * z, xy = x * y, xz = x * z, yz = y * z, wx = w * x, wy = w * y, wz = w * z;
  Mat3 R;
  R.m[0] = 1.f - 2.f * (y2 + z2); R.m[1] = 2.f * (xy - wz);       R.m[2] = 2.f * (xz + wy);
  R.m[3] = 2.f * (xy + wz);       R.m[4] = 1.f - 2.f * (x2 + z2); R.m[5] = 2.f * (yz - wx);
  R.m[6] = 2.f * (xz - wy);       R.m[7] = 2.f * (yz + wx);       R.m[8] = 1.f - 2.f * (x2 + y2);
  return R;
}

__device__ __forceinline__ bool finite3(float a, float b, float c) {
  return __builtin_isfinite(a) && __builtin_isfinite(b) && __builtin_isfinite(c);
}

// Wave-level helpers (wave64).
__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }
__device__ __forceinline__ int lane_id() { return __lane_id(); }
__device__ __forceinline__ uint32_t popc64(uint64_t m) { return (uint32_t)__popcll(m); }
// Number of set bits of m strictly below this lane.
__device__ __forceinline__ uint32_t mbcnt64(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

}  // namespace dev
}  // namespace b2c
