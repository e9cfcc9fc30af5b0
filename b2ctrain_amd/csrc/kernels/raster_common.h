// Helpers shared by the forward and backward raster kernels.
#pragma once
#include "device_math.h"

namespace b2c {
namespace dev {

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X (workgroup b runs on XCD b % 8), and
// each XCD has its own L2. Give every XCD a contiguous run of tiles (rows of the image) so splats shared
// by neighbouring tiles are fetched once per XCD rather than once per tile. The grid has 8 * per blocks;
// blocks mapped past n_tiles return.
constexpr int NUM_XCD = 8;
__host__ __device__ inline int xcd_tiles_per(int n_tiles) { return (n_tiles + NUM_XCD - 1) / NUM_XCD; }
__device__ __forceinline__ int xcd_tile(int block, int n_tiles) {
  const int per = xcd_tiles_per(n_tiles);
  return (block % NUM_XCD) * per + block / NUM_XCD;
}

constexpr float LOG2E = 1.44269504088896341f;

// A fragment's Mahalanobis half-distance sigma = a dx^2 + b dx dy + c dy^2 (a = c00 / 2, b = c01,
// c = c11 / 2; d = pixel centre - splat centre), evaluated as dx (a dx + b dy) + (c dy) dy with two fused
// multiply-adds. The forward, both backward modes and the CPU restatement (oracle/b2c_oracle.c) evaluate
// exactly this sequence, so every fragment's cutoff decision 0 <= sigma <= power agrees everywhere. lin =
// a dx + b dy and cdy = c dy are kept for the backward: d sigma / d dx = lin + a dx, d sigma / d dy =
// b dx + 2 cdy.
struct FragGeom {
  float dx, dy, lin, cdy, sigma;
};

__device__ __forceinline__ FragGeom frag_geom(float mx, float my, float a, float b, float c, float pcx, float pcy) {
#pragma clang fp contract(off)
  FragGeom f;
  f.dx = pcx - mx;
  f.dy = pcy - my;
  f.lin = __builtin_fmaf(a, f.dx, b * f.dy);
  f.cdy = c * f.dy;
  f.sigma = __builtin_fmaf(f.dx, f.lin, f.cdy * f.dy);
  return f;
}

// A fragment's sigma as a quadratic in the pixel centre's offset (u, v) from its tile's centre: with
// (mxr, myr) the splat centre relative to the tile centre and a = c00 / 2, b = c01, c = c11 / 2,
//   sigma = a (u - mxr)^2 + b (u - mxr)(v - myr) + c (v - myr)^2 = a uu + b uv + c vv + D u + E v + F,
// D = -(2a mxr + b myr), E = -(b mxr + 2c myr) and F the sigma at the tile centre (frag_geom's arithmetic at
// dx = -mxr, dy = -myr). D, E and F are formed once per (splat, tile); a pixel then costs five fused
// multiply-adds (u, v, uu, uv, vv are exact: u, v are +-0.5 .. +-3.5). Every kernel that tests or replays a
// fragment (forward, both backward modes, evidence, depth probe) and the CPU restatement evaluate exactly
// these operations, so all of them agree on which fragments pass. Rounding can leave sigma slightly
// negative where the exact value is 0 (a pixel centre on the splat centre): a fragment passes when
// sigma <= power, which keeps it, as the exact value would.
struct PixelPoly {
  float u, v, uu, uv, vv;
};

__device__ __forceinline__ PixelPoly pixel_poly(float u, float v) { return PixelPoly{u, v, u * u, u * v, v * v}; }

__device__ __forceinline__ float3 sigma_coefs(float mx, float my, float a, float b, float c, float tcx, float tcy) {
#pragma clang fp contract(off)
  const float mxr = mx - tcx, myr = my - tcy;
  const float D = -__builtin_fmaf(a + a, mxr, b * myr);
  const float E = -__builtin_fmaf(b, mxr, (c + c) * myr);
  const float F = __builtin_fmaf(mxr, __builtin_fmaf(a, mxr, b * myr), (c * myr) * myr);
  return make_float3(D, E, F);
}

__device__ __forceinline__ float poly_sigma(float a, float b, float c, float D, float E, float F, const PixelPoly& pp) {
  return __builtin_fmaf(a, pp.uu, __builtin_fmaf(b, pp.uv, __builtin_fmaf(c, pp.vv,
                                                 __builtin_fmaf(D, pp.u, __builtin_fmaf(E, pp.v, F)))));
}

// e^-sigma on the hardware exponential (v_exp_f32 is 2^x): the Gaussian factor of the opacity gradient.
__device__ __forceinline__ float gauss_weight(float sigma) { return __builtin_amdgcn_exp2f(sigma * -LOG2E); }

// log2 of a splat's opacity, precomputed once per splat for fragment_alpha.
__device__ __forceinline__ float log2_opacity(float opacity) { return __builtin_amdgcn_logf(opacity); }

// Unclamped alpha of a fragment, opacity * e^-sigma, as 2^(log2(opacity) - sigma log2 e): one fma and one
// v_exp_f32. Forward and backward must use this same expression: the backward recovers the forward's
// transmittance by dividing by (1 - alpha).
__device__ __forceinline__ float fragment_alpha(float sigma, float log2_op) {
  return __builtin_amdgcn_exp2f(__builtin_fmaf(sigma, -LOG2E, log2_op));
}

// Hollow loss (splat_math.cuh:14-17): a fragment at camera depth z behind a pixel's reference surface
// z_ref is penalised by h = clamp((z - z_ref - margin) / margin, 0, 1) (margin floored at 1e-4), and 0 when
// that quotient is not finite (no surface: z_ref = +inf). Evaluated as (z - (z_ref + margin)) / margin with
// the reciprocal taken once per pixel: the same value up to rounding, and the same bits in the forward,
// both backward modes and the CPU restatement.
struct HollowRef {
  float zm, inv_m;  // z_ref + margin, 1 / max(margin, 1e-4)
};
__device__ __forceinline__ HollowRef hollow_ref(float z_ref, float margin) {
  return HollowRef{z_ref + margin, 1.f / fmaxf(margin, 1e-4f)};
}
__device__ __forceinline__ float hollow_h(float z, HollowRef h) {
  const float d = (z - h.zm) * h.inv_m;
  return __builtin_isfinite(d) ? fminf(fmaxf(d, 0.f), 1.f) : 0.f;
}

// Quadrant culling. A raster wave covers an 8x8 tile as four 4x4 quadrants of 16 lanes; bit q = 2 qy + qx
// of the mask is set when the splat's ellipse {sigma <= power} can reach a pixel centre of quadrant (qx, qy).
// sigma = ah dx^2 + ch dy^2 + b dx dy (ah = c00 / 2, ch = c11 / 2) is convex, so its minimum over the box
// spanned by the quadrant's pixel centres is 0 when the centre lies inside and is otherwise attained on an
// edge that the centre lies beyond (sigma falls along the segment from the minimising point to the centre,
// so that segment leaves the box there): the left edge only if the centre is left of it, and so on - at most
// one vertical and one horizontal edge, where the minimum is a clamped one-dimensional one. The box minimum is at most sigma at any pixel centre
// of the quadrant; it is compared with power less a margin of 1e-5 of the terms' magnitude, far above the
// rounding of this evaluation. The per-pixel sigma (poly_sigma, the quadratic about the tile centre) rounds
// on the scale of its own terms, which near the splat centre can be much larger than sigma's: power is
// raised by 1e-5 of the sum of their magnitudes over the tile (the magnitudes of F, 3.5 |D|, 3.5 |E| and
// 12.25 (a + |b| + c), with F, D, E bounded term by term). So a quadrant is dropped only when no pixel of it
// can pass the cutoff. A fragment in a dropped quadrant would have had alpha = 0, so culling changes no
// result. Degenerate conics and a non-finite centre keep every quadrant. (x0, y0) is the tile's first
// pixel centre.
__device__ __forceinline__ float edge_sigma_lb(float ah, float b, float ch, float dx, float dy) {
  const float t1 = ah * dx * dx, t2 = ch * dy * dy, t3 = b * dx * dy;
  return (t1 + t2 + t3) - 1e-5f * (fabsf(t1) + fabsf(t2) + fabsf(t3));
}

__device__ __forceinline__ uint32_t quadrant_mask(float mx, float my, float ah, float b, float ch, float power,
                                                  float x0, float y0) {
  if (!(ah > 0.f && ch > 0.f) || !(mx - mx == 0.f) || !(my - my == 0.f)) return 0xFu;
  const float ky = -b / (2.f * ch), kx = -b / (2.f * ah);  // minimising dy for a given dx, and dx for dy
  const float mxr = fabsf(mx - (x0 + 3.5f)), myr = fabsf(my - (y0 + 3.5f)), bb = fabsf(b);
  const float scale = ((ah * mxr + bb * myr) * mxr + ch * myr * myr) +
                      3.5f * ((2.f * ah + bb) * mxr + (bb + 2.f * ch) * myr) + 12.25f * (ah + bb + ch);
  const float pw = power + 1e-5f * scale;
  const float ex[4] = {x0 - mx, x0 + 3.f - mx, x0 + 4.f - mx, x0 + 7.f - mx};
  const float ey[4] = {y0 - my, y0 + 3.f - my, y0 + 4.f - my, y0 + 7.f - my};
  uint32_t mask = 0;
#pragma unroll
  for (int qy = 0; qy < 2; qy++) {
#pragma unroll
    for (int qx = 0; qx < 2; qx++) {
      const float xlo = ex[2 * qx], xhi = ex[2 * qx + 1], ylo = ey[2 * qy], yhi = ey[2 * qy + 1];
      // the centre is left of the box when xlo > 0, right of it when xhi < 0 (above / below likewise)
      const bool fv = (xlo > 0.f) | (xhi < 0.f), fh = (ylo > 0.f) | (yhi < 0.f);
      const float xe = xlo > 0.f ? xlo : xhi, ye = ylo > 0.f ? ylo : yhi;
      const float mv = edge_sigma_lb(ah, b, ch, xe, fminf(fmaxf(ky * xe, ylo), yhi));
      const float mh = edge_sigma_lb(ah, b, ch, fminf(fmaxf(kx * ye, xlo), xhi), ye);
      // inside: neither edge faces the centre; a NaN edge minimum keeps the quadrant (bitwise: no branches)
      const bool reach = (!fv & !fh) | (fv & !(mv > pw)) | (fh & !(mh > pw));
      mask |= reach ? 1u << (2 * qy + qx) : 0u;
    }
  }
  return mask;
}

// DPP controls (GCN/CDNA): row_shr:n = 0x110 + n, row_ror:n = 0x120 + n, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143, wave_shl:1 = 0x130, wave_shr:1 = 0x138. Lanes whose source is outside the row mask or
// the wave get `fill`.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x, uint32_t fill) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)fill, (int)x, CTRL, ROW_MASK, 0xF, false);
}

constexpr uint32_t NO_RUN = 0xFFFFFFFFu;  // the run id of a lane outside every run

// One Hillis-Steele step of a segmented inclusive scan across the wave: add the partial of the DPP source
// lane when it lies in the same run (runs are contiguous, so equal ids at both ends mean no run boundary in
// between). Each value takes one v_fmac_f32 whose first operand is read through the DPP shift: v += m * v[src],
// with m = 1 when the source lane lies in the same run (and, for the row broadcasts, in a row the step
// feeds) and 0 otherwise; a lane whose source is outside its row or the wave reads 0 (bound_ctrl). Adding
// m * t with m in {0, 1} rounds exactly as the plain sum does. One asm block holds the step's values in a
// fixed order, so a value's DPP read comes at least NV - 1 instructions after the previous step wrote it;
// the leading s_nop gives the two wait states a DPP read needs after a VALU write of its source for the
// first step.
#define B2C_FD(i, C) "v_fmac_f32_dpp %" #i ", %" #i ", %[m] " C " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
#define B2C_FD3(C) B2C_FD(0, C) B2C_FD(1, C) B2C_FD(2, C)
#define B2C_FD11(C) \
  B2C_FD3(C) B2C_FD(3, C) B2C_FD(4, C) B2C_FD(5, C) B2C_FD(6, C) B2C_FD(7, C) B2C_FD(8, C) B2C_FD(9, C) B2C_FD(10, C)
#define B2C_FD14(C) B2C_FD11(C) B2C_FD(11, C) B2C_FD(12, C) B2C_FD(13, C)
#define B2C_OP3(v) "+v"(v[0]), "+v"(v[1]), "+v"(v[2])
#define B2C_OP11(v) \
  B2C_OP3(v), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10])
#define B2C_OP14(v) B2C_OP11(v), "+v"(v[11]), "+v"(v[12]), "+v"(v[13])
#define B2C_SEG_STEP(C)                                                                      \
  do {                                                                                       \
    if constexpr (NV == 3)                                                                   \
      asm("s_nop 1\n\t" B2C_FD3(C) : B2C_OP3(v) : [m] "v"(m));                               \
    else if constexpr (NV == 11)                                                             \
      asm("s_nop 1\n\t" B2C_FD11(C) : B2C_OP11(v) : [m] "v"(m));                             \
    else                                                                                     \
      asm("s_nop 1\n\t" B2C_FD14(C) : B2C_OP14(v) : [m] "v"(m));                             \
  } while (0)

// m for one step: 1 where the DPP source lane holds the same run id (and the lane lies in a row the step
// feeds), else 0.
template <int CTRL>
__device__ __forceinline__ float seg_scan_m(uint32_t id, bool row_ok) {
  const uint32_t src = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)id, CTRL, 0xF, 0xF, true);
  return (row_ok && src == id) ? 1.f : 0.f;
}

template <int NV>
__device__ __forceinline__ void seg_scan(uint32_t id, float (&v)[NV]) {
  static_assert(NV == 3 || NV == 11 || NV == 14, "the scan's asm steps cover 3, 11 and 14 values");
  const int lane = (int)__lane_id();
  float m;
  m = seg_scan_m<0x111>(id, true);  // row_shr:1
  B2C_SEG_STEP("row_shr:1");
  m = seg_scan_m<0x112>(id, true);  // row_shr:2
  B2C_SEG_STEP("row_shr:2");
  m = seg_scan_m<0x114>(id, true);  // row_shr:4
  B2C_SEG_STEP("row_shr:4");
  m = seg_scan_m<0x118>(id, true);  // row_shr:8
  B2C_SEG_STEP("row_shr:8");
  m = seg_scan_m<0x142>(id, (lane & 16) != 0);  // row_bcast:15 into rows 1 and 3
  B2C_SEG_STEP("row_bcast:15");
  m = seg_scan_m<0x143>(id, (lane & 32) != 0);  // row_bcast:31 into rows 2 and 3
  B2C_SEG_STEP("row_bcast:31");
}
#undef B2C_SEG_STEP
#undef B2C_OP14
#undef B2C_OP11
#undef B2C_OP3
#undef B2C_FD14
#undef B2C_FD11
#undef B2C_FD3
#undef B2C_FD

}  // namespace dev
}  // namespace b2c
