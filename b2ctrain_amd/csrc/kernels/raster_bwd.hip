// Backward through compositing: per-pixel reverse replay from the shrunk range end (the transmittance
// recovered as T / (1 - alpha), the colour behind carried as one scalar contracted with v_rgb), then a
// per-splat reduction of the fragment gradients over the tile's 64 pixels into v_splat[n][13].
//
// mode 0 (replaces raster_bwd_kernel, src/gpu/raster_bwd.cu:10-156): per-fragment gradient lanes summed over
//   the wave by shuffles, fp32 throughout. The correctness anchor.
// mode 1 (replaces raster_bwd_tc_kernel, src/gpu/raster_bwd_tc.cu:29-225): each lane writes four scalars
//   per fragment (vis, v_alpha*gauss, v_sigma, refine) for a group of 16 splats; the reduction over pixels
//   is the product basis^T (16 x 64 px) * S (64 px x 16 splats) on v_mfma_f32_16x16x32_f16, with both
//   operands split hi/lo in fp16 (lo scaled by 2^11 and accumulated separately in fp32), which keeps ~22
//   bits of the fp32 inputs. The basis is [v_rgb, v_feat, 1, u, v, u^2, uv, v^2] in tile-centred pixel
//   coordinates (u, v and their products are exact in fp16); conic and mean gradients come from the
//   moments of v_sigma about the splat centre.
#include "b2c_kernels.h"
#include "raster_common.h"

namespace b2c {
namespace dev {
namespace {

constexpr float R_SCALE = 1.f / 64.f;  // refine statistic pre-scale (raster_bwd_tc.cu:17)
constexpr float LO_SCALE = 2048.f;     // 2^11: lo parts live in the normal fp16 range

struct PixelState {
  bool inside;
  float pcx, pcy;
  float T, inv_final_a, v_o_w;
  float4 vo;
  uint32_t last;
  float4 vf;      // dL/d(feature lanes) (FEAT)
  HollowRef href;  // the pixel's reference surface (HOLLOW)
};

template <bool FEAT, bool HOLLOW>
__device__ __forceinline__ PixelState load_pixel(const b2c_raster_bwd_args& a, int px, int py, uint32_t range_x,
                                                 const uint32_t* last_idx) {
  PixelState s;
  s.inside = px < a.W && py < a.H;
  s.pcx = px + 0.5f;
  s.pcy = py + 0.5f;
  s.T = 0.f;
  s.last = range_x;
  s.vo = make_float4(0.f, 0.f, 0.f, 0.f);
  s.vf = make_float4(0.f, 0.f, 0.f, 0.f);
  s.v_o_w = 0.f;
  float final_a = 0.f, z_ref = __builtin_inff();
  if (s.inside) {
    const int pix = py * a.W + px;
    final_a = reinterpret_cast<const float4*>(a.out_rgba)[pix].w;
    s.T = reinterpret_cast<const float4*>(a.out_feat)[pix].w;
    s.last = last_idx[pix];
    s.vo = reinterpret_cast<const float4*>(a.v_out)[pix];
    if constexpr (FEAT) s.vf = reinterpret_cast<const float4*>(a.v_feat)[pix];
    if constexpr (HOLLOW) z_ref = a.hollow_z[pix];
    s.v_o_w = (s.vo.w - (a.bg[0] * s.vo.x + a.bg[1] * s.vo.y + a.bg[2] * s.vo.z)) * s.T;
  }
  s.inv_final_a = 1.f / fmaxf(final_a, 1e-5f);
  s.href = hollow_ref(z_ref, a.hollow_margin);
  return s;
}

// ------------------------------------------------------------------------------------------------------
// mode 0: the fp32 anchor
// ------------------------------------------------------------------------------------------------------
// The replay walks each pixel's list back to front carrying its transmittance T (T before a fragment is
// T after it over 1 - alpha) and one scalar Q: the sum over the composited fragments behind of
// vis * (colour . v_rgb), started at the background / alpha term -v_o_w. Then for a fragment
// dL/dalpha = T_before (colour . v_rgb) - Q / (1 - alpha), the colour remainder contracted with v_rgb once
// instead of carried per channel. Each lane's eleven per-fragment values (g0..g9 and the blend weight) are
// summed over the wave by a shuffle-down tree and lane 0 adds them to v_splat with float atomics, the
// reference's accumulation (raster_bwd.cu:130-139). The order of those atomic adds varies between runs; the
// mode-1 path below is the deterministic one. The per-splat inputs come from proj0..2 (the reference's
// buffers), not from the raster record the other kernels read, so this path also checks that record.
//
// Feature lanes (FEAT) are composited like the colour but without a background, so their share of
// dL/dalpha folds into the same scalar: (colour . v_rgb) becomes (colour . v_rgb + feature . v_feat), and
// the splat's feature gradient is the sum of vis * v_feat. The hollow penalty (HOLLOW) adds
// lam (T_before h - S_h / (1 - alpha)) to dL/dalpha, with S_h the vis-weighted penalty of the fragments
// behind (raster_bwd.cu:101); the refine statistic keeps the dL/dalpha without it.

__device__ __forceinline__ float wave_total_to_lane0(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_down(v, o);
  return v;
}

template <bool FEAT, bool HOLLOW>
__global__ void __launch_bounds__(64) raster_bwd_fp32_kernel(b2c_raster_bwd_args a) {
  // per-fragment sums: g0..g9, the blend weight, and with FEAT the three feature lanes
  constexpr int ANCHOR_VALS = FEAT ? 14 : 11;
  __shared__ float4 s_geo[64], s_shape[64], s_rgb[64];  // proj0, proj1, proj2 of the batch's splats
  __shared__ float2 s_f3[FEAT ? 64 : 1];                  // proj3 (feature y, z)
  __shared__ uint32_t s_id[64];
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const uint2 range = reinterpret_cast<const uint2*>(a.tile_ranges)[tile];
  if (range.y <= range.x) return;
  const int lane = threadIdx.x;
  const int px = (tile % a.tiles_x) * RT_W + (lane & 7), py = (tile / a.tiles_x) * RT_W + (lane >> 3);
  const PixelState ps = load_pixel<FEAT, HOLLOW>(a, px, py, range.x, a.last_idx);
  const float tcx = (tile % a.tiles_x) * RT_W + RT_W * 0.5f, tcy = (tile / a.tiles_x) * RT_W + RT_W * 0.5f;
  const PixelPoly pp = pixel_poly(ps.pcx - tcx, ps.pcy - tcy);
  const float Wf = (float)a.W, Hf = (float)a.H;
  float T = ps.T;
  float Q = -ps.v_o_w;
  float Sh = 0.f;  // sum over composited fragments behind of vis * penalty
  for (uint32_t hi = range.y; hi > range.x;) {
    const uint32_t lo = hi - range.x > 64u ? hi - 64u : range.x;
    const int count = (int)(hi - lo);
    __syncthreads();  // the previous batch is consumed
    if (lane < count) {
      const uint32_t id = a.vals_sorted[lo + lane];
      s_id[lane] = id;
      s_geo[lane] = reinterpret_cast<const float4*>(a.proj0)[id];
      s_shape[lane] = reinterpret_cast<const float4*>(a.proj1)[id];
      s_rgb[lane] = reinterpret_cast<const float4*>(a.proj2)[id];
      if constexpr (FEAT) s_f3[lane] = reinterpret_cast<const float2*>(a.proj3)[id];
    }
    __syncthreads();
    for (int j = count - 1; j >= 0; j--) {
      const float4 geo = s_geo[j], shape = s_shape[j];  // (mx, my, c00, c01), (c11, opacity, depth, power)
      // halving c00 and c11 is exact: the same sigma as the forward's (its tile-centred quadratic); the
      // gradient terms use the offsets from the splat centre
      const FragGeom fg = frag_geom(geo.x, geo.y, 0.5f * geo.z, geo.w, 0.5f * shape.x, ps.pcx, ps.pcy);
      const float3 def = sigma_coefs(geo.x, geo.y, 0.5f * geo.z, geo.w, 0.5f * shape.x, tcx, tcy);
      const float sigma = poly_sigma(0.5f * geo.z, geo.w, 0.5f * shape.x, def.x, def.y, def.z, pp);
      const bool in = ps.inside && lo + (uint32_t)j < ps.last && sigma <= shape.w;
      if (ballot64(in) == 0ull) continue;  // uniform
      float val[ANCHOR_VALS];
#pragma unroll
      for (int k = 0; k < ANCHOR_VALS; k++) val[k] = 0.f;
      if (in) {
        const float4 col = s_rgb[j];
        const float araw = fragment_alpha(sigma, log2_opacity(shape.y));
        const float alpha = fminf(ALPHA_MAX, araw);
        const float keep = 1.f - alpha;
        const float Tb = T / keep;
        const float vis = alpha * Tb;
        float cv = fmaxf(col.x, 0.f) * ps.vo.x + fmaxf(col.y, 0.f) * ps.vo.y + fmaxf(col.z, 0.f) * ps.vo.z;
        if constexpr (FEAT) {
          const float2 f12 = s_f3[j];
          cv = cv + (col.w * ps.vf.x + f12.x * ps.vf.y + f12.y * ps.vf.z);
        }
        const float v_alpha_photo = Tb * cv - Q / keep;
        float v_alpha = v_alpha_photo, hh = 0.f;
        if constexpr (HOLLOW) {
          hh = hollow_h(shape.z, ps.href);
          v_alpha = v_alpha + a.hollow_lam * (Tb * hh - Sh / keep);
        }
        if (araw <= ALPHA_MAX) {  // a clamped alpha does not depend on sigma
          const float dx = fg.dx, dy = fg.dy;
          const float v_sigma = -alpha * v_alpha;
          // d sigma / d mean = -(d sigma / d d) = -(2a dx + b dy, b dx + 2c dy)
          const float ex = __builtin_fmaf(0.5f * geo.z, dx, fg.lin), ey = __builtin_fmaf(geo.w, dx, fg.cdy + fg.cdy);
          const float gmx = -v_sigma * ex;
          const float gmy = -v_sigma * ey;
          val[0] = gmx;
          val[1] = gmy;
          val[2] = 0.5f * v_sigma * dx * dx;
          val[3] = v_sigma * dx * dy;
          val[4] = 0.5f * v_sigma * dy * dy;
          val[8] = v_alpha * gauss_weight(sigma);
          // the refine statistic: the mean gradient of the photometric (and feature) terms only
          const float vsp = -alpha * v_alpha_photo;
          const float px_ = -vsp * ex, py_ = -vsp * ey;
          val[9] = sqrtf((px_ * Wf) * (px_ * Wf) + (py_ * Hf) * (py_ * Hf)) * ps.inv_final_a;
        }
        val[5] = col.x >= 0.f ? vis * ps.vo.x : 0.f;
        val[6] = col.y >= 0.f ? vis * ps.vo.y : 0.f;
        val[7] = col.z >= 0.f ? vis * ps.vo.z : 0.f;
        val[10] = vis;
        if constexpr (FEAT) {
          val[11] = vis * ps.vf.x;
          val[12] = vis * ps.vf.y;
          val[13] = vis * ps.vf.z;
        }
        T = Tb;
        Q = Q + vis * cv;
        if constexpr (HOLLOW) Sh = Sh + vis * hh;
      }
#pragma unroll
      for (int k = 0; k < ANCHOR_VALS; k++) val[k] = wave_total_to_lane0(val[k]);
      if (lane == 0) {
        const uint32_t id = s_id[j];
        a.vis_flag[id] = 1u;
        if (a.vis_weight) atomicAdd(a.vis_weight + id, val[10]);
        float* dst = a.v_splat + (size_t)id * GRAD_LANES;
#pragma unroll
        for (int k = 0; k < 10; k++)
          if (val[k] != 0.f) atomicAdd(dst + k, val[k] * a.inv_gscale);
        if constexpr (FEAT) {
#pragma unroll
          for (int k = 0; k < 3; k++)
            if (val[11 + k] != 0.f) atomicAdd(dst + 10 + k, val[11 + k] * a.inv_gscale);
        }
      }
    }
    hi = lo;
  }
}

// ------------------------------------------------------------------------------------------------------
// mode 1: MFMA reduction into per-(tile, splat) rows, then a per-splat reduce (no atomics)
// ------------------------------------------------------------------------------------------------------
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Splats staged in LDS per step: 48 keeps the plain kernel's LDS at 8 KB, so five one-wave workgroups fit
// per SIMD instead of four (a batch is a whole number of groups, cut from the list end, so the groups of 8
// are the same splats whatever the batch size).
constexpr int BATCH = 48;
constexpr int G = 8;       // splats per MFMA group
static_assert(BATCH % G == 0, "batches of whole groups");
constexpr int SROW = 68;   // pixel stride of the per-fragment scalar rows (64 + 4: spreads the B reads over banks)
constexpr int SROW_H = 72;  // pixel stride of the fp16 refine rows (a multiple of 8: 16-byte aligned reads)
// (tile, splat) row: raw moments of the tile's fragments about the tile centre, 12 floats in three 16-byte
// quarters, each written by one lane with one store: sum v_sigma * [v, u^2, uv, v^2] | sum v_sigma * [1, u],
// sum vis, refine sum | sum vis * v_rgb, the tag word row_tag | tile (bits); with feature lanes a fourth
// quarter sum vis * v_feat, 0. Rows are ROW_FLOATS<FEAT> floats apart.
template <bool FEAT>
constexpr int ROW_FLOATS = FEAT ? 16 : 12;
// basis rows (M) of operand A: 0-2 v_rgb, 3-5 v_feat (zero without FEAT), 6 one, 7 u, 8 v, 9 u^2, 10 uv,
// 11 v^2, 12-15 zero
constexpr int B_ONE = 6, B_U = 7, B_V = 8, B_UU = 9, B_UV = 10, B_VV = 11;


typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Two fp32 values to fp16, rounding toward zero (v_cvt_pkrtz_f16_f32: one instruction per pair; values
// beyond the fp16 range saturate to the largest finite value instead of becoming infinite).
__device__ __forceinline__ half2v pk_rtz(float a, float b) {
  return __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(a, b));
}

// Split 8 fp32 values into fp16 hi (truncated) and 2^11-scaled fp16 lo parts: x - hi is exact, and the
// truncated lo keeps the pair to ~2^-21 relative. 2^11 (x - hi) is formed as fma(-hi, 2^11, 2^11 x), exact
// like (x - hi) 2^11 (both products are exact), which the compiler issues as one v_fma_mix_f32 reading hi
// straight from its fp16 half: three instructions per value instead of four.
__device__ __forceinline__ void split8(const float* x, half8& hi, half8& lo) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const half2v h = pk_rtz(x[e], x[e + 1]);
    hi[e] = h.x;
    hi[e + 1] = h.y;
    const half2v l = pk_rtz(__builtin_fmaf(-(float)h.x, LO_SCALE, x[e] * LO_SCALE),
                            __builtin_fmaf(-(float)h.y, LO_SCALE, x[e + 1] * LO_SCALE));
    lo[e] = l.x;
    lo[e + 1] = l.y;
  }
}

__device__ __forceinline__ void load8(const float* p, float* x) {
  const float4 q0 = reinterpret_cast<const float4*>(p)[0], q1 = reinterpret_cast<const float4*>(p)[1];
  x[0] = q0.x; x[1] = q0.y; x[2] = q0.z; x[3] = q0.w; x[4] = q1.x; x[5] = q1.y; x[6] = q1.z; x[7] = q1.w;
}

// One wave64 per 8x8 tile, one lane per pixel. The tile's list is replayed back to front in batches of 48
// splats staged in LDS and groups of 8: for each splat of a group every lane writes three scalars of its
// fragment (blend weight vis, v_sigma, refine) into LDS; then two 16x16x32 f16 MFMA products per 32 pixels
// contract them against the per-pixel basis (columns 0-7 vis, 8-15 v_sigma of the group's splats; second
// product: refine, fp16 only), with hi/lo fp16 splits so ~22 bits of the fp32 inputs survive. The opacity lane needs
// no product of its own: where a fragment is unclamped v_alpha * gauss = -v_sigma / opacity, and both are
// zero where it is clamped, so g8 = -(sum v_sigma) / opacity.
template <bool FEAT, bool HOLLOW>
__global__ void __launch_bounds__(64) raster_bwd_mfma_kernel(b2c_raster_bwd_args a) {
  constexpr bool EXT = FEAT || HOLLOW;
  constexpr int ROW = ROW_FLOATS<FEAT>;
  __shared__ float4 s_g0[BATCH];   // (D, E, F, c00 / 2): sigma_coefs at this tile
  __shared__ float4 s_g1[BATCH];   // (c01, c11 / 2, power, log2 opacity)
  __shared__ float4 s_col[BATCH];  // (max(r, 0), max(g, 0), max(b, 0), sign bits of r, g, b)
  __shared__ float4 s_ext[EXT ? BATCH : 1];  // (feature xyz, camera depth)
  __shared__ uint32_t s_slot[BATCH];
  __shared__ __attribute__((aligned(16))) float sS[2 * G][SROW];  // rows 0-7 vis, 8-15 v_sigma
  // the refine products, already the fp16 operand of their MFMA (truncated as the conversion of fp32 rows
  // would be)
  __shared__ __attribute__((aligned(16))) _Float16 sR[G][SROW_H];
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  // with the forward's compacted lists: the entries some pixel composited, the pixels' ends in them
  const bool compact = a.cvals != nullptr;  // uniform
  uint2 range = reinterpret_cast<const uint2*>(a.tile_ranges)[tile];
  if (compact) range.y = a.cend[tile];
  const uint32_t* list_vals = compact ? a.cvals : a.vals_sorted;
  const uint32_t* list_slots = compact ? a.cslots : a.slot_sorted;
  const int lane = threadIdx.x;
  // pairs past the shrunk end (or left out of the compacted list) never composited: they get no row, and the
  // reduce does not read theirs
  if (range.y <= range.x) return;
  const int tx = tile % a.tiles_x, ty = tile / a.tiles_x;
  const int lx = lane & 7, ly = lane >> 3;
  const int px = tx * RT_W + lx, py = ty * RT_W + ly;
  const float u = lx + 0.5f - RT_W * 0.5f, v = ly + 0.5f - RT_W * 0.5f;  // offset from the tile centre
  const float tcx = tx * RT_W + RT_W * 0.5f, tcy = ty * RT_W + RT_W * 0.5f;
  const PixelPoly pp = pixel_poly(u, v);
  const float u2 = u + u, v2 = v + v;
  PixelState ps = load_pixel<FEAT, HOLLOW>(a, px, py, range.x, compact ? a.clast : a.last_idx);
  // refine: sqrt(W^2 gx^2 + H^2 gy^2) = W sqrt(gx^2 + rho gy^2), W folded into the per-pixel scale
  const float rho = ((float)a.H * (float)a.H) / ((float)a.W * (float)a.W);
  const float r_scale = ps.inv_final_a * R_SCALE * (float)a.W;
  const float cv_x = ps.vo.x, cv_y = ps.vo.y, cv_z = ps.vo.z;

  // Basis operand A (16 rows x 64 px), built once per tile through sS as scratch.
  const int nl = lane & 15, kg = lane >> 4;
  half8 A_hi[2], A_lo[2];
  {
    float* bm = &sS[0][0];  // [16][SROW]
    const float row[16] = {cv_x, cv_y, cv_z, ps.vf.x, ps.vf.y, ps.vf.z, 1.f, u, v, u * u, u * v, v * v, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 16; m++) bm[m * SROW + lane] = row[m];
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      float x[8];
      load8(&bm[nl * SROW + kb * 32 + kg * 8], x);
      split8(x, A_hi[kb], A_lo[kb]);
    }
    __syncthreads();
  }

  float T = ps.T;
  float Q = -ps.v_o_w;  // sum over composited splats behind of (colour . v_rgb) * vis, minus the v_o_w term
  float Sh = 0.f;       // HOLLOW: sum over composited splats behind of vis * penalty
  const bool live_px = ps.inside;
  for (uint32_t batch_end = range.y; batch_end > range.x;) {
    const uint32_t batch_start = batch_end > range.x + BATCH ? batch_end - BATCH : range.x;
    const int count = (int)(batch_end - batch_start);
    __syncthreads();
    const int ngroups = (count + G - 1) / G;
    if (lane < count) {
      const uint32_t gid = list_vals[batch_start + lane];
      s_slot[lane] = list_slots[batch_start + lane];
      const float4* rec = reinterpret_cast<const float4*>(a.raster_rec) + (size_t)gid * 4;
      const float4 r0 = rec[0], r1 = rec[1], r2 = rec[2];
      const float3 def = sigma_coefs(r0.x, r0.y, r0.z, r0.w, r1.x, tcx, tcy);
      s_g0[lane] = make_float4(def.x, def.y, def.z, r0.z);
      s_g1[lane] = make_float4(r0.w, r1.x, r1.z, r2.w);
      s_col[lane] = make_float4(r2.x, r2.y, r2.z, r1.w);
      if constexpr (EXT) s_ext[lane] = rec[3];
    } else if (lane < ngroups * G) {  // pad the last group with null splats, never composited: power = 0
      s_g0[lane] = make_float4(0.f, 0.f, 1.f, 0.f);  // and sigma = F = 1
      s_g1[lane] = make_float4(0.f, 0.f, 0.f, 0.f);
      s_col[lane] = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (EXT) s_ext[lane] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    for (int grp = ngroups - 1; grp >= 0; grp--) {
      const int gbase = grp * G;
      const int gcount = min(G, count - gbase);
      // ---- replay: this pixel's three scalars for each splat of the group (zero when not composited)
      // the group's LDS byte offset, kept in one VGPR for the whole group (immediate offsets per splat)
      uint32_t goff = (uint32_t)gbase * 16u;
      asm volatile("" : "+v"(goff));
      const char* lds_g0 = reinterpret_cast<const char*>(s_g0) + goff;
      const char* lds_g1 = reinterpret_cast<const char*>(s_g1) + goff;
      const char* lds_col = reinterpret_cast<const char*>(s_col) + goff;
      const char* lds_ext = reinterpret_cast<const char*>(s_ext) + goff;
      // the last list index of the group this pixel composited, relative to the group start
      const int last_rel = (int)ps.last - (int)(batch_start + (uint32_t)gbase);
#pragma unroll
      for (int jj = G - 1; jj >= 0; jj--) {
        float o_vis = 0.f, o_vs = 0.f, o_r = 0.f;
        {
          const float4 g0 = *reinterpret_cast<const float4*>(lds_g0 + jj * 16);
          const float4 g1 = *reinterpret_cast<const float4*>(lds_g1 + jj * 16);
          const float sigma = poly_sigma(g0.w, g1.x, g1.y, g0.x, g0.y, g0.z, pp);
          // the forward's test: sigma <= power (a NaN sigma fails)
          const bool in = live_px & (jj < last_rel) & (sigma <= g1.z);
          {  // straight-line: a lane without this fragment computes zeros (alpha = 0)
            // a lane without this fragment runs the same arithmetic with alpha = 0: ra = 1, vis = 0,
            // v_sigma = 0 and T, Q unchanged (every operand stays finite)
            const float araw = fragment_alpha(sigma, g1.w);
            const float alpha = in ? fminf(ALPHA_MAX, araw) : 0.f;
            const float ra = __builtin_amdgcn_rcpf(1.f - alpha);
            const float Tb = T * ra;
            const float vis = alpha * Tb;
            const float4 col = *reinterpret_cast<const float4*>(lds_col + jj * 16);
            float cv = col.x * cv_x + col.y * cv_y + col.z * cv_z;
            float4 ext = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (EXT) ext = *reinterpret_cast<const float4*>(lds_ext + jj * 16);
            if constexpr (FEAT) cv = cv + (ext.x * ps.vf.x + ext.y * ps.vf.y + ext.z * ps.vf.z);
            const float v_alpha_photo = Tb * cv - ra * Q;
            float v_alpha = v_alpha_photo, hh = 0.f;
            if constexpr (HOLLOW) {
              hh = hollow_h(ext.w, ps.href);
              v_alpha = v_alpha + a.hollow_lam * (Tb * hh - ra * Sh);
            }
            const bool unclamped = araw <= ALPHA_MAX;  // clamped: no sigma gradient
            const float v_sigma = unclamped ? -alpha * v_alpha : 0.f;
            // refine statistic: |d(loss)/d(mean2d)| scaled to pixels, over the final alpha, from the
            // photometric (and feature) terms only
            const float v_sigma_photo = HOLLOW ? (unclamped ? -alpha * v_alpha_photo : 0.f) : v_sigma;
            // the sigma gradient in pixels: 2a u + b v + D, b u + 2c v + E
            const float gx = __builtin_fmaf(g0.w, u2, __builtin_fmaf(g1.x, v, g0.x));
            const float gy = __builtin_fmaf(g1.x, u, __builtin_fmaf(g1.y, v2, g0.y));
            o_r = fabsf(v_sigma_photo) * __builtin_amdgcn_sqrtf(gx * gx + rho * gy * gy) * r_scale;
            o_vis = vis;
            o_vs = v_sigma;
            T = Tb;
            Q = Q + vis * cv;
            if constexpr (HOLLOW) Sh = Sh + vis * hh;
          }
        }
        sS[jj][lane] = o_vis;
        sS[G + jj][lane] = o_vs;
        sR[jj][lane] = pk_rtz(o_r, 0.f).x;
      }
      __syncthreads();
      // ---- reduction over the 64 pixels on MFMA
      floatx4 d0_hi = {0.f, 0.f, 0.f, 0.f}, d0_lo = {0.f, 0.f, 0.f, 0.f};
      floatx4 d1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        float x[8];
        half8 b_hi, b_lo;
        load8(&sS[nl][kb * 32 + kg * 8], x);
        split8(x, b_hi, b_lo);
        d0_hi = __builtin_amdgcn_mfma_f32_16x16x32_f16(A_hi[kb], b_hi, d0_hi, 0, 0, 0);
        d0_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(A_hi[kb], b_lo, d0_lo, 0, 0, 0);
        d0_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(A_lo[kb], b_hi, d0_lo, 0, 0, 0);
        const half8 rb = *reinterpret_cast<const half8*>(&sR[nl & (G - 1)][kb * 32 + kg * 8]);  // columns 8-15 of d1 are unused
        d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A_hi[kb], rb, d1, 0, 0, 0);
      }
      // D layout: lane (nl, kg) holds rows 4 kg .. 4 kg + 3 of column nl. Three lanes per splat j store the
      // (tile, splat) row's raw moments (the reduce turns them into gradients), one 16-byte quarter each:
      // (j + 8, kg 2) the v_sigma column's rows 8-11; (j, kg 1) the v_sigma column's rows 6-7, taken from
      // lane j + 8 of its row of 16 lanes, then the vis column's row 6 and the refine product's row 6;
      // (j, kg 0) the vis column's rows 0-2 and the tag word.
      {
        const int j = nl & (G - 1);
        float dv[4];
#pragma unroll
        for (int rr = 0; rr < 4; rr++) dv[rr] = d0_hi[rr] + d0_lo[rr] * (1.f / LO_SCALE);
        // row_ror:8 within each row of 16 lanes: lane nl gets lane nl ^ 8 (every lane takes part)
        const float sv = __uint_as_float(dpp_u32<0x128, 0xF>(__float_as_uint(dv[2]), 0u));
        const float svu = __uint_as_float(dpp_u32<0x128, 0xF>(__float_as_uint(dv[3]), 0u));
        // FEAT: the vis column's rows 3-5 (sum vis * v_feat) sit in lane (j, kg 0) row 3 and lane (j, kg 1)
        // rows 4-5; the first moves 16 lanes up to join the others
        float fx = 0.f;
        if constexpr (FEAT) fx = __shfl_up(dv[3], 16);
        if (j < gcount) {
          float4* row = reinterpret_cast<float4*>(a.isect_rows) + (size_t)s_slot[gbase + j] * (ROW / 4);
          if (nl >= G && kg == 2) row[0] = make_float4(dv[0], dv[1], dv[2], dv[3]);
          if (nl < G && kg == 1) row[1] = make_float4(sv, svu, dv[2], d1[2]);
          if (nl < G && kg == 0) {
            row[2] = make_float4(dv[0], dv[1], dv[2], __uint_as_float(a.row_tag | (uint32_t)tile));
            if (a.row_live) a.row_live[s_slot[gbase + j]] = a.row_tag | (uint32_t)tile;
          }
          if constexpr (FEAT)
            if (nl < G && kg == 1) row[3] = make_float4(fx, dv[0], dv[1], 0.f);
        }
      }
    }
    batch_end = batch_start;
  }
}

// Per-splat sum of the (tile, splat) rows. In emit order the rows of one splat are one contiguous run and
// isect_vals[slot] (the emitted splat id) names the run, so this is a segmented reduction over a
// contiguous array, in two kernels:
//  * isect_reduce_kernel: one wave per aligned window of RED_WIN rows (256, or 1024 with the live-row
//    index), walked as 64-row sub-windows (coalesced 48-byte rows; a row without this pass's tag, a pair past its tile's shrunk end,
//    counts as zero), each a segmented inclusive scan across lanes on DPP row shifts and row broadcasts;
//    the sums of a run that continues into the next sub-window are carried in
//    registers. A run that starts and ends inside the window is finished there: its last lane adds the
//    sums to v_splat[0..9], vis_weight and vis_flag (the raster_bwd_tc.cu:195-198 updates, without
//    atomics). A run crossing a window edge leaves its per-window partial sums in isect_part (first run of
//    the window, last run of the window) with flags.
//  * isect_fixup_kernel: one thread per window; the window where a crossing run starts adds the partials
//    of the following windows the run covers, in order, and finishes the run (the whole wave helps with
//    runs over many windows).
// Every window does the same amount of work whatever the run lengths (splats spanning thousands of tiles
// do not serialise), and the summation order is fixed: the result is deterministic.
// Values carried per row: g0..g9 and the blend-weight sum, and with FEAT the three feature lanes (g10..g12).
template <bool FEAT>
constexpr int RED_VALS = FEAT ? 14 : 11;
// Partial-sum quarters per run piece (three or four float4) and per window (two pieces: the window's first
// run and its last run; the last piece's third quarter carries the head slot in .w).
template <bool FEAT>
constexpr int PART_Q = FEAT ? 4 : 3;
constexpr uint32_t W_CONT_BEFORE = 1u, W_CONT_AFTER = 2u, W_HAS_HEAD = 4u;
// 64-row sub-windows per reduce wave (one window): 4 when every row is read, 16 with the live-row index,
// where most rows are skipped and longer windows leave fewer runs to the fixup (config 4: reduce 4.84 ->
// 4.22 ms per 8-view step, config 5: 0.303 -> 0.281 ms; with every row read, 16 measured 127.6 against
// 124.6 us at config 3).
template <bool LIVE>
constexpr int RED_SUB = LIVE ? 16 : 4;
template <bool LIVE>
constexpr uint32_t RED_WIN = 64u * RED_SUB<LIVE>;  // rows per window (one wave)


template <bool FEAT>
__device__ __forceinline__ void prefetch_old(const b2c_raster_bwd_args& a, uint32_t id, float (&old)[RED_VALS<FEAT>]) {
  const float* dst = a.v_splat + (size_t)id * GRAD_LANES;
  const bool zero = a.v_splat_zero != 0;  // uniform
#pragma unroll
  for (int k = 0; k < 10; k++) old[k] = zero ? 0.f : dst[k];
  old[10] = (a.vis_weight && !a.defer_vis) ? a.vis_weight[id] : 0.f;
  if constexpr (FEAT) {
#pragma unroll
    for (int k = 0; k < 3; k++) old[11 + k] = zero ? 0.f : dst[10 + k];
  }
}

// Adds a finished run's sums to v_splat / vis_weight (previous contents in `old`) and flags the splat; with
// defer_vis (no feature lanes, v_splat known zero) the blend-weight sum goes to v_splat lane 10 instead, for
// the projection VJP to flag the splat and add it to vis_weight.
template <bool FEAT>
__device__ __forceinline__ void finish_run(const b2c_raster_bwd_args& a, uint32_t id, const float (&v)[RED_VALS<FEAT>],
                                           const float (&old)[RED_VALS<FEAT>]) {
  if (!(v[10] > 0.f)) return;  // no composited fragment: every lane of the run is zero
  float* dst = a.v_splat + (size_t)id * GRAD_LANES;
#pragma unroll
  for (int k = 0; k < 10; k++) dst[k] = old[k] + v[k];
  if constexpr (FEAT) {
#pragma unroll
    for (int k = 0; k < 3; k++) dst[10 + k] = old[11 + k] + v[11 + k];
  } else {
    if (a.defer_vis) {  // uniform
      dst[10] = v[10];
      return;
    }
  }
  a.vis_flag[id] = 1u;
  if (a.vis_weight) a.vis_weight[id] = old[10] + v[10];
}

template <bool FEAT>
__device__ __forceinline__ void store_part(float4* p, const float (&v)[RED_VALS<FEAT>]) {
  p[0] = make_float4(v[0], v[1], v[2], v[3]);
  p[1] = make_float4(v[4], v[5], v[6], v[7]);
  p[2] = make_float4(v[8], v[9], v[10], 0.f);
  if constexpr (FEAT) p[3] = make_float4(v[11], v[12], v[13], 0.f);
}

template <bool FEAT>
__device__ __forceinline__ void add_part(const float4* p, float (&v)[RED_VALS<FEAT>]) {
  const float4 q0 = p[0], q1 = p[1], q2 = p[2];
  v[0] += q0.x; v[1] += q0.y; v[2] += q0.z; v[3] += q0.w; v[4] += q1.x; v[5] += q1.y; v[6] += q1.z; v[7] += q1.w;
  v[8] += q2.x; v[9] += q2.y; v[10] += q2.z;
  if constexpr (FEAT) {
    const float4 q3 = p[3];
    v[11] += q3.x; v[12] += q3.y; v[13] += q3.z;
  }
}

// Gradient lanes g0..g9 and the blend-weight sum of one (tile, splat) row from its raw moments about the
// tile centre (raster_bwd_tc.cu:172-198 accumulates the same quantities per fragment): with (mx, my) the
// splat centre relative to the tile centre, the first and second moments of v_sigma about the splat centre
// give the mean and conic gradients, the vis moments the colour gradients, and where a fragment is
// unclamped v_alpha * gauss = -v_sigma / opacity gives g8. The row's tag word holds the tile; returns
// whether the tag is this pass's (otherwise the row was not written by it and v is to be discarded).
template <bool FEAT>
__device__ __forceinline__ bool row_gradients(const b2c_raster_bwd_args& a, uint32_t s, uint32_t id,
                                              float (&v)[RED_VALS<FEAT>]) {
  const float4* rw = reinterpret_cast<const float4*>(a.isect_rows) + (size_t)s * (ROW_FLOATS<FEAT> / 4);
  const float4 q0 = rw[0], q1 = rw[1], q2 = rw[2];
  const float4* rec = reinterpret_cast<const float4*>(a.raster_rec) + (size_t)id * 4;
  const float4 r0 = rec[0], r1 = rec[1];  // (mx, my, c00 / 2, c01), (c11 / 2, opacity, power, sign bits)
  const uint32_t word = __float_as_uint(q2.w);
  const uint32_t t = word & a.tile_mask;
  const uint32_t ty = t / (uint32_t)a.tiles_x, tx = t - ty * (uint32_t)a.tiles_x;
  const float mx = r0.x - ((float)(tx * RT_W) + RT_W * 0.5f), my = r0.y - ((float)(ty * RT_W) + RT_W * 0.5f);
  const float sv = q1.x, svu = q1.y, svv = q0.x, svuu = q0.y, svuv = q0.z, svvv = q0.w;
  const float sc = a.inv_gscale;
  const float m1u = svu - mx * sv, m1v = svv - my * sv;  // sum v_sigma (u - mx), (v - my)
  const float m2uu = svuu - 2.f * mx * svu + mx * mx * sv;
  const float m2uv = svuv - my * svu - mx * svv + mx * my * sv;
  const float m2vv = svvv - 2.f * my * svv + my * my * sv;
  const uint32_t sgn = __float_as_uint(r1.w);
  v[0] = -(2.f * r0.z * m1u + r0.w * m1v) * sc;
  v[1] = -(r0.w * m1u + 2.f * r1.x * m1v) * sc;
  v[2] = 0.5f * m2uu * sc;
  v[3] = m2uv * sc;
  v[4] = 0.5f * m2vv * sc;
  v[5] = (sgn & 1u) ? q2.x * sc : 0.f;
  v[6] = (sgn & 2u) ? q2.y * sc : 0.f;
  v[7] = (sgn & 4u) ? q2.z * sc : 0.f;
  v[8] = -sv / r1.y * sc;
  v[9] = q1.w * (1.f / R_SCALE) * sc;  // the raster pre-scales refine terms into the fp16 range
  v[10] = q1.z;
  if constexpr (FEAT) {
    const float4 q3 = rw[3];
    v[11] = q3.x * sc;
    v[12] = q3.y * sc;
    v[13] = q3.z * sc;
  }
  return (word & ~a.tile_mask) == a.row_tag;
}

// LIVE: rows are read through the live-row index (a.row_live).
template <bool FEAT, bool LIVE>
__global__ void __launch_bounds__(256) isect_reduce_kernel(b2c_raster_bwd_args a) {
  constexpr int RED_VALS = ::b2c::dev::RED_VALS<FEAT>;
  constexpr int PQ = PART_Q<FEAT>;
  const uint32_t m = a.num_isect;
  const int lane = threadIdx.x & 63;
  const uint32_t w = blockIdx.x * 4u + (threadIdx.x >> 6);
  constexpr uint32_t WIN = RED_WIN<LIVE>;
  const uint32_t wlo = w * WIN;
  if (wlo >= m) return;
  const uint32_t* ids = a.isect_vals;
  const uint32_t before = wlo == 0 ? NO_RUN : ids[wlo - 1];
  // wave-uniform state across the window's 64-row sub-windows: the partial sums of the run that continues
  // into the next sub-window, whether that run started before the window, and where it started
  float carry[RED_VALS];
#pragma unroll
  for (int k = 0; k < RED_VALS; k++) carry[k] = 0.f;
  bool carry_from_before = false;
  uint32_t carry_head = 0;
  uint32_t prev_id = before;
  bool window_cont_before = false, window_has_head = false;
  float4* part = reinterpret_cast<float4*>(a.isect_part) + (size_t)w * (2 * PQ);
  // with the live-row index, where most rows are not read, the next sub-window's splat ids and live-row
  // words are loaded while this one is processed (without it, the row loads dominate and this measured
  // slower)
  uint32_t nxt_id = NO_RUN, nxt_word = 0u;
  if (LIVE && wlo + lane < m) {
    nxt_id = ids[wlo + lane];
    nxt_word = a.row_live[wlo + lane];
  }
  for (int sub = 0; sub < RED_SUB<LIVE>; sub++) {
    const uint32_t lo = wlo + 64u * (uint32_t)sub;
    if (lo >= m) break;
    const uint32_t s = lo + lane;
    const bool valid = s < m;
    uint32_t id, word = 0u;
    if constexpr (LIVE) {
      id = nxt_id;  // valid ? ids[s] : NO_RUN
      word = nxt_word;
      const uint32_t s1 = s + 64u;
      const bool more = sub + 1 < RED_SUB<LIVE> && s1 < m;
      nxt_id = more ? ids[s1] : NO_RUN;
      nxt_word = more ? a.row_live[s1] : 0u;
    } else {
      id = valid ? ids[s] : NO_RUN;
    }
    const uint32_t next_id = lo + 64u < m ? ids[lo + 64u] : NO_RUN;
    float v[RED_VALS];
    // a row without this pass's tag (a pair past its tile's shrunk end, or a sentinel) counts as zero; with
    // the live-row index only the rows it marks are read
    bool live;
    // the kernel without the index keeps the test as a runtime branch (never taken: the host passes no
    // index to it); the compiler's schedule of that form measured 3 us faster at 6M rows than without it
    if (LIVE || a.row_live) {
      if (!LIVE) word = valid ? a.row_live[s] : 0u;
#pragma unroll
      for (int k = 0; k < RED_VALS; k++) v[k] = 0.f;
      live = valid && (word & ~a.tile_mask) == a.row_tag;
      if (live) live = row_gradients<FEAT>(a, s, id, v);
    } else {
      live = row_gradients<FEAT>(a, valid ? s : 0u, valid ? id : 0u, v) && valid;
    }
#pragma unroll
    for (int k = 0; k < RED_VALS; k++) v[k] = live ? v[k] : 0.f;
    const uint32_t prev = dpp_u32<0x138, 0xF>(id, prev_id);  // wave_shr:1; lane 0 gets the row before
    const bool head = valid && id != prev;
    const uint64_t heads = ballot64(head);
    const uint32_t id63 = (uint32_t)__builtin_amdgcn_readlane((int)id, 63);
    const bool cont_after = id63 != NO_RUN && next_id == id63;
    const bool cont_before = (heads & 1ull) == 0;  // row 0 continues the run of the row before
    if (sub == 0) window_cont_before = cont_before;
    window_has_head = window_has_head || heads != 0ull;
    const uint32_t nid = dpp_u32<0x130, 0xF>(id, cont_after ? id63 : NO_RUN);  // wave_shl:1; lane 63 gets the fill
    const bool tail = valid && nid != id;
    // the first run of the sub-window ends at the lane before the second head (or at the last valid row)
    const uint64_t later_heads = heads & ~1ull;
    const int last_valid = (int)min(63u, m - 1u - lo);
    const int first_tail = later_heads ? __builtin_ctzll(later_heads) - 1 : last_valid;
    const bool in_first = lane <= first_tail;
    const bool last_is_first = later_heads == 0ull;  // the sub-window holds one run only
    // the first run started before the window (then it is the window's first piece, finished by the fixup)
    const bool first_from_before = cont_before && (sub == 0 ? before != NO_RUN : carry_from_before);
    const bool is_first = lane == first_tail;
    const bool is_last = lane == 63;
    const bool crosses_window = cont_after && sub == RED_SUB<LIVE> - 1;
    const bool complete = tail && !(is_first && first_from_before);
    // a sub-window without a row of this pass scans to zeros: skip the scan (wave-uniform); a run ending in
    // it then has sums only if it carries some from the previous sub-window
    const bool any_live = ballot64(live) != 0ull;
    const bool carried = cont_before && sub > 0 && in_first;
    float old[RED_VALS];
    if (complete && (any_live || (carried && carry[10] > 0.f))) prefetch_old<FEAT>(a, id, old);
    if (any_live) seg_scan(valid ? id : NO_RUN, v);
    if (carried) {  // the run carried from the previous sub-window
#pragma unroll
      for (int k = 0; k < RED_VALS; k++) v[k] += carry[k];
    }
    if (complete) finish_run<FEAT>(a, id, v, old);
    if (is_first && first_from_before && (!cont_after || !last_is_first || sub == RED_SUB<LIVE> - 1))
      store_part<FEAT>(part, v);  // the window's first piece ends here (or spans the whole window)
    // the last run of the sub-window continues: carry it, or leave it for the fixup at the window's edge
    const uint32_t last_head = lo + 63u - (heads ? (uint32_t)__builtin_clzll(heads) : 63u);
    const bool last_from_before = last_is_first ? first_from_before : false;
    if (cont_after) {
      if (!crosses_window) {
#pragma unroll
        for (int k = 0; k < RED_VALS; k++) carry[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[k]), 63));
        carry_from_before = last_from_before;
        carry_head = (heads && !(last_is_first && cont_before)) ? last_head : carry_head;
      } else if (is_last && !last_from_before) {  // a run that starts in this window: sums and head slot
        store_part<FEAT>(part + PQ, v);
        part[PQ + 2].w = __uint_as_float((heads && !(last_is_first && cont_before)) ? last_head : carry_head);
      }
    }
    prev_id = id63;
    if (!cont_after) carry_from_before = false;
  }
  const uint32_t wend = min(wlo + WIN, m);
  const bool window_cont_after = wend < m && ids[wend - 1] == ids[wend];
  if (lane == 0)
    a.isect_part_flags[w] = (window_cont_before && before != NO_RUN ? W_CONT_BEFORE : 0u) |
                            (window_cont_after ? W_CONT_AFTER : 0u) | (window_has_head ? W_HAS_HEAD : 0u);
}

// One thread per window: the window where a crossing run starts (it has a head and continues into the next
// window) sums its own piece and the partials of the windows the run covers (the last one follows from the
// run length), in window order, and finishes the run. A run over more than SHORT_SPAN further windows (a
// splat covering hundreds of tiles) is summed by the whole wave instead, 64 windows a step, in a fixed
// order: one wave step per such run, so no lane walks a long chain alone.
constexpr uint32_t SHORT_SPAN = 4;

template <bool FEAT, bool LIVE>
__global__ void __launch_bounds__(64) isect_fixup_kernel(b2c_raster_bwd_args a) {
  constexpr int RED_VALS = ::b2c::dev::RED_VALS<FEAT>;
  constexpr int PQ = PART_Q<FEAT>;
  constexpr uint32_t WIN = RED_WIN<LIVE>;
  const uint32_t nwin = (a.num_isect + WIN - 1u) / WIN;
  const uint32_t w = blockIdx.x * 64u + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const float4* part = reinterpret_cast<const float4*>(a.isect_part);
  // Memory round trip 1: the window's flags, last id and head slot, its own tail partials and the head
  // partials of the next SHORT_SPAN windows. Round trip 2: the run's tile count and previous sums. Every
  // load is unconditional, from a clamped window or id, so no branch splits the loads from their waits.
  const uint32_t wc = min(w, nwin - 1u);
  const uint32_t f = a.isect_part_flags[wc];
  const uint32_t run_ld = a.isect_vals[min(wc * WIN + WIN - 1u, a.num_isect - 1u)];
  const uint32_t head = __float_as_uint(part[(size_t)wc * (2 * PQ) + PQ + 2].w);
  float4 tail[PQ], nxt[SHORT_SPAN][PQ];
#pragma unroll
  for (int k = 0; k < PQ; k++) tail[k] = part[(size_t)wc * (2 * PQ) + PQ + k];
#pragma unroll
  for (uint32_t d = 1; d <= SHORT_SPAN; d++)
#pragma unroll
    for (int k = 0; k < PQ; k++) nxt[d - 1][k] = part[(size_t)min(wc + d, nwin - 1u) * (2 * PQ) + k];
  const bool owner = w < nwin && (f & W_CONT_AFTER) && (f & W_HAS_HEAD);
  const uint32_t run = owner ? run_ld : NO_RUN;
  const uint32_t tc = a.tile_count[run_ld];
  float old_s[RED_VALS];
  prefetch_old<FEAT>(a, run_ld, old_s);
  // the run covers emit positions [head, head + tile_count)
  const uint32_t last_win = owner ? min((head + tc - 1u) / WIN, nwin - 1u) : 0u;
  const bool short_run = owner && last_win - w <= SHORT_SPAN;
  if (short_run) {
    float v[RED_VALS];
#pragma unroll
    for (int k = 0; k < RED_VALS; k++) v[k] = 0.f;
    add_part<FEAT>(tail, v);
#pragma unroll
    for (uint32_t d = 1; d <= SHORT_SPAN; d++)
      if (w + d <= last_win) add_part<FEAT>(nxt[d - 1], v);  // the run's rows at the start of w + d
    finish_run<FEAT>(a, run, v, old_s);
  }
  // long runs: every lane of the wave stays to here (no early exit), so the cross-lane sums are whole
  uint64_t longs = ballot64(owner && !short_run);
  while (longs) {
    const int src = __builtin_ctzll(longs);
    longs &= longs - 1ull;
    const uint32_t lw = (uint32_t)__builtin_amdgcn_readlane((int)w, src);
    const uint32_t lrun = (uint32_t)__builtin_amdgcn_readlane((int)run, src);
    const uint32_t llast = (uint32_t)__builtin_amdgcn_readlane((int)last_win, src);
    float v[RED_VALS];
#pragma unroll
    for (int k = 0; k < RED_VALS; k++) v[k] = 0.f;
    for (uint32_t x0 = lw + 1; x0 <= llast; x0 += 64u) {
      const uint32_t x = x0 + (uint32_t)lane;
      if (x <= llast) add_part<FEAT>(part + (size_t)x * (2 * PQ), v);
    }
#pragma unroll
    for (int k = 0; k < RED_VALS; k++) {
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) v[k] += __shfl_xor(v[k], o);
    }
    if (lane == src) {
      add_part<FEAT>(part + (size_t)lw * (2 * PQ) + PQ, v);
      float old[RED_VALS];
      prefetch_old<FEAT>(a, lrun, old);
      finish_run<FEAT>(a, lrun, v, old);
    }
  }
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" int b2c_hip_raster_bwd(const b2c_raster_bwd_args* a, hipStream_t stream) {
  const int n_tiles = a->tiles_x * a->tiles_y;
  if (n_tiles <= 0) return 0;
  const dim3 grid(NUM_XCD * xcd_tiles_per(n_tiles)), block(64);
  const bool feat = a->feat != 0, hollow = a->hollow_z != nullptr && a->hollow_lam != 0.f;
  if (feat && !a->v_feat) return (int)hipErrorInvalidValue;
  if (a->defer_vis && (a->mode != 1 || feat || !a->v_splat_zero)) return (int)hipErrorInvalidValue;
  if (a->mode == 0) {
    if (feat && !a->proj3) return (int)hipErrorInvalidValue;
    if (feat) {
      if (hollow) raster_bwd_fp32_kernel<true, true><<<grid, block, 0, stream>>>(*a);
      else raster_bwd_fp32_kernel<true, false><<<grid, block, 0, stream>>>(*a);
    } else {
      if (hollow) raster_bwd_fp32_kernel<false, true><<<grid, block, 0, stream>>>(*a);
      else raster_bwd_fp32_kernel<false, false><<<grid, block, 0, stream>>>(*a);
    }
  } else {
    if (!a->slot_sorted || !a->isect_rows || !a->isect_vals || !a->tile_count || !a->raster_rec)
      return (int)hipErrorInvalidValue;
    if (a->cvals && (!a->cslots || !a->clast || !a->cend)) return (int)hipErrorInvalidValue;
    if (a->num_isect && (a->row_tag == 0u || (a->row_tag & a->tile_mask) != 0u))
      return (int)hipErrorInvalidValue;
    if (feat) {
      if (hollow) raster_bwd_mfma_kernel<true, true><<<grid, block, 0, stream>>>(*a);
      else raster_bwd_mfma_kernel<true, false><<<grid, block, 0, stream>>>(*a);
    } else {
      if (hollow) raster_bwd_mfma_kernel<false, true><<<grid, block, 0, stream>>>(*a);
      else raster_bwd_mfma_kernel<false, false><<<grid, block, 0, stream>>>(*a);
    }
    if (a->split_event) {
      const int e = (int)hipEventRecord(static_cast<hipEvent_t>(a->split_event), stream);
      if (e) return e;
    }
    const bool live = a->row_live != nullptr;
    const uint32_t win = live ? RED_WIN<true> : RED_WIN<false>;
    const uint32_t windows = (a->num_isect + win - 1u) / win;
    if (windows) {
      if (!a->isect_part || !a->isect_part_flags) return (int)hipErrorInvalidValue;
      const dim3 rgrid((windows + 3u) / 4u), rblock(256), fgrid((windows + 63u) / 64u), fblock(64);
      if (feat) {
        if (live) {
          isect_reduce_kernel<true, true><<<rgrid, rblock, 0, stream>>>(*a);
          isect_fixup_kernel<true, true><<<fgrid, fblock, 0, stream>>>(*a);
        } else {
          isect_reduce_kernel<true, false><<<rgrid, rblock, 0, stream>>>(*a);
          isect_fixup_kernel<true, false><<<fgrid, fblock, 0, stream>>>(*a);
        }
      } else {
        if (live) {
          isect_reduce_kernel<false, true><<<rgrid, rblock, 0, stream>>>(*a);
          isect_fixup_kernel<false, true><<<fgrid, fblock, 0, stream>>>(*a);
        } else {
          isect_reduce_kernel<false, false><<<rgrid, rblock, 0, stream>>>(*a);
          isect_fixup_kernel<false, false><<<fgrid, fblock, 0, stream>>>(*a);
        }
      }
    }
  }
  return (int)hipGetLastError();
}
