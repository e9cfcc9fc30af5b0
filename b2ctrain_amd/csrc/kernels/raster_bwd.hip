// Backward through compositing: per-pixel reverse replay from the shrunk range end (T_before = T/(1-alpha),
// running colour remainder S), then a per-splat reduction of the fragment gradients over the tile's 64
// pixels, accumulated into v_splat[n][13] with one global atomic per lane per (tile, contributing splat).
//
// mode 0 (replaces raster_bwd_kernel, src/gpu/raster_bwd.cu:10-156): the 13 lanes + blend weight are
//   reduced with wave64 butterfly shuffles, fp32 throughout. The correctness anchor.
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
};

__device__ __forceinline__ PixelState load_pixel(const b2c_raster_bwd_args& a, int px, int py, uint32_t range_x) {
  PixelState s;
  s.inside = px < a.W && py < a.H;
  s.pcx = px + 0.5f;
  s.pcy = py + 0.5f;
  s.T = 0.f;
  s.last = range_x;
  s.vo = make_float4(0.f, 0.f, 0.f, 0.f);
  s.v_o_w = 0.f;
  float final_a = 0.f;
  if (s.inside) {
    const int pix = py * a.W + px;
    final_a = reinterpret_cast<const float4*>(a.out_rgba)[pix].w;
    s.T = reinterpret_cast<const float4*>(a.out_feat)[pix].w;
    s.last = a.last_idx[pix];
    s.vo = reinterpret_cast<const float4*>(a.v_out)[pix];
    s.v_o_w = (s.vo.w - (a.bg[0] * s.vo.x + a.bg[1] * s.vo.y + a.bg[2] * s.vo.z)) * s.T;
  }
  s.inv_final_a = 1.f / fmaxf(final_a, 1e-5f);
  return s;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ------------------------------------------------------------------------------------------------------
// mode 0: fp32 butterfly reduction
// ------------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) raster_bwd_fp32_kernel(b2c_raster_bwd_args a) {
  __shared__ float4 s0[64], s1[64], s2[64];
  __shared__ uint32_t s_gid[64];
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const uint2 range = reinterpret_cast<const uint2*>(a.tile_ranges)[tile];
  if (range.y <= range.x) return;
  const int lane = threadIdx.x;
  const int tx = tile % a.tiles_x, ty = tile / a.tiles_x;
  const int px = tx * RT_W + (lane & 7), py = ty * RT_W + (lane >> 3);
  PixelState ps = load_pixel(a, px, py, range.x);
  const float Wf = (float)a.W, Hf = (float)a.H;
  float Sx = 0.f, Sy = 0.f, Sz = 0.f;
  const float4* proj0 = reinterpret_cast<const float4*>(a.proj0);
  const float4* proj1 = reinterpret_cast<const float4*>(a.proj1);
  const float4* proj2 = reinterpret_cast<const float4*>(a.proj2);
  for (uint32_t batch_end = range.y; batch_end > range.x;) {
    const uint32_t batch_start = batch_end > range.x + 64 ? batch_end - 64 : range.x;
    const uint32_t count = batch_end - batch_start;
    __syncthreads();
    if ((uint32_t)lane < count) {
      const uint32_t gid = a.vals_sorted[batch_start + lane];
      s_gid[lane] = gid;
      s0[lane] = proj0[gid];
      s1[lane] = proj1[gid];
      s2[lane] = proj2[gid];
    }
    __syncthreads();
    for (int j = (int)count - 1; j >= 0; j--) {
      const uint32_t idx = batch_start + j;
      float g[GRAD_LANES];
#pragma unroll
      for (int k = 0; k < GRAD_LANES; k++) g[k] = 0.f;
      float visw = 0.f;
      bool contrib = ps.inside && idx < ps.last;
      if (contrib) {
        const float4 p0 = s0[j], p1 = s1[j];
        const float dx = ps.pcx - p0.x, dy = ps.pcy - p0.y;
        const float sigma = calc_sigma(ps.pcx, ps.pcy, p0.z, p0.w, p1.x, p0.x, p0.y);
        contrib = sigma >= 0.f && sigma <= p1.w;
        if (contrib) {
          const float gauss = gauss_weight(sigma);
          const float alpha = fminf(ALPHA_MAX, p1.y * gauss);
          const float ra = 1.f / (1.f - alpha);
          const float T_before = ps.T * ra;
          const float vis = alpha * T_before;
          const float4 col = s2[j];
          const float cr = fmaxf(col.x, 0.f), cg = fmaxf(col.y, 0.f), cb = fmaxf(col.z, 0.f);
          g[5] = col.x >= 0.f ? vis * ps.vo.x : 0.f;
          g[6] = col.y >= 0.f ? vis * ps.vo.y : 0.f;
          g[7] = col.z >= 0.f ? vis * ps.vo.z : 0.f;
          const float v_alpha = (T_before * cr - Sx * ra) * ps.vo.x + (T_before * cg - Sy * ra) * ps.vo.y +
                                (T_before * cb - Sz * ra) * ps.vo.z + ps.v_o_w * ra;
          const float v_sigma = -alpha * v_alpha;
          if (p1.y * gauss <= ALPHA_MAX) {
            g[2] = 0.5f * v_sigma * dx * dx;
            g[3] = v_sigma * dx * dy;
            g[4] = 0.5f * v_sigma * dy * dy;
            g[0] = -v_sigma * (p0.z * dx + p0.w * dy);
            g[1] = -v_sigma * (p0.w * dx + p1.x * dy);
            g[8] = v_alpha * gauss;
            g[9] = sqrtf(g[0] * Wf * g[0] * Wf + g[1] * Hf * g[1] * Hf) * ps.inv_final_a;
          }
          Sx += cr * vis; Sy += cg * vis; Sz += cb * vis;
          ps.T = T_before;
          visw = vis;
        }
      }
      if (ballot64(contrib) == 0) continue;
      const float sv = wave_sum(visw);
      float sums[GRAD_LANES];
#pragma unroll
      for (int k = 0; k < GRAD_LANES; k++) sums[k] = wave_sum(g[k]);
      if (lane == 0) {
        const uint32_t gid = s_gid[j];
        a.vis_flag[gid] = 1u;
        if (a.vis_weight) atomicAdd(a.vis_weight + gid, sv);
        float* dst = a.v_splat + (size_t)gid * GRAD_LANES;
#pragma unroll
        for (int k = 0; k < GRAD_LANES; k++) {
          const float v = sums[k] * a.inv_gscale;
          if (v != 0.f) atomicAdd(dst + k, v);
        }
      }
    }
    batch_end = batch_start;
  }
}

// ------------------------------------------------------------------------------------------------------
// mode 1: MFMA reduction
// ------------------------------------------------------------------------------------------------------
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int GROUP = 16;  // splats per MFMA group (N)
constexpr int NTYPES = 4;  // vis, v_alpha * gauss, v_sigma, refine
// basis rows (M): 0-2 v_rgb, 3-5 v_feat, 6 one, 7 u, 8 v, 9 u^2, 10 uv, 11 v^2, 12-15 zero
constexpr int B_ONE = 6, B_U = 7, B_V = 8, B_UU = 9, B_UV = 10, B_VV = 11;

__device__ __forceinline__ float clamp_h(float x) {
  return __builtin_isfinite(x) ? fminf(fmaxf(x, -60000.f), 60000.f) : 0.f;
}

// Split 8 fp32 values into fp16 hi and 2^11-scaled fp16 lo parts.
__device__ __forceinline__ void split8(const float* x, half8& hi, half8& lo) {
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float v = clamp_h(x[e]);
    const _Float16 h = (_Float16)v;
    hi[e] = h;
    lo[e] = (_Float16)((v - (float)h) * LO_SCALE);
  }
}

__global__ void __launch_bounds__(64) raster_bwd_mfma_kernel(b2c_raster_bwd_args a) {
  __shared__ float4 s0[64], s1[64], s2[64];
  __shared__ uint32_t s_gid[64];
  __shared__ __attribute__((aligned(16))) float sS[NTYPES][GROUP][64];  // per-fragment scalars, [type][splat][pixel]
  __shared__ float sC[NTYPES][16][GROUP];                              // reduced [type][basis row][splat]
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const uint2 range = reinterpret_cast<const uint2*>(a.tile_ranges)[tile];
  if (range.y <= range.x) return;
  const int lane = threadIdx.x;
  const int tx = tile % a.tiles_x, ty = tile / a.tiles_x;
  const int lx = lane & 7, ly = lane >> 3;
  const int px = tx * RT_W + lx, py = ty * RT_W + ly;
  const float ox = tx * RT_W + RT_W * 0.5f, oy = ty * RT_W + RT_W * 0.5f;  // tile centre
  const float u = lx + 0.5f - RT_W * 0.5f, v = ly + 0.5f - RT_W * 0.5f;
  PixelState ps = load_pixel(a, px, py, range.x);
  const float Wf = (float)a.W, Hf = (float)a.H;

  // Basis operand A (16 rows x 64 px), built once per tile through sS[0] as scratch.
  {
    float* bm = &sS[0][0][0];  // [16][64]
    const float row[16] = {ps.vo.x, ps.vo.y, ps.vo.z, 0.f, 0.f, 0.f, 1.f, u, v, u * u, u * v, v * v, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 16; m++) bm[m * 64 + lane] = row[m];
  }
  __syncthreads();
  const int nl = lane & 15, kg = lane >> 4;
  half8 A_hi[2], A_lo[2];
  {
    const float* bm = &sS[0][0][0];
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; e++) x[e] = bm[nl * 64 + kb * 32 + kg * 8 + e];
      split8(x, A_hi[kb], A_lo[kb]);
    }
  }
  __syncthreads();

  float Sx = 0.f, Sy = 0.f, Sz = 0.f;
  const float4* proj0 = reinterpret_cast<const float4*>(a.proj0);
  const float4* proj1 = reinterpret_cast<const float4*>(a.proj1);
  const float4* proj2 = reinterpret_cast<const float4*>(a.proj2);
  for (uint32_t batch_end = range.y; batch_end > range.x;) {
    const uint32_t batch_start = batch_end > range.x + 64 ? batch_end - 64 : range.x;
    const int count = (int)(batch_end - batch_start);
    __syncthreads();
    if (lane < count) {
      const uint32_t gid = a.vals_sorted[batch_start + lane];
      s_gid[lane] = gid;
      s0[lane] = proj0[gid];
      s1[lane] = proj1[gid];
      s2[lane] = proj2[gid];
    }
    __syncthreads();
    const int ngroups = (count + GROUP - 1) / GROUP;
    for (int grp = ngroups - 1; grp >= 0; grp--) {
      const int gbase = grp * GROUP;
      const int gcount = min(GROUP, count - gbase);
      // ---- replay: this pixel's four scalars for each splat of the group (zero when not contributing)
      for (int j = GROUP - 1; j >= 0; j--) {
        float s_vis = 0.f, s_va = 0.f, s_vs = 0.f, s_r = 0.f;
        const int sj = gbase + j;
        if (j < gcount && ps.inside && batch_start + (uint32_t)sj < ps.last) {
          const float4 p0 = s0[sj], p1 = s1[sj];
          const float sigma = calc_sigma(ps.pcx, ps.pcy, p0.z, p0.w, p1.x, p0.x, p0.y);
          if (sigma >= 0.f && sigma <= p1.w) {
            const float dx = ps.pcx - p0.x, dy = ps.pcy - p0.y;
            const float gauss = gauss_weight(sigma);
            const float alpha = fminf(ALPHA_MAX, p1.y * gauss);
            const float ra = __builtin_amdgcn_rcpf(1.f - alpha);
            const float T_before = ps.T * ra;
            const float vis = alpha * T_before;
            const float4 col = s2[sj];
            const float cr = fmaxf(col.x, 0.f), cg = fmaxf(col.y, 0.f), cb = fmaxf(col.z, 0.f);
            const float v_alpha = (T_before * cr - Sx * ra) * ps.vo.x + (T_before * cg - Sy * ra) * ps.vo.y +
                                  (T_before * cb - Sz * ra) * ps.vo.z + ps.v_o_w * ra;
            const float v_sigma = -alpha * v_alpha;
            if (p1.y * gauss <= ALPHA_MAX) {
              s_va = v_alpha * gauss;
              s_vs = v_sigma;
              const float vx = -v_sigma * (p0.z * dx + p0.w * dy), vy = -v_sigma * (p0.w * dx + p1.x * dy);
              s_r = __builtin_amdgcn_sqrtf(vx * Wf * vx * Wf + vy * Hf * vy * Hf) * ps.inv_final_a * R_SCALE;
            }
            Sx += cr * vis; Sy += cg * vis; Sz += cb * vis;
            ps.T = T_before;
            s_vis = vis;
          }
        }
        sS[0][j][lane] = s_vis;
        sS[1][j][lane] = s_va;
        sS[2][j][lane] = s_vs;
        sS[3][j][lane] = s_r;
      }
      __syncthreads();
      // ---- reduction over the 64 pixels on MFMA: D[t] (16 basis rows x 16 splats) = A (16 x 64) * S[t]^T
      floatx4 acc_hi[NTYPES], acc_lo[NTYPES];
#pragma unroll
      for (int t = 0; t < NTYPES; t++) {
        acc_hi[t] = floatx4{0.f, 0.f, 0.f, 0.f};
        acc_lo[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
#pragma unroll
        for (int t = 0; t < NTYPES; t++) {
          const float4* src = reinterpret_cast<const float4*>(&sS[t][nl][kb * 32 + kg * 8]);
          const float4 q0 = src[0], q1 = src[1];
          const float x[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
          half8 b_hi, b_lo;
          split8(x, b_hi, b_lo);
          acc_hi[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A_hi[kb], b_hi, acc_hi[t], 0, 0, 0);
          acc_lo[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A_hi[kb], b_lo, acc_lo[t], 0, 0, 0);
          if (t == 0) acc_lo[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A_lo[kb], b_hi, acc_lo[t], 0, 0, 0);
        }
      }
      // D layout: this lane holds rows 4*kg .. 4*kg+3 of column nl
#pragma unroll
      for (int t = 0; t < NTYPES; t++)
#pragma unroll
        for (int rr = 0; rr < 4; rr++) sC[t][kg * 4 + rr][nl] = acc_hi[t][rr] + acc_lo[t][rr] * (1.f / LO_SCALE);
      __syncthreads();
      // ---- per-splat gradients: lane = (part, splat); 16 splats x 4 parts
      {
        const int j = nl, part = kg;
        const float sum_vis = sC[0][B_ONE][j];
        if (j < gcount && sum_vis > 0.f) {
          const int sj = gbase + j;
          const uint32_t gid = s_gid[sj];
          float* dst = a.v_splat + (size_t)gid * GRAD_LANES;
          const float sc = a.inv_gscale;
          if (part == 0 || part == 1) {
            const float4 p0 = s0[sj], p1 = s1[sj];
            const float mx = p0.x - ox, my = p0.y - oy;
            const float sv = sC[2][B_ONE][j], svu = sC[2][B_U][j], svv = sC[2][B_V][j];
            if (part == 0) {
              const float m1u = svu - mx * sv, m1v = svv - my * sv;  // sum v_sigma (u - mx), (v - my)
              const float g0 = -(p0.z * m1u + p0.w * m1v), g1 = -(p0.w * m1u + p1.x * m1v);
              if (g0 != 0.f) atomicAdd(dst + 0, g0 * sc);
              if (g1 != 0.f) atomicAdd(dst + 1, g1 * sc);
            } else {
              const float svuu = sC[2][B_UU][j], svuv = sC[2][B_UV][j], svvv = sC[2][B_VV][j];
              const float m2uu = svuu - 2.f * mx * svu + mx * mx * sv;
              const float m2uv = svuv - my * svu - mx * svv + mx * my * sv;
              const float m2vv = svvv - 2.f * my * svv + my * my * sv;
              const float g2 = 0.5f * m2uu, g3 = m2uv, g4 = 0.5f * m2vv;
              if (g2 != 0.f) atomicAdd(dst + 2, g2 * sc);
              if (g3 != 0.f) atomicAdd(dst + 3, g3 * sc);
              if (g4 != 0.f) atomicAdd(dst + 4, g4 * sc);
            }
          } else if (part == 2) {
            const float4 col = s2[sj];
            const float g5 = col.x >= 0.f ? sC[0][0][j] : 0.f;
            const float g6 = col.y >= 0.f ? sC[0][1][j] : 0.f;
            const float g7 = col.z >= 0.f ? sC[0][2][j] : 0.f;
            if (g5 != 0.f) atomicAdd(dst + 5, g5 * sc);
            if (g6 != 0.f) atomicAdd(dst + 6, g6 * sc);
            if (g7 != 0.f) atomicAdd(dst + 7, g7 * sc);
          } else {
            const float g8 = sC[1][B_ONE][j];
            const float g9 = sC[3][B_ONE][j] * (1.f / R_SCALE);
            if (g8 != 0.f) atomicAdd(dst + 8, g8 * sc);
            if (g9 != 0.f) atomicAdd(dst + 9, g9 * sc);
            a.vis_flag[gid] = 1u;
            if (a.vis_weight) atomicAdd(a.vis_weight + gid, sum_vis);
          }
        }
      }
    }
    batch_end = batch_start;
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
  if (a->mode == 0)
    raster_bwd_fp32_kernel<<<grid, block, 0, stream>>>(*a);
  else
    raster_bwd_mfma_kernel<<<grid, block, 0, stream>>>(*a);
  return (int)hipGetLastError();
}
