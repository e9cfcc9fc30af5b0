// Consumers of the tile lists (replaces src/train/evidence.cu:47-183 and src/gpu/probe.cu:7-53): per-view
// evidence (each splat's front-to-back weight on the view's pixels, split by the pixel's mask, residual and
// loss weight), the per-class label vote, and the per-pixel depth probe. They reuse the render's bit-exact
// lists and, for the evidence, the forward's last_idx: one wave64 per 8x8 tile, one lane per pixel, the
// list staged through LDS 64 splats at a time, the same sigma, cutoff and alpha as the forward kernel, so a
// replayed fragment carries exactly the blend weight the render gave it.
#include "b2c_kernels.h"
#include "raster_common.h"

namespace b2c {
namespace dev {
namespace {

constexpr int VSTRIDE = 65;  // row stride of the [splat][pixel] weight matrix in LDS (conflict-free columns)
constexpr uint32_t LABEL_NONE = 0xFFFFFFFFu;  // a pixel that takes no part in the label vote

__device__ __forceinline__ float byte_chan(uint32_t p, int c) { return (float)((p >> (8 * c)) & 0xffu) * (1.f / 255.f); }

// Evidence and label vote of one view. Per pixel: m = target alpha * weight (the in-mask mass), m * res with
// res the mean absolute colour residual of the render (plus the weighted normal residual with FEAT), and
// k = (target alpha if the view is masked with alpha, else 1) * weight. Each lane replays its pixel's list
// up to last_idx and writes every fragment's blend weight vis into a [64 splats][64 pixels] LDS matrix; the
// lane of splat j then contracts row j with the pixel vectors (m, m res, k) and adds the three sums to the
// view accumulator (float atomics, once per (tile, splat), as the reference adds them). With LABELS the
// same rows are summed per class over the tile's distinct label values into the splat's class bins.
template <bool FEAT, bool LABELS>
__global__ void __launch_bounds__(64) evidence_kernel(b2c_evidence_args a) {
  __shared__ float4 s_g0[64], s_g1[64];
  __shared__ uint32_t s_id[64];
  __shared__ float s_vis[64 * VSTRIDE];
  __shared__ float s_m[64], s_mr[64], s_k[64];
  __shared__ uint32_t s_lab[64];
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const uint2 range = reinterpret_cast<const uint2*>(a.tile_ranges)[tile];
  if (range.y <= range.x) return;
  const int lane = threadIdx.x;
  const int px = (tile % a.tiles_x) * RT_W + (lane & 7), py = (tile / a.tiles_x) * RT_W + (lane >> 3);
  const bool inside = px < a.W && py < a.H;
  const float pcx = px + 0.5f, pcy = py + 0.5f;
  float m = 0.f, mres = 0.f, k = 0.f;
  uint32_t last = range.x, lab = LABEL_NONE;
  if (inside) {
    const int pix = py * a.W + px;
    const uint32_t g = a.gt[pix];
    const float ga = byte_chan(g, 3);
    const float wp = a.weights ? (float)a.weights[pix] * (1.f / 255.f) : 1.f;
    const float4 o = reinterpret_cast<const float4*>(a.out_rgba)[pix];
    float res = (fabsf(o.x - byte_chan(g, 0)) + fabsf(o.y - byte_chan(g, 1)) + fabsf(o.z - byte_chan(g, 2))) * (1.f / 3.f);
    if constexpr (FEAT) {
      const uint32_t gn = a.normals[pix];
      if (((gn >> 24) & 0xffu) > 127u) {  // the normal loss's residual (loss.cu:218-223), weighted
        const float nx = (float)(gn & 0xffu) * (2.f / 255.f) - 1.f;
        const float ny = 1.f - (float)((gn >> 8) & 0xffu) * (2.f / 255.f);
        const float nz = 1.f - (float)((gn >> 16) & 0xffu) * (2.f / 255.f);
        const float4 f = reinterpret_cast<const float4*>(a.out_feat)[pix];
        const float pl = fmaxf(sqrtf(f.x * f.x + f.y * f.y + f.z * f.z), 1e-6f);
        const float nl = fmaxf(sqrtf(nx * nx + ny * ny + nz * nz), 1e-6f);
        const float nres = fabsf(f.x - nx) + fabsf(f.y - ny) + fabsf(f.z - nz) + 1.f - (f.x * nx + f.y * ny + f.z * nz) / (pl * nl);
        res += a.normal_weight * nres;
      }
    }
    m = ga * wp;
    mres = m * res;
    k = (a.masked_has_alpha ? ga : 1.f) * wp;
    last = a.last_idx[pix];
    if constexpr (LABELS) {
      lab = a.labels[pix];
      if (lab >= (uint32_t)B2C_LABEL_BINS || !(k != 0.f)) lab = LABEL_NONE;
    }
  }
  s_m[lane] = m;
  s_mr[lane] = mres;
  s_k[lane] = k;
  if constexpr (LABELS) s_lab[lane] = lab;
  float T = 1.f;
  for (uint32_t start = range.x; start < range.y; start += 64) {
    const uint32_t count = min(64u, range.y - start);
    __syncthreads();  // the previous batch's LDS is consumed
    if ((uint32_t)lane < count) {
      const uint32_t gid = a.vals_sorted[start + lane];
      s_id[lane] = gid;
      const float4* rec = reinterpret_cast<const float4*>(a.raster_rec) + (size_t)gid * 4;
      const float4 r1 = rec[1], r2 = rec[2];
      s_g0[lane] = rec[0];
      s_g1[lane] = make_float4(r1.x, r2.w, r1.z, 0.f);  // (c11 / 2, log2 opacity, power)
    }
    __syncthreads();
    for (uint32_t j = 0; j < count; j++) {
      const float4 g0 = s_g0[j], g1 = s_g1[j];
      const float sigma = frag_geom(g0.x, g0.y, g0.z, g0.w, g1.x, pcx, pcy).sigma;
      const bool valid = inside & (start + j < last) & (sigma >= 0.f) & (sigma <= g1.z);
      const float alpha = valid ? fminf(ALPHA_MAX, fragment_alpha(sigma, g1.y)) : 0.f;
      const float vis = alpha * T;
      T = T * (1.f - alpha);
      s_vis[j * VSTRIDE + lane] = vis;
    }
    __syncthreads();
    if ((uint32_t)lane < count) {
      const float* row = s_vis + lane * VSTRIDE;
      float a0 = 0.f, a1 = 0.f, a2 = 0.f;
#pragma unroll 8
      for (int p = 0; p < 64; p++) {
        const float v = row[p];
        a0 += v * s_m[p];
        a1 += v * s_mr[p];
        a2 += v * s_k[p];
      }
      float* dst = a.view_acc + (size_t)s_id[lane] * 3;
      if (a0 != 0.f) atomicAdd(dst, a0);
      if (a1 != 0.f) atomicAdd(dst + 1, a1);
      if (a2 != 0.f) atomicAdd(dst + 2, a2);
      if constexpr (LABELS) {
        // the tile's distinct classes, one pass each (labels are spatially coherent: usually one or two)
        uint64_t todo = ~0ull;
        while (true) {
          uint32_t b = LABEL_NONE;
          for (int p = 0; p < 64; p++)
            if (((todo >> p) & 1ull) && s_lab[p] != LABEL_NONE) { b = s_lab[p]; break; }
          if (b == LABEL_NONE) break;
          float sum = 0.f;
          for (int p = 0; p < 64; p++)
            if (s_lab[p] == b) {
              sum += row[p] * s_k[p];
              todo &= ~(1ull << p);
            }
          if (sum != 0.f) atomicAdd(a.label_acc + (size_t)s_id[lane] * B2C_LABEL_BINS + b, sum);
        }
      }
    }
  }
}

// fold_view_kernel (evidence.cu:114-126): the view's sums into the running evidence: w_in, w_all, err, the
// sum of w_in^2 (for the effective view count) and the w_in-weighted unit direction towards the camera.
__global__ void __launch_bounds__(256) fold_view_kernel(int n, const float* __restrict__ view_acc,
                                                        const float* __restrict__ pos_op, float cx, float cy, float cz,
                                                        float* __restrict__ ev) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float w_in = view_acc[(size_t)i * 3], err = view_acc[(size_t)i * 3 + 1], w_all = view_acc[(size_t)i * 3 + 2];
  float* e = ev + (size_t)i * B2C_EVIDENCE_STRIDE;
  e[0] += w_in;
  e[1] += w_all;
  e[2] += err;
  e[7] += w_in * w_in;
  if (w_in != 0.f) {
    const float4 p = reinterpret_cast<const float4*>(pos_op)[i];
    const float dx = cx - p.x, dy = cy - p.y, dz = cz - p.z;
    const float il = 1.f / fmaxf(sqrtf(dx * dx + dy * dy + dz * dz), 1e-12f);
    e[4] += w_in * dx * il;
    e[5] += w_in * dy * il;
    e[6] += w_in * dz * il;
  }
}

// Depth probe (probe.cu:7-53) over the full lists of a projected and binned view: per pixel the accumulated
// alpha, the depth at which it first reaches tau (tau <= 0: the alpha-weighted mean depth, when the pixel is
// more than 5% covered), the weight arriving from more than delta behind that first surface, and the weight
// from more than margin behind the reference depth (if given). The transmittance stop ends a pixel as in the
// forward.
__global__ void __launch_bounds__(64) probe_kernel(b2c_probe_args a) {
  __shared__ float4 s_g0[64], s_g1[64];
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const uint2 range = reinterpret_cast<const uint2*>(a.tile_ranges)[tile];
  const int lane = threadIdx.x;
  const int px = (tile % a.tiles_x) * RT_W + (lane & 7), py = (tile / a.tiles_x) * RT_W + (lane >> 3);
  const bool inside = px < a.W && py < a.H;
  const float pcx = px + 0.5f, pcy = py + 0.5f;
  const bool mean_mode = a.tau <= 0.f;
  float T = 1.f, z_first = __builtin_inff(), deep = 0.f, behind = 0.f, zsum = 0.f;
  const float zr = (inside && a.ref_z) ? a.ref_z[py * a.W + px] : __builtin_inff();
  bool live = inside;
  for (uint32_t start = range.x; start < range.y; start += 64) {
    if (ballot64(live) == 0ull) break;
    const uint32_t count = min(64u, range.y - start);
    __syncthreads();
    if ((uint32_t)lane < count) {
      const uint32_t gid = a.vals_sorted[start + lane];
      const float4* rec = reinterpret_cast<const float4*>(a.raster_rec) + (size_t)gid * 4;
      const float4 r1 = rec[1], r2 = rec[2], r3 = rec[3];
      s_g0[lane] = rec[0];
      s_g1[lane] = make_float4(r1.x, r2.w, r1.z, r3.w);  // (c11 / 2, log2 opacity, power, depth)
    }
    __syncthreads();
    for (uint32_t j = 0; j < count; j++) {
      const float4 g0 = s_g0[j], g1 = s_g1[j];
      const float sigma = frag_geom(g0.x, g0.y, g0.z, g0.w, g1.x, pcx, pcy).sigma;
      if (!live || !(sigma >= 0.f && sigma <= g1.z)) continue;
      const float alpha = fminf(ALPHA_MAX, fragment_alpha(sigma, g1.y));
      const float next_T = T * (1.f - alpha);
      if (next_T <= T_CUTOFF) {
        live = false;
        continue;
      }
      const float vis = alpha * T;
      const float z = g1.w;
      if (__builtin_isfinite(z_first) && z > z_first + a.delta) deep += vis;
      if (z > zr + a.margin) behind += vis;
      if (mean_mode) zsum = fmaf(vis, z, zsum);
      T = next_T;
      if (!__builtin_isfinite(z_first) && 1.f - T >= a.tau) z_first = z;
    }
  }
  if (mean_mode) z_first = (1.f - T) > 0.05f ? zsum / (1.f - T) : __builtin_inff();
  if (inside) reinterpret_cast<float4*>(a.out)[py * a.W + px] = make_float4(1.f - T, z_first, deep, behind);
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" int b2c_hip_evidence_view(const b2c_evidence_args* a, hipStream_t stream) {
  const int n_tiles = a->tiles_x * a->tiles_y;
  if (n_tiles <= 0) return 0;
  if (!a->raster_rec || !a->view_acc || !a->gt || !a->out_rgba || !a->last_idx) return (int)hipErrorInvalidValue;
  const bool feat = a->normals && a->normal_weight > 0.f;
  const bool labels = a->labels && a->label_acc;
  if (feat && !a->out_feat) return (int)hipErrorInvalidValue;
  const dim3 grid(NUM_XCD * xcd_tiles_per(n_tiles)), block(64);
  if (feat) {
    if (labels) evidence_kernel<true, true><<<grid, block, 0, stream>>>(*a);
    else evidence_kernel<true, false><<<grid, block, 0, stream>>>(*a);
  } else {
    if (labels) evidence_kernel<false, true><<<grid, block, 0, stream>>>(*a);
    else evidence_kernel<false, false><<<grid, block, 0, stream>>>(*a);
  }
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_evidence_fold(int n, const float* view_acc, const float* pos_op, const float cam_pos[3],
                                     float* evidence, hipStream_t stream) {
  if (n <= 0) return 0;
  fold_view_kernel<<<(n + 255) / 256, 256, 0, stream>>>(n, view_acc, pos_op, cam_pos[0], cam_pos[1], cam_pos[2],
                                                       evidence);
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_probe_depth(const b2c_probe_args* a, hipStream_t stream) {
  const int n_tiles = a->tiles_x * a->tiles_y;
  if (n_tiles <= 0) return 0;
  if (!a->raster_rec || !a->out) return (int)hipErrorInvalidValue;
  probe_kernel<<<dim3(NUM_XCD * xcd_tiles_per(n_tiles)), dim3(64), 0, stream>>>(*a);
  return (int)hipGetLastError();
}
