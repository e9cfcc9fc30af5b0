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

constexpr int VSTRIDE = 68;  // row stride of the [splat][pixel] weight matrix in LDS (16-byte rows; a row's
                             // 16-byte reads by consecutive lanes start 4 banks apart)
constexpr uint32_t LABEL_NONE = 0xFFFFFFFFu;  // a pixel that takes no part in the label vote

__device__ __forceinline__ float byte_chan(uint32_t p, int c) { return (float)((p >> (8 * c)) & 0xffu) * (1.f / 255.f); }

// Evidence and label vote of one view. Per pixel: m = target alpha * weight (the in-mask mass), m * res with
// res the mean absolute colour residual of the render (plus the weighted normal residual with FEAT), and
// k = (target alpha if the view is masked with alpha, else 1) * weight. Each lane replays its pixel's list
// up to last_idx and writes every fragment's blend weight vis into a [64 splats][64 pixels] LDS matrix; the
// lane of splat j then contracts row j with the pixel vectors (m, m res, k) and stores the three sums as the
// (tile, splat) row at the entry's emit position (the reference adds them to the splat with float atomics,
// which MI355X performs past the per-XCD L2; evidence_reduce_kernel sums each splat's rows instead). With
// LABELS the tile's distinct classes are found once (ballots: labels are spatially coherent, a tile usually
// holds one or two), each with a pixel vector k * [pixel in the class]; the same rows are contracted with
// those vectors and added to the splat's class bins with float atomics. Classes beyond the first MAXC of a
// tile take a slower pass over the pixels.
constexpr int MAXC = 4;  // classes per tile with their own pixel vector

template <bool FEAT, bool LABELS>
__global__ void __launch_bounds__(64) evidence_kernel(b2c_evidence_args a) {
  __shared__ float4 s_g0[64], s_g1[64];
  __shared__ uint32_t s_id[64];
  __shared__ __attribute__((aligned(16))) float s_vis[64 * VSTRIDE];
  __shared__ __attribute__((aligned(16))) float s_m[64], s_mr[64], s_k[64];
  __shared__ __attribute__((aligned(16))) float s_kc[LABELS ? MAXC : 1][64];  // k of the tile's c-th class's pixels, else 0
  __shared__ uint32_t s_lab[64];                 // class of the pixels beyond the first MAXC classes
  __shared__ uint32_t s_slot[64];
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const uint2 range = reinterpret_cast<const uint2*>(a.tile_ranges)[tile];
  const int lane = threadIdx.x;
  float4* rows = reinterpret_cast<float4*>(a.rows);
  // entries past the shrunk end composited nowhere: they get no row (the sum reads a row without this
  // pass's tag as zero)
  if (range.y <= range.x) return;
  const int px = (tile % a.tiles_x) * RT_W + (lane & 7), py = (tile / a.tiles_x) * RT_W + (lane >> 3);
  const bool inside = px < a.W && py < a.H;
  const float pcx = px + 0.5f, pcy = py + 0.5f;
  const float tcx = (tile % a.tiles_x) * RT_W + RT_W * 0.5f, tcy = (tile / a.tiles_x) * RT_W + RT_W * 0.5f;
  const PixelPoly pp = pixel_poly(pcx - tcx, pcy - tcy);
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
  uint32_t cls[MAXC] = {0u, 0u, 0u, 0u};  // wave-uniform: the tile's first classes, in pixel order
  int ncls = 0;
  bool rest = false;  // a pixel's class is not among them
  if constexpr (LABELS) {
    uint64_t todo = ballot64(lab != LABEL_NONE);
    int my_c = -1;
    while (todo != 0ull && ncls < MAXC) {
      const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)lab, __builtin_ctzll(todo));
      const uint64_t hit = ballot64(lab == b);
      if (lab == b) my_c = ncls;
      cls[ncls++] = b;
      todo &= ~hit;
    }
    rest = todo != 0ull;
#pragma unroll
    for (int c = 0; c < MAXC; c++) s_kc[c][lane] = my_c == c ? k : 0.f;
    s_lab[lane] = my_c < 0 ? lab : LABEL_NONE;
  }
  float T = 1.f;
  for (uint32_t start = range.x; start < range.y; start += 64) {
    const uint32_t count = min(64u, range.y - start);
    __syncthreads();  // the previous batch's LDS is consumed
    if ((uint32_t)lane < count) {
      const uint32_t gid = a.vals_sorted[start + lane];
      s_id[lane] = gid;
      s_slot[lane] = a.slot_sorted[start + lane];
      const float4* rec = reinterpret_cast<const float4*>(a.raster_rec) + (size_t)gid * 4;
      const float4 r0 = rec[0], r1 = rec[1], r2 = rec[2];
      const float3 def = sigma_coefs(r0.x, r0.y, r0.z, r0.w, r1.x, tcx, tcy);
      s_g0[lane] = make_float4(def.x, def.y, def.z, r0.z);
      s_g1[lane] = make_float4(r0.w, r2.w, r1.z, r1.x);  // (c01, log2 opacity, power, c11 / 2)
    }
    __syncthreads();
    for (uint32_t j = 0; j < count; j++) {
      const float4 g0 = s_g0[j], g1 = s_g1[j];
      const float sigma = poly_sigma(g0.w, g1.x, g1.w, g0.x, g0.y, g0.z, pp);
      const bool valid = inside & (start + j < last) & (sigma <= g1.z);
      const float alpha = valid ? fminf(ALPHA_MAX, fragment_alpha(sigma, g1.y)) : 0.f;
      const float vis = alpha * T;
      T = T * (1.f - alpha);
      s_vis[j * VSTRIDE + lane] = vis;
    }
    __syncthreads();
    if ((uint32_t)lane < count) {
      const float* row = s_vis + lane * VSTRIDE;
      // four pixels per 16-byte LDS read: the row, and the pixel vectors (broadcast to every lane)
      const float4* row4 = reinterpret_cast<const float4*>(row);
      float a0 = 0.f, a1 = 0.f, a2 = 0.f;
#pragma unroll 4
      for (int q = 0; q < 16; q++) {
        const float4 v = row4[q];
        const float4 m4 = reinterpret_cast<const float4*>(s_m)[q], r4 = reinterpret_cast<const float4*>(s_mr)[q],
                     k4 = reinterpret_cast<const float4*>(s_k)[q];
        a0 += v.x * m4.x; a0 += v.y * m4.y; a0 += v.z * m4.z; a0 += v.w * m4.w;
        a1 += v.x * r4.x; a1 += v.y * r4.y; a1 += v.z * r4.z; a1 += v.w * r4.w;
        a2 += v.x * k4.x; a2 += v.y * k4.y; a2 += v.z * k4.z; a2 += v.w * k4.w;
      }
      rows[s_slot[lane]] = make_float4(a0, a1, a2, __uint_as_float(a.row_tag));
      if constexpr (LABELS) {
        float* bins = a.label_acc + (size_t)s_id[lane] * B2C_LABEL_BINS;
        if (ncls == 1) {
          float c0 = 0.f;
#pragma unroll 4
          for (int q = 0; q < 16; q++) {
            const float4 v = row4[q], k4 = reinterpret_cast<const float4*>(s_kc[0])[q];
            c0 += v.x * k4.x; c0 += v.y * k4.y; c0 += v.z * k4.z; c0 += v.w * k4.w;
          }
          if (c0 != 0.f) atomicAdd(bins + cls[0], c0);
        } else if (ncls > 1) {
          float cc[MAXC] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
          for (int q = 0; q < 16; q++) {
            const float4 v = row4[q];
#pragma unroll
            for (int c = 0; c < MAXC; c++) {
              const float4 k4 = reinterpret_cast<const float4*>(s_kc[c])[q];
              cc[c] += v.x * k4.x; cc[c] += v.y * k4.y; cc[c] += v.z * k4.z; cc[c] += v.w * k4.w;
            }
          }
#pragma unroll
          for (int c = 0; c < MAXC; c++)
            if (c < ncls && cc[c] != 0.f) atomicAdd(bins + cls[c], cc[c]);
        }
        if (rest) {  // classes past the first MAXC of the tile: one pass each
          uint64_t todo = ~0ull;
          while (true) {
            uint32_t b = LABEL_NONE;
            for (int p = 0; p < 64; p++)
              if (((todo >> p) & 1ull) && s_lab[p] != LABEL_NONE) {
                b = s_lab[p];
                break;
              }
            if (b == LABEL_NONE) break;
            float sum = 0.f;
            for (int p = 0; p < 64; p++)
              if (s_lab[p] == b) {
                sum += row[p] * s_k[p];
                todo &= ~(1ull << p);
              }
            if (sum != 0.f) atomicAdd(bins + b, sum);
          }
        }
      }
    }
  }
}

// The view's per-splat sums: one lane per emit position, a segmented inclusive scan across the wave over
// the splat ids of the emit order (a splat's rows are contiguous), and the last lane of each run piece adds
// the piece's sums to the splat's view accumulator (one float atomic per piece and value: about one per
// splat instead of one per (tile, splat) pair).
__global__ void __launch_bounds__(256) evidence_reduce_kernel(b2c_evidence_sum_args a) {
  const uint32_t s = blockIdx.x * 256u + threadIdx.x;
  const bool valid = s < a.m;
  const uint32_t id = valid ? a.ids[s] : NO_RUN;
  float v[3] = {0.f, 0.f, 0.f};
  const float4 r = reinterpret_cast<const float4*>(a.rows)[valid ? s : 0u];
  if (valid && __float_as_uint(r.w) == a.row_tag) {  // another tag: past its tile's shrunk end, zero
    v[0] = r.x;
    v[1] = r.y;
    v[2] = r.z;
  }
  seg_scan(id, v);
  const uint32_t next = dpp_u32<0x130, 0xF>(id, NO_RUN);  // wave_shl:1: the next lane's id (lane 63: none)
  if (valid && next != id && id < (uint32_t)a.n) {
    float* dst = a.view_acc + (size_t)id * 3;
#pragma unroll
    for (int k = 0; k < 3; k++)
      if (v[k] != 0.f) atomicAdd(dst + k, v[k]);
  }
}

// fold_view_kernel (evidence.cu:114-126): the view's sums into the running evidence: w_in, w_all, err, the
// sum of w_in^2 (for the effective view count) and the w_in-weighted unit direction towards the camera.
__global__ void __launch_bounds__(256) fold_view_kernel(b2c_evidence_sum_args a) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  const float w_in = a.view_acc[(size_t)i * 3], err = a.view_acc[(size_t)i * 3 + 1], w_all = a.view_acc[(size_t)i * 3 + 2];
  float* e = a.evidence + (size_t)i * B2C_EVIDENCE_STRIDE;
  e[0] += w_in;
  e[1] += w_all;
  e[2] += err;
  e[7] += w_in * w_in;
  if (w_in != 0.f) {
    const float4 p = reinterpret_cast<const float4*>(a.pos_op)[i];
    const float dx = a.cam_pos[0] - p.x, dy = a.cam_pos[1] - p.y, dz = a.cam_pos[2] - p.z;
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
// forward, and the walk is the forward's: per 4x4 quadrant lists of each batch (a splat whose ellipse cannot
// reach a quadrant composites nothing there), two list entries per step, no branch per fragment.
__global__ void __launch_bounds__(64) probe_kernel(b2c_probe_args a) {
  // lanes by quadrant as in the forward: lane 16 q + p is pixel p (row-major 4x4) of quadrant q; slot 64
  // is a null splat that pads the shorter quadrant lists
  __shared__ float4 s_g0[65], s_g1[65];
  __shared__ float s_z[65];  // camera depth
  __shared__ uint32_t s_list[4][66];  // per quadrant: LDS byte offsets of its splats, in depth order
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const uint2 range = reinterpret_cast<const uint2*>(a.tile_ranges)[tile];
  const int lane = threadIdx.x;
  const int q = lane >> 4, p = lane & 15;
  const int tx = tile % a.tiles_x, ty = tile / a.tiles_x;
  const int px = tx * RT_W + (q & 1) * 4 + (p & 3), py = ty * RT_W + (q >> 1) * 4 + (p >> 2);
  const float x0 = tx * RT_W + 0.5f, y0 = ty * RT_W + 0.5f;  // the tile's first pixel centre
  const bool inside = px < a.W && py < a.H;
  const float pcx = px + 0.5f, pcy = py + 0.5f;
  const float tcx = tx * RT_W + RT_W * 0.5f, tcy = ty * RT_W + RT_W * 0.5f;  // the tile centre
  const PixelPoly pp = pixel_poly(pcx - tcx, pcy - tcy);
  const bool mean_mode = a.tau <= 0.f;
  float T = 1.f, z_first = __builtin_inff(), deep = 0.f, behind = 0.f, zsum = 0.f;
  const float zr = (inside && a.ref_z) ? a.ref_z[py * a.W + px] : __builtin_inff();
  bool live = inside;
  if (lane < 8) s_list[lane >> 1][64 + (lane & 1)] = 64u * 16u;  // read by the last pair's prefetch
  if (lane == 0) {  // power = 0 and sigma = F = 1: fails the cutoff
    s_g0[64] = make_float4(0.f, 0.f, 1.f, 0.f);
    s_g1[64] = make_float4(0.f, 0.f, 0.f, 0.f);
    s_z[64] = 0.f;
  }
  const char* lds_g0 = reinterpret_cast<const char*>(s_g0);
  const char* lds_g1 = reinterpret_cast<const char*>(s_g1);
  const char* lds_z = reinterpret_cast<const char*>(s_z);
  for (uint32_t start = range.x; start < range.y; start += 64) {
    if (ballot64(live) == 0ull) break;
    const uint32_t remaining = min(64u, range.y - start);
    __syncthreads();
    uint32_t qmask = 0;
    if ((uint32_t)lane < remaining) {
      const uint32_t gid = a.vals_sorted[start + lane];
      const float4* rec = reinterpret_cast<const float4*>(a.raster_rec) + (size_t)gid * 4;
      const float4 r0 = rec[0], r1 = rec[1], r2 = rec[2], r3 = rec[3];
      const float3 def = sigma_coefs(r0.x, r0.y, r0.z, r0.w, r1.x, tcx, tcy);
      s_g0[lane] = make_float4(def.x, def.y, def.z, r0.z);
      s_g1[lane] = make_float4(r0.w, r2.w, r1.z, r1.x);  // (c01, log2 opacity, power, c11 / 2)
      s_z[lane] = r3.w;
      qmask = quadrant_mask(r0.x, r0.y, r0.z, r0.w, r1.x, r1.z, x0, y0);
    }
    uint32_t n_iter = 0;
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (int qq = 0; qq < 4; qq++) {
      const bool mine = (qmask >> qq) & 1u;
      const uint64_t bal = ballot64(mine);
      const uint32_t c = popc64(bal);
      if (mine) s_list[qq][popc64(bal & below)] = (uint32_t)lane * 16u;
      if ((uint32_t)lane >= c) s_list[qq][lane] = 64u * 16u;
      n_iter = max(n_iter, c);
    }
    n_iter = __builtin_amdgcn_readfirstlane(n_iter);
    __syncthreads();
    const uint32_t* my_list = s_list[q];
    uint32_t off0 = my_list[0], off1 = my_list[1];
    // One step, straight-line as in the forward: an invalid fragment, a stopped lane or a null splat
    // contributes alpha = 0 and leaves every sum unchanged. A composited fragment (valid and not stopping the
    // lane) adds its weight to the depth sums and may set z_first.
#define B2C_PROBE_STEP(off, next)                                                                       \
  do {                                                                                                  \
    const float4 g0 = *reinterpret_cast<const float4*>(lds_g0 + (off));                                 \
    const float4 g1 = *reinterpret_cast<const float4*>(lds_g1 + (off));                                 \
    const float sigma = poly_sigma(g0.w, g1.x, g1.w, g0.x, g0.y, g0.z, pp);                             \
    const bool valid = live & (sigma <= g1.z);                                                          \
    float a_cl = fminf(ALPHA_MAX, fragment_alpha(sigma, g1.y));                                         \
    asm volatile("" : "+v"(a_cl));                                                                      \
    const float alpha = valid ? a_cl : 0.f;                                                             \
    const float next_T = __builtin_fmaf(-alpha, T, T);                                                       \
    const bool stop = next_T <= T_CUTOFF;                                                               \
    live = live & !stop;                                                                                \
    const bool comp = valid & !stop;                                                                    \
    const float vis = comp ? alpha * T : 0.f;                                                           \
    const float z = *reinterpret_cast<const float*>(lds_z + ((off) >> 2));                              \
    deep += (__builtin_isfinite(z_first) & (z > z_first + a.delta)) ? vis : 0.f;                        \
    behind += (z > zr + a.margin) ? vis : 0.f;                                                          \
    zsum = comp ? fmaf(vis, z, zsum) : zsum;                                                            \
    T = comp ? next_T : T;                                                                              \
    z_first = (comp & !__builtin_isfinite(z_first) & (1.f - T >= a.tau)) ? z : z_first;                \
    (off) = my_list[next];                                                                              \
  } while (0)
    for (uint32_t i = 0; i < n_iter; i += 2) {
      B2C_PROBE_STEP(off0, i + 2);
      B2C_PROBE_STEP(off1, i + 3);
    }
#undef B2C_PROBE_STEP
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
  if (!a->raster_rec || !a->rows || !a->slot_sorted || !a->gt || !a->out_rgba || !a->last_idx || a->row_tag == 0u)
    return (int)hipErrorInvalidValue;
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

extern "C" int b2c_hip_evidence_sum(const b2c_evidence_sum_args* a, hipStream_t stream) {
  if (a->n <= 0) return 0;
  if (!a->ids || !a->rows || !a->view_acc || !a->pos_op || !a->evidence || a->row_tag == 0u)
    return (int)hipErrorInvalidValue;
  const int fill = b2c_hip_fill_u32(reinterpret_cast<uint32_t*>(a->view_acc), 0u, (size_t)a->n * 3, stream);
  if (fill) return fill;
  if (a->m) evidence_reduce_kernel<<<(a->m + 255) / 256, 256, 0, stream>>>(*a);
  fold_view_kernel<<<(a->n + 255) / 256, 256, 0, stream>>>(*a);
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_probe_depth(const b2c_probe_args* a, hipStream_t stream) {
  const int n_tiles = a->tiles_x * a->tiles_y;
  if (n_tiles <= 0) return 0;
  if (!a->raster_rec || !a->out) return (int)hipErrorInvalidValue;
  probe_kernel<<<dim3(NUM_XCD * xcd_tiles_per(n_tiles)), dim3(64), 0, stream>>>(*a);
  return (int)hipGetLastError();
}
