// Projection (replaces src/gpu/project.cu:8-126): one thread per splat, EWA projection, SH colour, the
// feature lanes (pseudo-normal or a caller's buffer), exact ellipse/8x8-tile test over the splat's tile
// bounding box. Splats of at most 64 bbox tiles (the reference's limit is 32, a warp's mask) are tested by
// the wave together, into a 64-bit hit mask; splats with more than 64 bbox tiles are not counted by their
// own thread (one thread walking hundreds of tiles stalls its whole wave): they are appended to a list, and
// the workgroup counts their bboxes in chunks of up to 64 * B2C_BIG_CHUNKS tiles, one wave per chunk.
#pragma clang fp contract(off)
#include "b2c_kernels.h"
#include "device_math.h"
#include "screen_splat.h"
#include "raster_common.h"

namespace b2c {
namespace dev {
namespace {

// Four waves per workgroup: with ~92 VGPRs five waves fit per SIMD, and small workgroups desynchronise, so
// one workgroup's memory waits overlap another's arithmetic (1024-thread workgroups, one per CU, ran 25%
// slower). One big-list append per workgroup (same-address atomics serialise).
constexpr int PROJ_BLOCK = 256;

// Tile tests of the wave's small splats (bbox of at most 64 tiles) are shared out over all 64 lanes: the
// splats' bbox areas are prefix-summed across the wave, test t goes to lane t mod 64, which finds the
// owning splat by binary search over the prefix and sets the hit bit in the owner's mask in LDS. A wave
// then costs ceil(sum of areas / 64) tile tests per lane instead of its largest bbox.
struct WaveRec {
  float mx, my, c00, c01, c11, power;
  uint32_t origin;  // min_x | min_y << 16
  uint32_t bwm;     // bbox width (bits 0-15); a small splat's also (32768 / width + 1) << 16: bit / width =
                    // (bit * that) >> 15 for every bit < 64 (width <= 64: the error bit / 32768 stays below
                    // 1 / width)
};

__device__ __forceinline__ uint32_t pack_small_bw(int bw) {
  return (uint32_t)bw | ((32768u / (uint32_t)max(bw, 1) + 1u) << 16);  // (an empty bbox has no tests)
}

// A big splat's entry (bbox origin min_x | min_y << 16, width, area, chunk length): ceil(area / len) chunks
// of len tiles, len = 64 up to 64 * B2C_BIG_CHUNKS tiles and a multiple of 64 beyond, so no splat has more
// than B2C_BIG_CHUNKS chunks.
__device__ __forceinline__ uint32_t big_bbox_of_len(uint32_t area) {
  const uint32_t per = (area + B2C_BIG_CHUNKS - 1) / B2C_BIG_CHUNKS;
  return per <= 64u ? 64u : ((per + 63u) / 64u) * 64u;
}

__device__ __forceinline__ uint4 big_bbox_of(const TileBox& bb) {
  const uint32_t bw = (uint32_t)(bb.max_x - bb.min_x);
  const uint32_t area = bw * (uint32_t)(bb.max_y - bb.min_y);
  return make_uint4((uint32_t)bb.min_x | ((uint32_t)bb.min_y << 16), bw, area, big_bbox_of_len(area));
}

__device__ __forceinline__ uint32_t big_nchunks(uint4 info) { return (info.z + info.w - 1u) / info.w; }

// FEAT: feature lanes (feat_mode 1 or 2); the plain variant writes zeros there and keeps the registers the
// pseudo-normal would hold free (one more resident wave per SIMD at SH degree 3).
template <int DEG, bool HALF, bool FEAT>
__global__ void __launch_bounds__(PROJ_BLOCK) project_kernel(b2c_project_args a) {
  __shared__ WaveRec s_rec[PROJ_BLOCK];
  __shared__ uint32_t s_incl[PROJ_BLOCK];
  __shared__ uint32_t s_mask[2][PROJ_BLOCK];  // hit mask bits 0-31, 32-63
  const int i = blockIdx.x * PROJ_BLOCK + threadIdx.x;
  const int lane = lane_id();
  const int wbase = threadIdx.x & ~63;
  // the pair of counters the next projection appends to (nothing touches it in this one)
  if (a.clear_next && i == 0) *reinterpret_cast<unsigned long long*>(a.clear_next) = 0ull;
  bool big = false;
  bool small = false;
  uint32_t area = 0;
  TileBox bb{0, 0, 0, 0};
  if (i < a.n) {
    const float4 po = reinterpret_cast<const float4*>(a.pos_op)[i];
    const float4 q = reinterpret_cast<const float4*>(a.quat)[i];
    const float4 ls = reinterpret_cast<const float4*>(a.lscale)[i];
    constexpr int K = (DEG + 1) * (DEG + 1);
    float coef[3 * K];
    {
      const ShView sv{a.sh.dc, reinterpret_cast<const _Float16*>(a.sh.hi16), a.sh.hi32, a.sh.stride};
      sv.load_all<DEG, HALF>(i, coef);
    }
    const ScreenSplat pr = screen_splat(po, q, ls, a.cam);
    if (!pr.ok) {
      a.tile_count[i] = 0u;
      a.depth_bits[i] = 0xFFFFFFFFu;  // no tiles: sorts last
    } else {
      const float power = det_logf(pr.opacity * 255.f);
      bb = tile_bbox(pr.px, pr.py, pr.ex, pr.ey, a.tiles_x, a.tiles_y);
      const int bw = bb.max_x - bb.min_x, bh = bb.max_y - bb.min_y;
      big = bw * bh > 64;
      small = !big;
      if (small) {
        area = (uint32_t)(bw * bh);
        s_rec[threadIdx.x] = WaveRec{pr.px, pr.py, pr.conic.c00, pr.conic.c01, pr.conic.c11, power,
                                     (uint32_t)bb.min_x | ((uint32_t)bb.min_y << 16), pack_small_bw(bw)};
      } else {  // big: the geometry as the emit reads it back from the raster record (halved diagonal)
        s_rec[threadIdx.x] = WaveRec{pr.px, pr.py, 2.f * (0.5f * pr.conic.c00), pr.conic.c01,
                                     2.f * (0.5f * pr.conic.c11), power,
                                     (uint32_t)bb.min_x | ((uint32_t)bb.min_y << 16), (uint32_t)bw};
      }
      // SH colour at the camera-to-splat direction (project.cu:44-55)
      const float vl = sqrtf((pr.d[0] * pr.d[0] + pr.d[1] * pr.d[1]) + pr.d[2] * pr.d[2]);
      const float inv = 1.f / fmaxf(vl, 1e-12f);
      const float vx = pr.d[0] * inv, vy = pr.d[1] * inv, vz = pr.d[2] * inv;
      float b[K];
      sh_basis<DEG>(vx, vy, vz, b);
      const int ka = a.active_deg >= DEG ? K : (a.active_deg + 1) * (a.active_deg + 1);
      float cr = coef[0] * b[0], cg = coef[1] * b[0], cb = coef[2] * b[0];
#pragma unroll
      for (int k = 1; k < K; k++) {
        if (k < ka) {  // uniform: the active degree
          cr = cr + coef[k * 3] * b[k];
          cg = cg + coef[k * 3 + 1] * b[k];
          cb = cb + coef[k * 3 + 2] * b[k];
        }
      }
      cr = cr + 0.5f; cg = cg + 0.5f; cb = cb + 0.5f;
      cr = __builtin_isfinite(cr) ? fminf(fmaxf(cr, -100.f), 100.f) : 0.f;
      cg = __builtin_isfinite(cg) ? fminf(fmaxf(cg, -100.f), 100.f) : 0.f;
      cb = __builtin_isfinite(cb) ? fminf(fmaxf(cb, -100.f), 100.f) : 0.f;
      float f0 = 0.f, f1 = 0.f, f2 = 0.f;
      if (!FEAT) {
      } else if (a.feat_mode == 1) {
        // the pseudo-normal (project.cu:63-71): the local axis of the smallest log scale (the first of
        // equal ones), a column of R(q), as a unit vector turned towards the camera, in camera coordinates
        const AxisPick ax = smallest_axis(ls.x, ls.y, ls.z);
        const float* m = pr.rot.m;
        const float nx = ax.of(m[0], m[1], m[2]), ny = ax.of(m[3], m[4], m[5]), nz = ax.of(m[6], m[7], m[8]);
        const float il = 1.f / fmaxf(sqrtf((nx * nx + ny * ny) + nz * nz), 1e-12f);
        const float sx = nx * il, sy = ny * il, sz = nz * il;
        // pr.d runs from the camera to the splat: the axis faces the camera when it points against it
        const float face = ((sx * -pr.d[0] + sy * -pr.d[1]) + sz * -pr.d[2]) >= 0.f ? 1.f : -1.f;
        const float wx = sx * face, wy = sy * face, wz = sz * face;
        const float* R = a.cam.R;
        f0 = (R[0] * wx + R[1] * wy) + R[2] * wz;
        f1 = (R[3] * wx + R[4] * wy) + R[5] * wz;
        f2 = (R[6] * wx + R[7] * wy) + R[8] * wz;
      } else if (a.feat_mode == 2) {  // a caller's per-splat feature, clamped as a colour is
        f0 = a.feat_buffer[(size_t)i * 3];
        f1 = a.feat_buffer[(size_t)i * 3 + 1];
        f2 = a.feat_buffer[(size_t)i * 3 + 2];
        f0 = __builtin_isfinite(f0) ? fminf(fmaxf(f0, -100.f), 100.f) : 0.f;
        f1 = __builtin_isfinite(f1) ? fminf(fmaxf(f1, -100.f), 100.f) : 0.f;
        f2 = __builtin_isfinite(f2) ? fminf(fmaxf(f2, -100.f), 100.f) : 0.f;
      }
      a.depth_bits[i] = __float_as_uint(pr.c[2]);
      if (a.proj0) {  // the reference's projection buffers, for callers that read them
        reinterpret_cast<float4*>(a.proj0)[i] = make_float4(pr.px, pr.py, pr.conic.c00, pr.conic.c01);
        reinterpret_cast<float4*>(a.proj1)[i] = make_float4(pr.conic.c11, pr.opacity, pr.c[2], power);
        reinterpret_cast<float4*>(a.proj2)[i] = make_float4(cr, cg, cb, f0);
        reinterpret_cast<float2*>(a.proj3)[i] = make_float2(f1, f2);
      }
      {  // halving the conic diagonal is exact: the raster evaluates the reference's sigma
        float4* rec = reinterpret_cast<float4*>(a.raster_rec) + (size_t)i * 4;
        const uint32_t sgn = (cr >= 0.f ? 1u : 0u) | (cg >= 0.f ? 2u : 0u) | (cb >= 0.f ? 4u : 0u);
        rec[0] = make_float4(pr.px, pr.py, 0.5f * pr.conic.c00, pr.conic.c01);
        rec[1] = make_float4(0.5f * pr.conic.c11, pr.opacity, power, __uint_as_float(sgn));
        rec[2] = make_float4(fmaxf(cr, 0.f), fmaxf(cg, 0.f), fmaxf(cb, 0.f), log2_opacity(pr.opacity));
        rec[3] = make_float4(f0, f1, f2, pr.c[2]);  // read by the feature and hollow-loss variants and the depth probe
      }
      if (a.max_screen) {
        float ms = fmaxf(pr.ex / (float)a.cam.W, pr.ey / (float)a.cam.H);
        a.max_screen[i] = fmaxf(a.max_screen[i], ms);
      }
    }
  }
  // ---- wave-cooperative tile tests of the small splats
  uint32_t incl = area;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  const uint32_t total = __shfl(incl, 63);
  s_incl[threadIdx.x] = incl;
  s_mask[0][threadIdx.x] = 0u;
  s_mask[1][threadIdx.x] = 0u;
  __syncthreads();
  for (uint32_t t0 = 0; t0 < total; t0 += 64) {
    const uint32_t t = t0 + (uint32_t)lane;
    if (t < total) {
      int lo = 0, hi = 63;  // owner: the first lane whose inclusive prefix exceeds t
#pragma unroll
      for (int step = 0; step < 6; step++) {
        const int mid = (lo + hi) >> 1;
        if (s_incl[wbase + mid] > t) hi = mid; else lo = mid + 1;
      }
      const int owner = lo;
      const WaveRec rec = s_rec[wbase + owner];
      const uint32_t prev = owner == 0 ? 0u : s_incl[wbase + owner - 1];
      const uint32_t bit = t - prev;
      const uint32_t bw = rec.bwm & 0xFFFFu;
      const uint32_t row = (bit * (rec.bwm >> 16)) >> 15;  // bit / bw
      const int tx = (int)(rec.origin & 0xFFFFu) + (int)(bit - row * bw);
      const int ty = (int)(rec.origin >> 16) + (int)row;
      const float rx = tx * (float)RT_W, ry = ty * (float)RT_W;
      if (tile_hit(rx, ry, rx + RT_W, ry + RT_W, rec.mx, rec.my, Sym2{rec.c00, rec.c01, rec.c11}, rec.power))
        atomicOr(&s_mask[bit >> 5][wbase + owner], 1u << (bit & 31u));
    }
  }
  __syncthreads();
  if (small || big) {
    const uint32_t info = (uint32_t)bb.min_x | ((uint32_t)bb.min_y << 12) | ((uint32_t)(bb.max_x - bb.min_x) << 24);
    const uint32_t lo = small ? s_mask[0][threadIdx.x] : 0u, hi = small ? s_mask[1][threadIdx.x] : 0u;
    // The mask word of hit_info keeps the reference's meaning (binning.cu:37): the mask of a bbox of at
    // most 32 tiles, or 0xFFFFFFFF ("recompute"). A bbox of 33 to 64 tiles, or a full 32-tile mask (which
    // reads as "recompute"), keeps its mask in hit_wide; a big splat marks hit_wide (0, 0).
    const bool wide = big || area > 32u || lo == 0xFFFFFFFFu;
    reinterpret_cast<uint2*>(a.hit_info)[i] = make_uint2(wide ? 0xFFFFFFFFu : lo, info);
    if (wide) reinterpret_cast<uint2*>(a.hit_wide)[i] = make_uint2(lo, hi);
    if (small) {
      const uint32_t count = (uint32_t)(__popc(lo) + __popc(hi));
      a.tile_count[i] = count;
      if (count == 0u) a.depth_bits[i] = 0xFFFFFFFFu;  // no tiles: sorts last
    }
  }
  // Big splats: a big-list entry each (bbox, chunk length) and one work item per chunk of the bbox, both
  // appended with one device-scope atomic per workgroup (contended atomics on one address are serialised
  // at the memory side and cost ~10 ns each). The workgroup then counts the hits of its own big splats'
  // chunks, one wave per chunk (the emit needs each chunk's count), and writes their tile counts.
  const uint64_t bm = ballot64(big);
  if (__syncthreads_or(big ? 1 : 0)) {  // uniform per workgroup: the barriers below are reached by all or none
    __shared__ uint32_t s_wcount[PROJ_BLOCK / 64], s_witems[PROJ_BLOCK / 64];
    __shared__ uint32_t s_base, s_item_base, s_nbig, s_nitems;
    // by workgroup-local big index: the thread (its s_rec slot), bbox area, first chunk, hits counted
    __shared__ uint32_t s_bthread[PROJ_BLOCK], s_barea[PROJ_BLOCK], s_cstart[PROJ_BLOCK], s_btot[PROJ_BLOCK];
    uint4 info = make_uint4(0u, 0u, 0u, 0u);
    uint32_t nch = 0;
    if (big) {
      info = big_bbox_of(bb);
      nch = big_nchunks(info);
    }
    uint32_t incl = nch;  // inclusive prefix of the chunk counts across the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t t = __shfl_up(incl, o);
      if (lane >= o) incl += t;
    }
    const int w = threadIdx.x >> 6;
    if (lane == 63) {
      s_wcount[w] = popc64(bm);
      s_witems[w] = incl;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t tot = 0, items = 0;
      for (int k = 0; k < PROJ_BLOCK / 64; k++) {
        const uint32_t c = s_wcount[k], it = s_witems[k];
        s_wcount[k] = tot;
        s_witems[k] = items;
        tot += c;
        items += it;
      }
      // both counters in one atomic: a second contended atomic per workgroup on the same cache line costs
      // as much again (they are serialised at the memory side)
      const unsigned long long got =
          atomicAdd(reinterpret_cast<unsigned long long*>(a.big_count), (unsigned long long)tot | ((unsigned long long)items << 32));
      s_base = (uint32_t)got;
      s_item_base = (uint32_t)(got >> 32);
      s_nbig = tot;
      s_nitems = items;
    }
    __syncthreads();
    uint32_t lb = 0;  // workgroup-local big index
    if (big) {
      lb = s_wcount[w] + mbcnt64(bm);
      const uint32_t e = s_base + lb;
      a.big_list[e] = (uint32_t)i;
      reinterpret_cast<uint4*>(a.big_info)[e] = info;
      const uint32_t first = s_witems[w] + incl - nch;
      for (uint32_t k = 0; k < nch; k++) a.big_items[s_item_base + first + k] = (e << 5) | k;
      s_bthread[lb] = threadIdx.x;
      s_barea[lb] = info.z;
      s_cstart[lb] = first;
      s_btot[lb] = 0u;
    }
    __syncthreads();
    // chunk q of the workgroup's chunks goes to wave q mod 4; q is wave-uniform
    const uint32_t nbig = s_nbig, nitems = s_nitems;
    for (uint32_t q = (uint32_t)w; q < nitems; q += PROJ_BLOCK / 64) {
      uint32_t lo = 0, hi = nbig - 1;  // the last local big whose first chunk is <= q
      while (lo < hi) {
        const uint32_t mid = (lo + hi + 1u) >> 1;
        if (s_cstart[mid] <= q) lo = mid; else hi = mid - 1u;
      }
      const WaveRec rec = s_rec[s_bthread[lo]];
      const uint32_t ar = s_barea[lo];
      const uint32_t len = big_bbox_of_len(ar);
      const uint32_t k = q - s_cstart[lo];
      const uint32_t begin = k * len, end = min(begin + len, ar);
      const int min_x = (int)(rec.origin & 0xFFFFu), min_y = (int)(rec.origin >> 16), rbw = (int)(rec.bwm & 0xFFFFu);
      uint32_t hits = 0;
      for (uint32_t b0 = begin; b0 < end; b0 += 64) {
        const uint32_t b = b0 + (uint32_t)lane;
        bool h = false;
        if (b < end) {
          const int tx = min_x + (int)(b % (uint32_t)rbw), ty = min_y + (int)(b / (uint32_t)rbw);
          const float rx = tx * (float)RT_W, ry = ty * (float)RT_W;
          h = tile_hit(rx, ry, rx + RT_W, ry + RT_W, rec.mx, rec.my, Sym2{rec.c00, rec.c01, rec.c11}, rec.power);
        }
        hits += popc64(ballot64(h));
      }
      if (lane == 0) {
        a.big_chunk[(size_t)(s_base + lo) * B2C_BIG_CHUNKS + k] = hits;
        atomicAdd(&s_btot[lo], hits);
      }
    }
    __syncthreads();
    if (big) {
      const uint32_t total = s_btot[lb];
      a.tile_count[i] = total;
      if (total == 0u) a.depth_bits[i] = 0xFFFFFFFFu;  // no tiles: sorts last
    }
  }
}

__global__ void clear_counters_kernel(uint32_t* a, uint32_t* b) {
  *a = 0u;
  if (b) *b = 0u;
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" int b2c_hip_fill_u32(uint32_t* p, uint32_t value, size_t count, hipStream_t stream) {
  if (count == 0) return 0;
  size_t blocks = (count + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  fill_u32_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(p, value, count);
  return (int)hipGetLastError();
}

template <bool FEAT>
void launch_project(const b2c_project_args& a, dim3 grid, dim3 block, bool half, hipStream_t stream) {
  switch (a.degree * 2 + (half ? 1 : 0)) {
    case 0: project_kernel<0, false, FEAT><<<grid, block, 0, stream>>>(a); break;
    case 2: project_kernel<1, false, FEAT><<<grid, block, 0, stream>>>(a); break;
    case 3: project_kernel<1, true, FEAT><<<grid, block, 0, stream>>>(a); break;
    case 4: project_kernel<2, false, FEAT><<<grid, block, 0, stream>>>(a); break;
    case 5: project_kernel<2, true, FEAT><<<grid, block, 0, stream>>>(a); break;
    case 6: project_kernel<3, false, FEAT><<<grid, block, 0, stream>>>(a); break;
    case 7: project_kernel<3, true, FEAT><<<grid, block, 0, stream>>>(a); break;
    case 8: project_kernel<4, false, FEAT><<<grid, block, 0, stream>>>(a); break;
    default: project_kernel<4, true, FEAT><<<grid, block, 0, stream>>>(a); break;
  }
}

extern "C" int b2c_hip_project(const b2c_project_args* a, hipStream_t stream) {
  if (a->n <= 0) return 0;
  if (a->degree < 0 || a->degree > 4) return (int)hipErrorInvalidValue;
  if (!a->big_count || !a->big_list || !a->hit_wide || !a->raster_rec || !a->depth_bits || !a->big_info ||
      !a->big_chunk || !a->big_items || a->big_items_count != a->big_count + 1 ||
      (reinterpret_cast<uintptr_t>(a->big_count) & 7u))
    return (int)hipErrorInvalidValue;
  if (a->feat_mode < 0 || a->feat_mode > 2 || (a->feat_mode == 2 && !a->feat_buffer)) return (int)hipErrorInvalidValue;
  if (a->clear_next && (reinterpret_cast<uintptr_t>(a->clear_next) & 7u)) return (int)hipErrorInvalidValue;
  // the counters start at zero: cleared by a launch of their own, or (clear_next) by the previous projection
  if (!a->clear_next) clear_counters_kernel<<<1, 1, 0, stream>>>(a->big_count, a->big_items_count);
  dim3 grid((unsigned)((a->n + PROJ_BLOCK - 1) / PROJ_BLOCK)), block(PROJ_BLOCK);
  const bool half = a->degree > 0 && !a->sh.hi32;  // fp16 bands
  if (a->feat_mode) launch_project<true>(*a, grid, block, half, stream);
  else launch_project<false>(*a, grid, block, half, stream);
  return (int)hipGetLastError();
}
