// Forward compositing (replaces src/gpu/raster_fwd.cu:8-90): one wave64 per 8x8 tile, one lane per pixel,
// the tile's depth-ordered list staged through LDS 64 splats at a time and split per 4x4 quadrant,
// front-to-back alpha blending with the 1/255 cutoff (sigma <= power), the 0.999 clamp and the 1e-4
// transmittance stop. The whole wave leaves as soon as every lane is done. With bwd_info the tile's range
// end is shrunk to one past the last fragment any pixel composited. FEAT composites the three feature
// lanes as the colour is (without background); HOLLOW sums each pixel's hollow penalty.
#include "b2c_kernels.h"
#include "raster_common.h"

namespace b2c {
namespace dev {
namespace {

// Lanes are grouped by quadrant: lane 16 q + p is pixel p (row-major 4x4) of quadrant q (2x2 over the
// tile). Each batch of up to 64 splats is staged in LDS together with one list per quadrant of the splats
// whose ellipse can reach it (quadrant_mask), in depth order; the wave then runs max over quadrants of the
// list lengths iterations, each lane group taking the next splat of its own quadrant's list. A splat that
// reaches no pixel of a quadrant would contribute alpha = 0 there, so the result equals the plain sweep.
// The loop is branch-free: a lane that has terminated, has run out of its list, or whose fragment fails
// the cutoff contributes alpha = 0, which leaves T, the colour and the last index unchanged. Per splat the
// LDS holds (D, E, F, c00/2), (c01, log2 opacity, power, c11/2) and the colour clamped at 0, staged from
// the projection's 64-byte per-splat record (one cache line per gather): sigma is the tile-centred
// quadratic of raster_common.h (sigma_coefs once per splat and tile, poly_sigma per fragment).

// COMPACT: the tile's compacted list for the MFMA backward (the entries some pixel composited). Each lane
// marks the steps of its quadrant's list where it composited (one bit per step pair, even and odd steps
// apart); after the batch the marks are OR-ed over the quadrant's 16 lanes, each lane flags in LDS the
// splats at four of its quadrant's list positions that the quadrant composited, and splat j of the batch
// is kept when some quadrant flagged it.
template <bool FEAT, bool HOLLOW, bool COMPACT>
__global__ void __launch_bounds__(64) raster_fwd_kernel(b2c_raster_fwd_args a) {
  constexpr bool EXT = FEAT || HOLLOW;
  // slot 64 is a null splat (no fragment passes) that pads the shorter quadrant lists
  __shared__ float4 s_g0[65], s_g1[65], s_col[65];
  __shared__ float4 s_ext[EXT ? 65 : 1];  // (feature xyz, camera depth)
  __shared__ uint32_t s_list[4][66];  // per quadrant: LDS byte offsets of its splats, in depth order
  __shared__ uint32_t s_flag[COMPACT ? 65 : 1];  // COMPACT: splat j of the batch was composited (64: the null splat)
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const int lane = threadIdx.x;
  const int q = lane >> 4, p = lane & 15;
  const int tx = tile % a.tiles_x, ty = tile / a.tiles_x;
  const int px = tx * RT_W + (q & 1) * 4 + (p & 3), py = ty * RT_W + (q >> 1) * 4 + (p >> 2);
  const float x0 = tx * RT_W + 0.5f, y0 = ty * RT_W + 0.5f;  // the tile's first pixel centre
  const bool inside = px < a.W && py < a.H;
  const float pcx = px + 0.5f, pcy = py + 0.5f;
  const float tcx = tx * RT_W + RT_W * 0.5f, tcy = ty * RT_W + RT_W * 0.5f;  // the tile centre
  const PixelPoly pp = pixel_poly(pcx - tcx, pcy - tcy);
  uint2* ranges = reinterpret_cast<uint2*>(a.tile_ranges);
  const uint2 range = ranges[tile];
  float T = 1.f, r = 0.f, g = 0.f, b = 0.f;
  float f0 = 0.f, f1 = 0.f, f2 = 0.f, pen = 0.f;
  HollowRef href{};
  if constexpr (HOLLOW) href = hollow_ref(inside ? a.hollow_z[py * a.W + px] : __builtin_inff(), a.hollow_margin);
  bool live = inside;
  uint32_t last = range.x;
  uint32_t clast = range.x, cbase = 0;  // COMPACT: this pixel's end in the compacted list; entries kept so far
  if (lane < 8) s_list[lane >> 1][64 + (lane & 1)] = 64u * 16u;  // read by the last pair's prefetch
  if constexpr (COMPACT) s_flag[lane] = 0u;
  if (lane == 0) {  // power = 0 and sigma = F = 1: fails the cutoff
    s_g0[64] = make_float4(0.f, 0.f, 1.f, 0.f);
    s_g1[64] = make_float4(0.f, 0.f, 0.f, 0.f);
    s_col[64] = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (EXT) s_ext[64] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const char* lds_g0 = reinterpret_cast<const char*>(s_g0);
  const char* lds_g1 = reinterpret_cast<const char*>(s_g1);
  const char* lds_col = reinterpret_cast<const char*>(s_col);
  const char* lds_ext = reinterpret_cast<const char*>(s_ext);
  constexpr uint32_t NO_OFF = 0xFFFFFFFFu;
  for (uint32_t start = range.x; start < range.y; start += 64) {
    if (ballot64(live) == 0) break;
    const uint32_t remaining = min(64u, range.y - start);
    __syncthreads();
    uint32_t qmask = 0, gid = 0, gslot = 0;
    if ((uint32_t)lane < remaining) {
      gid = a.vals_sorted[start + lane];
      if constexpr (COMPACT) gslot = a.slot_sorted[start + lane];
      const float4* rec = reinterpret_cast<const float4*>(a.raster_rec) + (size_t)gid * 4;
      const float4 r0 = rec[0], r1 = rec[1], r2 = rec[2];
      const float3 def = sigma_coefs(r0.x, r0.y, r0.z, r0.w, r1.x, tcx, tcy);
      s_g0[lane] = make_float4(def.x, def.y, def.z, r0.z);
      s_g1[lane] = make_float4(r0.w, r2.w, r1.z, r1.x);
      s_col[lane] = r2;
      if constexpr (EXT) s_ext[lane] = rec[3];
      qmask = quadrant_mask(r0.x, r0.y, r0.z, r0.w, r1.x, r1.z, x0, y0);
    }
    // per-quadrant lists: the lanes with bit qq set, in lane (depth) order, padded with the null splat
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
    // The lists are walked in pairs (an odd count runs one null entry more); each offset register is
    // reloaded with the entry two ahead at the end of its step, while the other step of the pair runs.
    uint32_t off0 = my_list[0], off1 = my_list[1];
    // The steps this lane composited, as two shift registers (even and odd steps): each step shifts its
    // register left and brings in 1 when the lane composited (a select and a shift-or), so after the batch's
    // n_pairs step pairs bit b stands for pair n_pairs - 1 - b. They give the lane's last composited entry
    // (and, COMPACT, the kept entries) without a select per step.
    uint32_t marks_even = 0, marks_odd = 0;
    // One step: sigma <= power (a NaN sigma fails), bitwise & so the compiler does not branch on the
    // compares; the exp is kept out of an exec-masked branch (a lane whose fragment fails has its alpha
    // discarded by the select); only a valid fragment can stop a lane. The transmittance after a fragment is
    // fma(-alpha, T, T): T (1 - alpha) rounded once (the depth probe's walk does the same). A fragment is
    // composited (vis > 0) exactly when it is valid and does not stop the lane: a valid alpha is at least
    // 1/255 and a live lane's T is above the cutoff.
#define B2C_COMPOSITE(off, next, marks)                                                                \
  do {                                                                                                 \
    const float4 g0 = *reinterpret_cast<const float4*>(lds_g0 + (off));                                \
    const float4 g1 = *reinterpret_cast<const float4*>(lds_g1 + (off));                                \
    const float4 col = *reinterpret_cast<const float4*>(lds_col + (off));                              \
    const float sigma = poly_sigma(g0.w, g1.x, g1.w, g0.x, g0.y, g0.z, pp);                            \
    const bool valid = live & (sigma <= g1.z);                                                         \
    float a_cl = fminf(ALPHA_MAX, fragment_alpha(sigma, g1.y));                                        \
    asm volatile("" : "+v"(a_cl));                                                                     \
    const float alpha = valid ? a_cl : 0.f;                                                            \
    const float next_T = __builtin_fmaf(-alpha, T, T);                                                      \
    const bool stop = next_T <= T_CUTOFF;                                                              \
    live = live & !stop;                                                                               \
    const float vis = stop ? 0.f : alpha * T;                                                          \
    r += col.x * vis;                                                                                  \
    g += col.y * vis;                                                                                  \
    b += col.z * vis;                                                                                  \
    if constexpr (EXT) {                                                                               \
      const float4 ext = *reinterpret_cast<const float4*>(lds_ext + (off));                            \
      if constexpr (FEAT) {                                                                            \
        f0 += ext.x * vis;                                                                             \
        f1 += ext.y * vis;                                                                             \
        f2 += ext.z * vis;                                                                             \
      }                                                                                                \
      if constexpr (HOLLOW) pen += vis * hollow_h(ext.w, href);                                        \
    }                                                                                                  \
    T = stop ? T : next_T;                                                                             \
    (marks) = ((marks) << 1) | ((valid & !stop) ? 1u : 0u);                                           \
    (off) = my_list[next];                                                                             \
  } while (0)
    for (uint32_t i = 0; i < n_iter; i += 2) {
      B2C_COMPOSITE(off0, i + 2, marks_even);
      B2C_COMPOSITE(off1, i + 3, marks_odd);
    }
#undef B2C_COMPOSITE
    const int n_pairs = (int)(n_iter + 1u) >> 1;
    // this lane's last composited step (the latest pair is the lowest set bit), and its splat's LDS offset
    uint32_t last_off = NO_OFF;
    if (marks_even | marks_odd) {
      const int se = marks_even ? 2 * (n_pairs - 1 - __builtin_ctz(marks_even)) : -2;
      const int so = marks_odd ? 2 * (n_pairs - 1 - __builtin_ctz(marks_odd)) + 1 : -1;
      last_off = my_list[max(se, so)];
      last = start + (last_off >> 4) + 1u;
    }
    if constexpr (COMPACT) {
      // the quadrant's marks: OR over its 16 lanes (one DPP row)
      marks_even |= dpp_u32<0x128, 0xF>(marks_even, 0u);  // row_ror:8, 4, 2, 1
      marks_odd |= dpp_u32<0x128, 0xF>(marks_odd, 0u);
      marks_even |= dpp_u32<0x124, 0xF>(marks_even, 0u);
      marks_odd |= dpp_u32<0x124, 0xF>(marks_odd, 0u);
      marks_even |= dpp_u32<0x122, 0xF>(marks_even, 0u);
      marks_odd |= dpp_u32<0x122, 0xF>(marks_odd, 0u);
      marks_even |= dpp_u32<0x121, 0xF>(marks_even, 0u);
      marks_odd |= dpp_u32<0x121, 0xF>(marks_odd, 0u);
      // lane p of quadrant q flags the splats at positions p, p + 16, p + 32, p + 48 of q's list that q
      // composited (position pos is pair pos / 2, bit n_pairs - 1 - pos / 2; its parity is p's)
      const uint32_t m = (p & 1) ? marks_odd : marks_even;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int pos = p + 16 * j;
        if (pos < (int)n_iter && ((m >> ((n_pairs - 1 - (pos >> 1)) & 31)) & 1u)) s_flag[my_list[pos] >> 4] = 1u;
      }
      __syncthreads();
      const bool kept = s_flag[lane] != 0u;
      s_flag[lane] = 0u;  // cleared for the next batch (its flags are written after its lists are built)
      const uint64_t keep = ballot64(kept);
      if (kept) {
        const uint32_t c = range.x + cbase + popc64(keep & below);
        a.cvals[c] = gid;
        a.cslots[c] = gslot;
      }
      // a lane that composited in this batch: its last composited splat is kept
      if (last_off != NO_OFF) clast = range.x + cbase + popc64(keep & ((1ull << (last_off >> 4)) - 1ull)) + 1u;
      cbase += popc64(keep);
    }
  }
  if (inside) {
    const int pix = py * a.W + px;
    reinterpret_cast<float4*>(a.out_rgba)[pix] = make_float4(r + T * a.bg[0], g + T * a.bg[1], b + T * a.bg[2], 1.f - T);
    reinterpret_cast<float4*>(a.out_feat)[pix] = make_float4(f0, f1, f2, T);
    if constexpr (HOLLOW) a.hollow_pen[pix] = pen;
    if (a.bwd_info) a.last_idx[pix] = last;
    if constexpr (COMPACT) a.clast[pix] = clast;
  }
  if (a.bwd_info) {
    uint32_t m = last;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = max(m, (uint32_t)__shfl_xor(m, o));
    if (lane == 0) ranges[tile].y = m;
  }
  if constexpr (COMPACT)
    if (lane == 0) a.cend[tile] = range.x + cbase;
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" int b2c_hip_raster_fwd(const b2c_raster_fwd_args* a, hipStream_t stream) {
  const int n_tiles = a->tiles_x * a->tiles_y;
  if (n_tiles <= 0) return 0;
  if (!a->raster_rec || (a->hollow_z && !a->hollow_pen)) return (int)hipErrorInvalidValue;
  const dim3 grid(NUM_XCD * xcd_tiles_per(n_tiles)), block(64);
  const bool hollow = a->hollow_z != nullptr;
  const bool compact = a->bwd_info && a->cvals != nullptr;
  if (compact && (!a->cslots || !a->slot_sorted || !a->clast || !a->cend)) return (int)hipErrorInvalidValue;
  const int variant = (a->feat ? 4 : 0) | (hollow ? 2 : 0) | (compact ? 1 : 0);
  switch (variant) {
    case 0: raster_fwd_kernel<false, false, false><<<grid, block, 0, stream>>>(*a); break;
    case 1: raster_fwd_kernel<false, false, true><<<grid, block, 0, stream>>>(*a); break;
    case 2: raster_fwd_kernel<false, true, false><<<grid, block, 0, stream>>>(*a); break;
    case 3: raster_fwd_kernel<false, true, true><<<grid, block, 0, stream>>>(*a); break;
    case 4: raster_fwd_kernel<true, false, false><<<grid, block, 0, stream>>>(*a); break;
    case 5: raster_fwd_kernel<true, false, true><<<grid, block, 0, stream>>>(*a); break;
    case 6: raster_fwd_kernel<true, true, false><<<grid, block, 0, stream>>>(*a); break;
    default: raster_fwd_kernel<true, true, true><<<grid, block, 0, stream>>>(*a); break;
  }
  return (int)hipGetLastError();
}
