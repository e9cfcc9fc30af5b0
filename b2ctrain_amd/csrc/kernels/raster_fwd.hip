// Forward compositing (replaces src/gpu/raster_fwd.cu:8-90, FEAT none, HOLLOW none): one wave64 per 8x8
// tile, one lane per pixel, the tile's depth-ordered list staged through LDS 64 splats at a time,
// front-to-back alpha blending with the 1/255 cutoff (sigma <= power), the 0.999 clamp and the 1e-4
// transmittance stop. The whole wave leaves as soon as every lane is done. With bwd_info the tile's range
// end is shrunk to one past the last fragment any pixel composited.
#include "b2c_kernels.h"
#include "raster_common.h"

namespace b2c {
namespace dev {
namespace {

// The splat loop is wave-uniform and branch-free: a lane that has terminated (or a fragment that fails the
// cutoff) contributes alpha = 0, which leaves T, the colour and the last index unchanged. Per splat the LDS
// holds (mx, my, c00/2, c01), (c11/2, log2 opacity, power, 0) and the colour clamped at 0, staged from the
// projection's 64-byte per-splat record (one cache line per gather); halving c00 and c11 is exact, so
// sigma is the reference's 0.5 (c00 dx^2 + c11 dy^2) + c01 dx dy bit for bit (uncontracted).
__global__ void __launch_bounds__(64) raster_fwd_kernel(b2c_raster_fwd_args a) {
  __shared__ float4 s_g0[64], s_g1[64], s_col[64];
  const int n_tiles = a.tiles_x * a.tiles_y;
  const int tile = xcd_tile(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const int lane = threadIdx.x;
  const int tx = tile % a.tiles_x, ty = tile / a.tiles_x;
  const int px = tx * RT_W + (lane & 7), py = ty * RT_W + (lane >> 3);
  const bool inside = px < a.W && py < a.H;
  const float pcx = px + 0.5f, pcy = py + 0.5f;
  uint2* ranges = reinterpret_cast<uint2*>(a.tile_ranges);
  const uint2 range = ranges[tile];
  float T = 1.f, r = 0.f, g = 0.f, b = 0.f;
  bool live = inside;
  uint32_t last = range.x;
  for (uint32_t start = range.x; start < range.y; start += 64) {
    if (ballot64(live) == 0) break;
    const uint32_t remaining = min(64u, range.y - start);
    __syncthreads();
    if ((uint32_t)lane < remaining) {
      const uint32_t gid = a.vals_sorted[start + lane];
      const float4* rec = reinterpret_cast<const float4*>(a.raster_rec) + (size_t)gid * 4;
      const float4 r1 = rec[1], r2 = rec[2];
      s_g0[lane] = rec[0];
      s_g1[lane] = make_float4(r1.x, r2.w, r1.z, 0.f);
      s_col[lane] = r2;
    }
    __syncthreads();
    const uint32_t n_splats = __builtin_amdgcn_readfirstlane(remaining);  // scalar loop bound
    for (uint32_t t = 0; t < n_splats; t++) {
      const float4 g0 = s_g0[t], g1 = s_g1[t], col = s_col[t];
      float sigma;
      {
#pragma clang fp contract(off)
        const float dx = pcx - g0.x, dy = pcy - g0.y;
        sigma = ((g0.z * dx) * dx + (g1.x * dy) * dy) + (g0.w * dx) * dy;
      }
      // straight-line: every lane evaluates every splat; failing lanes carry alpha = 0 (bitwise & keeps the
      // compiler from branching on the compares)
      const bool valid = live & (sigma >= 0.f) & (sigma <= g1.z);
      float a_cl = fminf(ALPHA_MAX, fragment_alpha(sigma, g1.y));  // sigma < 0: discarded by the select
      asm volatile("" : "+v"(a_cl));  // keeps the exp out of an exec-masked branch
      const float alpha = valid ? a_cl : 0.f;
      const float next_T = T * (1.f - alpha);
      const bool stop = next_T <= T_CUTOFF;  // only a valid fragment can stop a lane
      live = live & !stop;
      const float vis = stop ? 0.f : alpha * T;
      r += col.x * vis;
      g += col.y * vis;
      b += col.z * vis;
      T = stop ? T : next_T;
      last = vis > 0.f ? start + t + 1 : last;
    }
  }
  if (inside) {
    const int pix = py * a.W + px;
    reinterpret_cast<float4*>(a.out_rgba)[pix] = make_float4(r + T * a.bg[0], g + T * a.bg[1], b + T * a.bg[2], 1.f - T);
    reinterpret_cast<float4*>(a.out_feat)[pix] = make_float4(0.f, 0.f, 0.f, T);
    if (a.bwd_info) a.last_idx[pix] = last;
  }
  if (a.bwd_info) {
    uint32_t m = last;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = max(m, (uint32_t)__shfl_xor(m, o));
    if (lane == 0) ranges[tile].y = m;
  }
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" int b2c_hip_raster_fwd(const b2c_raster_fwd_args* a, hipStream_t stream) {
  const int n_tiles = a->tiles_x * a->tiles_y;
  if (n_tiles <= 0) return 0;
  if (!a->raster_rec) return (int)hipErrorInvalidValue;
  raster_fwd_kernel<<<dim3(NUM_XCD * xcd_tiles_per(n_tiles)), dim3(64), 0, stream>>>(*a);
  return (int)hipGetLastError();
}
