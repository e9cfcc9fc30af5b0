// The losses beside the photometric one (replaces src/gpu/loss.cu:197-293 and hollow_loss / normal_loss /
// eval_metrics, 317-338): the normal-map supervision of the feature lanes, the hollow-penalty sum and the
// eval metrics (squared error and SSIM of the 8-bit prediction). Each workgroup leaves its sums in a
// partials array that one final workgroup adds up in a fixed order in double precision, so every result is
// deterministic (the reference adds per-warp sums with float atomics).
#pragma clang fp contract(off)
#include "b2c_kernels.h"
#include "device_math.h"
#include "ssim_common.h"

namespace b2c {
namespace dev {
namespace {

constexpr int AUX_BLOCK = 256;
constexpr int AUX_GRID_MAX = 2048;  // grid-stride kernels: at most this many workgroups (and partials)

// Sum of one value over a 256-thread workgroup: wave shuffles, then the four wave totals in LDS, added by
// thread 0 in wave order.
__device__ __forceinline__ float block_sum(float v, float* s_red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();  // s_red may still be read from a previous call
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];
}

// Normal supervision (loss.cu:206-238) for the pixels whose normal map is opaque (alpha byte above 127):
// with the target decoded as n = (2 r - 1, 1 - 2 g, 1 - 2 b) (r, g, b in [0, 1]; the [+X, -Y, -Z]
// convention) and the rendered feature p, the loss is k (|p - n|_1 + 1 - cos(p, n)), k = scale * weight, with
// both lengths floored at 1e-6. Its gradient, times grad_scale, is
//   k (sign(p - n) - n / (|p| |n|) + p (p . n) / (|p|^3 |n|)).
// Other pixels get a zero gradient.
__global__ void __launch_bounds__(AUX_BLOCK) normal_loss_kernel(b2c_normal_loss_args a) {
  __shared__ float s_red[4];
  const int npix = a.W * a.H;
  float local = 0.f;
  for (int pix = blockIdx.x * AUX_BLOCK + threadIdx.x; pix < npix; pix += gridDim.x * AUX_BLOCK) {
    const uint32_t nm = a.normals[pix];
    float4 out = make_float4(0.f, 0.f, 0.f, 0.f);
    if (((nm >> 24) & 0xffu) > 127u) {
      const float wp = a.weights ? (float)a.weights[pix] * (1.f / 255.f) : 1.f;
      const float k = a.scale * wp;
      const float nx = (float)(nm & 0xffu) * (2.f / 255.f) - 1.f;
      const float ny = 1.f - (float)((nm >> 8) & 0xffu) * (2.f / 255.f);
      const float nz = 1.f - (float)((nm >> 16) & 0xffu) * (2.f / 255.f);
      const float4 f = reinterpret_cast<const float4*>(a.feat)[pix];
      const float pl = fmaxf(sqrtf((f.x * f.x + f.y * f.y) + f.z * f.z), 1e-6f);
      const float nl = fmaxf(sqrtf((nx * nx + ny * ny) + nz * nz), 1e-6f);
      const float dot = (f.x * nx + f.y * ny) + f.z * nz;
      const float plnl = pl * nl;
      const float dx = f.x - nx, dy = f.y - ny, dz = f.z - nz;
      local = local + k * ((((fabsf(dx) + fabsf(dy)) + fabsf(dz)) + 1.f) - dot / plnl);
      const float inv = 1.f / plnl, radial = dot / ((pl * pl) * plnl);
      const float kg = k * a.grad_scale;
      const float sx = dx > 0.f ? 1.f : (dx < 0.f ? -1.f : 0.f);
      const float sy = dy > 0.f ? 1.f : (dy < 0.f ? -1.f : 0.f);
      const float sz = dz > 0.f ? 1.f : (dz < 0.f ? -1.f : 0.f);
      out = make_float4(kg * ((sx - nx * inv) + f.x * radial), kg * ((sy - ny * inv) + f.y * radial),
                        kg * ((sz - nz * inv) + f.z * radial), 0.f);
    }
    reinterpret_cast<float4*>(a.v_feat)[pix] = out;
  }
  const float t = block_sum(local, s_red);
  if (threadIdx.x == 0) a.partials[blockIdx.x] = t;
}

// Per-workgroup sums of the hollow penalty (loss.cu:197-204).
__global__ void __launch_bounds__(AUX_BLOCK) hollow_sum_kernel(const float* __restrict__ pen, int npix,
                                                               float* __restrict__ partials) {
  __shared__ float s_red[4];
  float local = 0.f;
  for (int pix = blockIdx.x * AUX_BLOCK + threadIdx.x; pix < npix; pix += gridDim.x * AUX_BLOCK)
    local = local + pen[pix];
  const float t = block_sum(local, s_red);
  if (threadIdx.x == 0) partials[blockIdx.x] = t;
}

// Eval metrics (loss.cu:240-286): one 256-thread workgroup per 16 x 16 tile and channel. The prediction is
// clamped to [0, 1] and rounded to 8 bits; the 26 x 26 input footprint (5-pixel halo, zero outside the
// image) goes to LDS, the horizontal 11-tap pass of the five SSIM statistics over its 26 rows and 16
// columns to LDS, then each thread takes one output pixel's vertical pass, its clamped SSIM and squared
// error (both weighted by the target alpha when mask_weighted). The workgroup's two sums go to partials.
constexpr int ET = 16;                // output tile edge
constexpr int EIN = ET + 2 * HALO;    // 26: input footprint edge
constexpr int ESTATS = 5;             // E[x], E[x^2], E[y], E[y^2], E[xy]

__global__ void __launch_bounds__(AUX_BLOCK) eval_kernel(b2c_eval_args a, int tiles_x) {
  __shared__ float s_p[EIN * EIN], s_g[EIN * EIN];
  __shared__ float s_h[EIN * ET * ESTATS];
  __shared__ float s_red[4];
  const int c = blockIdx.y;
  const int tile = blockIdx.x;
  const int x0 = (tile % tiles_x) * ET, y0 = (tile / tiles_x) * ET;
  const int tid = threadIdx.x;
  for (int i = tid; i < EIN * EIN; i += AUX_BLOCK) {
    const int gy = y0 - HALO + i / EIN, gx = x0 - HALO + i % EIN;
    float p = 0.f, g = 0.f;
    if (gx >= 0 && gx < a.W && gy >= 0 && gy < a.H) {
      const int pix = gy * a.W + gx;
      const float4 pv = reinterpret_cast<const float4*>(a.pred)[pix];
      const float pc = c == 0 ? pv.x : (c == 1 ? pv.y : pv.z);
      p = __builtin_rintf(fminf(fmaxf(pc, 0.f), 1.f) * 255.f) / 255.f;
      g = gt_channel(a.gt[pix], c);
    }
    s_p[i] = p;
    s_g[i] = g;
  }
  __syncthreads();
  for (int i = tid; i < EIN * ET; i += AUX_BLOCK) {
    const int row = i / ET, col = i % ET;
    float sx = 0.f, sxx = 0.f, sy = 0.f, syy = 0.f, sxy = 0.f;
#pragma unroll
    for (int d = 0; d < 11; d++) {
      const float w = gw_tap(d);
      const float x = s_p[row * EIN + col + d], y = s_g[row * EIN + col + d];
      sx = sx + w * x;
      sxx = sxx + (w * x) * x;
      sy = sy + w * y;
      syy = syy + (w * y) * y;
      sxy = sxy + (w * x) * y;
    }
    float* h = s_h + i * ESTATS;
    h[0] = sx; h[1] = sxx; h[2] = sy; h[3] = syy; h[4] = sxy;
  }
  __syncthreads();
  float se = 0.f, ss = 0.f;
  {
    const int ly = tid / ET, lx = tid % ET;
    const int gy = y0 + ly, gx = x0 + lx;
    if (gx < a.W && gy < a.H) {
      float st[ESTATS] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < 11; d++) {
        const float w = gw_tap(d);
        const float* h = s_h + ((ly + d) * ET + lx) * ESTATS;
#pragma unroll
        for (int k = 0; k < ESTATS; k++) st[k] = st[k] + w * h[k];
      }
      const float mu1 = st[0], mu2 = st[2];
      const float s1 = fmaxf(0.f, st[1] - mu1 * mu1), s2 = fmaxf(0.f, st[3] - mu2 * mu2), s12 = st[4] - mu1 * mu2;
      const float num = ((2.f * mu1) * mu2 + C1) * (2.f * s12 + C2);
      const float den = ((mu1 * mu1 + mu2 * mu2) + C1) * ((s1 + s2) + C2);
      const float ssim = fminf(fmaxf(num / den, -1.f), 1.f);
      const int li = (ly + HALO) * EIN + lx + HALO;
      const float d = fabsf(s_p[li] - s_g[li]);
      const float m = a.mask_weighted ? gt_channel(a.gt[gy * a.W + gx], 3) : 1.f;
      se = (d * m) * (d * m);
      ss = ssim * m;
    }
  }
  const float tse = block_sum(se, s_red);
  const float tss = block_sum(ss, s_red);
  if (tid == 0) {
    const size_t wg = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
    a.partials[2 * wg] = tse;
    a.partials[2 * wg + 1] = tss;
  }
}

// Fixed-order double-precision sums of `count` partials (every `stride`-th from `first`) times `factor`,
// added to accum[slot]; with two = 1 also the interleaved second value into accum[slot + 1].
__global__ void __launch_bounds__(1024) aux_reduce_kernel(const float* __restrict__ partials, int count, int two,
                                                          float factor, float* __restrict__ accum, int slot) {
  __shared__ double s_red[2][16];
  double acc0 = 0.0, acc1 = 0.0;
  const int stride = two ? 2 : 1;
  for (int i = threadIdx.x; i < count; i += 1024) {
    acc0 += (double)partials[(size_t)i * stride];
    if (two) acc1 += (double)partials[(size_t)i * stride + 1];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    acc0 += __shfl_xor(acc0, o);
    acc1 += __shfl_xor(acc1, o);
  }
  if ((threadIdx.x & 63) == 0) {
    s_red[0][threadIdx.x >> 6] = acc0;
    s_red[1][threadIdx.x >> 6] = acc1;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double t0 = 0.0, t1 = 0.0;
    for (int k = 0; k < 16; k++) {
      t0 += s_red[0][k];
      t1 += s_red[1][k];
    }
    accum[slot] = (float)((double)accum[slot] + (double)factor * t0);
    if (two) accum[slot + 1] = (float)((double)accum[slot + 1] + (double)factor * t1);
  }
}

int aux_grid(int npix) {
  const int blocks = (npix + AUX_BLOCK - 1) / AUX_BLOCK;
  return blocks < AUX_GRID_MAX ? blocks : AUX_GRID_MAX;
}

int eval_tiles(int W, int H) { return ((W + ET - 1) / ET) * ((H + ET - 1) / ET); }

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" size_t b2c_aux_partials(int W, int H) {
  if (W <= 0 || H <= 0) return 0;
  const size_t ev = (size_t)2 * 3 * (size_t)eval_tiles(W, H);
  return ev > (size_t)AUX_GRID_MAX ? ev : (size_t)AUX_GRID_MAX;
}

extern "C" int b2c_hip_normal_loss(const b2c_normal_loss_args* a, hipStream_t stream) {
  const int npix = a->W * a->H;
  if (npix <= 0) return 0;
  if (!a->feat || !a->normals || !a->v_feat || !a->loss_accum || !a->partials) return (int)hipErrorInvalidValue;
  const int grid = aux_grid(npix);
  normal_loss_kernel<<<grid, AUX_BLOCK, 0, stream>>>(*a);
  aux_reduce_kernel<<<1, 1024, 0, stream>>>(a->partials, grid, 0, 1.f, a->loss_accum, 1);
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_hollow_loss(const float* hollow_pen, int W, int H, float lam, float* loss_accum,
                                   float* partials, hipStream_t stream) {
  const int npix = W * H;
  if (npix <= 0) return 0;
  if (!hollow_pen || !loss_accum || !partials) return (int)hipErrorInvalidValue;
  const int grid = aux_grid(npix);
  hollow_sum_kernel<<<grid, AUX_BLOCK, 0, stream>>>(hollow_pen, npix, partials);
  aux_reduce_kernel<<<1, 1024, 0, stream>>>(partials, grid, 0, lam, loss_accum, 0);
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_eval_metrics(const b2c_eval_args* a, hipStream_t stream) {
  if (a->W <= 0 || a->H <= 0) return 0;
  if (!a->pred || !a->gt || !a->loss_accum || !a->partials) return (int)hipErrorInvalidValue;
  const int tiles_x = (a->W + ET - 1) / ET;
  const int tiles = eval_tiles(a->W, a->H);
  eval_kernel<<<dim3(tiles, 3), AUX_BLOCK, 0, stream>>>(*a, tiles_x);
  aux_reduce_kernel<<<1, 1024, 0, stream>>>(a->partials, tiles * 3, 1, 1.f, a->loss_accum, 4);
  return (int)hipGetLastError();
}
