// Fused photometric loss (replaces photometric_kernel, src/gpu/loss.cu:18-195, 296-315): per 16x16 output
// tile and channel, a 36x36 footprint of prediction and effective target in LDS (zero outside the image),
// separable 11-tap Gaussian (sigma 1.5) statistics at the 26x26 positions the output's SSIM gradient
// depends on, SSIM and its five partial maps, a second separable blur, L1 sign, and the alpha-match lane.
// The per-pixel gradient goes to v_out (times grad_scale); the loss value is reduced per workgroup and
// added to loss_accum[0]. A footprint where prediction equals target exactly has SSIM 1 and zero gradient
// and is finished without the blurs (loss.cu:51-74).
#include "b2c_kernels.h"
#include "device_math.h"

namespace b2c {
namespace dev {
namespace {

constexpr int TILE_W = 16, TILE_PX = TILE_W * TILE_W;
constexpr int HALO = 5;
constexpr int STAT_W = TILE_W + 2 * HALO;  // 26
constexpr int IN_W = STAT_W + 2 * HALO;    // 36
constexpr float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;

struct Gauss11 { float w[11]; };

__device__ __forceinline__ float gt_channel(uint32_t packed, int c) {
  return (float)((packed >> (8 * c)) & 0xffu) * (1.f / 255.f);
}

// Effective target of channel c (loss.cu:85-87), uncontracted: the L1 sign compares the prediction with
// exactly this fp32 value, so it must round the same way everywhere.
__device__ __forceinline__ float gt_effective(uint32_t gp, int c, bool composite, float bg_c) {
#pragma clang fp contract(off)
  float g = gt_channel(gp, c);
  if (composite) g = g + (1.f - gt_channel(gp, 3)) * bg_c;
  return g;
}

__device__ __forceinline__ void store_partial(const b2c_loss_args& a, float t) {
  if (a.partials)
    a.partials[blockIdx.y * gridDim.x + blockIdx.x] = t;
  else if (t != 0.f)
    atomicAdd(a.loss_accum, t);
}

__device__ __forceinline__ float block_sum_256(float v, float* s_red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
  if (threadIdx.x == 0)
    for (int i = 0; i < TILE_PX / 64; i++) t += s_red[i];
  return t;
}

__global__ void __launch_bounds__(TILE_PX) photometric_kernel(b2c_loss_args a, Gauss11 gw, int tiles_x) {
  __shared__ float s_in[2][IN_W * IN_W];
  __shared__ float s_h[IN_W * STAT_W * 5];
  __shared__ float s_v[STAT_W * STAT_W * 5];
  __shared__ float s_red[TILE_PX / 64];
  const int c = blockIdx.y;
  const int tile = blockIdx.x;
  const int tx0 = (tile % tiles_x) * TILE_W, ty0 = (tile / tiles_x) * TILE_W;
  const int tid = threadIdx.x;
  const int W = a.W, H = a.H;
  const float4* pred = reinterpret_cast<const float4*>(a.pred);
  const float bg_c = a.composite ? a.bg[c] : 0.f;
  // The statistics are accumulated for p - c1 and g - c2, with c1 / c2 the values at the tile centre:
  // variances and covariances are shift-invariant, and in the gradient 2p*blur(B) - 2*blur(B*mu1) the shift
  // cancels exactly, so both lose far less to fp32 cancellation than the unshifted form (loss.cu:122-170).
  float c1, c2;
  {
    const int cpix = min(ty0 + TILE_W / 2, H - 1) * W + min(tx0 + TILE_W / 2, W - 1);
    const float4 pv = pred[cpix];
    c1 = c == 0 ? pv.x : (c == 1 ? pv.y : pv.z);
    c2 = gt_effective(a.gt[cpix], c, a.composite, bg_c);
  }
  float flat_diff = 0.f;
  for (int i = tid; i < IN_W * IN_W; i += TILE_PX) {
    const int ly = i / IN_W, lx = i % IN_W;
    const int gy = ty0 + ly - 2 * HALO, gx = tx0 + lx - 2 * HALO;
    float p = 0.f, g = 0.f;
    if (gy >= 0 && gy < H && gx >= 0 && gx < W) {
      const int pix = gy * W + gx;
      const float4 pv = pred[pix];
      p = c == 0 ? pv.x : (c == 1 ? pv.y : pv.z);
      g = gt_effective(a.gt[pix], c, a.composite, bg_c);
    }
    s_in[0][i] = p - c1;
    s_in[1][i] = g - c2;
    flat_diff = fmaxf(flat_diff, fabsf(p - g));
  }
  if (c == 0 && a.alpha_lane) {
    const int gy = ty0 + tid / TILE_W, gx = tx0 + tid % TILE_W;
    if (gy < H && gx < W) {
      const int pix = gy * W + gx;
      flat_diff = fmaxf(flat_diff, fabsf(pred[pix].w - gt_channel(a.gt[pix], 3)));
    }
  }
  const float norm = a.scale / (3.f * (float)W * (float)H);
  if (__syncthreads_or(flat_diff > 0.f) == 0) {
    const int gy = ty0 + tid / TILE_W, gx = tx0 + tid % TILE_W;
    float loss_local = 0.f;
    if (gy < H && gx < W) {
      const int pix = gy * W + gx;
      const uint32_t gp = a.gt[pix];
      const float wp = a.weights ? a.weights[pix] * (1.f / 255.f) : 1.f;
      const float M = wp * (a.mask ? gt_channel(gp, 3) : 1.f) * norm;
      loss_local = M * a.ssim_w;  // SSIM == 1 exactly
      a.v_out[(size_t)pix * 4 + c] = 0.f;
      if (c == 0) a.v_out[(size_t)pix * 4 + 3] = 0.f;
    }
    const float t = block_sum_256(loss_local, s_red);
    if (tid == 0) store_partial(a, t);
    return;
  }
  // horizontal blur of the five statistics: rows 0..35, output columns 0..25
  for (int i = tid; i < IN_W * STAT_W; i += TILE_PX) {
    const int ly = i / STAT_W, ox = i % STAT_W;
    float sx = 0.f, sx2 = 0.f, sy = 0.f, sy2 = 0.f, sxy = 0.f;
#pragma unroll
    for (int d = 0; d < 11; d++) {
      const float w = gw.w[d];
      const float x = s_in[0][ly * IN_W + ox + d], y = s_in[1][ly * IN_W + ox + d];
      sx += w * x; sx2 += w * x * x; sy += w * y; sy2 += w * y * y; sxy += w * x * y;
    }
    float* o = s_h + i * 5;
    o[0] = sx; o[1] = sx2; o[2] = sy; o[3] = sy2; o[4] = sxy;
  }
  __syncthreads();
  // vertical blur -> statistics at 26x26, SSIM, and the partial maps scaled by M * ssim_w
  float loss_local = 0.f;
  for (int i = tid; i < STAT_W * STAT_W; i += TILE_PX) {
    const int oy = i / STAT_W, ox = i % STAT_W;
    float st[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 11; d++) {
      const float w = gw.w[d];
      const float* h = s_h + ((oy + d) * STAT_W + ox) * 5;
#pragma unroll
      for (int k = 0; k < 5; k++) st[k] += w * h[k];
    }
    const int gy = ty0 + oy - HALO, gx = tx0 + ox - HALO;
    float A = 0.f, B = 0.f, Bm = 0.f, Cc = 0.f, Cm = 0.f;
    if (gy >= 0 && gy < H && gx >= 0 && gx < W) {
      const int pix = gy * W + gx;
      const uint32_t gp = a.gt[pix];
      const float wp = a.weights ? a.weights[pix] * (1.f / 255.f) : 1.f;
      const float M = wp * (a.mask ? gt_channel(gp, 3) : 1.f) * norm;
      const float mu1 = st[0] + c1, mu2 = st[2] + c2;  // st[0], st[2]: shifted means
      const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2;
      const float s1_raw = st[1] - st[0] * st[0], s2_raw = st[3] - st[2] * st[2];
      const float sigma1_sq = fmaxf(0.f, s1_raw), sigma2_sq = fmaxf(0.f, s2_raw);
      const float sigma12 = st[4] - st[0] * st[2];
      const float A1 = 2.f * mu1 * mu2 + C1, A2 = 2.f * sigma12 + C2;
      const float B1 = mu1_sq + mu2_sq + C1, B2 = sigma1_sq + sigma2_sq + C2;
      const float raw = (A1 * A2) / (B1 * B2);
      const float ssim = fminf(fmaxf(raw, -1.f), 1.f);
      if (oy >= HALO && oy < HALO + TILE_W && ox >= HALO && ox < HALO + TILE_W) {
        const float4 pv = pred[pix];
        const float p = c == 0 ? pv.x : (c == 1 ? pv.y : pv.z);
        const float g = gt_effective(gp, c, a.composite, bg_c);
        loss_local += M * (a.l1_w * fabsf(p - g) + a.ssim_w * ssim);
      }
      if (raw > -1.f && raw < 1.f) {
        const float k = M * a.ssim_w;
        const float inv_BB = 1.f / (B1 * B2);
        const float d_mu1 = 2.f * mu2 * A2 * inv_BB - 2.f * mu1 * ssim / B1;
        const float d_s1 = s1_raw > 0.f ? -ssim / B2 : 0.f;
        const float d_s12 = 2.f * A1 * inv_BB;
        A = k * d_mu1; B = k * d_s1; Bm = B * st[0]; Cc = k * d_s12; Cm = Cc * st[2];
      }
    }
    float* o = s_v + i * 5;
    o[0] = A; o[1] = B; o[2] = Bm; o[3] = Cc; o[4] = Cm;
  }
  __syncthreads();
  // second blur, horizontal: rows 0..25, output columns 0..15
  for (int i = tid; i < STAT_W * TILE_W; i += TILE_PX) {
    const int ly = i / TILE_W, ox = i % TILE_W;
    float acc[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 11; d++) {
      const float w = gw.w[d];
      const float* v = s_v + (ly * STAT_W + ox + d) * 5;
#pragma unroll
      for (int k = 0; k < 5; k++) acc[k] += w * v[k];
    }
    float* o = s_h + i * 5;
#pragma unroll
    for (int k = 0; k < 5; k++) o[k] = acc[k];
  }
  __syncthreads();
  // vertical, one output pixel per thread
  {
    const int ly = tid / TILE_W, lx = tid % TILE_W;
    const int gy = ty0 + ly, gx = tx0 + lx;
    if (gy < H && gx < W) {
      float acc[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < 11; d++) {
        const float w = gw.w[d];
        const float* v = s_h + ((ly + d) * TILE_W + lx) * 5;
#pragma unroll
        for (int k = 0; k < 5; k++) acc[k] += w * v[k];
      }
      const int pix = gy * W + gx;
      // shifted values for the SSIM terms, exact ones for the L1 sign
      const float ps = s_in[0][(ly + 2 * HALO) * IN_W + lx + 2 * HALO], gs = s_in[1][(ly + 2 * HALO) * IN_W + lx + 2 * HALO];
      const float4 pv = pred[pix];
      const float p = c == 0 ? pv.x : (c == 1 ? pv.y : pv.z);
      const uint32_t gp = a.gt[pix];
      const float g = gt_effective(gp, c, a.composite, bg_c);
      const float gt_a = gt_channel(gp, 3);
      const float wp = a.weights ? a.weights[pix] * (1.f / 255.f) : 1.f;
      const float M = wp * (a.mask ? gt_a : 1.f) * norm;
      const float sgn = p > g ? 1.f : (p < g ? -1.f : 0.f);
      const float grad = M * a.l1_w * sgn + acc[0] + 2.f * ps * acc[1] - 2.f * acc[2] + gs * acc[3] - acc[4];
      a.v_out[(size_t)pix * 4 + c] = grad * a.grad_scale;
      if (c == 0) {
        float va = 0.f;
        if (a.alpha_lane) {
          const float da = pred[pix].w - gt_a;
          const float sa = da > 0.f ? 1.f : (da < 0.f ? -1.f : 0.f);
          const float Ma = wp * a.match_alpha_weight * a.scale / ((float)W * (float)H);
          va = Ma * sa * a.grad_scale;
          loss_local += Ma * fabsf(da);
        }
        a.v_out[(size_t)pix * 4 + 3] = va;
      }
    }
  }
  const float t = block_sum_256(loss_local, s_red);
  if (tid == 0) store_partial(a, t);
}

// Fixed-order double-precision sum of the per-workgroup partials into loss_accum[0].
__global__ void __launch_bounds__(1024) reduce_partials_kernel(const float* __restrict__ partials, int count,
                                                                float* __restrict__ loss_accum) {
  __shared__ double s_red[16];
  double acc = 0.0;
  for (int i = threadIdx.x; i < count; i += 1024) acc += (double)partials[i];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int k = 0; k < 16; k++) t += s_red[k];
    loss_accum[0] = (float)((double)loss_accum[0] + t);
  }
}

__global__ void accumulate_kernel(float* acc) {
  acc[2] += acc[0] + acc[1];
  acc[3] += 1.f;
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" int b2c_hip_photometric(const b2c_loss_args* a, hipStream_t stream) {
  if (a->W <= 0 || a->H <= 0) return 0;
  Gauss11 g;
  double w[11], sum = 0.0;
  for (int i = 0; i < 11; i++) {
    const double x = i - 5.0;
    w[i] = __builtin_exp(-x * x / (2.0 * 1.5 * 1.5));
    sum += w[i];
  }
  for (int i = 0; i < 11; i++) g.w[i] = (float)(w[i] / sum);
  const int tiles_x = (a->W + TILE_W - 1) / TILE_W, tiles_y = (a->H + TILE_W - 1) / TILE_W;
  photometric_kernel<<<dim3(tiles_x * tiles_y, 3), dim3(TILE_PX), 0, stream>>>(*a, g, tiles_x);
  if (a->partials) reduce_partials_kernel<<<1, 1024, 0, stream>>>(a->partials, tiles_x * tiles_y * 3, a->loss_accum);
  return (int)hipGetLastError();
}

extern "C" size_t b2c_loss_partials(int W, int H) {
  return (size_t)((W + TILE_W - 1) / TILE_W) * ((H + TILE_W - 1) / TILE_W) * 3;
}

extern "C" int b2c_hip_accumulate_loss(float* loss_accum, hipStream_t stream) {
  accumulate_kernel<<<1, 1, 0, stream>>>(loss_accum);
  return (int)hipGetLastError();
}
