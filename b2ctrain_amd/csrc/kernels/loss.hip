// Fused photometric loss (replaces photometric_kernel, src/gpu/loss.cu:18-195, 296-315): L1 + SSIM
// (separable 11-tap Gaussian, sigma 1.5, zero padding, C1 = 1e-4, C2 = 9e-4) with the alpha-match lane.
// The per-pixel gradient (SSIM partial maps through the second blur, L1 sign, alpha sign) goes to v_out
// times grad_scale; the loss value is summed per wave into `partials` and reduced in a fixed order in
// double precision. A footprint where prediction equals target exactly gives SSIM = 1 and a zero gradient
// by the same arithmetic (the reference's early exit, loss.cu:51-74, is an optimisation only).
#include "b2c_kernels.h"
#include "device_math.h"
#include "ssim_common.h"
#include "loss_sum.h"

#include <stdlib.h>
#include <string.h>

#include <mutex>

namespace b2c {
namespace dev {
namespace {


// Effective target of channel c (loss.cu:85-87), uncontracted: the L1 sign compares the prediction with
// exactly this fp32 value, so it must round the same way everywhere.
__device__ __forceinline__ float gt_effective(uint32_t gp, int c, bool composite, float bg_c) {
#pragma clang fp contract(off)
  float g = gt_channel(gp, c);
  if (composite) g = g + (1.f - gt_channel(gp, 3)) * bg_c;
  return g;
}

// One wave64 per (strip, channel): a strip is SW = 54 output columns by SH output rows. Lane l owns
// statistics column x0 - 5 + l and walks down the rows: each step loads one input row (p, g shifted by the
// strip's centre values) into a one-row LDS buffer, blurs it horizontally at the lane's column (11 taps,
// five statistics), pushes the result into an 11-row register ring and, once 11 rows are in, blurs the
// ring vertically: SSIM and its partial maps at that row (three: the terms without a per-pixel factor are
// summed before the blur). The partial-map row goes through a second
// one-row LDS buffer for the horizontal pass of the second blur, whose results fill a second register
// ring; its vertical pass gives the gradient five rows further down. The loop is unrolled by 11 so that
// the ring slots are static registers.
// SH + 4 HALO input rows are walked per strip (the unrolled loop runs whole rings of 11 rows and skips the
// steps past the strip's last row). Taller strips repeat fewer halo rows but make fewer, longer waves; the
// launcher picks SH per image size and device (see pick_strip_rows).
constexpr int SW = 54;
constexpr int SH_MIN = 35, SH_MAX = 128;

struct PixelIn {
  float p, g;
};

__device__ __forceinline__ bool in_image(const b2c_loss_args& a, int x, int y) {
  return x >= 0 && x < a.W && y >= 0 && y < a.H;
}

__device__ __forceinline__ PixelIn load_in(const b2c_loss_args& a, int c, float bg_c, int gx, int gy) {
  PixelIn v{0.f, 0.f};
  if (in_image(a, gx, gy)) {
    const int pix = gy * a.W + gx;
    v.p = a.pred[(size_t)pix * 4 + c];
    v.g = gt_effective(a.gt[pix], c, a.composite, bg_c);
  }
  return v;
}

// The raw words one step of the walk reads from memory: the input row (this lane's column and, for lanes
// 0-9, the 10 columns past 64), the SSIM row's weight inputs and L1 operands, and the output row's
// operands. They are fetched one step ahead so the loads overlap the previous step's arithmetic.
// Every field is loaded unconditionally and converted only where it is used: a conversion next to its
// load (say of an optional weight, under a branch) would make the wave wait for all loads in flight,
// the next step's prefetch included.
struct StepRaw {
  float p_in, p_in2, a_out;
  uint32_t g_in, g_in2, g_ss, g_out;
  uint32_t w_ss, w_out;  // weight bytes (without weights: a byte of gt, unused)
};

// Buffer views of the inputs. A load adds the row's byte offset (wave-uniform, a scalar register) to the
// lane's column offset (fixed for the whole walk), so it costs no per-lane address arithmetic. Rows and
// columns are clamped into the image, so every load is in bounds; a pixel outside the image is read from
// its clamped neighbour and then discarded by the caller's in-image test (zero padding).
constexpr uint32_t BUF_WORD3 = 0x00020000u;  // gfx9 raw buffer: 32-bit data format, no swizzle

struct LossBufs {
  __amdgpu_buffer_rsrc_t pred, gt, w;
};

__device__ __forceinline__ LossBufs loss_bufs(const b2c_loss_args& a) {
  const uint32_t P = (uint32_t)a.W * (uint32_t)a.H;  // the launcher checks 16 P < 2^32
  LossBufs b;
  b.pred = __builtin_amdgcn_make_buffer_rsrc((void*)a.pred, (short)0, (int)(P * 16u), (int)BUF_WORD3);
  b.gt = __builtin_amdgcn_make_buffer_rsrc((void*)a.gt, (short)0, (int)(P * 4u), (int)BUF_WORD3);
  b.w = __builtin_amdgcn_make_buffer_rsrc((void*)(a.weights ? a.weights : (const uint8_t*)a.gt), (short)0, (int)P,
                                          (int)BUF_WORD3);
  return b;
}

// This lane's clamped columns: the input column, the input column 64 further (used by lanes 0-9), and the
// statistics / output column.
struct LaneCols {
  uint32_t in, in2, s;
};

__device__ __forceinline__ float ld_pred(const LossBufs& b, uint32_t col, int c, uint32_t row_words) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(b.pred, (int)(col * 16u + 4u * (uint32_t)c),
                                                              (int)(row_words * 16u), 0));
}

__device__ __forceinline__ uint32_t ld_gt(const LossBufs& b, uint32_t col, uint32_t row_words) {
  return __builtin_amdgcn_raw_buffer_load_b32(b.gt, (int)(col * 4u), (int)(row_words * 4u), 0);
}

__device__ __forceinline__ uint32_t ld_weight(const LossBufs& b, uint32_t col, uint32_t row_words) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(b.w, (int)col, (int)row_words, 0);
}

__device__ __forceinline__ float weight_of(const b2c_loss_args& a, uint32_t raw) {
  return a.weights ? (float)raw * (1.f / 255.f) : 1.f;
}

__device__ __forceinline__ int clamp_row(const b2c_loss_args& a, int y) { return min(max(y, 0), a.H - 1); }

__device__ __forceinline__ StepRaw fetch_step(const b2c_loss_args& a, const LossBufs& b, const LaneCols& lc, int c,
                                              int y0, int r) {
  StepRaw f;
  const int y_in = y0 - 2 * HALO + r;
  const uint32_t ri = (uint32_t)clamp_row(a, y_in) * (uint32_t)a.W;
  const uint32_t rs = (uint32_t)clamp_row(a, y_in - HALO) * (uint32_t)a.W;
  const uint32_t ro = (uint32_t)clamp_row(a, y_in - 2 * HALO) * (uint32_t)a.W;
  f.p_in = ld_pred(b, lc.in, c, ri);
  f.g_in = ld_gt(b, lc.in, ri);
  f.p_in2 = ld_pred(b, lc.in2, c, ri);
  f.g_in2 = ld_gt(b, lc.in2, ri);
  f.g_ss = ld_gt(b, lc.s, rs);
  f.w_ss = ld_weight(b, lc.s, rs);
  f.a_out = ld_pred(b, lc.s, 3, ro);
  f.g_out = ld_gt(b, lc.s, ro);
  f.w_out = ld_weight(b, lc.s, ro);
  return f;
}

// Workgroup b runs on XCD b mod 8; each XCD gets a contiguous band of strips, and the three channel waves of
// a strip are consecutive on their XCD, so the strip's input lines are read from that XCD's L2 three times
// rather than from memory.
__global__ void __launch_bounds__(64) photometric_kernel(b2c_loss_args a, int strips_x, int nstrips, int SH) {
  // rows walked: SH + 4 HALO rounded up to whole rings; the `extra` rows this adds are walked first, above
  // the strip's top halo, and only loaded and blurred horizontally (their statistics rows lie outside
  // every window of the strip, so the ring simply holds them until they are overwritten)
  const int ROWS = (SH + 4 * HALO + 10) / 11 * 11;
  const int extra = ROWS - (SH + 4 * HALO);
  __shared__ float s_p[2][64 + 2 * HALO], s_g[2][64 + 2 * HALO];  // one input row (double buffered)
  // the last 11 input rows, unshifted: prediction and effective target, read back 5 rows later as the
  // SSIM row's L1 operands and 10 rows later as the output row's (slot = row mod 11, static when unrolled)
  __shared__ float s_rp[11][64 + 2 * HALO], s_rg[11][64 + 2 * HALO];
  __shared__ float s_pm[2][3][64];                                 // one partial-map row (double buffered)
  constexpr int NXCD = 8;
  const int per = (nstrips * 3 + NXCD - 1) / NXCD;  // work items per XCD
  const int item = (blockIdx.x % NXCD) * per + blockIdx.x / NXCD;
  if (item >= nstrips * 3) return;
  const int strip = item / 3, c = item % 3;
  const int lane = threadIdx.x;
  const int x0 = (strip % strips_x) * SW, y0 = (strip / strips_x) * SH;
  const int W = a.W, H = a.H;
  const float bg_c = a.composite ? a.bg[c] : 0.f;
  const float norm = a.scale / (3.f * (float)W * (float)H);
  const float alpha_norm = a.match_alpha_weight * a.scale / ((float)W * (float)H);
  // statistics are accumulated for p - c1 and g - c2 (values at the strip centre): variances and
  // covariances are shift-invariant, and in the gradient 2p*blur(B) - 2*blur(B*mu1) the shift cancels
  // exactly, so both lose far less to fp32 cancellation (loss.cu:122-170)
  float c1, c2;
  {
    const PixelIn cv = load_in(a, c, bg_c, min(x0 + SW / 2, W - 1), min(y0 + SH / 2, H - 1));
    c1 = cv.p;
    c2 = cv.g;
  }
  const int xs = x0 - HALO + lane;  // this lane's statistics column
  const bool out_lane = lane >= HALO && lane < HALO + SW;
  float ring1[11][5];  // horizontal blur of the statistics, by row mod 11
  float ring2[11][3];  // horizontal blur of the partial maps, by row mod 11
  float loss_local = 0.f;
  const LossBufs bufs = loss_bufs(a);
  const int xi0 = x0 - 2 * HALO + lane;
  const LaneCols lc{(uint32_t)min(max(xi0, 0), W - 1), (uint32_t)min(xi0 + 64, W - 1), (uint32_t)min(max(xs, 0), W - 1)};
  StepRaw nxt = fetch_step(a, bufs, lc, c, y0, -extra);
  for (int base = 0; base < ROWS; base += 11) {
#pragma unroll
    for (int j = 0; j < 11; j++) {
      const int rw = base + j;   // step of the walk (ring slot j, LDS buffer rw & 1)
      const int r = rw - extra;  // input row y0 - 10 + r
      const int buf = rw & 1;
      const StepRaw cur = nxt;
      nxt = fetch_step(a, bufs, lc, c, y0, r + 1);  // clamped rows: in bounds past the strip's end too
      // ---- input row y_in: columns x0 - 10 .. x0 + 63
      const int y_in = y0 - 2 * HALO + r;
      {
        const int xi = x0 - 2 * HALO + lane;
        const bool v1 = in_image(a, xi, y_in);
        const float pr = v1 ? cur.p_in : 0.f, gr = v1 ? gt_effective(cur.g_in, c, a.composite, bg_c) : 0.f;
        s_p[buf][lane] = pr - c1; s_g[buf][lane] = gr - c2;
        s_rp[j][lane] = pr; s_rg[j][lane] = gr;
        if (lane < 2 * HALO) {
          const bool v2 = in_image(a, xi + 64, y_in);
          const float pr2 = v2 ? cur.p_in2 : 0.f, gr2 = v2 ? gt_effective(cur.g_in2, c, a.composite, bg_c) : 0.f;
          s_p[buf][64 + lane] = pr2 - c1; s_g[buf][64 + lane] = gr2 - c2;
          s_rp[j][64 + lane] = pr2; s_rg[j][64 + lane] = gr2;
        }
      }
      __syncthreads();
      {
        float sx = 0.f, sx2 = 0.f, sy = 0.f, sy2 = 0.f, sxy = 0.f;
#pragma unroll
        for (int d = 0; d < 11; d++) {
          const float w = gw_tap(d);
          const float x = s_p[buf][lane + d], y = s_g[buf][lane + d];
          const float wx = w * x, wy = w * y;
          sx += wx; sx2 += wx * x; sy += wy; sy2 += wy * y; sxy += wx * y;
        }
        ring1[j][0] = sx; ring1[j][1] = sx2; ring1[j][2] = sy; ring1[j][3] = sy2; ring1[j][4] = sxy;
      }
      if (r >= 2 * HALO) {
        // ---- statistics row ys complete: vertical blur, SSIM, partial maps
        const int ys = y_in - HALO;
        float st[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < 11; d++) {
          const int slot = (j + 1 + d) % 11;  // oldest row first
          const float w = gw_tap(d);
#pragma unroll
          for (int k = 0; k < 5; k++) st[k] += w * ring1[slot][k];
        }
        float A = 0.f, B = 0.f, Bm = 0.f, Cc = 0.f, Cm = 0.f;
        if (in_image(a, xs, ys)) {
          const float M = weight_of(a, cur.w_ss) * (a.mask ? gt_channel(cur.g_ss, 3) : 1.f) * norm;
          const float mu1 = st[0] + c1, mu2 = st[2] + c2;
          const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2;
          const float s1_raw = st[1] - st[0] * st[0], s2_raw = st[3] - st[2] * st[2];
          const float sigma1_sq = fmaxf(0.f, s1_raw), sigma2_sq = fmaxf(0.f, s2_raw);
          const float sigma12 = st[4] - st[0] * st[2];
          const float A1 = 2.f * mu1 * mu2 + C1, A2 = 2.f * sigma12 + C2;
          const float B1 = mu1_sq + mu2_sq + C1, B2 = sigma1_sq + sigma2_sq + C2;
          const float raw = (A1 * A2) / (B1 * B2);
          const float ssim = fminf(fmaxf(raw, -1.f), 1.f);
          if (out_lane && ys >= y0 && ys < y0 + SH) {
            const int slot = (j + 6) % 11;  // input row r - 5
            const float g = s_rg[slot][lane + HALO];
            loss_local += M * (a.l1_w * fabsf(s_rp[slot][lane + HALO] - g) + a.ssim_w * ssim);
          }
          if (raw > -1.f && raw < 1.f) {
            // one reciprocal for the three quotients (1 / B1 = B2 / (B1 B2), 1 / B2 = B1 / (B1 B2)); the
            // SSIM value itself stays a correctly rounded quotient, so equal inputs give exactly 1
            const float k = M * a.ssim_w;
            const float inv_BB = __builtin_amdgcn_rcpf(B1 * B2);
            const float d_mu1 = 2.f * mu2 * A2 * inv_BB - 2.f * mu1 * ssim * (B2 * inv_BB);
            const float d_s1 = s1_raw > 0.f ? -ssim * (B1 * inv_BB) : 0.f;
            const float d_s12 = 2.f * A1 * inv_BB;
            A = k * d_mu1; B = k * d_s1; Bm = B * st[0]; Cc = k * d_s12; Cm = Cc * st[2];
          }
        }
        // the gradient is blur(A) + 2 p blur(B) - 2 blur(B mu1) + g blur(C) - blur(C mu2): the three terms
        // without a per-output factor are blurred as one map
        s_pm[buf][0][lane] = A - 2.f * Bm - Cm; s_pm[buf][1][lane] = B; s_pm[buf][2][lane] = Cc;
        __syncthreads();
        // ---- horizontal pass of the second blur at output column x0 + lane - 5
        const int j2 = (j + 1) % 11;  // slot of partial-map row ys (stats row index r - 10)
#pragma unroll
        for (int k = 0; k < 3; k++) ring2[j2][k] = 0.f;
        if (out_lane) {
#pragma unroll
          for (int d = 0; d < 11; d++) {
            const float w = gw_tap(d);
#pragma unroll
            for (int k = 0; k < 3; k++) ring2[j2][k] += w * s_pm[buf][k][lane - HALO + d];
          }
        }
        if (r >= 4 * HALO) {
          // ---- output row yo = ys - 5 complete: vertical pass, gradient
          const int yo = ys - HALO, xo = xs;
          float acc[3] = {0.f, 0.f, 0.f};
#pragma unroll
          for (int d = 0; d < 11; d++) {
            const int slot = (j2 + 1 + d) % 11;
            const float w = gw_tap(d);
#pragma unroll
            for (int k = 0; k < 3; k++) acc[k] += w * ring2[slot][k];
          }
          if (out_lane && yo < H && xo < W) {
            const int pix = yo * W + xo;
            const int slot = (j + 1) % 11;  // input row r - 10
            const float p = s_rp[slot][lane + HALO], g = s_rg[slot][lane + HALO];
            const float ps = p - c1, gs = g - c2;
            const float gt_a = gt_channel(cur.g_out, 3);
            const float M = weight_of(a, cur.w_out) * (a.mask ? gt_a : 1.f) * norm;
            const float sgn = p > g ? 1.f : (p < g ? -1.f : 0.f);
            const float grad = M * a.l1_w * sgn + acc[0] + 2.f * ps * acc[1] + gs * acc[2];
            a.v_out[(size_t)pix * 4 + c] = grad * a.grad_scale;
            if (c == 0) {
              float va = 0.f;
              if (a.alpha_lane) {
                const float da = cur.a_out - gt_a;
                const float sa = da > 0.f ? 1.f : (da < 0.f ? -1.f : 0.f);
                const float Ma = weight_of(a, cur.w_out) * alpha_norm;
                va = Ma * sa * a.grad_scale;
                loss_local += Ma * fabsf(da);
              }
              a.v_out[(size_t)pix * 4 + 3] = va;
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) loss_local += __shfl_xor(loss_local, o);
  if (lane == 0) {
    const int idx = item;
    if (a.partials)
      a.partials[idx] = loss_local;
    else if (loss_local != 0.f)
      atomicAdd(a.loss_accum, loss_local);
  }
}

// Fixed-order double-precision sum of the per-workgroup partials into loss_accum[0] (one wave).
__global__ void __launch_bounds__(64) reduce_partials_kernel(const float* __restrict__ partials, int count,
                                                              float* __restrict__ loss_accum, int assign,
                                                              int running) {
  loss_partials_store(partials, count, loss_accum, assign, running);
}

__global__ void accumulate_kernel(float* acc) {
  acc[2] += acc[0] + acc[1];
  acc[3] += 1.f;
}

__global__ void step_sums_kernel(float* acc) {
  acc[2] = acc[0] + acc[1];
  acc[3] = 1.f;
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

namespace {

// SIMDs of the device and the waves of the photometric kernel each holds at once (per-CU occupancy from
// the runtime; every workgroup is one wave).
struct LossSlots {
  int simds, per_simd;
};

LossSlots loss_slots() {
  static LossSlots cached{0, 0};
  if (cached.simds) return cached;
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, photometric_kernel, 64, 0) != hipSuccess || cus <= 0 ||
      per_cu < 4) {
    (void)hipGetLastError();
    return LossSlots{256 * 4, 3};  // MI355X: 256 CUs of 4 SIMDs, 3 waves of this size per SIMD
  }
  cached = LossSlots{cus * 4, per_cu / 4};
  return cached;
}

// Strip height. Every wave walks SH + 20 rows rounded up to whole rings, so the kernel takes about (rounds
// of resident waves) x (rows walked); pick the height in [SH_MIN, SH_MAX] that minimises it for this image
// and device, the tallest on ties (fewer waves). The kernel is VALU-bound: at 1080p heights 39 and 46 (one
// round, 66 rows walked) measured the same, 94.6 and 94.2 us, and 60 (under two waves per SIMD) 96.4 us.
// B2C_LOSS_STRIP_ROWS (a height in that range) overrides the choice, for tests and tuning.
int pick_strip_rows(int W, int H) {
  if (const char* env = getenv("B2C_LOSS_STRIP_ROWS")) {
    const int v = atoi(env);
    if (v >= SH_MIN && v <= SH_MAX) return v;
  }
  const LossSlots sl = loss_slots();
  const long slots = (long)sl.simds * sl.per_simd;
  const int strips_x = (W + SW - 1) / SW;
  int best = SH_MIN;
  long best_cost = -1;
  for (int sh = SH_MIN; sh <= SH_MAX; sh++) {
    const long waves = (long)strips_x * ((H + sh - 1) / sh) * 3;
    const long cost = ((waves + slots - 1) / slots) * ((sh + 4 * HALO + 10) / 11 * 11);
    if (best_cost < 0 || cost <= best_cost) {
      best_cost = cost;
      best = sh;
    }
  }
  return best;
}

}  // namespace

extern "C" int b2c_hip_photometric(const b2c_loss_args* a, hipStream_t stream) {
  if (a->W <= 0 || a->H <= 0) return 0;
  if ((uint64_t)a->W * (uint64_t)a->H * 16u > 0xFFFFFFFFull) return (int)hipErrorInvalidValue;  // 32-bit buffer offsets
  if (a->assign && !a->partials) return (int)hipErrorInvalidValue;  // float atomics can only add
  if (a->running && !a->assign) return (int)hipErrorInvalidValue;    // the running sum needs the final value
  // the kernel's constant weights must equal the double-precision Gaussian rounded to float
  static const bool weights_ok = [] {
    double w[11], sum = 0.0;
    for (int i = 0; i < 11; i++) {
      const double x = i - 5.0;
      w[i] = __builtin_exp(-x * x / (2.0 * 1.5 * 1.5));
      sum += w[i];
    }
    for (int i = 0; i < 11; i++) {
      const float f = (float)(w[i] / sum);
      uint32_t bits;
      memcpy(&bits, &f, 4);
      if (bits != GW_BITS[i]) return false;
    }
    return true;
  }();
  if (!weights_ok) return (int)hipErrorInvalidValue;
  const int strips_x = (a->W + SW - 1) / SW;
  const int sh = pick_strip_rows(a->W, a->H);
  const int nstrips = strips_x * ((a->H + sh - 1) / sh);
  const dim3 grid(8 * ((nstrips * 3 + 7) / 8)), block(64);
  photometric_kernel<<<grid, block, 0, stream>>>(*a, strips_x, nstrips, sh);
  if (a->partials && a->defer_sum_count)
    *a->defer_sum_count = nstrips * 3;  // the caller reduces them later (loss_partials_store)
  else if (a->partials)
    reduce_partials_kernel<<<1, 64, 0, stream>>>(a->partials, nstrips * 3, a->loss_accum, a->assign, a->running);
  return (int)hipGetLastError();
}

// ---- allocation-free entry point: the per-workgroup partials live in a fixed device array ----
// Each GPU the library runs on holds its own copy of `scratch` until the process ends. Host code must not
// pass the array's name to a kernel (on the host it is only a stand-in symbol): the device address comes
// from hipGetSymbolAddress, once per device with that device current, and is kept per device.
static __device__ __align__(256) float scratch[B2C_LOSS_STATIC_PARTIALS];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[MAX_DEVICES] = {};

hipError_t device_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace

extern "C" int b2c_hip_photometric_noalloc(const b2c_loss_args* a, hipStream_t stream) {
  if (a->W <= 0 || a->H <= 0) return 0;
  if (b2c_loss_partials(a->W, a->H) > (size_t)B2C_LOSS_STATIC_PARTIALS) return (int)hipErrorInvalidValue;
  if (a->defer_sum_count) return (int)hipErrorInvalidValue;  // its partials must be reduced before the next call
  float* partials = nullptr;
  const hipError_t e = device_scratch(&partials);
  if (e != hipSuccess) return (int)e;
  b2c_loss_args b = *a;
  b.partials = partials;  // every entry the reduce reads is written by this call's workgroups first
  return b2c_hip_photometric(&b, stream);
}

extern "C" int b2c_hip_step_loss_sums(float* loss_accum, hipStream_t stream) {
  step_sums_kernel<<<1, 1, 0, stream>>>(loss_accum);
  return (int)hipGetLastError();
}

extern "C" size_t b2c_loss_partials(int W, int H) {
  return (size_t)((W + SW - 1) / SW) * ((H + SH_MIN - 1) / SH_MIN) * 3;  // the most strips any choice makes
}

extern "C" int b2c_hip_accumulate_loss(float* loss_accum, hipStream_t stream) {
  accumulate_kernel<<<1, 1, 0, stream>>>(loss_accum);
  return (int)hipGetLastError();
}
