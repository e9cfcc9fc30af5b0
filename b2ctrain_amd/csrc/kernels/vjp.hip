// Projection VJP and fused optimizer (replaces optim_kernel, src/gpu/optim.cu:99-377): one thread per
// splat turns the 13 screen-space gradient lanes into parameter gradients [pos3, opacity, quat4,
// log-scale3, SH 3K]. Reads and clears v_splat and vis_flag (the consumed-and-zeroed contract of
// optim.cu:110-121). With grad_out set the gradients are written (optim.cu:292-296): accumulate = 1 adds
// into grad_out so gradients of several views can be summed; 0 overwrites like the reference, and with
// sparse set leaves the rows of splats without gradient alone as the reference's early return does
// (optim.cu:148). Without grad_out the same gradient row feeds the Adam / lazy sparse Adam / MCMC noise
// update of the splat's parameters (adam_update below).
// The chain is derived here from the semi-axis form of the projection (screen_splat.h): from the conic to
// the screen covariance, to the image-plane semi-axes u_j, and from those to the semi-axis lengths, the
// camera-frame rotation, the Jacobian scale and the ray tangents; the colour's view-direction term comes
// from the SH basis evaluated on dual numbers. No world-space covariance is formed. Evaluated without FMA
// contraction (the culling decisions of the recomputed projection must match the forward's bit for bit).
#pragma clang fp contract(off)
#include <cmath>

#include "b2c_kernels.h"
#include "device_math.h"
#include "screen_splat.h"
#include "adam_math.h"
#include "loss_sum.h"

namespace b2c {
namespace dev {
namespace {

// d L / d q for the unit quaternion q = (w, v) of R(q), given G = d L / d R (row major). Writing
// a = (G21 - G12, G02 - G20, G10 - G01) for the axial vector of G - G^T and S = G + G^T:
//   d L / d w = 2 v . a,   d L / d v = 2 (w a + S v - 2 tr(G) v),
// from differentiating R = (w^2 - v.v) I + 2 v v^T + 2 w [v]x entrywise on the unit sphere's embedding.
__device__ __forceinline__ float4 rotation_vjp(float w, float x, float y, float z, const float* G) {
  const float ax = G[7] - G[5], ay = G[2] - G[6], az = G[3] - G[1];
  const float tr2 = 2.f * ((G[0] + G[4]) + G[8]);
  const float s01 = G[1] + G[3], s02 = G[2] + G[6], s12 = G[5] + G[7];
  const float svx = 2.f * G[0] * x + s01 * y + s02 * z;
  const float svy = s01 * x + 2.f * G[4] * y + s12 * z;
  const float svz = s02 * x + s12 * y + 2.f * G[8] * z;
  return make_float4(2.f * ((x * ax + y * ay) + z * az), 2.f * (w * ax + svx - tr2 * x), 2.f * (w * ay + svy - tr2 * y),
                     2.f * (w * az + svz - tr2 * z));
}

// Through the normalisation q / |q|: the gradient's component along q vanishes, the rest scales by 1/|q|.
__device__ __forceinline__ float4 unit_quat_vjp(float4 qn, float inv_len, float4 g) {
  const float along = ((qn.x * g.x + qn.y * g.y) + qn.z * g.z) + qn.w * g.w;
  return make_float4((g.x - qn.x * along) * inv_len, (g.y - qn.y * along) * inv_len, (g.z - qn.z * along) * inv_len,
                     (g.w - qn.w * along) * inv_len);
}

// The per-splat rows of v_splat (13 floats) and grad_out (11 + 3K floats) are read and written through
// LDS by the whole workgroup, so consecutive lanes touch consecutive addresses (a lane-per-row access
// would touch one cache line per lane per instruction).
constexpr int VJP_BLOCK = 64;

// One Adam step on one parameter, after the lazy catch-up (optim.cu:301-315). A splat last updated s + 1
// steps ago would, under dense Adam with zero gradient, have seen its moments decay to beta1^s m and
// beta2^s v and moved by lr sum_{k=1..s} (beta1^k m) / sqrt(beta2^k v) = lr drift m / sqrt(v), with
// drift = r (1 - r^s) / (1 - r) and r = beta1 / sqrt(beta2) (the bias corrections held at this step's).
struct CatchUp {
  float skipped, d1, d2, drift;
};

__device__ __forceinline__ void adam_param(float& p, float& m, float& v, float g, float lr, const b2c_adam_step& s,
                                           const CatchUp& cu) {
  if (cu.skipped > 0.f) {
    p = p - ((lr * cu.drift) * (m * s.bc1)) / (sqrtf(v * s.bc2) + s.eps);
    m = m * cu.d1;
    v = v * cu.d2;
  }
  m = s.beta1 * m + (1.f - s.beta1) * g;
  v = s.beta2 * v + ((1.f - s.beta2) * g) * g;
  p = p - (lr * (m * s.bc1)) / (sqrtf(v * s.bc2) + s.eps);
}

__device__ __forceinline__ void adam_param4(float4& p, float4& m, float4& v, float4 g, float4 lr, const b2c_adam_step& s,
                                            const CatchUp& cu) {
  adam_param(p.x, m.x, v.x, g.x, lr.x, s, cu);
  adam_param(p.y, m.y, v.y, g.y, lr.y, s, cu);
  adam_param(p.z, m.z, v.z, g.z, lr.z, s, cu);
  adam_param(p.w, m.w, v.w, g.w, lr.w, s, cu);
}

// The fused optimizer (optim.cu:298-377) for splat i, given its gradient row g = [pos3, opacity logit,
// quat4, log-scale3, SH 3K] as the VJP built it, bsq = sum_k Y_k^2 over the active basis and the colour
// gradient (vcx, vcy, vcz) (both zero when the splat has no gradient):
//   - Adam with bias correction on pos_op (lr_mean for the mean, lr_opac for the logit), quat (lr_rot) and
//     the log scales (lr_scale; the frozen floor lscale.w and its moments stay as they are / zero);
//   - the SH: a first moment per lane, one second moment per splat from the lane-mean squared gradient
//     bsq |vc|^2 / 3K, lr_dc on the DC lanes and lr_sh_rest above; fp16 bands stored with stochastic rounding;
//   - in sparse mode the lazy catch-up of the steps the splat skipped, and last_step = t;
//   - MCMC noise on the means of visible splats: N(0, 1) per axis times noise_weight (1 - opacity)^150,
//     clamped to +-noise_clamp (optim.cu:361-375).
// A splat's float4 parameters with their moments, v_sh and last_step: loaded by the update kernel in its first
// memory round trip, together with the screen-space gradient, so their latency overlaps the VJP.
struct SplatState {
  float4 po, q, ls, mp, vp, mq, vq, ml, vl;
  float vsh;
  uint32_t last;
};

__device__ __forceinline__ SplatState load_state(const b2c_vjp_args& a, int i) {
  const b2c_adam_state& st = a.adam;
  SplatState x;
  x.po = reinterpret_cast<const float4*>(a.pos_op)[i];
  x.q = reinterpret_cast<const float4*>(a.quat)[i];
  x.ls = reinterpret_cast<const float4*>(a.lscale)[i];
  x.mp = reinterpret_cast<const float4*>(st.m_pos_op)[i];
  x.vp = reinterpret_cast<const float4*>(st.v_pos_op)[i];
  x.mq = reinterpret_cast<const float4*>(st.m_quat)[i];
  x.vq = reinterpret_cast<const float4*>(st.v_quat)[i];
  x.ml = reinterpret_cast<const float4*>(st.m_lscale)[i];
  x.vl = reinterpret_cast<const float4*>(st.v_lscale)[i];
  x.vsh = st.v_sh[i];
  x.last = a.step.sparse ? st.last_step[i] : 0u;
  return x;
}

template <int DEG, bool HALF>
__device__ __forceinline__ void adam_update(const b2c_vjp_args& a, int i, const float* g, bool visible, float bsq,
                                            float vcx, float vcy, float vcz, const SplatState& x) {
  constexpr int K = (DEG + 1) * (DEG + 1);
  constexpr int L = 3 * K;
  const b2c_adam_step& s = a.step;
  const b2c_adam_state& st = a.adam;
  float4* const P4 = reinterpret_cast<float4*>(a.pos_op);
  float4* const Q4 = reinterpret_cast<float4*>(a.quat);
  float4* const L4 = reinterpret_cast<float4*>(a.lscale);
  float4* const MP = reinterpret_cast<float4*>(st.m_pos_op);
  float4* const VP = reinterpret_cast<float4*>(st.v_pos_op);
  float4* const MQ = reinterpret_cast<float4*>(st.m_quat);
  float4* const VQ = reinterpret_cast<float4*>(st.v_quat);
  float4* const ML = reinterpret_cast<float4*>(st.m_lscale);
  float4* const VL = reinterpret_cast<float4*>(st.v_lscale);
  // The per-splat words were loaded before the VJP (load_state); every store here follows all loads,
  // since a store the compiler cannot prove disjoint from a later load holds that load back.
  float4 po = x.po, q = x.q, ls = x.ls, mp = x.mp, vp = x.vp, mq = x.mq, vq = x.vq, ml = x.ml, vl = x.vl;
  float vsh = x.vsh;
  const uint32_t last = x.last;
  CatchUp cu{0.f, 1.f, 1.f, 0.f};
  if (s.sparse) {
    cu.skipped = last == 0u ? 0.f : fmaxf(((float)s.t - (float)last) - 1.f, 0.f);
    if (cu.skipped > 0.f) {
      cu.d1 = det_expf(cu.skipped * s.ln_beta1);
      cu.d2 = det_expf(cu.skipped * s.ln_beta2);
      cu.drift = (s.ratio * (1.f - det_expf(cu.skipped * s.ln_ratio))) / (1.f - s.ratio);
    }
  }
  adam_param4(po, mp, vp, make_float4(g[0], g[1], g[2], g[3]), make_float4(s.lr_mean, s.lr_mean, s.lr_mean, s.lr_opac),
              s, cu);
  adam_param4(q, mq, vq, make_float4(g[4], g[5], g[6], g[7]), make_float4(s.lr_rot, s.lr_rot, s.lr_rot, s.lr_rot), s, cu);
  adam_param(ls.x, ml.x, vl.x, g[8], s.lr_scale, s, cu);
  adam_param(ls.y, ml.y, vl.y, g[9], s.lr_scale, s, cu);
  adam_param(ls.z, ml.z, vl.z, g[10], s.lr_scale, s, cu);
  ml.w = 0.f;
  vl.w = 0.f;
  const float gsq = (bsq * ((vcx * vcx + vcy * vcy) + vcz * vcz)) * (1.f / (float)L);
  vsh = vsh * cu.d2;
  const float denom_old = cu.skipped > 0.f ? (cu.drift * s.bc1) / (sqrtf(vsh * s.bc2) + s.eps) : 0.f;
  vsh = s.beta2 * vsh + (1.f - s.beta2) * gsq;
  const float denom = s.bc1 / (sqrtf(vsh * s.bc2) + s.eps);
  if (s.noise_weight > 0.f && visible) {
    const float sig = 1.f / (1.f + det_expf(-po.w));
    float comp = 1.f;
    if (ls.w > 0.f) {  // the floor's opacity factor, as the projection forms it
      const float f2 = ls.w * ls.w;
      const float vx = det_expf(2.f * ls.x), vy = det_expf(2.f * ls.y), vz = det_expf(2.f * ls.z);
      comp = sqrtf(((vx / (vx + f2)) * (vy / (vy + f2))) * (vz / (vz + f2)));
    }
    const float o = fminf(fmaxf(sig * comp, 0.f), 1.f);
    const float w = fminf(fmaxf(det_expf(150.f * det_logf(1.f - o)), 0.f), 1.f) * s.noise_weight;
    if (w > 0.f) {
      const uint32_t ns = s.seed ^ (s.step * 0x9E3779B9u);
      const float cl = s.noise_clamp;
      po.x = po.x + fminf(fmaxf(hash_gauss(ns, (uint32_t)i, 0u) * w, -cl), cl);
      po.y = po.y + fminf(fmaxf(hash_gauss(ns, (uint32_t)i, 1u) * w, -cl), cl);
      po.z = po.z + fminf(fmaxf(hash_gauss(ns, (uint32_t)i, 2u) * w, -cl), cl);
    }
  }
  P4[i] = po; Q4[i] = q; L4[i] = ls;
  MP[i] = mp; VP[i] = vp; MQ[i] = mq; VQ[i] = vq; ML[i] = ml; VL[i] = vl;
  st.v_sh[i] = vsh;
  if (s.sparse) st.last_step[i] = (uint32_t)s.t;
  // The SH lanes (planar, coalesced across the wave) in chunks: a chunk's parameters and moments are all
  // loaded before any of its stores, so each chunk is one memory round trip.
  const uint32_t sr_seed = (s.seed ^ (s.step * 0x9E3779B9u)) ^ 0x5A5A5A5Au;
  const b2c_sh_planes& pw = a.sh_out;
  const b2c_sh_planes& mw = st.m_sh;
  constexpr int CH = 16;
#pragma unroll
  for (int c0 = 0; c0 < L; c0 += CH) {
    float p[CH], m[CH];
#pragma unroll
    for (int j = 0; j < CH; j++) {
      const int lane = c0 + j;
      if (lane >= L) break;
      const size_t o = (size_t)(lane < 3 ? lane : lane - 3) * pw.stride + i;
      if (lane < 3) {
        p[j] = pw.dc[o];
        m[j] = mw.dc[o];
      } else if constexpr (HALF) {
        p[j] = f16_value(pw.hi16[o]);
        m[j] = f16_value(mw.hi16[o]);
      } else {
        p[j] = pw.hi32[o];
        m[j] = mw.hi32[o];
      }
    }
#pragma unroll
    for (int j = 0; j < CH; j++) {
      const int lane = c0 + j;
      if (lane >= L) break;
      const float lrk = lane < 3 ? s.lr_dc : s.lr_sh_rest;
      const size_t o = (size_t)(lane < 3 ? lane : lane - 3) * pw.stride + i;
      float pj = p[j], mj = m[j];
      if (cu.skipped > 0.f) {
        pj = pj - (lrk * denom_old) * mj;
        mj = mj * cu.d1;
      }
      mj = s.beta1 * mj + (1.f - s.beta1) * g[11 + lane];
      pj = pj - (lrk * denom) * mj;
      if (lane < 3) {
        mw.dc[o] = mj;
        pw.dc[o] = pj;
      } else if constexpr (HALF) {
        mw.hi16[o] = f16_bits(mj);
        pw.hi16[o] = f16_stochastic(pj, hash_unit(sr_seed, (uint32_t)i, (uint32_t)lane));
      } else {
        mw.hi32[o] = mj;
        pw.hi32[o] = pj;
      }
    }
  }
}

template <int DEG, bool HALF, bool ADAM>
__global__ void __launch_bounds__(VJP_BLOCK) vjp_kernel(b2c_vjp_args a) {
  constexpr int K = (DEG + 1) * (DEG + 1);
  constexpr int PER = 11 + 3 * K;
  __shared__ __attribute__((aligned(16))) float s_buf[VJP_BLOCK * PER];  // v_splat rows in, grad_out rows out
  __shared__ uint32_t s_vis[VJP_BLOCK], s_any[VJP_BLOCK];
  const int i0 = blockIdx.x * VJP_BLOCK;
  const int i = i0 + threadIdx.x;
  const int rows = min(VJP_BLOCK, a.n - i0);
  // a deferred loss reduction, in the first workgroup (one wave)
  if (a.loss_partials && blockIdx.x == 0)
    loss_partials_store(a.loss_partials, a.loss_count, a.loss_accum, a.loss_assign, a.loss_running);
  const bool in_range = i < a.n;
  // Memory round trip 1: this splat's flag, tile count and statistics, and the block's v_splat rows (one
  // contiguous, 16-byte aligned stretch of VJP_BLOCK * 13 floats), all issued before any is waited for.
  uint32_t vis = 0u, tc = 0u;
  float vcount = 0.f, rnorm = 0.f, vweight = 0.f;
  SplatState pre{};  // the update's per-splat words
  const bool from_row = a.vis_from_row != 0;  // uniform
  if (in_range) {
    if (!from_row) vis = a.vis_flag[i];
    else if (a.vis_weight) vweight = a.vis_weight[i];
    tc = a.tile_count[i];
    if (a.vis_count) vcount = a.vis_count[i];
    if (a.refine_norm) rnorm = a.refine_norm[i];
    if constexpr (ADAM) pre = load_state(a, i);
  }
  const int nin = rows * GRAD_LANES;
  const float* vin = a.v_splat + (size_t)i0 * GRAD_LANES;
  if (rows == VJP_BLOCK) {  // uniform: a whole block, a fixed number of loads per thread
    constexpr int N4 = VJP_BLOCK * GRAD_LANES / 4, FULL = N4 / VJP_BLOCK, REM = N4 - FULL * VJP_BLOCK;
    static_assert(VJP_BLOCK * GRAD_LANES % 4 == 0 && FULL == 3, "whole float4s per block, 3 + a remainder");
    const float4* v4 = reinterpret_cast<const float4*>(vin) + threadIdx.x;
    float4* b4 = reinterpret_cast<float4*>(s_buf) + threadIdx.x;
    const bool rem = threadIdx.x < REM;
    const float4 t0 = v4[0], t1 = v4[VJP_BLOCK], t2 = v4[2 * VJP_BLOCK];
    float4 t3 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (rem) t3 = v4[3 * VJP_BLOCK];
    b4[0] = t0; b4[VJP_BLOCK] = t1; b4[2 * VJP_BLOCK] = t2;
    if (rem) b4[3 * VJP_BLOCK] = t3;
  } else {
    for (int j = threadIdx.x; j < nin / 4; j += VJP_BLOCK)
      reinterpret_cast<float4*>(s_buf)[j] = reinterpret_cast<const float4*>(vin)[j];
    for (int j = (nin & ~3) + threadIdx.x; j < nin; j += VJP_BLOCK) s_buf[j] = vin[j];
  }
  __syncthreads();
  // a backward run with defer_vis left the blend-weight sum in lane 10 (a feature lane, zero otherwise)
  const float wsum = from_row && in_range ? s_buf[threadIdx.x * GRAD_LANES + 10] : 0.f;
  if (from_row) vis = wsum > 0.f ? 1u : 0u;
  float g[GRAD_LANES];
#pragma unroll
  for (int k = 0; k < GRAD_LANES; k++) g[k] = vis && !(from_row && k == 10) ? s_buf[threadIdx.x * GRAD_LANES + k] : 0.f;
  s_vis[threadIdx.x] = vis;
  __syncthreads();  // s_buf now holds the grad_out rows
  // Update the statistics, then clear the consumed flag and rows (optim.cu:110-121). The loaded words are
  // all used before the clearing loop: its store count is not known at compile time, so a use of an
  // earlier load after it would wait for every memory operation in flight.
  const bool visible = vis != 0u && tc != 0u;
  if (a.vis_count && in_range) a.vis_count[i] = vcount + (visible ? 1.f : 0.f);
  if (a.refine_norm && in_range) {
    const float rn = __builtin_isfinite(g[9]) ? fminf(fmaxf(g[9], 0.f), 1e32f) : 0.f;
    a.refine_norm[i] = fmaxf(rnorm, rn);
  }
  if (from_row) {
    if (vis && a.vis_weight) a.vis_weight[i] = vweight + wsum;
  } else if (vis) {
    a.vis_flag[i] = 0u;
  }
  for (int j = threadIdx.x; j < rows * GRAD_LANES; j += VJP_BLOCK)
    if (s_vis[j / GRAD_LANES]) a.v_splat[(size_t)i0 * GRAD_LANES + j] = 0.f;
  bool any = false;
#pragma unroll
  for (int k = 0; k < GRAD_LANES; k++) if (k != 9 && g[k] != 0.f) any = true;
  any = any && visible;
#pragma unroll
  for (int k = 0; k < GRAD_LANES; k++) if (!__builtin_isfinite(g[k])) any = false;

  // this splat's grad_out row is built in LDS as it is computed (the SH part first), so no 11 + 3K
  // register array stays live across the projection VJP
  float* out = s_buf + threadIdx.x * PER;
  bool done = false;
  float bsq_done = 0.f;
  if (any) {
    // Memory round trip 2: the splat's parameters (already loaded for the update) and all its SH
    // coefficients, issued together
    const float4 po = ADAM ? pre.po : reinterpret_cast<const float4*>(a.pos_op)[i];
    const float4 q = ADAM ? pre.q : reinterpret_cast<const float4*>(a.quat)[i];
    const float4 ls = ADAM ? pre.ls : reinterpret_cast<const float4*>(a.lscale)[i];
    const ShView sv{a.sh.dc, reinterpret_cast<const _Float16*>(a.sh.hi16), a.sh.hi32, a.sh.stride};
    float coef[3 * K];
    if constexpr (HALF)
      sv.load_all<DEG, true>(i, coef);
    else
      sv.load_all_either<DEG>(i, coef);
    const b2c_camera_gpu& cam = a.cam;
    // the camera-to-splat vector, as screen_splat forms it
    const float dvx = po.x - cam.pos[0], dvy = po.y - cam.pos[1], dvz = po.z - cam.pos[2];
    const float dl = sqrtf((dvx * dvx + dvy * dvy) + dvz * dvz);
    const float idl = 1.f / dl;
    const int kmax = a.active_deg >= DEG ? K : (a.active_deg + 1) * (a.active_deg + 1);
    const float vcr = g[5], vcg = g[6], vcb = g[7];
    // Colour = sum_k coef_k Y_k(dir) + 0.5: the SH rows are Y_k * v_rgb, and the direction gradient is
    // sum_k (coef_k . v_rgb) grad Y_k, taken on dual numbers; the SH half runs first, so the
    // coefficients are dead before the projection's registers are live.
    float gdx = 0.f, gdy = 0.f, gdz = 0.f;
    float bsq = 0.f;  // sum of the squared basis values (the SH second moment's share, optim.cu:337-339)
    {
      float wk[K];
#pragma unroll
      for (int k = 0; k < K; k++) wk[k] = k < kmax ? (coef[3 * k] * vcr + coef[3 * k + 1] * vcg) + coef[3 * k + 2] * vcb : 0.f;
      Dual3 yk[K];
      sh_basis<DEG>(Dual3{dvx * idl, 1.f, 0.f, 0.f}, Dual3{dvy * idl, 0.f, 1.f, 0.f}, Dual3{dvz * idl, 0.f, 0.f, 1.f}, yk);
#pragma unroll
      for (int k = 0; k < K; k++) {
        const float y = k < kmax ? yk[k].v : 0.f;
        out[11 + 3 * k] = y * vcr; out[12 + 3 * k] = y * vcg; out[13 + 3 * k] = y * vcb;
        if constexpr (ADAM) bsq = bsq + y * y;
        gdx = gdx + wk[k] * yk[k].x; gdy = gdy + wk[k] * yk[k].y; gdz = gdz + wk[k] * yk[k].z;
      }
    }
    const ScreenSplat sp = screen_splat(po, q, ls, cam);
    if (sp.ok) {
      // dir = d / |d|: only the gradient's part across dir moves it
      const float ux = dvx * idl, uy = dvy * idl, uz = dvz * idl;
      const float radial = (ux * gdx + uy * gdy) + uz * gdz;
      const float gsx = (gdx - ux * radial) * idl, gsy = (gdy - uy * radial) * idl, gsz = (gdz - uz * radial) * idl;
      // Conic C = Sigma'^-1: dL/dSigma' = -C Gc C (Gc = [[g2, g3/2], [g3/2, g4]]), and Sigma' = U U^T + 0.3 I gives
      // dL/du_j = 2 dL/dSigma' u_j = -2 C Gc (C u_j). C u_j is formed as adj(Sigma') u_j / det with
      // adj(Sigma') u_j = sum_{k != j} (u_j x u_k) (uy_k, -ux_k) + 0.3 u_j: for the long axis of an elongated
      // footprint, C u_j is small and the conic's entries would leave it as the difference of two nearly
      // equal products. With u_j = (jx e_j, jy f_j) a_j, e_j = W0j - tx W2j and f_j = W1j - ty W2j, collect
      // the gradients of the semi-axis lengths, of W, and of jx, jy, tx, ty.
      const float idet = sp.idet;
      const float h = 0.5f * g[3];
      const float xs[3][3] = {{0.f, sp.cross[0], sp.cross[1]}, {-sp.cross[0], 0.f, sp.cross[2]}, {-sp.cross[1], -sp.cross[2], 0.f}};
      float gaxis[3], gW[9];
      float gjx = 0.f, gjy = 0.f, gtx = 0.f, gty = 0.f;
#pragma unroll
      for (int j = 0; j < 3; j++) {
        float ax_ = 0.3f * sp.ux[j], ay_ = 0.3f * sp.uy[j];
#pragma unroll
        for (int k = 0; k < 3; k++) {
          if (k == j) continue;
          ax_ = ax_ + xs[j][k] * sp.uy[k];
          ay_ = ay_ - xs[j][k] * sp.ux[k];
        }
        const float cux = ax_ * idet, cuy = ay_ * idet;  // C u_j
        const float vx = g[2] * cux + h * cuy, vy = h * cux + g[4] * cuy;
        const float gux = -2.f * (sp.cov.c11 * vx - sp.cov.c01 * vy) * idet;
        const float guy = -2.f * (sp.cov.c00 * vy - sp.cov.c01 * vx) * idet;
        const float e = sp.w.m[j] - sp.tx * sp.w.m[6 + j], f = sp.w.m[3 + j] - sp.ty * sp.w.m[6 + j];
        gaxis[j] = gux * sp.jx * e + guy * sp.jy * f;
        const float ke = gux * sp.jx * sp.axis[j], kf = guy * sp.jy * sp.axis[j];  // dL/de_j, dL/df_j
        gW[j] = ke;
        gW[3 + j] = kf;
        gW[6 + j] = -(sp.tx * ke + sp.ty * kf);
        gjx = gjx + gux * e * sp.axis[j];
        gjy = gjy + guy * f * sp.axis[j];
        gtx = gtx - ke * sp.w.m[6 + j];
        gty = gty - kf * sp.w.m[6 + j];
      }
      // Pinhole: px = fx x/z + cx, jx = fx/z, tx = x/z unless clamped (likewise y). Camera-frame centre:
      const float iz = 1.f / sp.c[2];
      const float ax = g[0] * cam.fx + (sp.clip_x ? 0.f : gtx);  // dL/d(x/z)
      const float ay = g[1] * cam.fy + (sp.clip_y ? 0.f : gty);
      const float gcx = ax * iz, gcy = ay * iz;
      const float gcz = -iz * (((gjx * sp.jx + gjy * sp.jy) + ax * sp.tx_raw) + ay * sp.ty_raw);
      // c = R_view (p - o): world gradient R_view^T gc, plus the view direction's share
      const float* Rv = cam.R;
      float gpx = ((Rv[0] * gcx + Rv[3] * gcy) + Rv[6] * gcz) + gsx;
      float gpy = ((Rv[1] * gcx + Rv[4] * gcy) + Rv[7] * gcz) + gsy;
      float gpz = ((Rv[2] * gcx + Rv[5] * gcy) + Rv[8] * gcz) + gsz;
      // W = R_view R(q): dL/dR = R_view^T gW
      float gR[9];
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int j = 0; j < 3; j++) gR[3 * r + j] = (Rv[r] * gW[j] + Rv[3 + r] * gW[3 + j]) + Rv[6 + r] * gW[6 + j];
      // Feature lanes (optim.cu:235-250): the pseudo-normal f = R_view (s u), u = c / |c| with c the column
      // of R(q) along the smallest log scale and s = +-1 its facing sign (locally constant), so
      // dL/dc = s (I - u u^T) R_view^T dL/df / |c|, which joins that column of dL/dR(q).
      if (g[10] != 0.f || g[11] != 0.f || g[12] != 0.f) {
        const AxisPick ax = smallest_axis(ls.x, ls.y, ls.z);
        const float* m = sp.rot.m;
        const float nx = ax.of(m[0], m[1], m[2]), ny = ax.of(m[3], m[4], m[5]), nz = ax.of(m[6], m[7], m[8]);
        const float il = 1.f / fmaxf(sqrtf((nx * nx + ny * ny) + nz * nz), 1e-12f);
        const float ux = nx * il, uy = ny * il, uz = nz * il;
        const float face = ((ux * -dvx + uy * -dvy) + uz * -dvz) >= 0.f ? 1.f : -1.f;
        const float bx = ((Rv[0] * g[10] + Rv[3] * g[11]) + Rv[6] * g[12]) * face;
        const float by = ((Rv[1] * g[10] + Rv[4] * g[11]) + Rv[7] * g[12]) * face;
        const float bz = ((Rv[2] * g[10] + Rv[5] * g[11]) + Rv[8] * g[12]) * face;
        const float along = (ux * bx + uy * by) + uz * bz;
        const float cx = (bx - ux * along) * il, cy = (by - uy * along) * il, cz = (bz - uz * along) * il;
#pragma unroll
        for (int j = 0; j < 3; j++) {
          const bool on = j == 0 ? ax.x : (j == 1 ? ax.y : ax.z);
          gR[j] = on ? gR[j] + cx : gR[j];
          gR[3 + j] = on ? gR[3 + j] + cy : gR[3 + j];
          gR[6 + j] = on ? gR[6 + j] + cz : gR[6 + j];
        }
      }
      // semi-axes a_j = sqrt(exp(2 l_j) + f^2), and the floor's opacity factor prod_j sqrt(var_j / (var_j + f^2))
      const float v_op = g[8];
      const float f2 = ls.w * ls.w;
      float gl[3];
#pragma unroll
      for (int j = 0; j < 3; j++)
        gl[j] = gaxis[j] * sp.var[j] / sp.axis[j] + v_op * sp.opacity * f2 / (sp.var[j] + f2);
      float g_logit = v_op * sp.floor_comp * sp.sig * (1.f - sp.sig);
      const float qn2 = ((q.x * q.x + q.y * q.y) + q.z * q.z) + q.w * q.w;
      const float iq = 1.f / sqrtf(qn2);
      const float4 qn = make_float4(q.x * iq, q.y * iq, q.z * iq, q.w * iq);
      float4 gq = unit_quat_vjp(qn, iq, rotation_vjp(qn.x, qn.y, qn.z, qn.w, gR));
      const bool ok = finite3(gpx, gpy, gpz) && __builtin_isfinite(g_logit) && finite3(gl[0], gl[1], gl[2]) &&
                      __builtin_isfinite(gq.x + gq.y + gq.z + gq.w);
      if (!ok) {
        gpx = gpy = gpz = g_logit = gl[0] = gl[1] = gl[2] = 0.f;
        gq = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      out[0] = gpx; out[1] = gpy; out[2] = gpz; out[3] = g_logit;
      out[4] = gq.x; out[5] = gq.y; out[6] = gq.z; out[7] = gq.w;
      out[8] = gl[0]; out[9] = gl[1]; out[10] = gl[2];
      done = true;
      if constexpr (ADAM) bsq_done = bsq;
    }
  }
  if (!done) {
#pragma unroll
    for (int k = 0; k < PER; k++) out[k] = 0.f;
  }
  if constexpr (ADAM) {
    // the fused update of optim.cu:298-377 on this splat's gradient row; no barrier follows, so
    // threads without work leave here (sparse mode: splats without gradient keep all their state)
    if (!in_range || (a.step.sparse && !any)) return;
    adam_update<DEG, HALF>(a, i, out, visible, bsq_done, done ? g[5] : 0.f, done ? g[6] : 0.f, done ? g[7] : 0.f, pre);
    return;
  }
  s_any[threadIdx.x] = any ? 1u : 0u;
  __syncthreads();
  // the block's grad_out rows: one contiguous stretch, 16-byte aligned (VJP_BLOCK * PER floats per block)
  float* o = a.grad_out + (size_t)i0 * PER;
  const int nout = rows * PER;
  if (a.accumulate) {
    for (int j = threadIdx.x; j < nout; j += VJP_BLOCK)
      if (s_any[j / PER]) o[j] += s_buf[j];
  } else if (a.sparse) {  // the reference returns before the grad_out write for these splats
    for (int j = threadIdx.x; j < nout; j += VJP_BLOCK)
      if (s_any[j / PER]) o[j] = s_buf[j];
  } else {
    for (int j = threadIdx.x; j < nout / 4; j += VJP_BLOCK)
      reinterpret_cast<float4*>(o)[j] = reinterpret_cast<const float4*>(s_buf)[j];
    for (int j = (nout & ~3) + threadIdx.x; j < nout; j += VJP_BLOCK) o[j] = s_buf[j];
  }
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

namespace {
template <bool ADAM>
hipError_t launch_vjp(const b2c_vjp_args& a, hipStream_t stream) {
  const dim3 grid((unsigned)((a.n + VJP_BLOCK - 1) / VJP_BLOCK)), block(VJP_BLOCK);
  const bool half = a.degree > 0 && !a.sh.hi32;  // fp16 bands
  switch (a.degree * 2 + (half ? 1 : 0)) {
    case 0: vjp_kernel<0, false, ADAM><<<grid, block, 0, stream>>>(a); break;
    case 2: vjp_kernel<1, false, ADAM><<<grid, block, 0, stream>>>(a); break;
    case 3: vjp_kernel<1, true, ADAM><<<grid, block, 0, stream>>>(a); break;
    case 4: vjp_kernel<2, false, ADAM><<<grid, block, 0, stream>>>(a); break;
    case 5: vjp_kernel<2, true, ADAM><<<grid, block, 0, stream>>>(a); break;
    case 6: vjp_kernel<3, false, ADAM><<<grid, block, 0, stream>>>(a); break;
    case 7: vjp_kernel<3, true, ADAM><<<grid, block, 0, stream>>>(a); break;
    case 8: vjp_kernel<4, false, ADAM><<<grid, block, 0, stream>>>(a); break;
    case 9: vjp_kernel<4, true, ADAM><<<grid, block, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

extern "C" int b2c_hip_vjp(const b2c_vjp_args* a, hipStream_t stream) {
  static_assert(VJP_BLOCK == 64, "the deferred loss sum runs on the first workgroup's one wave");
  if (a->loss_partials && (!a->loss_accum || a->n <= 0)) return (int)hipErrorInvalidValue;
  if (a->n <= 0) return 0;
  if (a->grad_out) return (int)launch_vjp<false>(*a, stream);
  // the update writes the parameters, their moments and (sparse) last_step; the SH it writes are the ones it reads
  const b2c_adam_state& st = a->adam;
  if (!a->pos_op || !a->quat || !a->lscale || !st.m_pos_op || !st.v_pos_op || !st.m_quat || !st.v_quat ||
      !st.m_lscale || !st.v_lscale || !st.v_sh || !st.m_sh.dc || (a->step.sparse && !st.last_step) ||
      a->sh_out.dc != a->sh.dc || a->sh_out.stride != a->sh.stride || st.m_sh.stride != a->sh.stride)
    return (int)hipErrorInvalidValue;
  if (a->degree > 0) {
    const bool half = !a->sh.hi32;
    if (half ? (!a->sh_out.hi16 || a->sh_out.hi16 != a->sh.hi16 || !st.m_sh.hi16)
             : (a->sh_out.hi32 != a->sh.hi32 || !st.m_sh.hi32))
      return (int)hipErrorInvalidValue;
  }
  if (a->step.t < 1) return (int)hipErrorInvalidValue;
  return (int)launch_vjp<true>(*a, stream);
}

extern "C" void b2c_adam_step_constants(b2c_adam_step* s) {
  const double b1 = s->beta1, b2 = s->beta2, t = s->t;
  s->bc1 = (float)(1.0 / (1.0 - std::pow(b1, t)));
  s->bc2 = (float)(1.0 / (1.0 - std::pow(b2, t)));
  s->ln_beta1 = (float)std::log(b1);
  s->ln_beta2 = (float)std::log(b2);
  const double r = b1 / std::sqrt(b2);
  s->ratio = (float)r;
  s->ln_ratio = (float)std::log(r);
}
