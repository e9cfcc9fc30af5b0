// Projection VJP (replaces the gradient half of optim_kernel, src/gpu/optim.cu:99-253, with the grad_out
// write of 292-296): one thread per splat turns the 13 screen-space gradient lanes into parameter
// gradients [pos3, opacity, quat4, log-scale3, SH 3K]. Reads and clears v_splat and vis_flag (the
// consumed-and-zeroed contract of optim.cu:110-121). accumulate = 1 adds into grad_out so gradients of
// several views can be summed; 0 overwrites like the reference, and with sparse set leaves the rows of splats
// without gradient alone as the reference's early return does (optim.cu:148).
// Evaluated without FMA contraction, in the operation order of the reference's VJP: the chain through the
// 2x2 inverse and the 3x3 covariance amplifies rounding differences by the conic's condition number
// (large for the thin splats of the stress configuration), so the kernel keeps IEEE single-op rounding.
#pragma clang fp contract(off)
#include "b2c_kernels.h"
#include "device_math.h"
#include "project_one.h"

namespace b2c {
namespace dev {
namespace {

__device__ __forceinline__ float4 apply_normalize_vjp(float4 q, float4 g) {  // optim.cu:10-21
  const float lsq = q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w;
  const float l = sqrtf(lsq);
  const float inv = 1.f / (l * lsq);
  const float qw = q.x, qx = q.y, qy = q.z, qz = q.w;
  const float gw = g.x, gx = g.y, gy = g.z, gz = g.w;
  const float cc0 = -qw * qx, cc1 = -qx * qy, cc2 = -qy * qw, cs0 = -qw * qz, cs1 = -qx * qz, cs2 = -qy * qz;
  return make_float4(((lsq - qw * qw) * gw + cc0 * gx + cc2 * gy + cs0 * gz) * inv,
                     (cc0 * gw + (lsq - qx * qx) * gx + cc1 * gy + cs1 * gz) * inv,
                     (cc2 * gw + cc1 * gx + (lsq - qy * qy) * gy + cs2 * gz) * inv,
                     (cs0 * gw + cs1 * gx + cs2 * gy + (lsq - qz * qz) * gz) * inv);
}

__device__ __forceinline__ float4 quat_to_mat_vjp(float qw, float qx, float qy, float qz, const float* m) {  // optim.cu:24-33
  const float v00 = m[0], v01 = m[1], v02 = m[2], v10 = m[3], v11 = m[4], v12 = m[5], v20 = m[6], v21 = m[7], v22 = m[8];
  const float w_grad = qx * (v21 - v12) + qy * (v02 - v20) + qz * (v10 - v01);
  const float x_grad = -2.f * qx * (v11 + v22) + qy * (v10 + v01) + qz * (v20 + v02) + qw * (v21 - v12);
  const float y_grad = qx * (v10 + v01) - 2.f * qy * (v00 + v22) + qz * (v21 + v12) + qw * (v02 - v20);
  const float z_grad = qx * (v20 + v02) + qy * (v21 + v12) - 2.f * qz * (v00 + v11) + qw * (v10 - v01);
  return make_float4(2.f * w_grad, 2.f * x_grad, 2.f * y_grad, 2.f * z_grad);
}

__device__ __forceinline__ Sym2 inverse2x2_vjp(Sym2 minv, Sym2 v) {  // optim.cu:35-45
  const float tmp00 = -minv.c00 * v.c00 + -minv.c01 * v.c01;
  const float tmp01 = -minv.c01 * v.c00 + -minv.c11 * v.c01;
  const float tmp10 = -minv.c00 * v.c01 + -minv.c01 * v.c11;
  const float tmp11 = -minv.c01 * v.c01 + -minv.c11 * v.c11;
  Sym2 r;
  r.c00 = tmp00 * minv.c00 + tmp10 * minv.c01;
  r.c01 = tmp01 * minv.c00 + tmp11 * minv.c01;
  r.c11 = tmp01 * minv.c01 + tmp11 * minv.c11;
  return r;
}

// d colour / d view direction (optim.cu:48-88); dotc(k) = sum_ch c[k][ch] * vc[ch].
template <int DEG>
__device__ __forceinline__ void sh_viewdir_vjp(const float* coef, float x, float y, float z, float3 vc, int active,
                                               float& gx, float& gy, float& gz) {
  gx = gy = gz = 0.f;
  auto dotc = [&](int k) { return coef[k * 3] * vc.x + coef[k * 3 + 1] * vc.y + coef[k * 3 + 2] * vc.z; };
  if constexpr (DEG >= 1) if (active >= 1) {
    const float f0a = 0.4886025f;
    const float s_n1 = dotc(1), s_z0 = dotc(2), s_p1 = dotc(3);
    gx += -f0a * s_p1; gy += -f0a * s_n1; gz += f0a * s_z0;
    if constexpr (DEG >= 2) if (active >= 2) {
      const float c2 = -1.0925485f, f1a = 0.54627424f;
      const float s_n2 = dotc(4), s_n1b = dotc(5), s_z0b = dotc(6), s_p1b = dotc(7), s_p2 = dotc(8);
      gx += 2.f * f1a * y * s_n2 + c2 * z * s_p1b + 2.f * f1a * x * s_p2;
      gy += 2.f * f1a * x * s_n2 + c2 * z * s_n1b - 2.f * f1a * y * s_p2;
      gz += c2 * y * s_n1b + 2.f * 0.9461747f * z * s_z0b + c2 * x * s_p1b;
      if constexpr (DEG >= 3) if (active >= 3) {
        const float z2 = z * z, x2 = x * x, y2 = y * y;
        const float f2a = -0.5900436f, c1b = 1.4453057f, c0c = -2.285229f;
        const float f1b = c1b * z, f0c = c0c * z2 + 0.4570458f, f0c_dz = 2.f * c0c * z;
        const float s_n3 = dotc(9), s_n2c = dotc(10), s_n1c = dotc(11), s_z0c = dotc(12), s_p1c = dotc(13),
                    s_p2c = dotc(14), s_p3 = dotc(15);
        const float d12_z = 3.f * 1.8658817f * z2 - 1.119529f;
        gx += f2a * 6.f * x * y * s_n3 + 2.f * f1b * y * s_n2c + f0c * s_p1c + 2.f * f1b * x * s_p2c + f2a * 3.f * (x2 - y2) * s_p3;
        gy += f2a * 3.f * (x2 - y2) * s_n3 + 2.f * f1b * x * s_n2c + f0c * s_n1c + (-2.f) * f1b * y * s_p2c + f2a * (-6.f) * x * y * s_p3;
        gz += 2.f * c1b * x * y * s_n2c + f0c_dz * y * s_n1c + d12_z * s_z0c + f0c_dz * x * s_p1c + c1b * (x2 - y2) * s_p2c;
        if constexpr (DEG >= 4) if (active >= 4) {
          const float fc1 = x2 - y2, fs1 = 2.f * x * y, fc2 = x * fc1 - y * fs1, fs2 = x * fs1 + y * fc1;
          const float f0d = z * (-4.683326f * z2 + 2.0071396f), f0d_dz = -14.049978f * z2 + 2.0071396f;
          const float f1c = 3.3116114f * z2 - 0.47308735f, f1c_dz = 2.f * 3.3116114f * z;
          const float f2b_c = -1.7701308f, f2b = f2b_c * z, f3a = 0.62583575f;
          const float p12 = z * (1.8658817f * z2 - 1.119529f), dp12 = 3.f * 1.8658817f * z2 - 1.119529f;
          const float dp6 = 2.f * 0.9461747f * z;
          const float dp20 = 1.9843135f * (p12 + z * dp12) - 1.0062306f * dp6;
          const float s_n4 = dotc(16), s_n3d = dotc(17), s_n2d = dotc(18), s_n1d = dotc(19), s_z0d = dotc(20),
                      s_p1d = dotc(21), s_p2d = dotc(22), s_p3d = dotc(23), s_p4 = dotc(24);
          gx += f3a * 4.f * fs2 * s_n4 + f2b * 3.f * fs1 * s_n3d + f1c * 2.f * y * s_n2d + f0d * s_p1d + f1c * 2.f * x * s_p2d +
                f2b * 3.f * fc1 * s_p3d + f3a * 4.f * fc2 * s_p4;
          gy += f3a * 4.f * fc2 * s_n4 + f2b * 3.f * fc1 * s_n3d + f1c * 2.f * x * s_n2d + f0d * s_n1d + f1c * (-2.f) * y * s_p2d +
                f2b * (-3.f) * fs1 * s_p3d + f3a * (-4.f) * fs2 * s_p4;
          gz += f2b_c * fs2 * s_n3d + f1c_dz * fs1 * s_n2d + f0d_dz * y * s_n1d + dp20 * s_z0d + f0d_dz * x * s_p1d +
                f1c_dz * fc1 * s_p2d + f2b_c * fc2 * s_p3d;
        }
      }
    }
  }
}

// The per-splat rows of v_splat (13 floats) and grad_out (11 + 3K floats) are read and written through
// LDS by the whole workgroup, so consecutive lanes touch consecutive addresses (a lane-per-row access
// would touch one cache line per lane per instruction).
constexpr int VJP_BLOCK = 64;

template <int DEG, bool HALF>
__global__ void __launch_bounds__(VJP_BLOCK) vjp_kernel(b2c_vjp_args a) {
  constexpr int K = (DEG + 1) * (DEG + 1);
  constexpr int PER = 11 + 3 * K;
  __shared__ __attribute__((aligned(16))) float s_buf[VJP_BLOCK * PER];  // v_splat rows in, grad_out rows out
  __shared__ uint32_t s_vis[VJP_BLOCK], s_any[VJP_BLOCK];
  const int i0 = blockIdx.x * VJP_BLOCK;
  const int i = i0 + threadIdx.x;
  const int rows = min(VJP_BLOCK, a.n - i0);
  const bool in_range = i < a.n;
  // Memory round trip 1: this splat's flag, tile count and statistics, and the block's v_splat rows (one
  // contiguous, 16-byte aligned stretch of VJP_BLOCK * 13 floats), all issued before any is waited for.
  uint32_t vis = 0u, tc = 0u;
  float vcount = 0.f, rnorm = 0.f;
  if (in_range) {
    vis = a.vis_flag[i];
    tc = a.tile_count[i];
    if (a.vis_count) vcount = a.vis_count[i];
    if (a.refine_norm) rnorm = a.refine_norm[i];
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
  s_vis[threadIdx.x] = vis;
  __syncthreads();
  float g[GRAD_LANES];
#pragma unroll
  for (int k = 0; k < GRAD_LANES; k++) g[k] = vis ? s_buf[threadIdx.x * GRAD_LANES + k] : 0.f;
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
  if (vis) a.vis_flag[i] = 0u;
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
  if (any) {
    // Memory round trip 2: the splat's parameters and all its SH coefficients, issued together
    const float4 po = reinterpret_cast<const float4*>(a.pos_op)[i];
    const float4 q = reinterpret_cast<const float4*>(a.quat)[i];
    const float4 ls = reinterpret_cast<const float4*>(a.lscale)[i];
    const ShView sv{a.sh.dc, reinterpret_cast<const _Float16*>(a.sh.hi16), a.sh.hi32, a.sh.stride};
    float coef[3 * K];
    if constexpr (HALF)
      sv.load_all<DEG, true>(i, coef);
    else
      sv.load_all_either<DEG>(i, coef);
    const b2c_camera_gpu& cam = a.cam;
    // The SH half needs only the view direction: it runs first, so the coefficients are dead before the
    // projection's registers are live. Its row entries are zeroed below if the projection fails.
    const float ux = po.x - cam.pos[0], uy = po.y - cam.pos[1], uz = po.z - cam.pos[2];
    const float ul = sqrtf(ux * ux + uy * uy + uz * uz);
    const float iul = 1.f / ul;
    const float vx = ux * iul, vy = uy * iul, vz = uz * iul;
    const int kmax = a.active_deg >= DEG ? K : (a.active_deg + 1) * (a.active_deg + 1);
    const float3 vc = make_float3(g[5], g[6], g[7]);
    {
      float basis[K];
      sh_basis<DEG>(vx, vy, vz, basis);
#pragma unroll
      for (int k = 0; k < K; k++) {
        const float bk = k < kmax ? basis[k] : 0.f;
        out[11 + k * 3] = bk * vc.x; out[12 + k * 3] = bk * vc.y; out[13 + k * 3] = bk * vc.z;
      }
    }
    float vvx, vvy, vvz;
    sh_viewdir_vjp<DEG>(coef, vx, vy, vz, vc, a.active_deg, vvx, vvy, vvz);
    const float vdot = vx * vvx + vy * vvy + vz * vvz;
    const float msx = (vvx - vx * vdot) * (1.f / ul), msy = (vvy - vy * vdot) * (1.f / ul), msz = (vvz - vz * vdot) * (1.f / ul);
    const Proj pr = project_one(po, q, ls, a.cam);
    if (pr.ok) {
      const float v_alpha = g[8];
      float g_op = v_alpha * 1.f * pr.comp_floor * pr.sig * (1.f - pr.sig);
      const Sym2 v_cov = inverse2x2_vjp(pr.conic, Sym2{g[2], 0.5f * g[3], g[4]});
      const float* Rv = cam.R;
      float M[9];
#pragma unroll
      for (int r = 0; r < 3; r++) {
        M[r * 3] = pr.Rq.m[r * 3] * pr.s[0]; M[r * 3 + 1] = pr.Rq.m[r * 3 + 1] * pr.s[1]; M[r * 3 + 2] = pr.Rq.m[r * 3 + 2] * pr.s[2];
      }
      float covar[9];
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int cc = 0; cc < 3; cc++) covar[r * 3 + cc] = M[r * 3] * M[cc * 3] + M[r * 3 + 1] * M[cc * 3 + 1] + M[r * 3 + 2] * M[cc * 3 + 2];
      float RvC[9];
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int cc = 0; cc < 3; cc++) RvC[r * 3 + cc] = Rv[r * 3] * covar[cc] + Rv[r * 3 + 1] * covar[3 + cc] + Rv[r * 3 + 2] * covar[6 + cc];
      float cov_c[9];
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int cc = 0; cc < 3; cc++) cov_c[r * 3 + cc] = RvC[r * 3] * Rv[cc * 3] + RvC[r * 3 + 1] * Rv[cc * 3 + 1] + RvC[r * 3 + 2] * Rv[cc * 3 + 2];
      const float mcx = pr.mc[0], mcy = pr.mc[1], mcz = pr.mc[2];
      const float inv_z = 1.f / mcz, inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z;
      const float v2x = g[0], v2y = g[1];
      const float vcov[2][2] = {{v_cov.c00, v_cov.c01}, {v_cov.c01, v_cov.c11}};
      float tmp[2][3];
#pragma unroll
      for (int r = 0; r < 2; r++)
#pragma unroll
        for (int j = 0; j < 3; j++) tmp[r][j] = vcov[r][0] * pr.J[j] + vcov[r][1] * pr.J[3 + j];
      auto rowdot = [&](int r, int cr) { return tmp[r][0] * cov_c[cr * 3] + tmp[r][1] * cov_c[cr * 3 + 1] + tmp[r][2] * cov_c[cr * 3 + 2]; };
      const float vj00 = 2.f * rowdot(0, 0), vj11 = 2.f * rowdot(1, 1), vj20 = 2.f * rowdot(0, 2), vj21 = 2.f * rowdot(1, 2);
      const float rx = mcx * inv_z, ry = mcy * inv_z;
      const float txc = mcz * fminf(fmaxf(rx, cam.lim_neg_x), cam.lim_pos_x), tyc = mcz * fminf(fmaxf(ry, cam.lim_neg_y), cam.lim_pos_y);
      float v_mx = cam.fx * inv_z * v2x, v_my = cam.fy * inv_z * v2y;
      float v_mz = -(cam.fx * mcx * v2x + cam.fy * mcy * v2y) * inv_z2;
      if (!pr.clamp_x) v_mx += -cam.fx * inv_z2 * vj20; else v_mz += -cam.fx * inv_z3 * vj20 * txc;
      if (!pr.clamp_y) v_my += -cam.fy * inv_z2 * vj21; else v_mz += -cam.fy * inv_z3 * vj21 * tyc;
      v_mz += -cam.fx * inv_z2 * vj00 - cam.fy * inv_z2 * vj11 + 2.f * cam.fx * txc * inv_z3 * vj20 + 2.f * cam.fy * tyc * inv_z3 * vj21;
      float vcc[9];
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int cc = 0; cc < 3; cc++) {
          float s = 0.f;
#pragma unroll
          for (int p = 0; p < 2; p++)
#pragma unroll
            for (int q2 = 0; q2 < 2; q2++) s += pr.J[p * 3 + r] * vcov[p][q2] * pr.J[q2 * 3 + cc];
          vcc[r * 3 + cc] = s;
        }
      float t1[9];
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int cc = 0; cc < 3; cc++) t1[r * 3 + cc] = Rv[r] * vcc[cc] + Rv[3 + r] * vcc[3 + cc] + Rv[6 + r] * vcc[6 + cc];
      float v_covar[9];
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int cc = 0; cc < 3; cc++) v_covar[r * 3 + cc] = t1[r * 3] * Rv[cc] + t1[r * 3 + 1] * Rv[3 + cc] + t1[r * 3 + 2] * Rv[6 + cc];
      float v_M[9];
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int cc = 0; cc < 3; cc++)
          v_M[r * 3 + cc] = 2.f * (v_covar[r * 3] * M[cc] + v_covar[r * 3 + 1] * M[3 + cc] + v_covar[r * 3 + 2] * M[6 + cc]);
      float gpx = Rv[0] * v_mx + Rv[3] * v_my + Rv[6] * v_mz + msx;
      float gpy = Rv[1] * v_mx + Rv[4] * v_my + Rv[7] * v_mz + msy;
      float gpz = Rv[2] * v_mx + Rv[5] * v_my + Rv[8] * v_mz + msz;
      const float f2 = ls.w * ls.w;
      const float vs0 = pr.Rq.m[0] * v_M[0] + pr.Rq.m[3] * v_M[3] + pr.Rq.m[6] * v_M[6];
      const float vs1 = pr.Rq.m[1] * v_M[1] + pr.Rq.m[4] * v_M[4] + pr.Rq.m[7] * v_M[7];
      const float vs2 = pr.Rq.m[2] * v_M[2] + pr.Rq.m[5] * v_M[5] + pr.Rq.m[8] * v_M[8];
      float glx = vs0 * pr.s2_raw[0] / pr.s[0] + v_alpha * pr.opac * f2 / (pr.s2_raw[0] + f2);
      float gly = vs1 * pr.s2_raw[1] / pr.s[1] + v_alpha * pr.opac * f2 / (pr.s2_raw[1] + f2);
      float glz = vs2 * pr.s2_raw[2] / pr.s[2] + v_alpha * pr.opac * f2 / (pr.s2_raw[2] + f2);
      float vR[9];
#pragma unroll
      for (int r = 0; r < 3; r++) {
        vR[r * 3] = v_M[r * 3] * pr.s[0]; vR[r * 3 + 1] = v_M[r * 3 + 1] * pr.s[1]; vR[r * 3 + 2] = v_M[r * 3 + 2] * pr.s[2];
      }
      const float qn2 = q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w;
      const float inv_qn = 1.f / sqrtf(qn2);
      const float4 qg = quat_to_mat_vjp(q.x * inv_qn, q.y * inv_qn, q.z * inv_qn, q.w * inv_qn, vR);
      float4 gq = apply_normalize_vjp(q, qg);
      const bool ok = finite3(gpx, gpy, gpz) && __builtin_isfinite(g_op) && finite3(glx, gly, glz) &&
                      __builtin_isfinite(gq.x + gq.y + gq.z + gq.w);
      if (!ok) {
        gpx = gpy = gpz = g_op = glx = gly = glz = 0.f;
        gq = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      out[0] = gpx; out[1] = gpy; out[2] = gpz; out[3] = g_op;
      out[4] = gq.x; out[5] = gq.y; out[6] = gq.z; out[7] = gq.w;
      out[8] = glx; out[9] = gly; out[10] = glz;
      done = true;
    }
  }
  if (!done) {
#pragma unroll
    for (int k = 0; k < PER; k++) out[k] = 0.f;
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

extern "C" int b2c_hip_vjp(const b2c_vjp_args* a, hipStream_t stream) {
  if (a->n <= 0) return 0;
  const dim3 grid((unsigned)((a->n + VJP_BLOCK - 1) / VJP_BLOCK)), block(VJP_BLOCK);
  const bool half = a->degree > 0 && !a->sh.hi32;  // fp16 bands
  switch (a->degree * 2 + (half ? 1 : 0)) {
    case 0: vjp_kernel<0, false><<<grid, block, 0, stream>>>(*a); break;
    case 2: vjp_kernel<1, false><<<grid, block, 0, stream>>>(*a); break;
    case 3: vjp_kernel<1, true><<<grid, block, 0, stream>>>(*a); break;
    case 4: vjp_kernel<2, false><<<grid, block, 0, stream>>>(*a); break;
    case 5: vjp_kernel<2, true><<<grid, block, 0, stream>>>(*a); break;
    case 6: vjp_kernel<3, false><<<grid, block, 0, stream>>>(*a); break;
    case 7: vjp_kernel<3, true><<<grid, block, 0, stream>>>(*a); break;
    case 8: vjp_kernel<4, false><<<grid, block, 0, stream>>>(*a); break;
    case 9: vjp_kernel<4, true><<<grid, block, 0, stream>>>(*a); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}
