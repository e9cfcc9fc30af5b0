// Screen-space footprint of one splat. The semantics are the reference's projection
// (src/gpu/splat_math.cuh:224-293): the same culls, the 0.3 px dilation, the tangent clamp of the EWA
// Jacobian, the opacity-adaptive extent and the Mip-Splatting floor. The formulation is this file's own:
//
//   A splat's covariance is Sigma = A A^T with A = R(q) diag(a), whose columns are its semi-axes in world
//   space, a_j = sqrt(exp(2 l_j) + f^2) (f the frozen floor). The camera sees the centre at
//   c = R_view (p - o) (o the camera centre) and the axes' directions as W = R_view R(q). Near c the pinhole
//   map is affine with Jacobian J = [[fx/z, 0, -fx tx / z], [0, fy/z, -fy ty / z]], where (tx, ty) is the
//   ray's tangent (x/z, y/z) clamped to 15% beyond the frame. Each semi-axis lands on the image as
//   u_j = a_j J W_j, i.e. u_j = (fx/z (W_0j - tx W_2j) a_j, fy/z (W_1j - ty W_2j) a_j), and the screen
//   covariance is Sigma' = U U^T + 0.3 I with U = [u_0 u_1 u_2].
//
//   Its determinant comes from the Cauchy-Binet formula, det(U U^T) = sum_{j<k} (u_j x u_k)^2 (2D cross
//   products), plus 0.3 tr(U U^T) + 0.09, instead of c00 c11 - c01^2: for an elongated footprint (axes
//   hundreds of pixels against one) that difference cancels to a few digits and the conic's narrow
//   direction loses its accuracy, while every term here is a sum of non-negative numbers.
//
// Everything that decides a tile (centre, conic, opacity, power, extent) is evaluated without FMA
// contraction, with IEEE division and square root and with the exp/log of device_math.h, so the CPU
// restatement in oracle/b2c_oracle.c reproduces it bit for bit. The projection VJP (vjp.hip) differentiates
// this same formulation, reusing the intermediates kept here. Mip filtering is not part of this build (the
// reference's trainer rejects --render-mode mip, src/main.cpp:26).
#pragma once
#include "b2c_kernels.h"
#include "device_math.h"

namespace b2c {
namespace dev {

struct ScreenSplat {
  float d[3];          // p - o: the camera-to-splat vector in world space (also the SH view direction)
  float c[3];          // centre in camera coordinates, R_view d
  float var[3];        // exp(2 l_j): squared semi-axes without the floor
  float axis[3];       // semi-axis lengths a_j = sqrt(var_j + f^2)
  float floor_comp;    // opacity factor of the floor, sqrt(prod_j var_j / (var_j + f^2)); 1 without one
  Mat3 rot;            // R(q) of the normalised quaternion
  Mat3 w;              // R_view R(q)
  float jx, jy;        // fx / z, fy / z
  float tx_raw, ty_raw;  // x / z, y / z
  float tx, ty;        // the tangents clamped to the Jacobian limits
  bool clip_x, clip_y;   // the clamp is active (the Jacobian then stops following the centre)
  float ux[3], uy[3];  // image-plane semi-axes u_j
  float cross[3];      // u_0 x u_1, u_0 x u_2, u_1 x u_2
  Sym2 cov;            // Sigma', dilated
  float idet;          // 1 / det(Sigma')
  Sym2 conic;
  float sig, opacity;  // sigmoid of the logit; opacity = sig * floor_comp
  float px, py;        // image-plane centre
  float ex, ey;        // half extents of the cutoff ellipse {sigma <= power}
  bool ok;             // false: culled
};

__device__ __forceinline__ ScreenSplat screen_splat(float4 po, float4 q, float4 ls, const b2c_camera_gpu& cam) {
#pragma clang fp contract(off)
  ScreenSplat s;
  s.ok = false;
  s.d[0] = po.x - cam.pos[0];
  s.d[1] = po.y - cam.pos[1];
  s.d[2] = po.z - cam.pos[2];
#pragma unroll
  for (int r = 0; r < 3; r++) s.c[r] = (cam.R[3 * r] * s.d[0] + cam.R[3 * r + 1] * s.d[1]) + cam.R[3 * r + 2] * s.d[2];
  const float z = s.c[2];
  if (!(finite3(s.c[0], s.c[1], z) && z <= 1e10f)) return s;
  if (!(z >= 0.01f)) return s;
  const float f2 = ls.w * ls.w;
  const float lj[3] = {ls.x, ls.y, ls.z};
  float keep = 1.f;  // prod_j var_j / (var_j + f^2), as a product of ratios (no underflow for tiny axes)
#pragma unroll
  for (int j = 0; j < 3; j++) {
    s.var[j] = det_expf(2.f * lj[j]);
    const float vf = s.var[j] + f2;
    s.axis[j] = sqrtf(vf);
    keep = keep * (s.var[j] / vf);
  }
  s.floor_comp = ls.w > 0.f ? sqrtf(keep) : 1.f;
  if (!finite3(s.axis[0], s.axis[1], s.axis[2])) return s;
  const float qn2 = ((q.x * q.x + q.y * q.y) + q.z * q.z) + q.w * q.w;
  if (!(qn2 >= 1e-6f && __builtin_isfinite(qn2))) return s;
  if (!__builtin_isfinite(po.w)) return s;
  const float iq = 1.f / sqrtf(qn2);
  s.rot = quat_to_mat(q.x * iq, q.y * iq, q.z * iq, q.w * iq);
  // tangents, clamp and Jacobian scale
  s.tx_raw = s.c[0] / z;
  s.ty_raw = s.c[1] / z;
  s.clip_x = !(s.tx_raw <= cam.lim_pos_x && s.tx_raw >= cam.lim_neg_x);
  s.clip_y = !(s.ty_raw <= cam.lim_pos_y && s.ty_raw >= cam.lim_neg_y);
  s.tx = fminf(fmaxf(s.tx_raw, cam.lim_neg_x), cam.lim_pos_x);
  s.ty = fminf(fmaxf(s.ty_raw, cam.lim_neg_y), cam.lim_pos_y);
  s.jx = cam.fx / z;
  s.jy = cam.fy / z;
  // image-plane semi-axes and the screen covariance
  float q00 = 0.f, q01 = 0.f, q11 = 0.f;
#pragma unroll
  for (int j = 0; j < 3; j++) {
#pragma unroll
    for (int r = 0; r < 3; r++)
      s.w.m[3 * r + j] = (cam.R[3 * r] * s.rot.m[j] + cam.R[3 * r + 1] * s.rot.m[3 + j]) + cam.R[3 * r + 2] * s.rot.m[6 + j];
    s.ux[j] = s.jx * ((s.w.m[j] - s.tx * s.w.m[6 + j]) * s.axis[j]);
    s.uy[j] = s.jy * ((s.w.m[3 + j] - s.ty * s.w.m[6 + j]) * s.axis[j]);
    q00 = q00 + s.ux[j] * s.ux[j];
    q01 = q01 + s.ux[j] * s.uy[j];
    q11 = q11 + s.uy[j] * s.uy[j];
  }
  const float big = fmaxf(fabsf(q00), fmaxf(fabsf(q01), fabsf(q11)));
  if (big > 1e18f) {  // keep the determinant finite (the reference rescales the covariance the same way)
    const float k = sqrtf(1e18f / big);
    q00 = q01 = q11 = 0.f;
#pragma unroll
    for (int j = 0; j < 3; j++) {
      s.ux[j] = s.ux[j] * k;
      s.uy[j] = s.uy[j] * k;
      q00 = q00 + s.ux[j] * s.ux[j];
      q01 = q01 + s.ux[j] * s.uy[j];
      q11 = q11 + s.uy[j] * s.uy[j];
    }
  }
  s.cross[0] = s.ux[0] * s.uy[1] - s.uy[0] * s.ux[1];
  s.cross[1] = s.ux[0] * s.uy[2] - s.uy[0] * s.ux[2];
  s.cross[2] = s.ux[1] * s.uy[2] - s.uy[1] * s.ux[2];
  const float dil = 0.3f;  // 0.3 px dilation
  const float det = ((s.cross[0] * s.cross[0] + s.cross[1] * s.cross[1]) + s.cross[2] * s.cross[2]) + dil * (q00 + q11) +
                    dil * dil;
  s.cov = Sym2{q00 + dil, q01, q11 + dil};
  s.sig = 1.f / (1.f + det_expf(-po.w));
  s.opacity = s.sig * s.floor_comp;
  if (!(finite3(s.cov.c00, s.cov.c01, s.cov.c11) && __builtin_isfinite(det))) return s;
  if (!(det > 0.f)) return s;
  s.idet = 1.f / det;
  s.conic.c00 = s.cov.c11 * s.idet;
  s.conic.c01 = -s.cov.c01 * s.idet;
  s.conic.c11 = s.cov.c00 * s.idet;
  s.px = cam.fx * s.tx_raw + cam.cx;
  s.py = cam.fy * s.ty_raw + cam.cy;
  if (!(s.opacity >= ALPHA_CUTOFF)) return s;
  const float power = det_logf(s.opacity * 255.f);
  const float detc = s.conic.c00 * s.conic.c11 - s.conic.c01 * s.conic.c01;
  if (!(detc > 0.f)) return s;
  extent_from_conic(s.conic, power, s.ex, s.ey);
  if (!(s.ex >= 0.f && s.ey >= 0.f)) return s;
  const bool on_screen = s.px + s.ex > 0.f && s.px - s.ex < (float)cam.W && s.py + s.ey > 0.f && s.py - s.ey < (float)cam.H;
  s.ok = on_screen;
  return s;
}

}  // namespace dev
}  // namespace b2c
