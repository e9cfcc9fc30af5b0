// EWA projection of one splat (src/gpu/splat_math.cuh:199-293), evaluated without FMA contraction so
// that mean2d / conic / opacity / power / extent, and hence every tile decision, are reproducible bit for
// bit. Differences from the reference's arithmetic, all toward exactness: rsqrtf -> 1/sqrtf, __expf /
// __logf -> Cephes exp/log (det_expf / det_logf). Mip filtering is not part of this build (the reference's
// trainer rejects --render-mode mip, src/main.cpp:26).
#pragma once
#include "device_math.h"
#include "b2c_kernels.h"

namespace b2c {
namespace dev {

struct Proj {
  float mc[3];        // view-space mean
  float s[3];         // effective scales (with floor)
  float s2_raw[3];    // exp(2 log s)
  float comp_floor;   // floor opacity compensation
  Mat3 Rq;            // rotation of the normalised quaternion
  float J[6];         // 2x3 projection Jacobian, row major
  bool clamp_x, clamp_y;
  Sym2 conic;
  float opac, sig;
  float mean2d[2];
  float ex, ey;
  bool ok;
};

__device__ __forceinline__ Proj project_one(float4 po, float4 q, float4 ls, const b2c_camera_gpu& cam) {
#pragma clang fp contract(off)
  Proj r;
  r.ok = false;
  const float* Rv = cam.R;
  float mcx = Rv[0] * po.x + Rv[1] * po.y + Rv[2] * po.z;
  float mcy = Rv[3] * po.x + Rv[4] * po.y + Rv[5] * po.z;
  float mcz = Rv[6] * po.x + Rv[7] * po.y + Rv[8] * po.z;
  mcx = mcx + cam.t[0]; mcy = mcy + cam.t[1]; mcz = mcz + cam.t[2];
  r.mc[0] = mcx; r.mc[1] = mcy; r.mc[2] = mcz;
  if (!(finite3(mcx, mcy, mcz) && mcz <= 1e10f)) return r;
  if (!(mcz >= 0.01f)) return r;
  float s2x = det_expf(2.f * ls.x), s2y = det_expf(2.f * ls.y), s2z = det_expf(2.f * ls.z);
  r.s2_raw[0] = s2x; r.s2_raw[1] = s2y; r.s2_raw[2] = s2z;
  float f2 = ls.w * ls.w;
  float s2fx = s2x + f2, s2fy = s2y + f2, s2fz = s2z + f2;
  r.s[0] = sqrtf(s2fx); r.s[1] = sqrtf(s2fy); r.s[2] = sqrtf(s2fz);
  r.comp_floor = ls.w > 0.f ? sqrtf((s2x * s2y * s2z) / (s2fx * s2fy * s2fz)) : 1.f;
  if (!finite3(r.s[0], r.s[1], r.s[2])) return r;
  float qn2 = q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w;
  if (!(qn2 >= 1e-6f && __builtin_isfinite(qn2))) return r;
  if (!__builtin_isfinite(po.w)) return r;
  float inv_qn = 1.f / sqrtf(qn2);
  r.Rq = quat_to_mat(q.x * inv_qn, q.y * inv_qn, q.z * inv_qn, q.w * inv_qn);
  Mat3 Rm;
#pragma unroll
  for (int k = 0; k < 9; k++) Rm.m[k] = Rv[k];
  Mat3 M = mat3_mul(Rm, r.Rq);
#pragma unroll
  for (int i = 0; i < 3; i++) { M.m[i * 3] *= r.s[0]; M.m[i * 3 + 1] *= r.s[1]; M.m[i * 3 + 2] *= r.s[2]; }
  float inv_z = 1.f / mcz;
  float rx = mcx * inv_z, ry = mcy * inv_z;
  float cxr = fminf(fmaxf(rx, cam.lim_neg_x), cam.lim_pos_x), cyr = fminf(fmaxf(ry, cam.lim_neg_y), cam.lim_pos_y);
  r.clamp_x = !(rx <= cam.lim_pos_x && rx >= cam.lim_neg_x);
  r.clamp_y = !(ry <= cam.lim_pos_y && ry >= cam.lim_neg_y);
  float dx = cam.fx * inv_z, dy = cam.fy * inv_z;
  r.J[0] = dx; r.J[1] = 0.f; r.J[2] = -dx * cxr;
  r.J[3] = 0.f; r.J[4] = dy; r.J[5] = -dy * cyr;
  float V[6];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 3; j++) V[i * 3 + j] = r.J[i * 3] * M.m[j] + r.J[i * 3 + 1] * M.m[3 + j] + r.J[i * 3 + 2] * M.m[6 + j];
  float c00 = V[0] * V[0] + V[1] * V[1] + V[2] * V[2];
  float c01 = V[0] * V[3] + V[1] * V[4] + V[2] * V[5];
  float c11 = V[3] * V[3] + V[4] * V[4] + V[5] * V[5];
  float max_abs = fmaxf(fabsf(c00), fmaxf(fabsf(c01), fabsf(c11)));
  if (max_abs > 1e18f) { float k = 1e18f / max_abs; c00 *= k; c01 *= k; c11 *= k; }
  c00 += 0.3f; c11 += 0.3f;  // 0.3 px dilation (splat_math.cuh:264-265)
  r.sig = 1.f / (1.f + det_expf(-po.w));
  r.opac = r.sig * 1.f * r.comp_floor;
  if (!finite3(c00, c01, c11)) return r;
  float det = c00 * c11 - c01 * c01;
  if (!(det > 0.f)) return r;
  float inv_det = 1.f / det;
  r.conic.c00 = c11 * inv_det; r.conic.c01 = -c01 * inv_det; r.conic.c11 = c00 * inv_det;
  r.mean2d[0] = cam.fx * rx + cam.cx; r.mean2d[1] = cam.fy * ry + cam.cy;
  if (!(r.opac >= ALPHA_CUTOFF)) return r;
  float power = det_logf(r.opac * 255.f);
  float detc = r.conic.c00 * r.conic.c11 - r.conic.c01 * r.conic.c01;
  if (!(detc > 0.f)) return r;
  extent_from_conic(r.conic, power, r.ex, r.ey);
  if (!(r.ex >= 0.f && r.ey >= 0.f)) return r;
  bool on_screen = r.mean2d[0] + r.ex > 0.f && r.mean2d[0] - r.ex < (float)cam.W && r.mean2d[1] + r.ey > 0.f &&
                   r.mean2d[1] - r.ey < (float)cam.H;
  if (!on_screen) return r;
  r.ok = true;
  return r;
}

}  // namespace dev
}  // namespace b2c
