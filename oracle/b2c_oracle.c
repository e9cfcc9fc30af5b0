/*
 * TEST INFRASTRUCTURE ONLY — CPU restatement of Erant/b2ctrain's splat rasterizer (the checker).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
 * Build: gcc -O2 -std=c11 -ffp-contract=off (oracle/Makefile). Contraction must stay off: the
 * projection and binning below are bit-exact restatements that the HIP kernels must reproduce.
 */
#define _POSIX_C_SOURCE 199309L /* clock_gettime */
#include "b2c_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define RT_W 8
#define ALPHA_CUTOFF (1.0f / 255.0f) /* splat_math.cuh:7 */
#define T_CUTOFF 1e-4f              /* splat_math.cuh:8 */
#define ALPHA_MAX 0.999f            /* splat_math.cuh:9 */
#define GRAD_LANES 13               /* splat_math.cuh:10 */
#define SH_C0 0.28209479177387814f

/* ------------------------------------------------------------------------------------------------
 * Cephes single-precision exp and log (Stephen L. Moshier, Cephes Math Library, single/expf.c and
 * single/logf.c): Cody-Waite reduction by ln 2 split in two constants, then a degree-6 (exp) or
 * degree-9 (log) polynomial. Replaces the reference's __expf/__logf fast-math intrinsics
 * (splat_math.cuh:232,282; project.cu:31). Below -86 the result is returned as 0 so that no
 * subnormal is ever produced (the GPU version follows the same rule).
 * ---------------------------------------------------------------------------------------------- */
float orc_expf(float xx) {
  float x = xx;
  if (!(x <= 88.0f)) return x != x ? x : INFINITY;
  if (x < -86.0f) return 0.0f;
  float t = 1.44269504088896341f * x;
  t = t + 0.5f;
  float z = floorf(t);
  x = x - z * 0.693359375f;
  x = x - z * -2.12194440e-4f;
  int n = (int)z;
  z = x * x;
  float p = 1.9875691500e-4f;
  p = p * x + 1.3981999507e-3f;
  p = p * x + 8.3334519073e-3f;
  p = p * x + 4.1665795894e-2f;
  p = p * x + 1.6666665459e-1f;
  p = p * x + 5.0000001201e-1f;
  p = p * z;
  p = p + x;
  p = p + 1.0f;
  return ldexpf(p, n);
}

float orc_logf(float xx) {
  float x = xx;
  if (!(x > 0.0f)) return x == 0.0f ? -INFINITY : NAN;
  if (isinf(x)) return x;
  int e;
  x = frexpf(x, &e);
  if (x < 0.707106781186547524f) {
    e -= 1;
    x = x + x;
    x = x - 1.0f;
  } else {
    x = x - 1.0f;
  }
  float z = x * x;
  float y = 7.0376836292e-2f;
  y = y * x - 1.1514610310e-1f;
  y = y * x + 1.1676998740e-1f;
  y = y * x - 1.2420140846e-1f;
  y = y * x + 1.4249322787e-1f;
  y = y * x - 1.6668057665e-1f;
  y = y * x + 2.0000714765e-1f;
  y = y * x - 2.4999993993e-1f;
  y = y * x + 3.3333331174e-1f;
  y = y * x;
  y = y * z;
  float fe = (float)e;
  if (e) y = y + -2.12194440e-4f * fe;
  y = y + -0.5f * z;
  z = x + y;
  if (e) z = z + 0.693359375f * fe;
  return z;
}

/* ------------------------------------------------------------------------------------------------
 * Small fp32 helpers (util.cuh:210-243 semantics, left-to-right evaluation).
 * ---------------------------------------------------------------------------------------------- */
typedef struct { float c00, c01, c11; } sym2;

static int finitef(float a) { return isfinite(a) != 0; }

/* util.cuh:235-243: rotation matrix from a normalised (w, x, y, z) quaternion. */
static void quat_to_mat(const float q[4], float R[9]) {
  float w = q[0], x = q[1], y = q[2], z = q[3];
  float x2 = x * x, y2 = y * y, z2 = z * z, xy = x * y, xz = x * z, yz = y * z, wx = w * x, wy = w * y, wz = w * z;
  R[0] = 1.f - 2.f * (y2 + z2); R[1] = 2.f * (xy - wz);       R[2] = 2.f * (xz + wy);
  R[3] = 2.f * (xy + wz);       R[4] = 1.f - 2.f * (x2 + z2); R[5] = 2.f * (yz - wx);
  R[6] = 2.f * (xz - wy);       R[7] = 2.f * (yz + wx);       R[8] = 1.f - 2.f * (x2 + y2);
}

/* util.cuh:226-233 */
static void mat3_mul(const float A[9], const float B[9], float C[9]) {
  for (int i = 0; i < 3; i++)
    for (int j = 0; j < 3; j++) C[i * 3 + j] = A[i * 3] * B[j] + A[i * 3 + 1] * B[3 + j] + A[i * 3 + 2] * B[6 + j];
}

/* splat_math.cuh:21-24 */
static float calc_sigma(float px, float py, sym2 c, float mx, float my) {
  float dx = px - mx, dy = py - my;
  return 0.5f * (c.c00 * dx * dx + c.c11 * dy * dy) + c.c01 * dx * dy;
}

/* splat_math.cuh:27-41: conservative ellipse-vs-rectangle test (nearest edge point in the conic metric). */
static int tile_hit(float rmin_x, float rmin_y, float rmax_x, float rmax_y, float mx, float my, sym2 conic, float power) {
  int x_left = mx < rmin_x, x_right = mx > rmax_x, in_x = !(x_left || x_right);
  int y_above = my < rmin_y, y_below = my > rmax_y, in_y = !(y_above || y_below);
  if (in_x && in_y) return 1;
  float corner_x = x_left ? rmin_x : rmax_x, corner_y = y_above ? rmin_y : rmax_y;
  float width = rmax_x - rmin_x, height = rmax_y - rmin_y;
  float dxf = x_left ? width : -width, dyf = y_above ? height : -height;
  float diff_x = mx - corner_x, diff_y = my - corner_y;
  float tx_raw = (dxf * conic.c00 * diff_x + dxf * conic.c01 * diff_y) / (dxf * conic.c00 * dxf);
  float ty_raw = (dyf * conic.c01 * diff_x + dyf * conic.c11 * diff_y) / (dyf * conic.c11 * dyf);
  float tx = in_y ? 0.f : fminf(fmaxf(tx_raw, 0.f), 1.f);
  float ty = in_x ? 0.f : fminf(fmaxf(ty_raw, 0.f), 1.f);
  float px = corner_x + tx * dxf, py = corner_y + ty * dyf;
  return calc_sigma(px, py, conic, mx, my) <= power;
}

typedef struct { int min_x, min_y, max_x, max_y; } tilebox;

/* splat_math.cuh:43-53 */
static tilebox tile_bbox(float mx, float my, float ex, float ey, int tiles_x, int tiles_y) {
  float tw = (float)RT_W;
  float cx = mx / tw, cy = my / tw, dx = ex / tw, dy = ey / tw;
  tilebox b;
  b.min_x = (int)fminf(fmaxf(cx - dx, 0.f), (float)tiles_x);
  b.min_y = (int)fminf(fmaxf(cy - dy, 0.f), (float)tiles_y);
  b.max_x = (int)fminf(fmaxf(cx + dx + 1.f, 0.f), (float)tiles_x);
  b.max_y = (int)fminf(fmaxf(cy + dy + 1.f, 0.f), (float)tiles_y);
  return b;
}

/* splat_math.cuh:122-145: real SH basis (Sloan order) for degree <= 4 into b[0..(deg+1)^2). */
static void sh_basis_f(int deg, float vx, float vy, float vz, float* b) {
  b[0] = SH_C0;
  if (deg < 1) return;
  const float f0a = 0.4886025f;
  b[1] = -f0a * vy; b[2] = f0a * vz; b[3] = -f0a * vx;
  if (deg < 2) return;
  float z2 = vz * vz, f0b = -1.0925485f * vz, f1a = 0.54627424f;
  float fc1 = vx * vx - vy * vy, fs1 = 2.f * vx * vy;
  b[4] = f1a * fs1; b[5] = f0b * vy; b[6] = 0.9461747f * z2 - 0.31539157f; b[7] = f0b * vx; b[8] = f1a * fc1;
  if (deg < 3) return;
  float f0c = -2.285229f * z2 + 0.4570458f, f1b = 1.4453057f * vz, f2a = -0.5900436f;
  float fc2 = vx * fc1 - vy * fs1, fs2 = vx * fs1 + vy * fc1;
  b[9] = f2a * fs2; b[10] = f1b * fs1; b[11] = f0c * vy; b[12] = vz * (1.8658817f * z2 - 1.119529f);
  b[13] = f0c * vx; b[14] = f1b * fc1; b[15] = f2a * fc2;
  if (deg < 4) return;
  float f0d = vz * (-4.683326f * z2 + 2.0071396f), f1c = 3.3116114f * z2 - 0.47308735f, f2b = -1.7701308f * vz, f3a = 0.62583575f;
  float fc3 = vx * fc2 - vy * fs2, fs3 = vx * fs2 + vy * fc2;
  b[16] = f3a * fs3; b[17] = f2b * fs2; b[18] = f1c * fs1; b[19] = f0d * vy;
  b[20] = 1.9843135f * vz * b[12] - 1.0062306f * b[6];
  b[21] = f0d * vx; b[22] = f1c * fc1; b[23] = f2b * fc2; b[24] = f3a * fc3;
}

static int imin(int a, int b) { return a < b ? a : b; }

/* Everything the projection produces that the VJP needs (splat_math.cuh:199-217 lists the same
 * quantities). */
typedef struct {
  float mc[3], s[3], s2_raw[3], comp_floor;
  float Rq[9], J[6];
  int clamp_x, clamp_y;
  sym2 cov, conic;
  float opac, sig;
  float mean2d[2];
  float ex, ey;
  int ok;
} proj_t;

/* The projection of splat_math.cuh:224-293 (mip off), in the operation sequence of the HIP kernel's
 * screen_splat (b2ctrain_amd/csrc/kernels/screen_splat.h), so that, compiled without FMA contraction,
 * centre, conic, opacity, power and extent agree bit for bit: the camera-frame centre R (p - o) from the
 * camera centre o; per-axis variances exp(2 l) and semi-axes sqrt(var + f^2); the floor's opacity factor
 * as a product of per-axis ratios; the image-plane semi-axes u_j = (fx/z (W0j - tx W2j) a_j,
 * fy/z (W1j - ty W2j) a_j) with W = R_view R(q) and (tx, ty) the clamped tangents; the screen covariance
 * sum_j u_j u_j^T + 0.3 I with its determinant by Cauchy-Binet (no cancellation for elongated footprints,
 * where the reference's c00 c11 - c01^2 loses digits). The reference's rsqrtf is 1/sqrtf here and its __expf/__logf the Cephes
 * functions above; the reference's x * (1/z) tangents are true quotients. */
static void project_one(const float* po, const float* q, const float* ls, const orc_cam_t* cam, proj_t* r) {
  r->ok = 0;
  const float* Rv = cam->R;
  const float d[3] = {po[0] - cam->pos[0], po[1] - cam->pos[1], po[2] - cam->pos[2]};
  for (int k = 0; k < 3; k++) r->mc[k] = (Rv[3 * k] * d[0] + Rv[3 * k + 1] * d[1]) + Rv[3 * k + 2] * d[2];
  const float z = r->mc[2];
  if (!(finitef(r->mc[0]) && finitef(r->mc[1]) && finitef(z) && z <= 1e10f)) return;
  if (!(z >= 0.01f)) return;
  const float f2 = ls[3] * ls[3];
  float keep = 1.f;
  for (int j = 0; j < 3; j++) {
    r->s2_raw[j] = orc_expf(2.f * ls[j]);
    const float vf = r->s2_raw[j] + f2;
    r->s[j] = sqrtf(vf);
    keep = keep * (r->s2_raw[j] / vf);
  }
  r->comp_floor = ls[3] > 0.f ? sqrtf(keep) : 1.f;
  if (!(finitef(r->s[0]) && finitef(r->s[1]) && finitef(r->s[2]))) return;
  const float qn2 = ((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3];
  if (!(qn2 >= 1e-6f && finitef(qn2))) return;
  if (!finitef(po[3])) return;
  const float iq = 1.f / sqrtf(qn2);
  const float qn[4] = {q[0] * iq, q[1] * iq, q[2] * iq, q[3] * iq};
  quat_to_mat(qn, r->Rq);
  const float tx_raw = r->mc[0] / z, ty_raw = r->mc[1] / z;
  r->clamp_x = !(tx_raw <= cam->lim_pos_x && tx_raw >= cam->lim_neg_x);
  r->clamp_y = !(ty_raw <= cam->lim_pos_y && ty_raw >= cam->lim_neg_y);
  const float tx = fminf(fmaxf(tx_raw, cam->lim_neg_x), cam->lim_pos_x);
  const float ty = fminf(fmaxf(ty_raw, cam->lim_neg_y), cam->lim_pos_y);
  const float jx = cam->fx / z, jy = cam->fy / z;
  r->J[0] = jx; r->J[1] = 0.f; r->J[2] = -jx * tx;
  r->J[3] = 0.f; r->J[4] = jy; r->J[5] = -jy * ty;
  float ux[3], uy[3], q00 = 0.f, q01 = 0.f, q11 = 0.f;
  for (int j = 0; j < 3; j++) {
    float w[3];
    for (int k = 0; k < 3; k++) w[k] = (Rv[3 * k] * r->Rq[j] + Rv[3 * k + 1] * r->Rq[3 + j]) + Rv[3 * k + 2] * r->Rq[6 + j];
    ux[j] = jx * ((w[0] - tx * w[2]) * r->s[j]);
    uy[j] = jy * ((w[1] - ty * w[2]) * r->s[j]);
    q00 = q00 + ux[j] * ux[j];
    q01 = q01 + ux[j] * uy[j];
    q11 = q11 + uy[j] * uy[j];
  }
  const float big = fmaxf(fabsf(q00), fmaxf(fabsf(q01), fabsf(q11)));
  if (big > 1e18f) {
    const float k = sqrtf(1e18f / big);
    q00 = q01 = q11 = 0.f;
    for (int j = 0; j < 3; j++) {
      ux[j] = ux[j] * k;
      uy[j] = uy[j] * k;
      q00 = q00 + ux[j] * ux[j];
      q01 = q01 + ux[j] * uy[j];
      q11 = q11 + uy[j] * uy[j];
    }
  }
  /* det(U U^T + 0.3 I) by Cauchy-Binet: sum of squared 2D cross products + 0.3 tr + 0.09 */
  const float x01 = ux[0] * uy[1] - uy[0] * ux[1], x02 = ux[0] * uy[2] - uy[0] * ux[2], x12 = ux[1] * uy[2] - uy[1] * ux[2];
  const float dil = 0.3f;
  const float det = ((x01 * x01 + x02 * x02) + x12 * x12) + dil * (q00 + q11) + dil * dil;
  const float c00 = q00 + dil, c01 = q01, c11 = q11 + dil;
  r->cov.c00 = c00; r->cov.c01 = c01; r->cov.c11 = c11;
  r->sig = 1.f / (1.f + orc_expf(-po[3]));
  r->opac = r->sig * r->comp_floor;
  if (!(finitef(c00) && finitef(c01) && finitef(c11) && finitef(det))) return;
  if (!(det > 0.f)) return;
  const float idet = 1.f / det;
  r->conic.c00 = c11 * idet; r->conic.c01 = -c01 * idet; r->conic.c11 = c00 * idet;
  r->mean2d[0] = cam->fx * tx_raw + cam->cx; r->mean2d[1] = cam->fy * ty_raw + cam->cy;
  if (!(r->opac >= ALPHA_CUTOFF)) return;
  const float power = orc_logf(r->opac * 255.f);
  const float detc = r->conic.c00 * r->conic.c11 - r->conic.c01 * r->conic.c01;
  if (!(detc > 0.f)) return;
  const float idetc = 1.f / detc;
  r->ex = sqrtf(2.f * power * r->conic.c11 * idetc);
  r->ey = sqrtf(2.f * power * r->conic.c00 * idetc);
  if (!(r->ex >= 0.f && r->ey >= 0.f)) return;
  r->ok = r->mean2d[0] + r->ex > 0.f && r->mean2d[0] - r->ex < (float)cam->W && r->mean2d[1] + r->ey > 0.f &&
          r->mean2d[1] - r->ey < (float)cam->H;
}

int orc_tile_bits(int n_tiles) {
  int b = 1;
  while ((1 << b) < n_tiles + 1) b++;
  return b;
}

/* project.cu:8-84 (DEG from the model, FEAT none). */
void orc_project_feat(const orc_model_t* m, const orc_cam_t* cam, int active_deg, int tiles_x, int tiles_y, float* proj0,
                      float* proj1, float* proj2, float* proj3, uint32_t* tile_count, uint32_t* hit_info, int feat_mode,
                      const float* feat_buffer) {
  const int K = (m->degree + 1) * (m->degree + 1);
  int deg = active_deg < m->degree ? active_deg : m->degree;
  if (deg < 0) deg = 0;
  const int Ka = (deg + 1) * (deg + 1);
  for (int i = 0; i < m->n; i++) {
    const float* po = m->pos_op + (size_t)i * 4;
    proj_t pr;
    project_one(po, m->quat + (size_t)i * 4, m->lscale + (size_t)i * 4, cam, &pr);
    if (!pr.ok) { tile_count[i] = 0; continue; }
    float power = orc_logf(pr.opac * 255.f);
    tilebox bb = tile_bbox(pr.mean2d[0], pr.mean2d[1], pr.ex, pr.ey, tiles_x, tiles_y);
    uint32_t hits = 0, mask = 0;
    int bw = bb.max_x - bb.min_x, bh = bb.max_y - bb.min_y;
    int small = bw * bh <= 32;
    int bit = 0;
    for (int ty = bb.min_y; ty < bb.max_y; ty++)
      for (int tx = bb.min_x; tx < bb.max_x; tx++, bit++) {
        float rx = tx * (float)RT_W, ry = ty * (float)RT_W;
        if (tile_hit(rx, ry, rx + RT_W, ry + RT_W, pr.mean2d[0], pr.mean2d[1], pr.conic, power)) {
          hits++;
          if (small) mask |= 1u << bit;
        }
      }
    tile_count[i] = hits;
    hit_info[i * 2] = small ? mask : 0xFFFFFFFFu;
    hit_info[i * 2 + 1] = (uint32_t)bb.min_x | ((uint32_t)bb.min_y << 12) | ((uint32_t)bw << 24);
    /* colour: view direction camera -> splat (project.cu:44-55) */
    float vx = po[0] - cam->pos[0], vy = po[1] - cam->pos[1], vz = po[2] - cam->pos[2];
    float vl = sqrtf(vx * vx + vy * vy + vz * vz);
    float inv = 1.f / fmaxf(vl, 1e-12f);
    vx = vx * inv; vy = vy * inv; vz = vz * inv;
    float b[25];
    sh_basis_f(deg, vx, vy, vz, b);
    const float* c = m->sh + (size_t)i * K * 3;
    float cr = c[0] * b[0], cg = c[1] * b[0], cb = c[2] * b[0];
    for (int k = 1; k < Ka; k++) {
      cr = cr + c[k * 3] * b[k];
      cg = cg + c[k * 3 + 1] * b[k];
      cb = cb + c[k * 3 + 2] * b[k];
    }
    cr = cr + 0.5f; cg = cg + 0.5f; cb = cb + 0.5f;
    cr = finitef(cr) ? fminf(fmaxf(cr, -100.f), 100.f) : 0.f;
    cg = finitef(cg) ? fminf(fmaxf(cg, -100.f), 100.f) : 0.f;
    cb = finitef(cb) ? fminf(fmaxf(cb, -100.f), 100.f) : 0.f;
    float* p0 = proj0 + (size_t)i * 4; float* p1 = proj1 + (size_t)i * 4; float* p2 = proj2 + (size_t)i * 4;
    p0[0] = pr.mean2d[0]; p0[1] = pr.mean2d[1]; p0[2] = pr.conic.c00; p0[3] = pr.conic.c01;
    p1[0] = pr.conic.c11; p1[1] = pr.opac; p1[2] = pr.mc[2]; p1[3] = power;
    /* feature lanes (project.cu:63-77) */
    float f0 = 0.f, f1 = 0.f, f2 = 0.f;
    const float* ls = m->lscale + (size_t)i * 4;
    if (feat_mode == 1) {
      const int ax = (ls[0] <= ls[1] && ls[0] <= ls[2]) ? 0 : (ls[1] <= ls[2] ? 1 : 2);
      const float nx = pr.Rq[ax], ny = pr.Rq[3 + ax], nz = pr.Rq[6 + ax];
      const float il = 1.f / fmaxf(sqrtf((nx * nx + ny * ny) + nz * nz), 1e-12f);
      const float sx = nx * il, sy = ny * il, sz = nz * il;
      const float d0 = po[0] - cam->pos[0], d1 = po[1] - cam->pos[1], d2 = po[2] - cam->pos[2];
      const float face = ((sx * -d0 + sy * -d1) + sz * -d2) >= 0.f ? 1.f : -1.f;
      const float wx = sx * face, wy = sy * face, wz = sz * face;
      const float* Rv = cam->R;
      f0 = (Rv[0] * wx + Rv[1] * wy) + Rv[2] * wz;
      f1 = (Rv[3] * wx + Rv[4] * wy) + Rv[5] * wz;
      f2 = (Rv[6] * wx + Rv[7] * wy) + Rv[8] * wz;
    } else if (feat_mode == 2) {
      f0 = feat_buffer[(size_t)i * 3]; f1 = feat_buffer[(size_t)i * 3 + 1]; f2 = feat_buffer[(size_t)i * 3 + 2];
      f0 = finitef(f0) ? fminf(fmaxf(f0, -100.f), 100.f) : 0.f;
      f1 = finitef(f1) ? fminf(fmaxf(f1, -100.f), 100.f) : 0.f;
      f2 = finitef(f2) ? fminf(fmaxf(f2, -100.f), 100.f) : 0.f;
    }
    p2[0] = cr; p2[1] = cg; p2[2] = cb; p2[3] = f0;
    proj3[(size_t)i * 2] = f1; proj3[(size_t)i * 2 + 1] = f2;
  }
}

void orc_project(const orc_model_t* m, const orc_cam_t* cam, int active_deg, int tiles_x, int tiles_y, float* proj0,
                 float* proj1, float* proj2, float* proj3, uint32_t* tile_count, uint32_t* hit_info) {
  orc_project_feat(m, cam, active_deg, tiles_x, tiles_y, proj0, proj1, proj2, proj3, tile_count, hit_info, 0, NULL);
}

/* project.cu:82-83: every splat that survives project_one's culls (whatever its tile count) raises its
 * max_screen to its larger screen-space half-extent as a fraction of the frame, max(ex / W, ey / H). */
void orc_max_screen(const orc_model_t* m, const orc_cam_t* cam, float* max_screen) {
  for (int i = 0; i < m->n; i++) {
    proj_t pr;
    project_one(m->pos_op + (size_t)i * 4, m->quat + (size_t)i * 4, m->lscale + (size_t)i * 4, cam, &pr);
    if (!pr.ok) continue;
    const float ms = fmaxf(pr.ex / (float)cam->W, pr.ey / (float)cam->H);
    max_screen[i] = fmaxf(max_screen[i], ms);
  }
}

/* ------------------------------------------------------------------------------------------------
 * Binning (binning.cu:10-143).
 * ---------------------------------------------------------------------------------------------- */
typedef struct { uint32_t key, idx; } kv_t;
static int kv_cmp(const void* a, const void* b) {
  const kv_t* x = (const kv_t*)a; const kv_t* y = (const kv_t*)b;
  if (x->key != y->key) return x->key < y->key ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

static uint32_t float_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

uint32_t orc_bin(int n, const uint32_t* tile_count, const uint32_t* hit_info, const float* proj0, const float* proj1,
                 int tiles_x, int tiles_y, uint32_t cap, uint32_t* order, uint32_t* tile_off, uint32_t* keys_sorted,
                 uint32_t* vals_sorted, uint32_t* tile_ranges) {
  const uint32_t n_tiles = (uint32_t)(tiles_x * tiles_y);
  memset(tile_ranges, 0, sizeof(uint32_t) * 2 * n_tiles);
  if (n == 0) return 0;
  /* 1. depth sort: key = z bits for splats with hits, 0xFFFFFFFF otherwise; stable (binning.cu:10-15,116-118).
   * Sorting on (key, index) is the same total order as a stable sort on key. */
  kv_t* kv = (kv_t*)malloc(sizeof(kv_t) * (size_t)n);
  for (int i = 0; i < n; i++) {
    kv[i].key = tile_count[i] ? float_bits(proj1[(size_t)i * 4 + 2]) : 0xFFFFFFFFu;
    kv[i].idx = (uint32_t)i;
  }
  qsort(kv, (size_t)n, sizeof(kv_t), kv_cmp);
  for (int r = 0; r < n; r++) order[r] = kv[r].idx;
  free(kv);
  /* 2. inclusive scan of counts in depth order (binning.cu:16-19,120-124). */
  uint32_t run = 0;
  for (int r = 0; r < n; r++) { run += tile_count[order[r]]; tile_off[r] = run; }
  const uint32_t M = run;
  if (M > cap || M == 0) return M;
  /* 3. emit in depth order (binning.cu:25-93): hit-mask bits in increasing (row-major bbox) order;
   * big splats re-test the bbox with ex/ey recomputed from proj0/proj1; shortfall gets the sentinel. */
  uint32_t* keys = (uint32_t*)malloc(sizeof(uint32_t) * M);
  uint32_t* vals = (uint32_t*)malloc(sizeof(uint32_t) * M);
  const uint32_t sentinel = n_tiles;
  for (int r = 0; r < n; r++) {
    uint32_t i = order[r];
    uint32_t cnt = tile_count[i];
    if (!cnt) continue;
    uint32_t base = tile_off[r] - cnt;
    uint32_t mask = hit_info[i * 2], info = hit_info[i * 2 + 1];
    if (mask != 0xFFFFFFFFu) {
      int min_x = (int)(info & 0xFFFu), min_y = (int)((info >> 12) & 0xFFFu), bw = (int)(info >> 24);
      uint32_t k = 0;
      for (int bit = 0; bit < 32 && k < cnt; bit++) {
        if (!(mask >> bit & 1u)) continue;
        int tx = min_x + bit % bw, ty = min_y + bit / bw;
        keys[base + k] = (uint32_t)(ty * tiles_x + tx); vals[base + k] = i; k++;
      }
      for (; k < cnt; k++) { keys[base + k] = sentinel; vals[base + k] = i; }
    } else {
      const float* a = proj0 + (size_t)i * 4; const float* b = proj1 + (size_t)i * 4;
      sym2 conic = {a[2], a[3], b[0]};
      float power = b[3];
      float detc = conic.c00 * conic.c11 - conic.c01 * conic.c01;
      float inv_detc = 1.f / detc;
      float ex = sqrtf(2.f * power * conic.c11 * inv_detc), ey = sqrtf(2.f * power * conic.c00 * inv_detc);
      tilebox bb = tile_bbox(a[0], a[1], ex, ey, tiles_x, tiles_y);
      uint32_t written = 0;
      for (int ty = bb.min_y; ty < bb.max_y && written < cnt; ty++)
        for (int tx = bb.min_x; tx < bb.max_x && written < cnt; tx++) {
          float rx = tx * (float)RT_W, ry = ty * (float)RT_W;
          if (tile_hit(rx, ry, rx + RT_W, ry + RT_W, a[0], a[1], conic, power)) {
            keys[base + written] = (uint32_t)(ty * tiles_x + tx); vals[base + written] = i; written++;
          }
        }
      for (; written < cnt; written++) { keys[base + written] = sentinel; vals[base + written] = i; }
    }
  }
  /* 4. stable sort by tile id (binning.cu:140-142): counting sort over n_tiles + 1 buckets. */
  uint32_t* start = (uint32_t*)calloc((size_t)n_tiles + 2, sizeof(uint32_t));
  for (uint32_t s = 0; s < M; s++) start[keys[s] + 1]++;
  for (uint32_t t = 0; t <= n_tiles; t++) start[t + 1] += start[t];
  for (uint32_t s = 0; s < M; s++) {
    uint32_t p = start[keys[s]]++;
    keys_sorted[p] = keys[s]; vals_sorted[p] = vals[s];
  }
  free(start); free(keys); free(vals);
  /* 5. per-tile [first, last) (binning.cu:95-105); absent tiles stay (0, 0). */
  for (uint32_t s = 0; s < M; s++) {
    uint32_t t = keys_sorted[s];
    if (t >= n_tiles) continue;
    if (s == 0 || keys_sorted[s - 1] != t) tile_ranges[t * 2] = s;
    if (s == M - 1 || keys_sorted[s + 1] != t) tile_ranges[t * 2 + 1] = s + 1;
  }
  return M;
}

/* ------------------------------------------------------------------------------------------------
 * Forward raster (raster_fwd.cu:8-71). Each pixel walks its tile's list front to back; the whole
 * tile's early exit only skips pixels that are already done, so a per-pixel loop is equivalent.
 * ---------------------------------------------------------------------------------------------- */
/* A fragment's sigma as the raster kernels evaluate it (raster_common.h sigma_coefs / poly_sigma): a
 * quadratic in the pixel centre's offset (u, v) from its 8x8 tile's centre. With a = c00 / 2, b = c01,
 * c = c11 / 2 (halving is exact) and (mxr, myr) the splat centre relative to the tile centre,
 *   sigma = fma(a, uu, fma(b, uv, fma(c, vv, fma(D, u, fma(E, v, F))))),
 *   D = -fma(2a, mxr, b myr), E = -fma(b, mxr, (2c) myr), F = fma(mxr, fma(a, mxr, b myr), (c myr) myr).
 * The reference's 0.5 (c00 dx^2 + c11 dy^2) + c01 dx dy (raster_fwd.cu:44) is the same quantity rounded
 * differently. A fragment passes when sigma <= power: rounding can leave sigma slightly below 0 where the
 * exact value is 0, and such a fragment is kept, as the exact value would be. */
static float frag_sigma(float mx, float my, float c00, float c01, float c11, float pcx, float pcy) {
  const float a = 0.5f * c00, b = c01, c = 0.5f * c11;
  const float tcx = floorf(pcx * (1.f / RT_W)) * RT_W + RT_W * 0.5f;
  const float tcy = floorf(pcy * (1.f / RT_W)) * RT_W + RT_W * 0.5f;
  const float mxr = mx - tcx, myr = my - tcy;
  const float D = -fmaf(a + a, mxr, b * myr);
  const float E = -fmaf(b, mxr, (c + c) * myr);
  const float F = fmaf(mxr, fmaf(a, mxr, b * myr), (c * myr) * myr);
  const float u = pcx - tcx, v = pcy - tcy;
  return fmaf(a, u * u, fmaf(b, u * v, fmaf(c, v * v, fmaf(D, u, fmaf(E, v, F)))));
}

void orc_frag_sigma(int n, const float* mx, const float* my, const float* c00, const float* c01, const float* c11,
                    const float* pcx, const float* pcy, float* out) {
  for (int i = 0; i < n; i++) out[i] = frag_sigma(mx[i], my[i], c00[i], c01[i], c11[i], pcx[i], pcy[i]);
}

/* Fragments the last orc_raster_fwd call composited (F_contrib: alpha >= 1/255, before termination). */
static uint64_t g_fwd_contrib = 0;
uint64_t orc_last_fwd_contrib(void) { return g_fwd_contrib; }

/* Host threads of the tiled raster passes (OpenMP over tiles). 1 (the default) keeps the backward's
 * double-precision sums in a fixed order; more threads add them atomically in a varying order. */
static int g_threads = 1;
void orc_set_threads(int n) { g_threads = n > 0 ? n : 1; }

static inline void acc_add(double* p, double v) {
  if (g_threads > 1) {
#pragma omp atomic
    *p += v;
  } else {
    *p += v;
  }
}

/* The hollow penalty of a fragment at depth z over a pixel's reference depth z_ref (splat_math.cuh:14-17),
 * as the HIP kernels evaluate it: (z - (z_ref + margin)) times 1 / max(margin, 1e-4), clamped to [0, 1],
 * 0 when not finite. */
static float hollow_pen_of(float z, float z_ref, float margin) {
  const float zm = z_ref + margin, inv = 1.f / fmaxf(margin, 1e-4f);
  const float d = (z - zm) * inv;
  return finitef(d) ? fminf(fmaxf(d, 0.f), 1.f) : 0.f;
}

void orc_raster_fwd(int W, int H, int tiles_x, int tiles_y, const float bg[3], uint32_t* tile_ranges,
                    const uint32_t* vals_sorted, const float* proj0, const float* proj1, const float* proj2,
                    float* out_rgba, float* out_T, uint32_t* last_idx) {
  orc_raster_fwd_ext(W, H, tiles_x, tiles_y, bg, tile_ranges, vals_sorted, proj0, proj1, proj2, out_rgba, out_T, last_idx,
                     NULL);
}

void orc_raster_fwd_ext(int W, int H, int tiles_x, int tiles_y, const float bg[3], uint32_t* tile_ranges,
                        const uint32_t* vals_sorted, const float* proj0, const float* proj1, const float* proj2,
                        float* out_rgba, float* out_T, uint32_t* last_idx, const orc_ext_t* ext) {
  const int feat = ext && ext->feat;
  const float* hz = ext ? ext->hollow_z : NULL;
  uint64_t contrib = 0;
#pragma omp parallel for num_threads(g_threads) schedule(dynamic, 16) reduction(+ : contrib)
  for (int tile = 0; tile < tiles_x * tiles_y; tile++) {
    int tx = tile % tiles_x, ty = tile / tiles_x;
    uint32_t rx = tile_ranges[tile * 2], ry = tile_ranges[tile * 2 + 1];
    uint32_t max_last = rx;
    for (int l = 0; l < RT_W * RT_W; l++) {
      int px = tx * RT_W + l % RT_W, py = ty * RT_W + l / RT_W;
      if (!(px < W && py < H)) continue;
      float pcx = px + 0.5f, pcy = py + 0.5f;
      float T = 1.f, r = 0.f, g = 0.f, b = 0.f, f0 = 0.f, f1 = 0.f, f2 = 0.f, pen = 0.f;
      const float z_ref = hz ? hz[(size_t)py * W + px] : INFINITY;
      uint32_t last = rx;
      for (uint32_t idx = rx; idx < ry; idx++) {
        uint32_t gid = vals_sorted[idx];
        const float* a = proj0 + (size_t)gid * 4; const float* c = proj1 + (size_t)gid * 4;
        float sigma = frag_sigma(a[0], a[1], a[2], a[3], c[0], pcx, pcy);
        if (!(sigma <= c[3])) continue;
        float alpha = fminf(ALPHA_MAX, c[1] * expf(-sigma));
        float next_T = T * (1.f - alpha);
        if (next_T <= T_CUTOFF) break;
        float vis = alpha * T;
        const float* col = proj2 + (size_t)gid * 4;
        r += fmaxf(col[0], 0.f) * vis; g += fmaxf(col[1], 0.f) * vis; b += fmaxf(col[2], 0.f) * vis;
        if (feat) {
          const float* f12 = ext->proj3 + (size_t)gid * 2;
          f0 += col[3] * vis; f1 += f12[0] * vis; f2 += f12[1] * vis;
        }
        if (hz) pen += vis * hollow_pen_of(c[2], z_ref, ext->hollow_margin);
        T = next_T;
        last = idx + 1;
        contrib++;
      }
      size_t pix = (size_t)py * W + px;
      out_rgba[pix * 4] = r + T * bg[0]; out_rgba[pix * 4 + 1] = g + T * bg[1]; out_rgba[pix * 4 + 2] = b + T * bg[2];
      out_rgba[pix * 4 + 3] = 1.f - T;
      out_T[pix] = T;
      last_idx[pix] = last;
      if (feat && ext->out_feat) { ext->out_feat[pix * 3] = f0; ext->out_feat[pix * 3 + 1] = f1; ext->out_feat[pix * 3 + 2] = f2; }
      if (hz && ext->hollow_pen) ext->hollow_pen[pix] = pen;
      if (last > max_last) max_last = last;
    }
    tile_ranges[tile * 2 + 1] = max_last;
  }
  g_fwd_contrib = contrib;
}

/* ------------------------------------------------------------------------------------------------
 * Photometric loss (loss.cu:18-195, 296-303), whole image, double precision.
 * ---------------------------------------------------------------------------------------------- */
static void gauss11(double w[11]) {
  double sum = 0;
  for (int i = 0; i < 11; i++) { double x = i - 5.0; w[i] = exp(-x * x / (2 * 1.5 * 1.5)); sum += w[i]; }
  for (int i = 0; i < 11; i++) w[i] /= sum;
}

/* separable 11-tap blur with zero padding outside the image */
static void blur_d(int W, int H, const double* w, const double* in, double* tmp, double* out) {
  for (int y = 0; y < H; y++)
    for (int x = 0; x < W; x++) {
      double s = 0;
      for (int d = -5; d <= 5; d++) { int xx = x + d; if (xx >= 0 && xx < W) s += w[d + 5] * in[(size_t)y * W + xx]; }
      tmp[(size_t)y * W + x] = s;
    }
  for (int y = 0; y < H; y++)
    for (int x = 0; x < W; x++) {
      double s = 0;
      for (int d = -5; d <= 5; d++) { int yy = y + d; if (yy >= 0 && yy < H) s += w[d + 5] * tmp[(size_t)yy * W + x]; }
      out[(size_t)y * W + x] = s;
    }
}

/* loss.cu:58 decodes with a multiply by 1/255; tests/reference.cpp:107 divides by 255. */
static double gtc(uint32_t packed, int c) { return (double)((packed >> (8 * c)) & 0xffu) * (1.0 / 255.0); }
/* loss.cu:58,85-87 in fp32: the effective target the kernel compares the prediction with (the L1 sign and
 * the alpha-lane sign are decided on these fp32 values). */
static float gt_chan_f(uint32_t packed, int c) { return (float)((packed >> (8 * c)) & 0xffu) * (1.0f / 255.0f); }
static float gt_eff_f(uint32_t packed, int c, int composite, float bg) {
  float g = gt_chan_f(packed, c);
  if (composite) g = g + (1.f - gt_chan_f(packed, 3)) * bg;
  return g;
}
static double gtc_div(uint32_t packed, int c) { return (double)((packed >> (8 * c)) & 0xffu) / 255.0; }

double orc_photometric(int W, int H, const float* pred, const uint32_t* gt, const uint8_t* weights,
                       const orc_loss_params_t* lp, float* v_out) {
  const size_t P = (size_t)W * H;
  double w[11];
  gauss11(w);
  const double C1 = 0.01 * 0.01, C2 = 0.03 * 0.03;
  const double norm = (double)lp->scale / (3.0 * (double)W * (double)H);
  double* buf = (double*)malloc(sizeof(double) * P * 17);
  double *X = buf, *Y = buf + P, *tmp = buf + 2 * P, *mu1 = buf + 3 * P, *mu2 = buf + 4 * P, *ex2 = buf + 5 * P,
         *ey2 = buf + 6 * P, *exy = buf + 7 * P, *A = buf + 8 * P, *B = buf + 9 * P, *Bm = buf + 10 * P,
         *Cc = buf + 11 * P, *Cm = buf + 12 * P, *bA = buf + 13 * P, *bB = buf + 14 * P, *bBm = buf + 15 * P,
         *bC = buf + 16 * P;
  double* bCm = (double*)malloc(sizeof(double) * P);
  double* sq = (double*)malloc(sizeof(double) * P);
  double loss = 0;
  for (int ch = 0; ch < 3; ch++) {
    for (size_t i = 0; i < P; i++) {
      X[i] = pred[i * 4 + ch];
      Y[i] = (double)gt_eff_f(gt[i], ch, lp->composite, lp->bg[ch]);
    }
    blur_d(W, H, w, X, tmp, mu1);
    blur_d(W, H, w, Y, tmp, mu2);
    for (size_t i = 0; i < P; i++) sq[i] = X[i] * X[i];
    blur_d(W, H, w, sq, tmp, ex2);
    for (size_t i = 0; i < P; i++) sq[i] = Y[i] * Y[i];
    blur_d(W, H, w, sq, tmp, ey2);
    for (size_t i = 0; i < P; i++) sq[i] = X[i] * Y[i];
    blur_d(W, H, w, sq, tmp, exy);
    for (size_t i = 0; i < P; i++) {
      double wp = weights ? weights[i] / 255.0 : 1.0;
      double M = wp * (lp->mask ? gtc(gt[i], 3) : 1.0) * norm;
      double m1 = mu1[i], m2 = mu2[i];
      double s1_raw = ex2[i] - m1 * m1, s2_raw = ey2[i] - m2 * m2;
      double s1 = s1_raw > 0 ? s1_raw : 0, s2 = s2_raw > 0 ? s2_raw : 0, s12 = exy[i] - m1 * m2;
      double A1 = 2 * m1 * m2 + C1, A2 = 2 * s12 + C2, B1 = m1 * m1 + m2 * m2 + C1, B2 = s1 + s2 + C2;
      double raw = (A1 * A2) / (B1 * B2);
      double ssim = raw < -1 ? -1 : (raw > 1 ? 1 : raw);
      loss += M * (lp->l1_w * fabs(X[i] - Y[i]) + lp->ssim_w * ssim);
      A[i] = B[i] = Bm[i] = Cc[i] = Cm[i] = 0;
      if (raw > -1 && raw < 1) { /* loss.cu:165-172 */
        double k = M * lp->ssim_w;
        double inv_BB = 1.0 / (B1 * B2);
        double d_mu1 = 2 * m2 * A2 * inv_BB - 2 * m1 * ssim / B1;
        double d_s1 = s1_raw > 0 ? -ssim / B2 : 0.0;
        double d_s12 = 2 * A1 * inv_BB;
        A[i] = k * d_mu1; B[i] = k * d_s1; Bm[i] = B[i] * m1; Cc[i] = k * d_s12; Cm[i] = Cc[i] * m2;
      }
    }
    if (v_out) {
      blur_d(W, H, w, A, tmp, bA); blur_d(W, H, w, B, tmp, bB); blur_d(W, H, w, Bm, tmp, bBm);
      blur_d(W, H, w, Cc, tmp, bC); blur_d(W, H, w, Cm, tmp, bCm);
      for (size_t i = 0; i < P; i++) {
        double wp = weights ? weights[i] / 255.0 : 1.0;
        double M = wp * (lp->mask ? gtc(gt[i], 3) : 1.0) * norm;
        double p = X[i], g = Y[i];
        double sgn = p > g ? 1.0 : (p < g ? -1.0 : 0.0);
        double grad = M * lp->l1_w * sgn + bA[i] + 2 * p * bB[i] - 2 * bBm[i] + g * bC[i] - bCm[i];  /* loss.cu:213 */
        v_out[i * 4 + ch] = (float)(grad * lp->grad_scale);
      }
    }
  }
  for (size_t i = 0; i < P; i++) { /* alpha lane (loss.cu:215-225); not masked */
    double va = 0;
    if (lp->alpha_lane) {
      double wp = weights ? weights[i] / 255.0 : 1.0;
      double da = (double)(pred[i * 4 + 3] - gt_chan_f(gt[i], 3));
      double sa = da > 0 ? 1.0 : (da < 0 ? -1.0 : 0.0);
      double Ma = wp * lp->match_alpha_weight * lp->scale / ((double)W * (double)H);
      va = Ma * sa * lp->grad_scale;
      loss += Ma * fabs(da);
    }
    if (v_out) v_out[i * 4 + 3] = (float)va;
  }
  free(buf); free(bCm); free(sq);
  return loss;
}

/* ------------------------------------------------------------------------------------------------
 * Backward raster (raster_bwd.cu:37-139): reverse replay per pixel from the shrunk range end,
 * T_before = T / (1 - alpha), 13 gradient lanes per fragment.
 * ---------------------------------------------------------------------------------------------- */
void orc_raster_bwd(int W, int H, int tiles_x, int tiles_y, const float bg[3], const uint32_t* tile_ranges,
                    const uint32_t* vals_sorted, const float* proj0, const float* proj1, const float* proj2,
                    const float* out_rgba, const float* out_T, const uint32_t* last_idx, const float* v_out,
                    float inv_gscale, double* v_splat, uint32_t* vis_flag, double* vis_weight) {
  orc_raster_bwd_ext(W, H, tiles_x, tiles_y, bg, tile_ranges, vals_sorted, proj0, proj1, proj2, out_rgba, out_T, last_idx,
                     v_out, inv_gscale, v_splat, vis_flag, vis_weight, NULL);
}

/* raster_bwd.cu:37-139 with the feature lanes (FEAT: v_feat back through the composited features into
 * v_splat[10..12] and into dL/dalpha) and the hollow penalty (HOLLOW: lam (T_before h - S_h / (1 - alpha))
 * added to dL/dalpha, the refine statistic kept photometric). */
void orc_raster_bwd_ext(int W, int H, int tiles_x, int tiles_y, const float bg[3], const uint32_t* tile_ranges,
                        const uint32_t* vals_sorted, const float* proj0, const float* proj1, const float* proj2,
                        const float* out_rgba, const float* out_T, const uint32_t* last_idx, const float* v_out,
                        float inv_gscale, double* v_splat, uint32_t* vis_flag, double* vis_weight, const orc_ext_t* ext) {
  const int feat = ext && ext->feat;
  const float* hz = ext ? ext->hollow_z : NULL;
  const float lam = ext ? ext->hollow_lam : 0.f;
  const float Wf = (float)W, Hf = (float)H;
#pragma omp parallel for num_threads(g_threads) schedule(dynamic, 16)
  for (int tile = 0; tile < tiles_x * tiles_y; tile++) {
    int tx = tile % tiles_x, ty = tile / tiles_x;
    uint32_t rx = tile_ranges[tile * 2], ry = tile_ranges[tile * 2 + 1];
    if (ry <= rx) continue;
    for (int l = 0; l < RT_W * RT_W; l++) {
      int px = tx * RT_W + l % RT_W, py = ty * RT_W + l / RT_W;
      if (!(px < W && py < H)) continue;
      size_t pix = (size_t)py * W + px;
      float pcx = px + 0.5f, pcy = py + 0.5f;
      float final_a = out_rgba[pix * 4 + 3], T = out_T[pix];
      uint32_t last = last_idx[pix];
      const float* vo = v_out + pix * 4;
      float v_o_w = (vo[3] - (bg[0] * vo[0] + bg[1] * vo[1] + bg[2] * vo[2])) * T;
      float Sx = 0.f, Sy = 0.f, Sz = 0.f, Sf0 = 0.f, Sf1 = 0.f, Sf2 = 0.f, Sh = 0.f;
      const float* vf = feat ? ext->v_feat + pix * 4 : NULL;
      const float z_ref = hz ? hz[pix] : INFINITY;
      const float inv_final_a = 1.f / fmaxf(final_a, 1e-5f);
      for (uint32_t idx = ry; idx-- > rx;) {
        if (!(idx < last)) continue;
        uint32_t gid = vals_sorted[idx];
        const float* a = proj0 + (size_t)gid * 4; const float* c = proj1 + (size_t)gid * 4;
        float dx = pcx - a[0], dy = pcy - a[1];
        float sigma = frag_sigma(a[0], a[1], a[2], a[3], c[0], pcx, pcy);
        if (!(sigma <= c[3])) continue;
        float g[GRAD_LANES];
        for (int k = 0; k < GRAD_LANES; k++) g[k] = 0.f;
        float gauss = expf(-sigma);
        float alpha = fminf(ALPHA_MAX, c[1] * gauss);
        float ra = 1.f / (1.f - alpha);
        float T_before = T * ra;
        float vis = alpha * T_before;
        const float* col = proj2 + (size_t)gid * 4;
        float cr = fmaxf(col[0], 0.f), cg = fmaxf(col[1], 0.f), cb = fmaxf(col[2], 0.f);
        g[5] = col[0] >= 0.f ? vis * vo[0] : 0.f;
        g[6] = col[1] >= 0.f ? vis * vo[1] : 0.f;
        g[7] = col[2] >= 0.f ? vis * vo[2] : 0.f;
        float v_alpha = (T_before * cr - Sx * ra) * vo[0] + (T_before * cg - Sy * ra) * vo[1] +
                        (T_before * cb - Sz * ra) * vo[2] + v_o_w * ra;
        float fx = 0.f, fy = 0.f, fz = 0.f, hh = 0.f;
        if (feat) {
          fx = col[3]; fy = ext->proj3[(size_t)gid * 2]; fz = ext->proj3[(size_t)gid * 2 + 1];
          g[10] = vis * vf[0]; g[11] = vis * vf[1]; g[12] = vis * vf[2];
          v_alpha += (T_before * fx - Sf0 * ra) * vf[0] + (T_before * fy - Sf1 * ra) * vf[1] + (T_before * fz - Sf2 * ra) * vf[2];
        }
        const float v_sigma_photo = -alpha * v_alpha;
        if (hz) {
          hh = hollow_pen_of(c[2], z_ref, ext->hollow_margin);
          v_alpha += lam * (T_before * hh - Sh * ra);
        }
        float v_sigma = -alpha * v_alpha;
        if (c[1] * gauss <= ALPHA_MAX) {
          g[2] = 0.5f * v_sigma * dx * dx; g[3] = v_sigma * dx * dy; g[4] = 0.5f * v_sigma * dy * dy;
          g[0] = -v_sigma * (a[2] * dx + a[3] * dy);
          g[1] = -v_sigma * (a[3] * dx + c[0] * dy);
          g[8] = v_alpha * gauss;
          const float rx_ = -v_sigma_photo * (a[2] * dx + a[3] * dy), ry_ = -v_sigma_photo * (a[3] * dx + c[0] * dy);
          float len = sqrtf(rx_ * Wf * rx_ * Wf + ry_ * Hf * ry_ * Hf);
          g[9] = len * inv_final_a;
        }
        Sx += cr * vis; Sy += cg * vis; Sz += cb * vis;
        if (feat) { Sf0 += fx * vis; Sf1 += fy * vis; Sf2 += fz * vis; }
        if (hz) Sh += hh * vis;
        T = T_before;
        vis_flag[gid] = 1u; /* every writer stores the same value */
        acc_add(&vis_weight[gid], (double)vis);
        for (int k = 0; k < GRAD_LANES; k++) acc_add(&v_splat[(size_t)gid * GRAD_LANES + k], (double)g[k] * (double)inv_gscale);
      }
    }
  }
}

/* ------------------------------------------------------------------------------------------------
 * Projection VJP (optim.cu:99-253) with the grad_out write (292-296), evaluated in double precision from
 * the float32 parameters and screen-space gradients: the accurate reference the HIP kernel's float32 VJP
 * is measured against. It follows the reference's chain through the world-space covariance
 * Sigma = M M^T (M = R(q) diag(s)) and the camera-frame covariance R_view Sigma R_view^T, a different
 * route from the kernel's (which differentiates the image-plane semi-axes). The colour's view-direction
 * term is a central difference of the double-precision SH basis on the unit sphere's tangent plane.
 * Splats culled by the float32 projection (the forward's decision) get zero rows.
 * ---------------------------------------------------------------------------------------------- */
typedef struct { double m[9]; } dmat3;

static dmat3 dm_mul(dmat3 A, dmat3 B) {
  dmat3 C;
  for (int r = 0; r < 3; r++)
    for (int c = 0; c < 3; c++) C.m[3 * r + c] = A.m[3 * r] * B.m[c] + A.m[3 * r + 1] * B.m[3 + c] + A.m[3 * r + 2] * B.m[6 + c];
  return C;
}

static dmat3 dm_t(dmat3 A) {
  dmat3 T;
  for (int r = 0; r < 3; r++)
    for (int c = 0; c < 3; c++) T.m[3 * r + c] = A.m[3 * c + r];
  return T;
}

static dmat3 dm_rot(const double q[4]) { /* unit quaternion (w, x, y, z) */
  const double w = q[0], x = q[1], y = q[2], z = q[3];
  dmat3 R = {{1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
              2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
              2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)}};
  return R;
}

static void sh_basis_d(int deg, double x, double y, double z, double* b);

/* colour(dir) . vc for the splat's coefficients (active degree deg) */
static double sh_colour_dot(int deg, const float* c, const double dir[3], const double vc[3]) {
  double b[25];
  sh_basis_d(deg, dir[0], dir[1], dir[2], b);
  double acc = 0.0;
  const int K = (deg + 1) * (deg + 1);
  for (int k = 0; k < K; k++) acc += b[k] * (c[3 * k] * vc[0] + c[3 * k + 1] * vc[1] + c[3 * k + 2] * vc[2]);
  return acc;
}

void orc_vjp(const orc_model_t* m, const orc_cam_t* cam, int active_deg, const float* v_splat, const uint32_t* vis_flag,
             const uint32_t* tile_count, float* grad_out) {
  const int K = (m->degree + 1) * (m->degree + 1);
  int deg = active_deg < m->degree ? active_deg : m->degree;
  if (deg < 0) deg = 0;
  const int kmax = (deg + 1) * (deg + 1);
  const int per = 11 + 3 * K;
  dmat3 Rv;
  for (int k = 0; k < 9; k++) Rv.m[k] = cam->R[k];
  const dmat3 RvT = dm_t(Rv);
  const double fx = cam->fx, fy = cam->fy;
  for (int i = 0; i < m->n; i++) {
    float* o = grad_out + (size_t)i * per;
    for (int k = 0; k < per; k++) o[k] = 0.f;
    const float* gl = v_splat + (size_t)i * GRAD_LANES;
    const int visible = vis_flag[i] != 0u && tile_count[i] != 0u;
    int any = 0, finite = 1;
    for (int k = 0; k < GRAD_LANES; k++) {
      const float v = vis_flag[i] ? gl[k] : 0.f;
      if (k != 9 && v != 0.f) any = 1;
      if (!finitef(v)) finite = 0;
    }
    if (!(any && visible && finite)) continue; /* optim.cu:110-148 */
    const float* po = m->pos_op + (size_t)i * 4;
    const float* qf = m->quat + (size_t)i * 4;
    const float* ls = m->lscale + (size_t)i * 4;
    proj_t pr;
    project_one(po, qf, ls, cam, &pr);
    if (!pr.ok) continue;
    double g[GRAD_LANES];
    for (int k = 0; k < GRAD_LANES; k++) g[k] = gl[k];
    /* ---- SH coefficients and the view-direction term */
    const double dv[3] = {(double)po[0] - cam->pos[0], (double)po[1] - cam->pos[1], (double)po[2] - cam->pos[2]};
    const double dlen = sqrt(dv[0] * dv[0] + dv[1] * dv[1] + dv[2] * dv[2]);
    const double dir[3] = {dv[0] / dlen, dv[1] / dlen, dv[2] / dlen};
    const double vc[3] = {g[5], g[6], g[7]};
    double basis[25];
    sh_basis_d(deg, dir[0], dir[1], dir[2], basis);
    for (int k = 0; k < kmax; k++)
      for (int ch = 0; ch < 3; ch++) o[11 + 3 * k + ch] = (float)(basis[k] * vc[ch]);
    double gpos[3] = {0, 0, 0};
    { /* d(colour . vc)/d p: moving p by dp turns dir by (I - dir dir^T) dp / |d| */
      const float* coef = m->sh + (size_t)i * K * 3;
      const double h = 1e-6;
      for (int a = 0; a < 3; a++) {
        double dp[3] = {dv[0], dv[1], dv[2]}, dm[3] = {dv[0], dv[1], dv[2]};
        dp[a] += h * dlen;
        dm[a] -= h * dlen;
        const double lp = sqrt(dp[0] * dp[0] + dp[1] * dp[1] + dp[2] * dp[2]);
        const double lm = sqrt(dm[0] * dm[0] + dm[1] * dm[1] + dm[2] * dm[2]);
        const double up[3] = {dp[0] / lp, dp[1] / lp, dp[2] / lp}, um[3] = {dm[0] / lm, dm[1] / lm, dm[2] / lm};
        gpos[a] = (sh_colour_dot(deg, coef, up, vc) - sh_colour_dot(deg, coef, um, vc)) / (2.0 * h * dlen);
      }
    }
    /* ---- the covariance chain */
    const double qn2 = (double)qf[0] * qf[0] + (double)qf[1] * qf[1] + (double)qf[2] * qf[2] + (double)qf[3] * qf[3];
    const double qlen = sqrt(qn2);
    const double qn[4] = {qf[0] / qlen, qf[1] / qlen, qf[2] / qlen, qf[3] / qlen};
    const dmat3 Rq = dm_rot(qn);
    const double f2 = (double)ls[3] * ls[3];
    double var[3], sc[3];
    for (int j = 0; j < 3; j++) {
      var[j] = exp(2.0 * (double)ls[j]);
      sc[j] = sqrt(var[j] + f2);
    }
    dmat3 M;
    for (int r = 0; r < 3; r++)
      for (int j = 0; j < 3; j++) M.m[3 * r + j] = Rq.m[3 * r + j] * sc[j];
    const dmat3 Sigma = dm_mul(M, dm_t(M));
    const dmat3 Sc = dm_mul(dm_mul(Rv, Sigma), RvT);
    double mc[3];
    for (int r = 0; r < 3; r++) mc[r] = Rv.m[3 * r] * po[0] + Rv.m[3 * r + 1] * po[1] + Rv.m[3 * r + 2] * po[2] + cam->t[r];
    const double z = mc[2], tx = mc[0] / z, ty = mc[1] / z;
    const int clip_x = !(tx <= cam->lim_pos_x && tx >= cam->lim_neg_x);
    const int clip_y = !(ty <= cam->lim_pos_y && ty >= cam->lim_neg_y);
    const double txc = fmin(fmax(tx, cam->lim_neg_x), cam->lim_pos_x), tyc = fmin(fmax(ty, cam->lim_neg_y), cam->lim_pos_y);
    const double J[2][3] = {{fx / z, 0.0, -fx * txc / z}, {0.0, fy / z, -fy * tyc / z}};
    double cov[2][2];
    for (int a = 0; a < 2; a++)
      for (int b = 0; b < 2; b++) {
        double acc = 0.0;
        for (int r = 0; r < 3; r++)
          for (int c = 0; c < 3; c++) acc += J[a][r] * Sc.m[3 * r + c] * J[b][c];
        cov[a][b] = acc + (a == b ? 0.3 : 0.0);
      }
    const double det = cov[0][0] * cov[1][1] - cov[0][1] * cov[1][0];
    const double Cn[2][2] = {{cov[1][1] / det, -cov[0][1] / det}, {-cov[1][0] / det, cov[0][0] / det}};
    /* dL/dcov = -C Gc C, Gc the symmetric conic gradient (off-diagonal lane g3 counts both entries) */
    const double Gc[2][2] = {{g[2], 0.5 * g[3]}, {0.5 * g[3], g[4]}};
    double T2[2][2], Gcov[2][2];
    for (int a = 0; a < 2; a++)
      for (int b = 0; b < 2; b++) T2[a][b] = Cn[a][0] * Gc[0][b] + Cn[a][1] * Gc[1][b];
    for (int a = 0; a < 2; a++)
      for (int b = 0; b < 2; b++) Gcov[a][b] = -(T2[a][0] * Cn[0][b] + T2[a][1] * Cn[1][b]);
    /* cov = J Sc J^T: dL/dJ = 2 Gcov J Sc, dL/dSc = J^T Gcov J */
    double GJ[2][3];
    for (int a = 0; a < 2; a++)
      for (int c = 0; c < 3; c++) {
        double acc = 0.0;
        for (int b = 0; b < 2; b++)
          for (int r = 0; r < 3; r++) acc += Gcov[a][b] * J[b][r] * Sc.m[3 * r + c];
        GJ[a][c] = 2.0 * acc;
      }
    dmat3 GSc;
    for (int r = 0; r < 3; r++)
      for (int c = 0; c < 3; c++) {
        double acc = 0.0;
        for (int a = 0; a < 2; a++)
          for (int b = 0; b < 2; b++) acc += J[a][r] * Gcov[a][b] * J[b][c];
        GSc.m[3 * r + c] = acc;
      }
    /* pinhole: mean2d = (fx tx + cx, fy ty + cy); J00 = fx/z, J02 = -fx txc/z with txc = tx unless clamped */
    double gmc[3];
    gmc[0] = fx / z * g[0] + (clip_x ? 0.0 : -fx / (z * z) * GJ[0][2]);
    gmc[1] = fy / z * g[1] + (clip_y ? 0.0 : -fy / (z * z) * GJ[1][2]);
    gmc[2] = -fx * mc[0] / (z * z) * g[0] - fy * mc[1] / (z * z) * g[1] - fx / (z * z) * GJ[0][0] - fy / (z * z) * GJ[1][1] +
             GJ[0][2] * (fx * txc / (z * z) + (clip_x ? 0.0 : fx * tx / (z * z))) +
             GJ[1][2] * (fy * tyc / (z * z) + (clip_y ? 0.0 : fy * ty / (z * z)));
    for (int a = 0; a < 3; a++) gpos[a] += RvT.m[3 * a] * gmc[0] + RvT.m[3 * a + 1] * gmc[1] + RvT.m[3 * a + 2] * gmc[2];
    /* Sc = R_view Sigma R_view^T, Sigma = M M^T */
    const dmat3 GSigma = dm_mul(dm_mul(RvT, GSc), Rv);
    dmat3 GM = dm_mul(GSigma, M);
    for (int k = 0; k < 9; k++) GM.m[k] *= 2.0;
    /* M = R(q) diag(s): dL/ds_j = column j of R(q) . column j of GM; dL/dR = GM diag(s) */
    double glog[3];
    const double opac = pr.opac, sigm = pr.sig;
    for (int j = 0; j < 3; j++) {
      const double gs = Rq.m[j] * GM.m[j] + Rq.m[3 + j] * GM.m[3 + j] + Rq.m[6 + j] * GM.m[6 + j];
      glog[j] = gs * var[j] / sc[j] + g[8] * opac * f2 / (var[j] + f2);
    }
    dmat3 GR;
    for (int r = 0; r < 3; r++)
      for (int j = 0; j < 3; j++) GR.m[3 * r + j] = GM.m[3 * r + j] * sc[j];
    /* feature lanes (optim.cu:235-250): the pseudo-normal R_view (s u), u = c / |c| with c the column of
     * R(q) along the smallest log scale and s the facing sign, so dL/dc = s (I - u u^T) R_view^T g_f / |c| */
    if (g[10] != 0.0 || g[11] != 0.0 || g[12] != 0.0) {
      const int ax = (ls[0] <= ls[1] && ls[0] <= ls[2]) ? 0 : (ls[1] <= ls[2] ? 1 : 2);
      const double cv[3] = {Rq.m[ax], Rq.m[3 + ax], Rq.m[6 + ax]};
      const double cl = fmax(sqrt(cv[0] * cv[0] + cv[1] * cv[1] + cv[2] * cv[2]), 1e-12);
      const double u[3] = {cv[0] / cl, cv[1] / cl, cv[2] / cl};
      const double face = -(dv[0] * u[0] + dv[1] * u[1] + dv[2] * u[2]) >= 0.0 ? 1.0 : -1.0;
      double bu[3];
      for (int r = 0; r < 3; r++) bu[r] = face * (RvT.m[3 * r] * g[10] + RvT.m[3 * r + 1] * g[11] + RvT.m[3 * r + 2] * g[12]);
      const double along = u[0] * bu[0] + u[1] * bu[1] + u[2] * bu[2];
      for (int r = 0; r < 3; r++) GR.m[3 * r + ax] += (bu[r] - u[r] * along) / cl;
    }
    /* quaternion: entrywise derivatives of R(q) (optim.cu:24-33), then through q / |q| (optim.cu:10-21) */
    const double w = qn[0], x = qn[1], y = qn[2], zq = qn[3];
    const double* G = GR.m;
    double gqn[4];
    gqn[0] = 2 * (x * (G[7] - G[5]) + y * (G[2] - G[6]) + zq * (G[3] - G[1]));
    gqn[1] = 2 * (-2 * x * (G[4] + G[8]) + y * (G[3] + G[1]) + zq * (G[6] + G[2]) + w * (G[7] - G[5]));
    gqn[2] = 2 * (x * (G[3] + G[1]) - 2 * y * (G[0] + G[8]) + zq * (G[7] + G[5]) + w * (G[2] - G[6]));
    gqn[3] = 2 * (x * (G[6] + G[2]) + y * (G[7] + G[5]) - 2 * zq * (G[0] + G[4]) + w * (G[3] - G[1]));
    const double along = qn[0] * gqn[0] + qn[1] * gqn[1] + qn[2] * gqn[2] + qn[3] * gqn[3];
    double gq[4];
    for (int k = 0; k < 4; k++) gq[k] = (gqn[k] - qn[k] * along) / qlen;
    const double glogit = g[8] * pr.comp_floor * sigm * (1.0 - sigm);
    const double outv[11] = {gpos[0], gpos[1], gpos[2], glogit, gq[0], gq[1], gq[2], gq[3], glog[0], glog[1], glog[2]};
    int ok = 1;
    for (int k = 0; k < 11; k++) ok = ok && isfinite(outv[k]);
    for (int k = 0; k < 11; k++) o[k] = ok ? (float)outv[k] : 0.f;
  }
}

/* ------------------------------------------------------------------------------------------------
 * fp64 brute force (tests/reference.cpp:34-143), photometric + alpha lane.
 * ---------------------------------------------------------------------------------------------- */
static void sh_basis_d(int deg, double x, double y, double z, double* b) { /* reference.cpp:16-30 (+ degree 4) */
  int K = (deg + 1) * (deg + 1);
  for (int k = 0; k < K; k++) b[k] = 0.0;
  b[0] = 0.28209479177387814;
  if (deg >= 1) { b[1] = -0.4886025 * y; b[2] = 0.4886025 * z; b[3] = -0.4886025 * x; }
  if (deg >= 2) {
    double z2 = z * z, f0b = -1.0925485 * z, f1a = 0.54627424, fc1 = x * x - y * y, fs1 = 2 * x * y;
    b[4] = f1a * fs1; b[5] = f0b * y; b[6] = 0.9461747 * z2 - 0.31539157; b[7] = f0b * x; b[8] = f1a * fc1;
    if (deg >= 3) {
      double f0c = -2.285229 * z2 + 0.4570458, f1b = 1.4453057 * z, f2a = -0.5900436, fc2 = x * fc1 - y * fs1, fs2 = x * fs1 + y * fc1;
      b[9] = f2a * fs2; b[10] = f1b * fs1; b[11] = f0c * y; b[12] = z * (1.8658817 * z2 - 1.119529); b[13] = f0c * x;
      b[14] = f1b * fc1; b[15] = f2a * fc2;
      if (deg >= 4) { /* extension: splat_math.cuh:136-141 */
        double f0d = z * (-4.683326 * z2 + 2.0071396), f1c = 3.3116114 * z2 - 0.47308735, f2b = -1.7701308 * z, f3a = 0.62583575;
        double fc3 = x * fc2 - y * fs2, fs3 = x * fs2 + y * fc2;
        b[16] = f3a * fs3; b[17] = f2b * fs2; b[18] = f1c * fs1; b[19] = f0d * y; b[20] = 1.9843135 * z * b[12] - 1.0062306 * b[6];
        b[21] = f0d * x; b[22] = f1c * fc1; b[23] = f2b * fc2; b[24] = f3a * fc3;
      }
    }
  }
}

typedef struct { int ok; double mx, my, c00, c01, c11, opac, depth, r, g, b, f[3]; } dproj_t;

static const dproj_t* g_sort_pr;
static int depth_cmp(const void* a, const void* b) {
  double da = g_sort_pr[*(const int*)a].depth, db = g_sort_pr[*(const int*)b].depth;
  if (da < db) return -1;
  if (da > db) return 1;
  return *(const int*)a - *(const int*)b;
}

/* Rows [y0, y1) of the brute-force render (reference.cpp:84-104): every depth-sorted projected splat is
 * tested at every pixel; with stride > 1 only the pixels whose row-major index is a multiple of it. */
static void ref_composite(const dproj_t* pr, const int* order, int no, int W, int y0, int y1, const double bg[3],
                          double* imgd, size_t stride, double* featd, const float* hollow_z, double hollow_margin,
                          double* hollow_sum) {
  for (int py = y0; py < y1; py++)
    for (int px = 0; px < W; px++) {
      if (stride > 1 && ((size_t)py * W + px) % stride) continue;
      double T = 1, r = 0, g = 0, b = 0, pcx = px + 0.5, pcy = py + 0.5, f0 = 0, f1 = 0, f2 = 0;
      const double zr = hollow_z ? (double)hollow_z[(size_t)py * W + px] : 0.0;
      for (int oi = 0; oi < no; oi++) {
        const dproj_t* q = &pr[order[oi]];
        double dx = pcx - q->mx, dy = pcy - q->my;
        double sigma = 0.5 * (q->c00 * dx * dx + q->c11 * dy * dy) + q->c01 * dx * dy;
        double alpha = fmin(0.999, q->opac * exp(-sigma));
        if (!(sigma >= 0 && alpha >= 1.0 / 255.0)) continue;
        double nT = T * (1 - alpha);
        if (nT <= 1e-4) break;
        double vis = alpha * T;
        r += fmax(q->r, 0.0) * vis; g += fmax(q->g, 0.0) * vis; b += fmax(q->b, 0.0) * vis;
        f0 += q->f[0] * vis; f1 += q->f[1] * vis; f2 += q->f[2] * vis;
        if (hollow_z) { /* reference.cpp:100 */
          const double d = (q->depth - zr - hollow_margin) / fmax(hollow_margin, 1e-4);
          if (isfinite(d)) *hollow_sum += vis * fmin(fmax(d, 0.0), 1.0);
        }
        T = nT;
      }
      size_t o = (size_t)py * W + px;
      imgd[o * 4] = r + T * bg[0]; imgd[o * 4 + 1] = g + T * bg[1]; imgd[o * 4 + 2] = b + T * bg[2]; imgd[o * 4 + 3] = 1 - T;
      if (featd) { featd[o * 3] = f0; featd[o * 3 + 1] = f1; featd[o * 3 + 2] = f2; }
    }
}

/* A bounded sample of the brute force for the CPU baseline: with a stride above 1, orc_ref_loss renders
 * only every stride-th pixel (row-major), times that (orc_ref_composite_seconds) and returns 0 without the
 * loss. */
static size_t g_ref_stride = 1;
static double g_ref_composite_s = 0.0;
void orc_ref_set_sample(uint64_t stride) { g_ref_stride = stride > 1 ? (size_t)stride : 1; }
double orc_ref_composite_seconds(void) { return g_ref_composite_s; }

double orc_ref_loss(int n, int degree, const double* pos, const double* log_scale, const double* quat, const double* opacity,
                    const double* sh, const double* floor_, const orc_cam_t* cam, int W, int H, const double bg[3],
                    const uint32_t* gt, const uint8_t* weights, int composite, int mask, int alpha_lane, double l1_w,
                    double ssim_w, double match_alpha_weight, double scale, int float_exp, double* out_img) {
  return orc_ref_loss_ext(n, degree, pos, log_scale, quat, opacity, sh, floor_, cam, W, H, bg, gt, weights, composite, mask,
                          alpha_lane, l1_w, ssim_w, match_alpha_weight, scale, float_exp, out_img, NULL);
}

double orc_ref_loss_ext(int n, int degree, const double* pos, const double* log_scale, const double* quat,
                        const double* opacity, const double* sh, const double* floor_, const orc_cam_t* cam, int W, int H,
                        const double bg[3], const uint32_t* gt, const uint8_t* weights, int composite, int mask,
                        int alpha_lane, double l1_w, double ssim_w, double match_alpha_weight, double scale, int float_exp,
                        double* out_img, const orc_ref_ext_t* rx) {
  const int normals = rx && rx->normals;
  const float* hollow_z = rx ? rx->hollow_z : NULL;
  double R[9];
  for (int i = 0; i < 9; i++) R[i] = cam->R[i];
  const double fx = cam->fx, fy = cam->fy, cx = cam->cx, cy = cam->cy;
  double lim_pos_x = (1.15 * W - cx) / fx, lim_neg_x = (-0.15 * W - cx) / fx;
  double lim_pos_y = (1.15 * H - cy) / fy, lim_neg_y = (-0.15 * H - cy) / fy;
  const int K = (degree + 1) * (degree + 1);
  dproj_t* pr = (dproj_t*)calloc((size_t)(n > 0 ? n : 1), sizeof(dproj_t));
  for (int i = 0; i < n; i++) {
    double mean[3] = {pos[i * 3], pos[i * 3 + 1], pos[i * 3 + 2]};
    double mc[3];
    for (int r = 0; r < 3; r++) mc[r] = R[r * 3] * mean[0] + R[r * 3 + 1] * mean[1] + R[r * 3 + 2] * mean[2] + cam->t[r];
    if (!(mc[2] >= 0.01)) continue;
    double s[3], f2 = floor_ ? floor_[i] * floor_[i] : 0.0, comp = 1.0;
    /* reference.cpp:45,56 pass float parameters to std::exp, which selects the float overload;
     * float_exp = 1 reproduces that, 0 keeps the exponentials in double (smooth for finite differences). */
    for (int k = 0; k < 3; k++) s[k] = float_exp ? (double)expf((float)log_scale[i * 3 + k]) : exp(log_scale[i * 3 + k]);
    if (f2 > 0) { /* extension: Mip-Splatting floor, splat_math.cuh:232-237 */
      double num = 1, den = 1;
      for (int k = 0; k < 3; k++) { double s2 = s[k] * s[k]; num *= s2; den *= s2 + f2; s[k] = sqrt(s2 + f2); }
      comp = sqrt(num / den);
    }
    double w = quat[i * 4], x = quat[i * 4 + 1], y = quat[i * 4 + 2], z = quat[i * 4 + 3];
    double qn = sqrt(w * w + x * x + y * y + z * z);
    w /= qn; x /= qn; y /= qn; z /= qn;
    double Rq[9] = {1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w),
                    2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w),
                    2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)};
    double M[9];
    for (int r = 0; r < 3; r++)
      for (int c = 0; c < 3; c++) {
        double v = 0;
        for (int k = 0; k < 3; k++) v += R[r * 3 + k] * Rq[k * 3 + c];
        M[r * 3 + c] = v * s[c];
      }
    double inv_z = 1.0 / mc[2], rx = mc[0] * inv_z, ry = mc[1] * inv_z;
    double cxr = fmin(fmax(rx, lim_neg_x), lim_pos_x), cyr = fmin(fmax(ry, lim_neg_y), lim_pos_y);
    double J[6] = {fx * inv_z, 0, -fx * inv_z * cxr, 0, fy * inv_z, -fy * inv_z * cyr};
    double V[6];
    for (int r = 0; r < 2; r++)
      for (int c = 0; c < 3; c++) V[r * 3 + c] = J[r * 3] * M[c] + J[r * 3 + 1] * M[3 + c] + J[r * 3 + 2] * M[6 + c];
    double c00 = V[0] * V[0] + V[1] * V[1] + V[2] * V[2] + 0.3, c01 = V[0] * V[3] + V[1] * V[4] + V[2] * V[5];
    double c11 = V[3] * V[3] + V[4] * V[4] + V[5] * V[5] + 0.3;
    double det = c00 * c11 - c01 * c01;
    if (!(det > 0)) continue;
    dproj_t q;
    q.c00 = c11 / det; q.c01 = -c01 / det; q.c11 = c00 / det;
    q.opac = 1.0 / (1.0 + (float_exp ? (double)expf(-(float)opacity[i]) : exp(-opacity[i]))) * comp;
    if (!(q.opac >= 1.0 / 255.0)) continue;
    q.mx = fx * rx + cx; q.my = fy * ry + cy; q.depth = mc[2];
    double power = log(q.opac * 255.0), detc = q.c00 * q.c11 - q.c01 * q.c01;
    double ex = sqrt(2 * power * q.c11 / detc), ey = sqrt(2 * power * q.c00 / detc);
    if (!(q.mx + ex > 0 && q.mx - ex < W && q.my + ey > 0 && q.my - ey < H)) continue;
    double v[3] = {mean[0] - cam->pos[0], mean[1] - cam->pos[1], mean[2] - cam->pos[2]};
    double vl = sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    v[0] /= vl; v[1] /= vl; v[2] /= vl;
    double b[25];
    sh_basis_d(degree, v[0], v[1], v[2], b);
    double col[3] = {0, 0, 0};
    for (int k = 0; k < K; k++)
      for (int ch = 0; ch < 3; ch++) col[ch] += b[k] * sh[((size_t)i * K + k) * 3 + ch];
    q.r = fmin(fmax(col[0] + 0.5, -100.0), 100.0);
    q.g = fmin(fmax(col[1] + 0.5, -100.0), 100.0);
    q.b = fmin(fmax(col[2] + 0.5, -100.0), 100.0);
    q.f[0] = q.f[1] = q.f[2] = 0.0;
    if (normals) { /* reference.cpp:75-83: the camera-facing shortest local axis in camera space */
      const double* l = log_scale + (size_t)i * 3;
      const int ax = (l[0] <= l[1] && l[0] <= l[2]) ? 0 : (l[1] <= l[2] ? 1 : 2);
      const double a[3] = {Rq[ax], Rq[3 + ax], Rq[6 + ax]};
      const double al = sqrt(a[0] * a[0] + a[1] * a[1] + a[2] * a[2]);
      const double u[3] = {a[0] / al, a[1] / al, a[2] / al};
      const double face = ((cam->pos[0] - mean[0]) * u[0] + (cam->pos[1] - mean[1]) * u[1] + (cam->pos[2] - mean[2]) * u[2]) >= 0 ? 1.0 : -1.0;
      for (int r = 0; r < 3; r++) q.f[r] = R[r * 3] * u[0] * face + R[r * 3 + 1] * u[1] * face + R[r * 3 + 2] * u[2] * face;
    }
    q.ok = 1;
    pr[i] = q;
  }
  int* order = (int*)malloc(sizeof(int) * (size_t)(n > 0 ? n : 1));
  int no = 0;
  for (int i = 0; i < n; i++) if (pr[i].ok) order[no++] = i;
  g_sort_pr = pr;
  qsort(order, (size_t)no, sizeof(int), depth_cmp);
  const size_t P = (size_t)W * H;
  float* img = (float*)malloc(sizeof(float) * P * 4);
  double* imgd = (double*)malloc(sizeof(double) * P * 4);
  if (g_ref_stride > 1) { /* bounded sample: every g_ref_stride-th pixel, then no loss */
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    ref_composite(pr, order, no, W, 0, H, bg, imgd, g_ref_stride, NULL, NULL, 0.0, NULL);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    g_ref_composite_s = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
    if (out_img) memcpy(out_img, imgd, sizeof(double) * P * 4);
    free(img); free(imgd); free(order); free(pr);
    return 0.0;
  }
  double* featd = normals ? (double*)malloc(sizeof(double) * P * 3) : NULL;
  double hollow_sum = 0.0;
  ref_composite(pr, order, no, W, 0, H, bg, imgd, 1, featd, hollow_z, rx ? rx->hollow_margin : 0.0, &hollow_sum);
  if (out_img) memcpy(out_img, imgd, sizeof(double) * P * 4);
  /* loss in double over the double image (reference.cpp:105-131) */
  double w[11];
  gauss11(w);
  double* X = (double*)malloc(sizeof(double) * P * 9);
  double *Y = X + P, *tmp = X + 2 * P, *mu1 = X + 3 * P, *mu2 = X + 4 * P, *ex2 = X + 5 * P, *ey2 = X + 6 * P, *exy = X + 7 * P, *sq = X + 8 * P;
  const double norm = scale / (3.0 * W * H);
  double loss = 0;
  for (int ch = 0; ch < 3; ch++) {
    for (size_t i = 0; i < P; i++) { X[i] = imgd[i * 4 + ch]; Y[i] = gtc_div(gt[i], ch) + (composite ? (1 - gtc_div(gt[i], 3)) * bg[ch] : 0.0); }
    blur_d(W, H, w, X, tmp, mu1);
    blur_d(W, H, w, Y, tmp, mu2);
    for (size_t i = 0; i < P; i++) sq[i] = X[i] * X[i];
    blur_d(W, H, w, sq, tmp, ex2);
    for (size_t i = 0; i < P; i++) sq[i] = Y[i] * Y[i];
    blur_d(W, H, w, sq, tmp, ey2);
    for (size_t i = 0; i < P; i++) sq[i] = X[i] * Y[i];
    blur_d(W, H, w, sq, tmp, exy);
    for (size_t i = 0; i < P; i++) {
      double s1 = fmax(0.0, ex2[i] - mu1[i] * mu1[i]), s2 = fmax(0.0, ey2[i] - mu2[i] * mu2[i]), s12 = exy[i] - mu1[i] * mu2[i];
      double ssim = ((2 * mu1[i] * mu2[i] + 1e-4) * (2 * s12 + 9e-4)) / ((mu1[i] * mu1[i] + mu2[i] * mu2[i] + 1e-4) * (s1 + s2 + 9e-4));
      ssim = fmin(fmax(ssim, -1.0), 1.0);
      double wp = weights ? weights[i] / 255.0 : 1.0;
      double Mw = wp * (mask ? gtc_div(gt[i], 3) : 1.0) * norm;
      loss += Mw * (l1_w * fabs(X[i] - Y[i]) + ssim_w * ssim);
    }
  }
  if (alpha_lane)
    for (size_t i = 0; i < P; i++) {
      double wp = weights ? weights[i] / 255.0 : 1.0;
      loss += wp * match_alpha_weight * scale / (double)(W * H) * fabs(imgd[i * 4 + 3] - gtc_div(gt[i], 3));
    }
  if (normals && rx->normal_scale > 0)
    for (size_t i = 0; i < P; i++) { /* reference.cpp:134-141 */
      const uint32_t g = rx->gtn[i];
      if (((g >> 24) & 0xffu) <= 127u) continue;
      const double wp = weights ? weights[i] / 255.0 : 1.0;
      const double gx = (g & 0xffu) * (2.0 / 255.0) - 1, gy = 1 - ((g >> 8) & 0xffu) * (2.0 / 255.0), gz = 1 - ((g >> 16) & 0xffu) * (2.0 / 255.0);
      const double px = featd[i * 3], py = featd[i * 3 + 1], pz = featd[i * 3 + 2];
      const double pl = fmax(sqrt(px * px + py * py + pz * pz), 1e-6), gl = fmax(sqrt(gx * gx + gy * gy + gz * gz), 1e-6);
      loss += rx->normal_scale * wp * (fabs(px - gx) + fabs(py - gy) + fabs(pz - gz) + 1 - (px * gx + py * gy + pz * gz) / (pl * gl));
    }
  if (hollow_z) loss += rx->hollow_lam * hollow_sum;
  free(featd);
  free(X); free(img); free(imgd); free(order); free(pr);
  return loss;
}

/* ------------------------------------------------------------------------------------------------
 * The other losses (loss.cu:197-293), per pixel in single precision exactly as the HIP kernels evaluate
 * them (the per-pixel outputs bit for bit), the sums in double.
 * ---------------------------------------------------------------------------------------------- */
double orc_normal_loss(int W, int H, const float* feat, const uint32_t* normals, const uint8_t* weights, float scale,
                       float grad_scale, float* v_feat) {
  double loss = 0.0;
  for (size_t pix = 0; pix < (size_t)W * H; pix++) {
    const uint32_t nm = normals[pix];
    float* out = v_feat + pix * 4;
    out[0] = out[1] = out[2] = out[3] = 0.f;
    if (((nm >> 24) & 0xffu) <= 127u) continue;
    const float wp = weights ? (float)weights[pix] * (1.f / 255.f) : 1.f;
    const float k = scale * wp;
    const float nx = (float)(nm & 0xffu) * (2.f / 255.f) - 1.f;
    const float ny = 1.f - (float)((nm >> 8) & 0xffu) * (2.f / 255.f);
    const float nz = 1.f - (float)((nm >> 16) & 0xffu) * (2.f / 255.f);
    const float* f = feat + pix * 4;
    const float pl = fmaxf(sqrtf((f[0] * f[0] + f[1] * f[1]) + f[2] * f[2]), 1e-6f);
    const float nl = fmaxf(sqrtf((nx * nx + ny * ny) + nz * nz), 1e-6f);
    const float dot = (f[0] * nx + f[1] * ny) + f[2] * nz;
    const float plnl = pl * nl;
    const float dx = f[0] - nx, dy = f[1] - ny, dz = f[2] - nz;
    loss += (double)(k * ((((fabsf(dx) + fabsf(dy)) + fabsf(dz)) + 1.f) - dot / plnl));
    const float inv = 1.f / plnl, radial = dot / ((pl * pl) * plnl);
    const float kg = k * grad_scale;
    const float sx = dx > 0.f ? 1.f : (dx < 0.f ? -1.f : 0.f);
    const float sy = dy > 0.f ? 1.f : (dy < 0.f ? -1.f : 0.f);
    const float sz = dz > 0.f ? 1.f : (dz < 0.f ? -1.f : 0.f);
    out[0] = kg * ((sx - nx * inv) + f[0] * radial);
    out[1] = kg * ((sy - ny * inv) + f[1] * radial);
    out[2] = kg * ((sz - nz * inv) + f[2] * radial);
  }
  return loss;
}

double orc_hollow_sum(int npix, const float* pen) {
  double s = 0.0;
  for (int i = 0; i < npix; i++) s += (double)pen[i];
  return s;
}

/* loss.cu:240-286: 8-bit prediction (clamped to [0, 1], rounded half to even), per channel and pixel the
 * squared error and the clamped SSIM of the 11-tap window (zero padding), alpha-weighted when
 * mask_weighted; the horizontal then vertical passes in the kernel's float order. */
void orc_eval(int W, int H, const float* pred, const uint32_t* gt, int mask_weighted, double* sum_se, double* sum_ssim) {
  double wd[11];
  gauss11(wd);
  float w[11];
  for (int d = 0; d < 11; d++) w[d] = (float)wd[d];
  const size_t P = (size_t)W * H;
  float* p = (float*)malloc(sizeof(float) * P);
  float* g = (float*)malloc(sizeof(float) * P);
  float* hs = (float*)malloc(sizeof(float) * P * 5);
  double se_t = 0.0, ss_t = 0.0;
  for (int c = 0; c < 3; c++) {
    for (size_t i = 0; i < P; i++) {
      const float pc = pred[i * 4 + c];
      p[i] = rintf(fminf(fmaxf(pc, 0.f), 1.f) * 255.f) / 255.f;
      g[i] = gt_chan_f(gt[i], c);
    }
    for (int y = 0; y < H; y++)
      for (int x = 0; x < W; x++) {
        float sx = 0.f, sxx = 0.f, sy = 0.f, syy = 0.f, sxy = 0.f;
        for (int d = 0; d < 11; d++) {
          const int xx = x - 5 + d;
          const float xv = (xx >= 0 && xx < W) ? p[(size_t)y * W + xx] : 0.f;
          const float yv = (xx >= 0 && xx < W) ? g[(size_t)y * W + xx] : 0.f;
          sx = sx + w[d] * xv; sxx = sxx + (w[d] * xv) * xv; sy = sy + w[d] * yv; syy = syy + (w[d] * yv) * yv;
          sxy = sxy + (w[d] * xv) * yv;
        }
        float* h = hs + ((size_t)y * W + x) * 5;
        h[0] = sx; h[1] = sxx; h[2] = sy; h[3] = syy; h[4] = sxy;
      }
    for (int y = 0; y < H; y++)
      for (int x = 0; x < W; x++) {
        float st[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
        for (int d = 0; d < 11; d++) {
          const int yy = y - 5 + d;
          for (int k = 0; k < 5; k++) st[k] = st[k] + w[d] * ((yy >= 0 && yy < H) ? hs[((size_t)yy * W + x) * 5 + k] : 0.f);
        }
        const float mu1 = st[0], mu2 = st[2];
        const float s1 = fmaxf(0.f, st[1] - mu1 * mu1), s2 = fmaxf(0.f, st[3] - mu2 * mu2), s12 = st[4] - mu1 * mu2;
        const float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f; /* as the kernels form them */
        const float num = ((2.f * mu1) * mu2 + C1) * (2.f * s12 + C2);
        const float den = ((mu1 * mu1 + mu2 * mu2) + C1) * ((s1 + s2) + C2);
        const float ssim = fminf(fmaxf(num / den, -1.f), 1.f);
        const size_t i = (size_t)y * W + x;
        const float d = fabsf(p[i] - g[i]);
        const float m = mask_weighted ? gt_chan_f(gt[i], 3) : 1.f;
        se_t += (double)((d * m) * (d * m));
        ss_t += (double)(ssim * m);
      }
  }
  *sum_se = se_t;
  *sum_ssim = ss_t;
  free(p); free(g); free(hs);
}

/* ------------------------------------------------------------------------------------------------
 * Replays of a rendered view's tile lists (evidence.cu:47-112, 141-183, probe.cu:7-45): per pixel the
 * forward's own walk, in single precision, with the forward oracle's alpha; the per-splat sums in double.
 * ---------------------------------------------------------------------------------------------- */
static float byte_f(uint32_t p, int c) { return (float)((p >> (8 * c)) & 0xffu) * (1.f / 255.f); }

void orc_evidence_view(int W, int H, int tiles_x, int tiles_y, const uint32_t* tile_ranges, const uint32_t* vals_sorted,
                       const float* proj0, const float* proj1, const float* out_rgba, const float* out_feat,
                       const uint32_t* last_idx, const uint32_t* gt, const uint32_t* normals, const uint8_t* weights,
                       const uint8_t* labels, int masked_has_alpha, float normal_weight, double* view_acc,
                       double* label_acc) {
  for (int tile = 0; tile < tiles_x * tiles_y; tile++) {
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const uint32_t rx = tile_ranges[tile * 2], ry = tile_ranges[tile * 2 + 1];
    for (int l = 0; l < RT_W * RT_W; l++) {
      const int px = tx * RT_W + l % RT_W, py = ty * RT_W + l / RT_W;
      if (!(px < W && py < H)) continue;
      const size_t pix = (size_t)py * W + px;
      const uint32_t g = gt[pix];
      const float ga = byte_f(g, 3);
      const float wp = weights ? (float)weights[pix] * (1.f / 255.f) : 1.f;
      const float* o = out_rgba + pix * 4;
      float res = (fabsf(o[0] - byte_f(g, 0)) + fabsf(o[1] - byte_f(g, 1)) + fabsf(o[2] - byte_f(g, 2))) * (1.f / 3.f);
      if (normals && normal_weight > 0.f && ((normals[pix] >> 24) & 0xffu) > 127u) { /* loss.cu:218-223 */
        const uint32_t gn = normals[pix];
        const float nx = (float)(gn & 0xffu) * (2.f / 255.f) - 1.f;
        const float ny = 1.f - (float)((gn >> 8) & 0xffu) * (2.f / 255.f);
        const float nz = 1.f - (float)((gn >> 16) & 0xffu) * (2.f / 255.f);
        const float* f = out_feat + pix * 3;
        const float pl = fmaxf(sqrtf(f[0] * f[0] + f[1] * f[1] + f[2] * f[2]), 1e-6f);
        const float nl = fmaxf(sqrtf(nx * nx + ny * ny + nz * nz), 1e-6f);
        const float nres = fabsf(f[0] - nx) + fabsf(f[1] - ny) + fabsf(f[2] - nz) + 1.f -
                           (f[0] * nx + f[1] * ny + f[2] * nz) / (pl * nl);
        res += normal_weight * nres;
      }
      const float m = ga * wp, mres = m * res, k = (masked_has_alpha ? ga : 1.f) * wp;
      const int lab = labels ? (int)labels[pix] : -1;
      const int vote = label_acc && lab >= 0 && lab < ORC_LABEL_BINS && k != 0.f;
      const float pcx = px + 0.5f, pcy = py + 0.5f;
      const uint32_t last = last_idx[pix];
      float T = 1.f;
      for (uint32_t idx = rx; idx < ry && idx < last; idx++) {
        const uint32_t gid = vals_sorted[idx];
        const float* a = proj0 + (size_t)gid * 4; const float* c = proj1 + (size_t)gid * 4;
        const float sigma = frag_sigma(a[0], a[1], a[2], a[3], c[0], pcx, pcy);
        if (!(sigma <= c[3])) continue;
        const float alpha = fminf(ALPHA_MAX, c[1] * expf(-sigma));
        const float vis = alpha * T;
        T *= 1.f - alpha;
        view_acc[(size_t)gid * 3] += (double)vis * m;
        view_acc[(size_t)gid * 3 + 1] += (double)vis * mres;
        view_acc[(size_t)gid * 3 + 2] += (double)vis * k;
        if (vote) label_acc[(size_t)gid * ORC_LABEL_BINS + lab] += (double)vis * k;
      }
    }
  }
}

void orc_probe(int W, int H, int tiles_x, int tiles_y, const uint32_t* tile_ranges, const uint32_t* vals_sorted,
               const float* proj0, const float* proj1, float tau, float delta, const float* ref_z, float margin,
               float* out) {
  const int mean_mode = tau <= 0.f;
  for (int tile = 0; tile < tiles_x * tiles_y; tile++) {
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const uint32_t rx = tile_ranges[tile * 2], ry = tile_ranges[tile * 2 + 1];
    for (int l = 0; l < RT_W * RT_W; l++) {
      const int px = tx * RT_W + l % RT_W, py = ty * RT_W + l / RT_W;
      if (!(px < W && py < H)) continue;
      const size_t pix = (size_t)py * W + px;
      const float pcx = px + 0.5f, pcy = py + 0.5f;
      const float zr = ref_z ? ref_z[pix] : INFINITY;
      float T = 1.f, z_first = INFINITY, deep = 0.f, behind = 0.f, zsum = 0.f;
      for (uint32_t idx = rx; idx < ry; idx++) {
        const uint32_t gid = vals_sorted[idx];
        const float* a = proj0 + (size_t)gid * 4; const float* c = proj1 + (size_t)gid * 4;
        const float sigma = frag_sigma(a[0], a[1], a[2], a[3], c[0], pcx, pcy);
        if (!(sigma <= c[3])) continue;
        const float alpha = fminf(ALPHA_MAX, c[1] * expf(-sigma));
        const float next_T = T * (1.f - alpha);
        if (next_T <= T_CUTOFF) break;
        const float vis = alpha * T, z = c[2];
        if (finitef(z_first) && z > z_first + delta) deep += vis;
        if (z > zr + margin) behind += vis;
        if (mean_mode) zsum = fmaf(vis, z, zsum);
        T = next_T;
        if (!finitef(z_first) && 1.f - T >= tau) z_first = z;
      }
      if (mean_mode) z_first = (1.f - T) > 0.05f ? zsum / (1.f - T) : INFINITY;
      out[pix * 4] = 1.f - T;
      out[pix * 4 + 1] = z_first;
      out[pix * 4 + 2] = deep;
      out[pix * 4 + 3] = behind;
    }
  }
}

/* ------------------------------------------------------------------------------------------------
 * Exports of internal pieces so the tests can pin them against closed forms.
 * ---------------------------------------------------------------------------------------------- */
void orc_sh_basis_f(int deg, float x, float y, float z, float* out) { sh_basis_f(deg, x, y, z, out); }
int orc_project_ok(const float* po, const float* q, const float* ls, const orc_cam_t* cam) {
  proj_t r;
  project_one(po, q, ls, cam, &r);
  return r.ok;
}
void orc_sh_basis_d(int deg, double x, double y, double z, double* out) { sh_basis_d(deg, x, y, z, out); }
void orc_quat_to_mat(const float* q, float* R) { quat_to_mat(q, R); }
int orc_tile_hit(float rmin_x, float rmin_y, float rmax_x, float rmax_y, float mx, float my, float c00, float c01,
                 float c11, float power) {
  sym2 c = {c00, c01, c11};
  return tile_hit(rmin_x, rmin_y, rmax_x, rmax_y, mx, my, c, power);
}
