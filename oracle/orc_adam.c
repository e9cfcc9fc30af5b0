/*
 * TEST INFRASTRUCTURE ONLY — the checker, never the product.
 *
 * CPU restatement of the fused optimizer of Erant/b2ctrain (src/gpu/optim.cu:104-148 bookkeeping and
 * 298-377 update; src/gpu/util.cuh:106-117 random streams and 148-162 stochastic fp16 rounding), one splat
 * at a time in single precision. Compiled with -ffp-contract=off, every operation is the one the HIP
 * kernel (b2ctrain_amd/csrc/kernels/vjp.hip, adam_update) evaluates, in the same order, so the GPU must
 * match it bit for bit. The reference's powf / __logf / __cosf are replaced as the kernel replaces them:
 * the step constants come from double-precision libm (orc_adam_constants), the per-splat powers are
 * e^(s ln beta) with the Cephes expf, and the Box-Muller logarithm / cosine are the Cephes logf and the
 * polynomials below. How each piece is pinned against something other than itself:
 * tests/test_oracle_adam.py.
 */
#include <math.h>
#include <string.h>

#include "b2c_oracle.h"

/* ---- random streams (util.cuh:106-117) ---- */

static uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

uint32_t orc_mix32(uint32_t x) { return mix32(x); }

float orc_hash_unit(uint32_t a, uint32_t b, uint32_t c) {
  const uint32_t h = mix32((a * 0x9E3779B1u) ^ mix32((b * 0x85EBCA77u) ^ mix32(c * 0xC2B2AE3Du)));
  return (float)(h >> 8) * (1.f / 16777216.f);
}

/* cos(2 pi u), u in [0, 1): exact reduction in turns to at most 1/8 turn, then the Cephes single-precision
 * cos / sin polynomials (S. L. Moshier, single/sinf.c). */
float orc_cos_turns(float u) {
  const float t = u >= 0.5f ? u - 1.f : u;
  float a = fabsf(t), sign = 1.f;
  if (a > 0.25f) {
    a = 0.5f - a;
    sign = -1.f;
  }
  const float two_pi = 6.28318530717958647692f;
  float r;
  if (a > 0.125f) {
    const float x = (0.25f - a) * two_pi, z = x * x;
    r = ((-1.9515295891e-4f * z + 8.3321608736e-3f) * z - 1.6666654611e-1f) * z * x + x;
  } else {
    const float x = a * two_pi, z = x * x;
    r = ((2.443315711809948e-5f * z - 1.388731625493765e-3f) * z + 4.166664568298827e-2f) * z * z;
    r = r - 0.5f * z;
    r = r + 1.f;
  }
  return sign * r;
}

/* Box-Muller over the counter pair (c, c + 0x1234567), u1 floored at 1e-7. */
float orc_hash_gauss(uint32_t a, uint32_t b, uint32_t c) {
  const float u1 = fmaxf(orc_hash_unit(a, b, c), 1e-7f), u2 = orc_hash_unit(a, b, c + 0x1234567u);
  return sqrtf(-2.f * orc_logf(u1)) * orc_cos_turns(u2);
}

/* ---- IEEE binary16 ---- */

static uint32_t fbits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float bitsf(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round to nearest even: normal results by the 13 dropped mantissa bits, subnormal ones by scaling the
 * magnitude to units of 2^-24 (exact) and rounding that to an integer. */
uint16_t orc_f16_bits(float v) {
  const uint32_t x = fbits(v), sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: overflows to infinity */
  if (ax < 0x38800000u) return (uint16_t)(sign | (uint32_t)rintf(bitsf(ax) * 16777216.f));
  uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
  const uint32_t rest = ax & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float orc_f16_value(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    const float mag = (float)m * (1.f / 16777216.f);
    return sign ? -mag : mag;
  }
  if (e == 31) return bitsf(sign | 0x7f800000u | (m << 13));
  return bitsf(sign | ((e + 112u) << 23) | (m << 13));
}

static uint16_t f16_next(uint16_t h, int up) {
  if ((h & 0x7fffu) == 0u) return up ? 0x0001u : 0x8001u;
  const int neg = (h & 0x8000u) != 0u;
  return (uint16_t)(up != neg ? h + 1u : h - 1u);
}

/* util.cuh:148-162: the lower neighbour lo, or the upper one with probability (v - lo) / (hi - lo). */
uint16_t orc_f16_stochastic(float v, float u01) {
  v = fminf(fmaxf(v, -65000.f), 65000.f);
  uint16_t h = orc_f16_bits(v);
  float lo = orc_f16_value(h);
  if (lo > v) {
    h = f16_next(h, 0);
    lo = orc_f16_value(h);
  }
  if (lo != v) {
    const uint16_t up = f16_next(h, 1);
    if (u01 * (orc_f16_value(up) - lo) < v - lo) h = up;
  }
  return h;
}

/* ---- the update ---- */

void orc_adam_constants(orc_adam_step_t* s) {
  const double b1 = s->beta1, b2 = s->beta2, t = s->t;
  s->bc1 = (float)(1.0 / (1.0 - pow(b1, t)));
  s->bc2 = (float)(1.0 / (1.0 - pow(b2, t)));
  s->ln_beta1 = (float)log(b1);
  s->ln_beta2 = (float)log(b2);
  const double r = b1 / sqrt(b2);
  s->ratio = (float)r;
  s->ln_ratio = (float)log(r);
}

typedef struct {
  float skipped, d1, d2, drift;
} catch_up_t;

/* optim.cu:301-315 for one parameter: the catch-up of skipped steps, then one bias-corrected Adam step. */
static void adam_param(float* p, float* m, float* v, float g, float lr, const orc_adam_step_t* s,
                       const catch_up_t* cu) {
  if (cu->skipped > 0.f) {
    *p = *p - ((lr * cu->drift) * (*m * s->bc1)) / (sqrtf(*v * s->bc2) + s->eps);
    *m = *m * cu->d1;
    *v = *v * cu->d2;
  }
  *m = s->beta1 * *m + (1.f - s->beta1) * g;
  *v = s->beta2 * *v + ((1.f - s->beta2) * g) * g;
  *p = *p - (lr * (*m * s->bc1)) / (sqrtf(*v * s->bc2) + s->eps);
}

void orc_adam_update(orc_adam_model_t* m, const orc_cam_t* cam, int active_deg, const float* v_splat,
                     const uint32_t* vis_flag, const uint32_t* tile_count, const float* grads,
                     const orc_adam_step_t* s) {
  const int K = (m->degree + 1) * (m->degree + 1), per = 11 + 3 * K;
  const int kmax = active_deg >= m->degree ? K : (active_deg + 1) * (active_deg + 1);
  for (int i = 0; i < m->n; i++) {
    /* optim.cu:110-131: the splat's screen-space gradient, visibility and "has a gradient" */
    const int vis = vis_flag[i] != 0u, visible = vis && tile_count[i] != 0u;
    float g[13];
    for (int k = 0; k < 13; k++) g[k] = vis ? v_splat[(size_t)i * 13 + k] : 0.f;
    int any = 0;
    for (int k = 0; k < 13; k++)
      if (k != 9 && g[k] != 0.f) any = 1;
    any = any && visible;
    for (int k = 0; k < 13; k++)
      if (!isfinite(g[k])) any = 0;
    if (s->sparse && !any) continue; /* optim.cu:148 */
    float* po = m->pos_op + 4 * (size_t)i;
    float* q = m->quat + 4 * (size_t)i;
    float* ls = m->lscale + 4 * (size_t)i;
    /* the SH second moment's share: sum of squared active basis values and the colour gradient, both zero
     * unless the splat has a gradient and survives the projection (optim.cu:152-170) */
    float bsq = 0.f, vc[3] = {0.f, 0.f, 0.f};
    if (any && orc_project_ok(po, q, ls, cam)) {
      const float dx = po[0] - cam->pos[0], dy = po[1] - cam->pos[1], dz = po[2] - cam->pos[2];
      const float idl = 1.f / sqrtf((dx * dx + dy * dy) + dz * dz);
      float b[25];
      orc_sh_basis_f(m->degree, dx * idl, dy * idl, dz * idl, b);
      for (int k = 0; k < K; k++) {
        const float y = k < kmax ? b[k] : 0.f;
        bsq = bsq + y * y;
      }
      vc[0] = g[5]; vc[1] = g[6]; vc[2] = g[7];
    }
    const float* G = grads + (size_t)i * per;
    /* optim.cu:142 and 298-308: the steps skipped since the last update (sparse mode) */
    catch_up_t cu = {0.f, 1.f, 1.f, 0.f};
    if (s->sparse) {
      const uint32_t last = m->last_step[i];
      cu.skipped = last == 0u ? 0.f : fmaxf(((float)s->t - (float)last) - 1.f, 0.f);
      m->last_step[i] = (uint32_t)s->t;
      if (cu.skipped > 0.f) {
        cu.d1 = orc_expf(cu.skipped * s->ln_beta1);
        cu.d2 = orc_expf(cu.skipped * s->ln_beta2);
        cu.drift = (s->ratio * (1.f - orc_expf(cu.skipped * s->ln_ratio))) / (1.f - s->ratio);
      }
    }
    /* optim.cu:316-335: means and opacity logit, rotation, log scales (floor lane kept, its moments zero) */
    const float lr_po[4] = {s->lr_mean, s->lr_mean, s->lr_mean, s->lr_opac};
    for (int c = 0; c < 4; c++)
      adam_param(&po[c], &m->m_pos_op[4 * (size_t)i + c], &m->v_pos_op[4 * (size_t)i + c], G[c], lr_po[c], s, &cu);
    for (int c = 0; c < 4; c++)
      adam_param(&q[c], &m->m_quat[4 * (size_t)i + c], &m->v_quat[4 * (size_t)i + c], G[4 + c], s->lr_rot, s, &cu);
    for (int c = 0; c < 3; c++)
      adam_param(&ls[c], &m->m_lscale[4 * (size_t)i + c], &m->v_lscale[4 * (size_t)i + c], G[8 + c], s->lr_scale, s,
                 &cu);
    m->m_lscale[4 * (size_t)i + 3] = 0.f;
    m->v_lscale[4 * (size_t)i + 3] = 0.f;
    /* optim.cu:336-359: SH, one second moment per splat */
    {
      const float gsq = (bsq * ((vc[0] * vc[0] + vc[1] * vc[1]) + vc[2] * vc[2])) * (1.f / (float)(3 * K));
      float vsh = m->v_sh[i] * cu.d2;
      const float denom_old = cu.skipped > 0.f ? (cu.drift * s->bc1) / (sqrtf(vsh * s->bc2) + s->eps) : 0.f;
      vsh = s->beta2 * vsh + (1.f - s->beta2) * gsq;
      m->v_sh[i] = vsh;
      const float denom = s->bc1 / (sqrtf(vsh * s->bc2) + s->eps);
      const uint32_t sr_seed = (s->seed ^ (s->step * 0x9E3779B9u)) ^ 0x5A5A5A5Au;
      for (int lane = 0; lane < 3 * K; lane++) {
        const float lrk = lane < 3 ? s->lr_dc : s->lr_sh_rest;
        float* P = m->sh + (size_t)i * 3 * K + lane;
        float* M = m->m_sh + (size_t)i * 3 * K + lane;
        float p = *P, mo = *M;
        if (cu.skipped > 0.f) {
          p = p - (lrk * denom_old) * mo;
          mo = mo * cu.d1;
        }
        mo = s->beta1 * mo + (1.f - s->beta1) * G[11 + lane];
        p = p - (lrk * denom) * mo;
        if (lane >= 3 && m->sh_half) {
          *M = orc_f16_value(orc_f16_bits(mo));
          *P = orc_f16_value(orc_f16_stochastic(p, orc_hash_unit(sr_seed, (uint32_t)i, (uint32_t)lane)));
        } else {
          *M = mo;
          *P = p;
        }
      }
    }
    /* optim.cu:361-375: MCMC noise on the means of visible splats, from the updated logit and scales */
    if (s->noise_weight > 0.f && visible) {
      const float sig = 1.f / (1.f + orc_expf(-po[3]));
      float comp = 1.f;
      if (ls[3] > 0.f) {
        const float f2 = ls[3] * ls[3];
        const float vx = orc_expf(2.f * ls[0]), vy = orc_expf(2.f * ls[1]), vz = orc_expf(2.f * ls[2]);
        comp = sqrtf(((vx / (vx + f2)) * (vy / (vy + f2))) * (vz / (vz + f2)));
      }
      const float o = fminf(fmaxf(sig * comp, 0.f), 1.f);
      const float w = fminf(fmaxf(orc_expf(150.f * orc_logf(1.f - o)), 0.f), 1.f) * s->noise_weight;
      if (w > 0.f) {
        const uint32_t ns = s->seed ^ (s->step * 0x9E3779B9u);
        const float cl = s->noise_clamp;
        for (int c = 0; c < 3; c++) po[c] = po[c] + fminf(fmaxf(orc_hash_gauss(ns, (uint32_t)i, (uint32_t)c) * w, -cl), cl);
      }
    }
  }
}
