// Device helpers of the fused Adam update (vjp.hip): counter-based random numbers, Gaussian samples and
// the stochastically rounded fp16 store of the SH bands. All of it is integer work or single-precision
// arithmetic evaluated without FMA contraction with IEEE square root and the Cephes exp/log of
// device_math.h, so the CPU restatement (oracle/orc_adam.c) reproduces every output bit for bit.
#pragma once
#include "device_math.h"

namespace b2c {
namespace dev {

// The random streams are the reference's (src/gpu/util.cuh:106-117), so one seed gives the same noise and
// rounding decisions: a 32-bit finaliser (xor-shift / multiply, "lowbias32" from C. Wellons'
// hash-prospector) applied in a chain over three counters, the top 24 bits scaled into [0, 1).
__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

__device__ __forceinline__ float hash_unit(uint32_t a, uint32_t b, uint32_t c) {
  const uint32_t h = mix32((a * 0x9E3779B1u) ^ mix32((b * 0x85EBCA77u) ^ mix32(c * 0xC2B2AE3Du)));
  return (float)(h >> 8) * (1.f / 16777216.f);
}

// cos(2 pi u) for u in [0, 1). The argument is reduced exactly in turns (each subtraction below is exact by
// Sterbenz's lemma): to t in [-1/2, 1/2), by symmetry to a in [0, 1/4], then to at most 1/8 turn (pi / 4),
// where the Cephes single-precision polynomials for cos and sin (S. L. Moshier, single/sinf.c) apply.
__device__ __forceinline__ float cos_turns(float u) {
#pragma clang fp contract(off)
  const float t = u >= 0.5f ? u - 1.f : u;
  float a = fabsf(t);
  float sign = 1.f;
  if (a > 0.25f) {  // cos(2 pi a) = -cos(2 pi (1/2 - a))
    a = 0.5f - a;
    sign = -1.f;
  }
  const float two_pi = 6.28318530717958647692f;
  float r;
  if (a > 0.125f) {  // cos(2 pi a) = sin(2 pi (1/4 - a))
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

// A standard normal sample by the Box-Muller transform of two uniforms drawn at counters c and
// c + 0x1234567 (the reference's pairing, util.cuh:114-117), u1 floored at 1e-7.
__device__ __forceinline__ float hash_gauss(uint32_t a, uint32_t b, uint32_t c) {
#pragma clang fp contract(off)
  const float u1 = fmaxf(hash_unit(a, b, c), 1e-7f), u2 = hash_unit(a, b, c + 0x1234567u);
  return sqrtf(-2.f * det_logf(u1)) * cos_turns(u2);
}

// IEEE binary16 bit patterns.
__device__ __forceinline__ uint16_t f16_bits(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }
__device__ __forceinline__ float f16_value(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// The next binary16 value toward +inf (up) or -inf: one step of the magnitude bits, across zero to the
// smallest subnormal of the other sign.
__device__ __forceinline__ uint16_t f16_next(uint16_t h, bool up) {
  if ((h & 0x7fffu) == 0u) return up ? (uint16_t)0x0001u : (uint16_t)0x8001u;
  const bool neg = (h & 0x8000u) != 0u;
  return (uint16_t)(up != neg ? h + 1u : h - 1u);
}

// Stochastic rounding to binary16 (util.cuh:148-162): v, clamped to +-65000, goes to its lower neighbour
// lo or upper neighbour hi with P(hi) = (v - lo) / (hi - lo), so the stored value is v in expectation. An
// update far below half an fp16 ulp (the 2e-4 SH learning rate against coefficients above ~0.25) then still
// moves the coefficient on average, where round-to-nearest would freeze it. u01 is uniform in [0, 1).
__device__ __forceinline__ uint16_t f16_stochastic(float v, float u01) {
#pragma clang fp contract(off)
  v = fminf(fmaxf(v, -65000.f), 65000.f);
  uint16_t h = f16_bits(v);  // nearest; step down when it lies above v, so h is the lower neighbour
  float lo = f16_value(h);
  if (lo > v) {
    h = f16_next(h, false);
    lo = f16_value(h);
  }
  if (lo != v) {
    const uint16_t up = f16_next(h, true);
    if (u01 * (f16_value(up) - lo) < v - lo) h = up;
  }
  return h;
}

}  // namespace dev
}  // namespace b2c
