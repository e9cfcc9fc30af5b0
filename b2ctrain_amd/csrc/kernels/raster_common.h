// Helpers shared by the forward and backward raster kernels.
#pragma once
#include "device_math.h"

namespace b2c {
namespace dev {

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X (workgroup b runs on XCD b % 8), and
// each XCD has its own L2. Give every XCD a contiguous run of tiles (rows of the image) so splats shared
// by neighbouring tiles are fetched once per XCD rather than once per tile. The grid has 8 * per blocks;
// blocks mapped past n_tiles return.
constexpr int NUM_XCD = 8;
__host__ __device__ inline int xcd_tiles_per(int n_tiles) { return (n_tiles + NUM_XCD - 1) / NUM_XCD; }
__device__ __forceinline__ int xcd_tile(int block, int n_tiles) {
  const int per = xcd_tiles_per(n_tiles);
  return (block % NUM_XCD) * per + block / NUM_XCD;
}

constexpr float LOG2E = 1.44269504088896341f;

// e^-sigma on the hardware exponential (v_exp_f32 is 2^x): the Gaussian factor of the opacity gradient.
__device__ __forceinline__ float gauss_weight(float sigma) { return __builtin_amdgcn_exp2f(sigma * -LOG2E); }

// log2 of a splat's opacity, precomputed once per splat for fragment_alpha.
__device__ __forceinline__ float log2_opacity(float opacity) { return __builtin_amdgcn_logf(opacity); }

// Unclamped alpha of a fragment, opacity * e^-sigma, as 2^(log2(opacity) - sigma log2 e): one fma and one
// v_exp_f32. Forward and backward must use this same expression: the backward recovers the forward's
// transmittance by dividing by (1 - alpha).
__device__ __forceinline__ float fragment_alpha(float sigma, float log2_op) {
  return __builtin_amdgcn_exp2f(__builtin_fmaf(sigma, -LOG2E, log2_op));
}

}  // namespace dev
}  // namespace b2c
