// Fixed-order double-precision sum of the photometric loss's per-workgroup partials into loss_accum, by one
// wave: lane l adds entries l, l + 64, ... in order, the lanes' sums meet in an xor butterfly, and lane 0's
// total is stored. The loss's own reduction launch and the fused training step (which hands the sum to the
// projection VJP's first workgroup instead of a launch of its own) both use it, so they give the same value.
#pragma once
#include "device_math.h"

namespace b2c {
namespace dev {

// assign: loss_accum[0] = loss, [1] = 0 (else [0] += loss); running (with assign): also [2] = [0] + [1] and
// [3] = 1, what the trainer's per-step clear and accumulate_kernel leave (loss.cu:317,324). Every lane of the
// wave must call it.
__device__ __forceinline__ void loss_partials_store(const float* __restrict__ partials, int count,
                                                    float* __restrict__ loss_accum, int assign, int running) {
  double acc = 0.0;
  for (int i = lane_id(); i < count; i += 64) acc += (double)partials[i];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane_id() == 0) {
    if (assign) {
      loss_accum[0] = (float)acc;
      loss_accum[1] = 0.f;
      if (running) {
        loss_accum[2] = loss_accum[0] + loss_accum[1];
        loss_accum[3] = 1.f;
      }
    } else {
      loss_accum[0] = (float)((double)loss_accum[0] + acc);
    }
  }
}

}  // namespace dev
}  // namespace b2c
