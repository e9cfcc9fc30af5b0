// Pieces shared by the SSIM kernels (the fused photometric loss in loss.hip, the eval metrics in
// aux_loss.hip): the 11-tap Gaussian window (sigma 1.5, loss.cu:296-303), the SSIM constants and the
// packed-RGBA8 channel decode (loss.cu:15).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace b2c {
namespace dev {

constexpr int HALO = 5;
constexpr float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;

// The 11 weights (double-precision exp(-d^2 / 4.5) normalised to sum 1, rounded to float), as compile-time
// constants: passed as kernel arguments they took 11 scalar registers and the kernel spilled others. The
// photometric launcher checks them bitwise against its own computation.
constexpr uint32_t GW_BITS[11] = {0x3a86cab6u, 0x3bf8ff01u, 0x3d13758cu, 0x3ddff87fu, 0x3e5a1e20u, 0x3e8832b0u,
                                  0x3e5a1e20u, 0x3ddff87fu, 0x3d13758cu, 0x3bf8ff01u, 0x3a86cab6u};
__device__ __forceinline__ float gw_tap(int d) { return __uint_as_float(GW_BITS[d]); }

__device__ __forceinline__ float gt_channel(uint32_t packed, int c) {
  return (float)((packed >> (8 * c)) & 0xffu) * (1.f / 255.f);
}

}  // namespace dev
}  // namespace b2c
