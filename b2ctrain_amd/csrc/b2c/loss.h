// Loss API of the drop-in (replaces src/gpu/loss.h:1-43). normal_loss, hollow_loss and eval_metrics keep
// their signatures and throw: feature lanes and evaluation are outside this build.
#pragma once
#include "render.h"

namespace b2c {

// A training view resident on the GPU (loss.h:7-18).
struct ViewGPU {
  const uint32_t* rgba = nullptr;     // packed RGBA8 (premultiplied for transparent views)
  const uint32_t* normals = nullptr;
  const uint8_t* weights = nullptr;   // per-pixel loss weight (w / 255) or nullptr
  const uint8_t* labels = nullptr;
  int W = 0, H = 0;
  bool has_alpha = false, masked = false;
  float alpha_coverage = 1.f;
  float normal_count = 0.f;
  const float2* warp = nullptr;
  int warp_w = 0, warp_h = 0;
};

struct LossParams {
  float l1_w = 0.8f, ssim_w = -0.2f;  // brush: (1 - ssim_weight), -ssim_weight
  float bg[3] = {0, 0, 0};
  bool composite = false;             // gt_eff = gt + (1 - gt.a) * bg
  bool mask = false;                  // multiply the loss map by gt.a
  bool alpha_lane = false;            // add match_alpha_weight * |pred.a - gt.a|
  float match_alpha_weight = 0.1f;
  float scale = 1.f;                  // multiplier on the whole photometric loss
  float normal_scale = 0.f;
  float grad_scale = 1.f;             // multiplies the per-pixel gradients (not the loss value)
  bool assign_loss = false;           // store into loss_accum[0] (and clear [1]) instead of adding
  bool running_sum = false;           // with assign_loss: also apply accumulate_loss's update in the same launch
};

// Fused L1 + SSIM (+ alpha lane): gradient into ctx.v_out, loss added to ctx.loss_accum[0] (stored, with
// loss_accum[1] cleared, when lp.assign_loss).
void photometric_loss(RenderCtx& ctx, const ViewGPU& view, const LossParams& lp, hipStream_t stream);
void normal_loss(RenderCtx& ctx, const ViewGPU& view, const LossParams& lp, hipStream_t stream);
// loss_accum[2] += loss_accum[0] + loss_accum[1]; loss_accum[3] += 1.
void accumulate_loss(RenderCtx& ctx, hipStream_t stream);
void hollow_loss(RenderCtx& ctx, float lam, hipStream_t stream);
void eval_metrics(RenderCtx& ctx, const ViewGPU& view, bool mask_weighted, hipStream_t stream);

}  // namespace b2c
