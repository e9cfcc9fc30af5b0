// Loss API of the drop-in (replaces src/gpu/loss.h:1-43): the fused photometric loss, the normal-map loss
// of the feature lanes, the hollow-penalty sum and the eval metrics.
#pragma once
#include "render.h"

namespace b2c {

// ViewGPU (loss.h:7-18): device pointers of one training image. The field set is the reference's; this
// build reads rgba, normals and weights.
struct ViewGPU {
  const uint32_t* rgba = nullptr;     // target pixels, r | g << 8 | b << 16 | a << 24; colour already scaled by a
                                      // when the view carries transparency
  const uint32_t* normals = nullptr;  // normal map, packed RGBA8 (normal_loss); alpha above 127 marks supervised pixels
  const uint8_t* weights = nullptr;   // per-pixel weight byte, weight = byte / 255 (times LossParams::scale);
                                      // nullptr: weight 1
  const uint8_t* labels = nullptr;    // evidence-pass input (not read here)
  int W = 0, H = 0;
  bool has_alpha = false, masked = false;
  float alpha_coverage = 1.f;
  float normal_count = 0.f;
  const float2* warp = nullptr;       // render-side alignment field (not supported here)
  int warp_w = 0, warp_h = 0;
};

// LossParams (loss.h:20-30), plus two flags of this build for the fused training step.
struct LossParams {
  float l1_w = 0.8f, ssim_w = -0.2f;  // weights of |p - g| and of SSIM; the trainer passes 1 - w and -w
  float bg[3] = {0, 0, 0};            // background the target is composited over when `composite`
  bool composite = false;             // target colour becomes g + (1 - g.a) bg
  bool mask = false;                  // each pixel's loss is multiplied by the target's alpha
  bool alpha_lane = false;            // adds match_alpha_weight |p.a - g.a| (not masked)
  float match_alpha_weight = 0.1f;
  float scale = 1.f;                  // factor on the photometric terms, applied where the weight is
  float normal_scale = 0.f;           // weight of normal_loss (the trainer's normal_loss_weight * every / count)
  float grad_scale = 1.f;             // factor on v_out only; the loss value is unscaled
  bool assign_loss = false;           // loss_accum[0] = this loss and loss_accum[1] = 0, instead of adding
  bool running_sum = false;           // with assign_loss: loss_accum[2] = loss_accum[0] + loss_accum[1] and
                                      // loss_accum[3] = 1 in the same launch, which is what the trainer's
                                      // per-step clear of [0..3] followed by accumulate_loss leaves
  bool defer_sum = false;             // this build: leave the reduction of the per-workgroup partials to the
                                      // next optimizer_step on the context (ctx.loss_pending), which runs it in
                                      // the VJP's first workgroup instead of a launch of its own
};

// Fused L1 + SSIM (+ alpha lane): per-pixel gradient into ctx.v_out, the loss added to ctx.loss_accum[0]
// (see assign_loss / running_sum).
void photometric_loss(RenderCtx& ctx, const ViewGPU& view, const LossParams& lp, hipStream_t stream);
// Normal-map supervision of the feature lanes (render with FeatureMode::Normals): scale * weight * (L1 +
// 1 - cos) over the pixels the map marks, gradient (times grad_scale) into ctx.v_feat, loss added to
// ctx.loss_accum[1].
void normal_loss(RenderCtx& ctx, const ViewGPU& view, const LossParams& lp, hipStream_t stream);
// loss_accum[2] += loss_accum[0] + loss_accum[1]; loss_accum[3] += 1.
void accumulate_loss(RenderCtx& ctx, hipStream_t stream);
// loss_accum[0] += lam * sum of ctx.hollow_pen (the forward's per-pixel penalties; the gradient is taken in
// the raster backward).
void hollow_loss(RenderCtx& ctx, float lam, hipStream_t stream);
// Metrics of the current render against the view: loss_accum[4] += sum over pixels and channels of the
// squared error of the 8-bit prediction, loss_accum[5] += sum of its SSIM (alpha-weighted when
// mask_weighted).
void eval_metrics(RenderCtx& ctx, const ViewGPU& view, bool mask_weighted, hipStream_t stream);

}  // namespace b2c
