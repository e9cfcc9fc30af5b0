// Loss entry points (replaces src/gpu/loss.cu:296-380).
#include "loss.h"

namespace b2c {

void photometric_loss(RenderCtx& ctx, const ViewGPU& view, const LossParams& lp, hipStream_t stream) {
  if (view.warp) throw std::runtime_error("photometric_loss: view warp fields are not supported by this build");
  b2c_loss_args a{};
  a.pred = reinterpret_cast<const float*>(ctx.out_rgba.ptr);
  a.gt = view.rgba;
  a.weights = view.weights;
  a.W = ctx.W; a.H = ctx.H;
  a.l1_w = lp.l1_w; a.ssim_w = lp.ssim_w;
  for (int k = 0; k < 3; k++) a.bg[k] = lp.bg[k];
  a.composite = lp.composite; a.mask = lp.mask; a.alpha_lane = lp.alpha_lane;
  a.match_alpha_weight = lp.match_alpha_weight; a.scale = lp.scale; a.grad_scale = lp.grad_scale;
  a.v_out = reinterpret_cast<float*>(ctx.v_out.ptr);
  a.loss_accum = ctx.loss_accum.ptr;
  a.partials = ctx.loss_partials.ptr;
  a.assign = lp.assign_loss ? 1 : 0;
  a.running = lp.running_sum ? 1 : 0;
  LAUNCH_CHECK(b2c_hip_photometric(&a, stream));
}

void accumulate_loss(RenderCtx& ctx, hipStream_t stream) { LAUNCH_CHECK(b2c_hip_accumulate_loss(ctx.loss_accum.ptr, stream)); }

void normal_loss(RenderCtx&, const ViewGPU&, const LossParams&, hipStream_t) {
  throw std::runtime_error("normal_loss: feature lanes are not supported by this build");
}
void hollow_loss(RenderCtx&, float, hipStream_t) {
  throw std::runtime_error("hollow_loss: not supported by this build");
}
void eval_metrics(RenderCtx&, const ViewGPU&, bool, hipStream_t) {
  throw std::runtime_error("eval_metrics: not supported by this build");
}

}  // namespace b2c
