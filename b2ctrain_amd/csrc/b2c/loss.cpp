// Loss entry points (replaces src/gpu/loss.cu:296-338).
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
  // a sum still pending here belonged to a step that failed before its VJP: this loss replaces it
  ctx.loss_pending = 0;
  if (lp.defer_sum) a.defer_sum_count = &ctx.loss_pending;
  LAUNCH_CHECK(b2c_hip_photometric(&a, stream));
  ctx.loss_pending_assign = a.assign;
  ctx.loss_pending_running = a.running;
}

void accumulate_loss(RenderCtx& ctx, hipStream_t stream) { LAUNCH_CHECK(b2c_hip_accumulate_loss(ctx.loss_accum.ptr, stream)); }

void normal_loss(RenderCtx& ctx, const ViewGPU& view, const LossParams& lp, hipStream_t stream) {
  if (!view.normals) throw std::runtime_error("normal_loss: the view has no normal map");
  b2c_normal_loss_args a{};
  a.feat = reinterpret_cast<const float*>(ctx.out_feat.ptr);
  a.normals = view.normals;
  a.weights = view.weights;
  a.W = ctx.W; a.H = ctx.H;
  a.scale = lp.normal_scale;
  a.grad_scale = lp.grad_scale;
  a.v_feat = reinterpret_cast<float*>(ctx.v_feat.ptr);
  a.loss_accum = ctx.loss_accum.ptr;
  a.partials = ctx.aux_partials.ptr;
  LAUNCH_CHECK(b2c_hip_normal_loss(&a, stream));
}

void hollow_loss(RenderCtx& ctx, float lam, hipStream_t stream) {
  LAUNCH_CHECK(b2c_hip_hollow_loss(ctx.hollow_pen.ptr, ctx.W, ctx.H, lam, ctx.loss_accum.ptr, ctx.aux_partials.ptr,
                                   stream));
}

void eval_metrics(RenderCtx& ctx, const ViewGPU& view, bool mask_weighted, hipStream_t stream) {
  b2c_eval_args a{};
  a.pred = reinterpret_cast<const float*>(ctx.out_rgba.ptr);
  a.gt = view.rgba;
  a.W = ctx.W; a.H = ctx.H;
  a.mask_weighted = mask_weighted ? 1 : 0;
  a.loss_accum = ctx.loss_accum.ptr;
  a.partials = ctx.aux_partials.ptr;
  LAUNCH_CHECK(b2c_hip_eval_metrics(&a, stream));
}

}  // namespace b2c
