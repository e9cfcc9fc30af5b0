// optimizer_step (replaces src/gpu/optim.cu:379-392 and the kernel body 99-377): one launch of the fused
// VJP kernel (kernels/vjp.hip), in gradient mode when grad_out is set, else in update mode.
#include "optim.h"

namespace b2c {

void optimizer_step(RenderCtx& ctx, Model& m, const OptimParams& op, hipStream_t stream) {
  if (m.n == 0) return;
  if (op.mip || op.pos_override || op.quat_override || op.lscale_override || op.sh_frame || op.canon_rot || op.spa_z ||
      op.stretch_w || op.g_app_out || op.g_pos_out || op.frozen || op.update_mask)
    throw std::runtime_error("optimizer_step: deformation / sparsify / appearance extensions are not supported by this build");
  if (m.degree < 0 || m.degree > 4) throw std::runtime_error("bad degree");
  b2c_vjp_args a{};
  a.n = m.n; a.degree = m.degree; a.active_deg = op.active_sh_degree;
  a.pos_op = reinterpret_cast<float*>(m.pos_op.ptr);
  a.quat = reinterpret_cast<float*>(m.quat.ptr);
  a.lscale = reinterpret_cast<float*>(m.lscale.ptr);
  a.sh = m.sh().view();
  a.cam = op.cam.dev();
  a.v_splat = ctx.v_splat;
  a.vis_flag = ctx.vis_flag;
  a.tile_count = ctx.tile_count;
  a.grad_out = op.grad_out;
  a.accumulate = op.grad_accumulate ? 1 : 0;
  a.sparse = op.sparse ? 1 : 0;
  a.refine_norm = m.refine_norm.ptr;
  a.vis_count = m.vis_count.ptr;
  a.vis_from_row = ctx.vis_in_rows ? 1 : 0;
  if (ctx.loss_pending) {
    a.loss_partials = ctx.loss_partials.ptr;
    a.loss_count = ctx.loss_pending;
    a.loss_assign = ctx.loss_pending_assign;
    a.loss_running = ctx.loss_pending_running;
    a.loss_accum = ctx.loss_accum.ptr;
  }
  a.vis_weight = m.vis_weight.ptr;
  if (!op.grad_out) {
    if (op.t < 1) throw std::runtime_error("optimizer_step: the Adam step t must be >= 1");
    if (!(op.beta1 >= 0.f && op.beta1 < 1.f && op.beta2 > 0.f && op.beta2 < 1.f))
      throw std::runtime_error("optimizer_step: beta1 must lie in [0, 1) and beta2 in (0, 1)");
    const ShBuf sh = m.sh();
    a.sh_out = b2c_sh_planes{sh.dc, m.sh_fp16 ? sh.hi : nullptr, m.sh_fp16 ? nullptr : sh.hi32, sh.stride};
    a.sh.hi16 = a.sh_out.hi16;
    a.sh.hi32 = a.sh_out.hi32;
    a.adam = m.adam_state();
    b2c_adam_step& s = a.step;
    s.t = op.t;
    s.sparse = op.sparse ? 1 : 0;
    s.beta1 = op.beta1; s.beta2 = op.beta2; s.eps = op.eps;
    s.lr_mean = op.lr_mean; s.lr_rot = op.lr_rot; s.lr_scale = op.lr_scale; s.lr_opac = op.lr_opac;
    s.lr_dc = op.lr_dc; s.lr_sh_rest = op.lr_sh_rest;
    s.noise_weight = op.noise_weight; s.noise_clamp = op.noise_clamp;
    s.seed = op.seed; s.step = op.step;
    b2c_adam_step_constants(&s);
  }
  LAUNCH_CHECK(b2c_hip_vjp(&a, stream));
  ctx.loss_pending = 0;
  // every row a backward wrote came with its splat's vis_flag (or, deferred, its lane-10 weight), and the
  // VJP cleared those rows
  ctx.v_splat_zero = true;
  ctx.vis_in_rows = false;
}

}  // namespace b2c
