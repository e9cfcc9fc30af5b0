// optimizer_step, gradient path (replaces src/gpu/optim.cu:434-442 launch + 99-253, 292-296).
#include "optim.h"

namespace b2c {

void optimizer_step(RenderCtx& ctx, Model& m, const OptimParams& op, hipStream_t stream) {
  if (m.n == 0) return;
  if (!op.grad_out) throw std::runtime_error("optimizer_step: the Adam update is not part of this build (set grad_out)");
  if (op.mip || op.pos_override || op.quat_override || op.lscale_override || op.sh_frame || op.canon_rot || op.spa_z ||
      op.stretch_w || op.g_app_out || op.g_pos_out)
    throw std::runtime_error("optimizer_step: deformation / sparsify / appearance extensions are not supported by this build");
  if (m.degree < 0 || m.degree > 4) throw std::runtime_error("bad degree");
  b2c_vjp_args a{};
  a.n = m.n; a.degree = m.degree; a.active_deg = op.active_sh_degree;
  a.pos_op = reinterpret_cast<const float*>(m.pos_op.ptr);
  a.quat = reinterpret_cast<const float*>(m.quat.ptr);
  a.lscale = reinterpret_cast<const float*>(m.lscale.ptr);
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
  LAUNCH_CHECK(b2c_hip_vjp(&a, stream));
}

}  // namespace b2c
