// Optimizer API of the drop-in (replaces src/gpu/optim.h:1-52). optimizer_step runs the projection VJP
// and then either writes [n][11 + 3K] parameter gradients (pos3, opacity, quat4, log-scale3, SH) when
// grad_out is set (the reference's test path, optim.cu:292-296), or applies the fused update: Adam with
// bias correction, the lazy catch-up of sparse Adam, the SH moments with stochastically rounded fp16 bands,
// and MCMC noise on the means (optim.cu:298-377). The cage / sparsify / appearance extensions
// (pos_override .. g_app_out) are outside this build and throw when requested.
#pragma once
#include "render.h"

namespace b2c {

struct OptimParams {
  CameraGPU cam;
  bool mip = false;
  int active_sh_degree = 3;
  int t = 1;
  float beta1 = 0.9f, beta2 = 0.999f, eps = 1e-15f;
  float lr_mean = 0.f;
  float lr_rot = 2e-3f, lr_scale = 5e-3f, lr_opac = 0.012f, lr_dc = 2e-3f, lr_sh_rest = 2e-4f;
  float noise_weight = 0.f;
  float noise_clamp = 0.f;
  uint32_t seed = 42, step = 0;
  const float4* pos_override = nullptr;
  float3* g_pos_out = nullptr;
  const float4* quat_override = nullptr;
  const float4* lscale_override = nullptr;
  const float4* sh_frame = nullptr;
  bool frozen = false;
  const uint8_t* update_mask = nullptr;
  const float4* canon_rot = nullptr;
  bool sparse = false;
  const float* spa_z = nullptr; const float* spa_u = nullptr; float spa_rho = 0.f;
  const float* stretch_w = nullptr; float stretch_log_tau = 0.f;
  float2* g_app_out = nullptr;
  float* grad_out = nullptr;  // write parameter gradients [n][11 + K*3] and skip the update
  bool grad_accumulate = false;  // this build: add into grad_out (gradients summed over several views)
};

// Projection backward + update; consumes and clears ctx.v_splat / ctx.vis_flag; updates Model::vis_count /
// refine_norm. Without grad_out it writes the model's parameters and Adam state (op.t >= 1).
void optimizer_step(RenderCtx& ctx, Model& m, const OptimParams& op, hipStream_t stream);

}  // namespace b2c
