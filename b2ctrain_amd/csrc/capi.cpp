// C ABI over the C++ drop-in API (declared in include/b2c.h).
#include "b2c.h"

#include <algorithm>
#include <cstring>
#include <vector>
#include <map>
#include <string>

#include "b2c/dataset.h"
#include "b2c/evidence.h"
#include "b2c/loss.h"
#include "b2c/optim.h"
#include "b2c/ply.h"
#include "b2c/png.h"
#include "b2c/resample.h"
#include "b2c/render.h"

struct b2c_model {
  b2c::Model m;
};

struct b2c_ctx {
  b2c::RenderCtx ctx;
  hipStream_t stream = nullptr;
  b2c::DevBuf<float> grads;
  int n = 0;
  int degree = 0;
  hipEvent_t ev[8] = {};
};

struct b2c_dataset {
  b2c::Dataset ds;
};

struct b2c_view {
  b2c::DevBuf<uint32_t> rgba, normals;
  b2c::DevBuf<uint8_t> weights, labels;
  b2c::ViewGPU view;
};

namespace {

thread_local std::string g_err;

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  } catch (...) {
    g_err = "unknown error";
    return -1;
  }
}

b2c::Camera to_camera(const b2c_camera& c) {
  b2c::Camera cam;
  cam.width = c.width; cam.height = c.height;
  cam.fx = c.fx; cam.fy = c.fy; cam.cx = c.cx; cam.cy = c.cy;
  for (int i = 0; i < 9; i++) cam.R[i] = c.R[i];
  for (int i = 0; i < 3; i++) cam.t[i] = c.t[i];
  cam.update_pos();
  return cam;
}

int train_step(b2c_ctx* c, b2c_model* m, const b2c_view* v, const b2c_render_opts* ro, const b2c_loss_opts* lo,
               int mode, int flags, const b2c_adam_opts* adam, b2c_step_times* times);
b2c::RenderParams to_params(const b2c_render_opts& o);

// OptimParams of an update step (optim.h:6-20 fields; op.t = ++model.adam_t when t is 0, trainer.cpp:512).
b2c::OptimParams to_optim(const b2c_render_opts& ro, const b2c_adam_opts& a, b2c::Model& m) {
  b2c::OptimParams op;
  op.cam = to_params(ro).cam;
  op.active_sh_degree = ro.sh_degree;
  if (a.t < 0) throw std::runtime_error("optimizer_step: negative Adam step");
  if (!(a.beta1 >= 0.f && a.beta1 < 1.f && a.beta2 > 0.f && a.beta2 < 1.f))
    throw std::runtime_error("optimizer_step: beta1 must lie in [0, 1) and beta2 in (0, 1)");
  op.t = a.t > 0 ? a.t : m.adam_t + 1;
  m.adam_t = op.t;
  op.beta1 = a.beta1; op.beta2 = a.beta2; op.eps = a.eps;
  op.lr_mean = a.lr_mean; op.lr_rot = a.lr_rot; op.lr_scale = a.lr_scale; op.lr_opac = a.lr_opac;
  op.lr_dc = a.lr_dc; op.lr_sh_rest = a.lr_sh_rest;
  op.noise_weight = a.noise_weight; op.noise_clamp = a.noise_clamp;
  op.seed = a.seed; op.step = a.step;
  op.sparse = a.sparse != 0;
  return op;
}

b2c::RenderParams to_params(const b2c_render_opts& o) {
  b2c::RenderParams p;
  p.cam = b2c::CameraGPU::from(to_camera(o.cam), o.W, o.H);
  for (int k = 0; k < 3; k++) p.bg[k] = o.bg[k];
  p.sh_degree = o.sh_degree;
  p.bwd_info = o.bwd_info != 0;
  if (o.feat_mode < 0 || o.feat_mode > 2) throw std::runtime_error("render opts: feat_mode must be 0, 1 or 2");
  p.feat = o.feat_mode == 1 ? b2c::FeatureMode::Normals : (o.feat_mode == 2 ? b2c::FeatureMode::Buffer : b2c::FeatureMode::None);
  p.feat_buffer = o.feat_buffer;
  p.hollow_z = o.hollow_z;
  p.hollow_margin = o.hollow_margin;
  p.hollow_lam = o.hollow_lam;
  return p;
}

b2c::LossParams to_loss(const b2c_loss_opts& o) {
  b2c::LossParams lp;
  lp.l1_w = o.l1_w; lp.ssim_w = o.ssim_w;
  for (int k = 0; k < 3; k++) lp.bg[k] = o.bg[k];
  lp.composite = o.composite != 0; lp.mask = o.mask != 0; lp.alpha_lane = o.alpha_lane != 0;
  lp.match_alpha_weight = o.match_alpha_weight; lp.scale = o.scale; lp.grad_scale = o.grad_scale;
  lp.normal_scale = o.normal_scale;
  return lp;
}

struct Field {
  void* ptr;
  size_t bytes;
};

Field ctx_field(b2c_ctx* c, const std::string& name) {
  b2c::RenderCtx& x = c->ctx;
  const size_t n = (size_t)c->n;
  const size_t P = (size_t)x.W * x.H;
  const size_t M = x.num_isect;
  std::map<std::string, Field> f = {
      {"proj0", {x.proj0.ptr, n * 16}},
      {"proj1", {x.proj1.ptr, n * 16}},
      {"proj2", {x.proj2.ptr, n * 16}},
      {"proj3", {x.proj3.ptr, n * 8}},
      {"raster_rec", {x.raster_rec.ptr, n * 64}},
      {"tile_count", {x.tile_count.ptr, n * 4}},
      {"tile_off", {x.tile_off.ptr, n * 4}},
      {"hit_info", {x.hit_info.ptr, n * 8}},
      {"hit_wide", {x.hit_wide.ptr, n * 8}},
      {"order", {x.order.ptr, n * 4}},
      {"depth_keys_sorted", {x.depth_keys_sorted.ptr, n * 4}},
      {"keys", {x.keys.ptr, M * 4}},
      {"vals", {x.vals.ptr, M * 4}},
      {"keys_sorted", {x.keys_sorted.ptr, M * 4}},
      {"vals_sorted", {x.vals_sorted.ptr, M * 4}},
      {"tile_ranges", {x.tile_ranges.ptr, (size_t)x.n_tiles * 8}},
      {"out_rgba", {x.out_rgba.ptr, P * 16}},
      {"out_feat", {x.out_feat.ptr, P * 16}},
      {"v_feat", {x.v_feat.ptr, P * 16}},
      {"hollow_pen", {x.hollow_pen.ptr, P * 4}},
      {"last_idx", {x.last_idx.ptr, P * 4}},
      {"v_out", {x.v_out.ptr, P * 16}},
      {"v_splat", {x.v_splat.ptr, n * b2c::GRAD_LANES * 4}},
      {"vis_flag", {x.vis_flag.ptr, n * 4}},
      {"loss_accum", {x.loss_accum.ptr, 16 * 4}},
      {"grads", {c->grads.ptr, c->grads.bytes()}},
      {"big_list", {x.big_list.ptr, n * 4}},
      {"big_base", {x.big_base.ptr, n * 4}},
      {"counters", {x.counters.ptr, x.counters.bytes()}},
      {"slot_sorted", {x.slot_sorted.ptr, M * 4}},
      {"cvals", {x.cvals.ptr, M * 4}},
      {"cslots", {x.cslots.ptr, M * 4}},
      {"clast", {x.clast.ptr, P * 4}},
      {"cend", {x.cend.ptr, (size_t)x.n_tiles * 4}},
      {"tile_end", {x.tile_end.ptr, ((size_t)x.n_tiles + 1) * 4}},
      {"isect_rows", {x.isect_rows.ptr, M * 48}},
      {"depth_keys", {x.depth_keys.ptr, n * 4}},
      {"order_in", {x.order_in.ptr, n * 4}},
      {"sort_tmp", {x.sort_tmp.ptr, x.sort_tmp.bytes()}},
  };
  auto it = f.find(name);
  if (it == f.end()) throw std::runtime_error("unknown context field: " + name);
  return it->second;
}

}  // namespace

extern "C" {

const char* b2c_last_error(void) { return g_err.c_str(); }

int b2c_get_device_count(int* count) {
  return guarded([&] { HIP_CHECK(hipGetDeviceCount(count)); });
}

int b2c_camera_gpu_from(const b2c_camera* cam, int W, int H, b2c_camera_gpu* out) {
  return guarded([&] { *out = b2c::CameraGPU::from(to_camera(*cam), W, H).dev(); });
}

b2c_model* b2c_model_create(void) { return new b2c_model(); }
void b2c_model_destroy(b2c_model* m) { delete m; }

int b2c_model_upload(b2c_model* m, int n, int degree, int sh_fp16, const float* pos, const float* log_scale,
                     const float* quat, const float* opacity, const float* sh, const float* floor_) {
  return guarded([&] {
    if (n < 0 || degree < 0 || degree > 4) throw std::runtime_error("model_upload: bad n or degree");
    b2c::SplatCloud c;
    c.resize((size_t)n, degree);
    std::memcpy(c.pos.data(), pos, sizeof(float) * 3 * n);
    std::memcpy(c.log_scale.data(), log_scale, sizeof(float) * 3 * n);
    std::memcpy(c.quat.data(), quat, sizeof(float) * 4 * n);
    std::memcpy(c.opacity.data(), opacity, sizeof(float) * n);
    std::memcpy(c.sh.data(), sh, sizeof(float) * 3 * (size_t)c.K() * n);
    m->m.sh_fp16 = sh_fp16 != 0;
    m->m.upload(c, nullptr, floor_);
  });
}

namespace {
Field model_field(const b2c_model* m, const std::string& name) {
  const b2c::Model& x = m->m;
  const size_t n = (size_t)x.n;
  const size_t cap = (size_t)x.cap, bands = 3 * (size_t)(x.K() - 1);
  std::map<std::string, Field> f = {
      {"pos_op", {x.pos_op.ptr, n * 16}},         {"quat", {x.quat.ptr, n * 16}},
      {"lscale", {x.lscale.ptr, n * 16}},         {"vis_weight", {x.vis_weight.ptr, n * 4}},
      {"vis_count", {x.vis_count.ptr, n * 4}},    {"refine_norm", {x.refine_norm.ptr, n * 4}},
      {"max_screen", {x.max_screen.ptr, n * 4}},
      {"m_pos_op", {x.m_pos_op.ptr, n * 16}},     {"v_pos_op", {x.v_pos_op.ptr, n * 16}},
      {"m_quat", {x.m_quat.ptr, n * 16}},         {"v_quat", {x.v_quat.ptr, n * 16}},
      {"m_lscale", {x.m_lscale.ptr, n * 16}},     {"v_lscale", {x.v_lscale.ptr, n * 16}},
      {"v_sh", {x.v_sh.ptr, n * 4}},              {"last_step", {x.last_step.ptr, n * 4}},
      // planar [lanes][cap] arrays, whole
      {"sh_dc", {x.sh_dc.ptr, 3 * cap * 4}},      {"m_sh_dc", {x.m_sh_dc.ptr, 3 * cap * 4}},
  };
  if (bands) {
    if (x.sh_fp16) {
      f["sh_hi"] = {x.sh_hi.ptr, bands * cap * 2};
      f["m_sh_hi"] = {x.m_sh_hi.ptr, bands * cap * 2};
    } else {
      f["sh_hi32"] = {x.sh_hi32.ptr, bands * cap * 4};
      f["m_sh_hi32"] = {x.m_sh_hi32.ptr, bands * cap * 4};
    }
  }
  auto it = f.find(name);
  if (it == f.end()) throw std::runtime_error("unknown model field: " + name);
  return it->second;
}
}  // namespace

int b2c_model_read(const b2c_model* m, const char* field, void* host, size_t bytes) {
  return guarded([&] {
    const Field f = model_field(m, field);
    if (bytes > f.bytes) throw std::runtime_error(std::string("model_read: too many bytes for ") + field);
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipMemcpy(host, f.ptr, bytes, hipMemcpyDeviceToHost));
  });
}

int b2c_model_write(b2c_model* m, const char* field, const void* host, size_t bytes) {
  return guarded([&] {
    const Field f = model_field(m, field);
    if (bytes > f.bytes) throw std::runtime_error(std::string("model_write: too many bytes for ") + field);
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipMemcpy(f.ptr, host, bytes, hipMemcpyHostToDevice));
  });
}

int b2c_model_zero_optimizer(b2c_model* m) {
  return guarded([&] {
    m->m.zero_optimizer(nullptr);
    HIP_CHECK(hipDeviceSynchronize());
  });
}

int b2c_model_adam_t(const b2c_model* m, int* t) {
  return guarded([&] { *t = m->m.adam_t; });
}

int b2c_model_device_ptr(const b2c_model* m, const char* field, void** ptr, size_t* bytes) {
  return guarded([&] {
    const Field f = model_field(m, field);
    *ptr = f.ptr;
    if (bytes) *bytes = f.bytes;
  });
}

int b2c_model_sh_view(const b2c_model* m, b2c_sh_view* out) {
  return guarded([&] { *out = m->m.sh().view(); });
}

b2c_ctx* b2c_ctx_create(void) {
  b2c_ctx* c = new b2c_ctx();
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    g_err = "hipStreamCreateWithFlags failed";
    delete c;
    return nullptr;
  }
  for (auto& e : c->ev) (void)hipEventCreate(&e);
  return c;
}

void b2c_ctx_destroy(b2c_ctx* c) {
  if (!c) return;
  (void)hipStreamSynchronize(c->stream);
  for (auto& e : c->ev) (void)hipEventDestroy(e);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

int b2c_ctx_setup(b2c_ctx* c, int W, int H, int n) {
  return guarded([&] {
    c->ctx.setup(W, H, n, c->stream);
    c->n = n;
    HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int b2c_ctx_info_get(const b2c_ctx* c, b2c_ctx_info* o) {
  const b2c::RenderCtx& x = c->ctx;
  o->W = x.W; o->H = x.H; o->tiles_x = x.tiles_x; o->tiles_y = x.tiles_y; o->n_tiles = x.n_tiles;
  o->tile_bits = x.tile_bits; o->num_isect = x.num_isect; o->isect_cap = x.isect_cap;
  return 0;
}

int b2c_ctx_device_ptr(b2c_ctx* c, const char* field, void** ptr, size_t* bytes) {
  return guarded([&] {
    const Field f = ctx_field(c, field);
    *ptr = f.ptr;
    if (bytes) *bytes = f.bytes;
    const std::string name(field);
    if (name == "v_splat" || name == "vis_flag") c->ctx.v_splat_shared = true;  // it may be written outside
  });
}

int b2c_ctx_read(b2c_ctx* c, const char* field, void* host, size_t bytes) {
  return guarded([&] {
    Field f = ctx_field(c, field);
    if (bytes > f.bytes) throw std::runtime_error(std::string("ctx_read: too many bytes for ") + field);
    HIP_CHECK(hipStreamSynchronize(c->stream));
    if (bytes) HIP_CHECK(hipMemcpy(host, f.ptr, bytes, hipMemcpyDeviceToHost));
  });
}

int b2c_ctx_write(b2c_ctx* c, const char* field, const void* host, size_t bytes) {
  return guarded([&] {
    Field f = ctx_field(c, field);
    if (bytes > f.bytes) throw std::runtime_error(std::string("ctx_write: too many bytes for ") + field);
    HIP_CHECK(hipStreamSynchronize(c->stream));
    if (bytes) HIP_CHECK(hipMemcpy(f.ptr, host, bytes, hipMemcpyHostToDevice));
    const std::string name(field);
    if (name == "v_splat" || name == "vis_flag") {
      c->ctx.v_splat_zero = false;
      c->ctx.v_splat_foreign = true;
      c->ctx.vis_in_rows = false;  // the caller's rows replace a deferred pass's
    }
  });
}

int b2c_ctx_zero(b2c_ctx* c, const char* field) {
  return guarded([&] {
    Field f = ctx_field(c, field);
    if (f.bytes % 4) throw std::runtime_error("ctx_zero: field size not a multiple of 4");
    if (f.bytes) LAUNCH_CHECK(b2c_hip_fill_u32(static_cast<uint32_t*>(f.ptr), 0u, f.bytes / 4, c->stream));
    if (std::string(field) == "v_splat") {
      c->ctx.v_splat_zero = true;
      c->ctx.v_splat_foreign = false;
      c->ctx.vis_in_rows = false;
    }
  });
}

int b2c_ctx_synchronize(b2c_ctx* c) {
  return guarded([&] { HIP_CHECK(hipStreamSynchronize(c->stream)); });
}

void* b2c_ctx_stream(b2c_ctx* c) { return c->stream; }

b2c_view* b2c_view_create(int W, int H, const uint32_t* rgba, const uint8_t* weights) {
  b2c_view* v = new b2c_view();
  int rc = guarded([&] {
    const size_t P = (size_t)W * H;
    v->rgba.upload(rgba, P);
    if (weights) v->weights.upload(weights, P);
    HIP_CHECK(hipDeviceSynchronize());
    v->view.rgba = v->rgba.ptr;
    v->view.weights = weights ? v->weights.ptr : nullptr;
    v->view.W = W;
    v->view.H = H;
  });
  if (rc) {
    delete v;
    return nullptr;
  }
  return v;
}

void b2c_view_destroy(b2c_view* v) { delete v; }

int b2c_view_set_normals(b2c_view* v, const uint32_t* normals) {
  return guarded([&] {
    const size_t P = (size_t)v->view.W * v->view.H;
    if (normals) {
      v->normals.upload(normals, P);
      HIP_CHECK(hipDeviceSynchronize());
      v->view.normals = v->normals.ptr;
    } else {
      v->view.normals = nullptr;
    }
  });
}

int b2c_view_set_labels(b2c_view* v, const uint8_t* labels) {
  return guarded([&] {
    const size_t P = (size_t)v->view.W * v->view.H;
    if (labels) {
      v->labels.upload(labels, P);
      HIP_CHECK(hipDeviceSynchronize());
      v->view.labels = v->labels.ptr;
    } else {
      v->view.labels = nullptr;
    }
  });
}

int b2c_view_set_flags(b2c_view* v, int has_alpha, int masked, float alpha_coverage, float normal_count) {
  return guarded([&] {
    v->view.has_alpha = has_alpha != 0;
    v->view.masked = masked != 0;
    v->view.alpha_coverage = alpha_coverage;
    v->view.normal_count = normal_count;
  });
}

int b2c_compute_evidence(b2c_ctx* c, const b2c_model* m, const b2c_view* const* views, const b2c_camera* cams,
                         int nviews, float normal_weight, int export_labels) {
  return guarded([&] {
    std::vector<b2c::ViewGPU> vs;
    std::vector<b2c::Camera> cs;
    for (int v = 0; v < nviews; v++) {
      vs.push_back(views[v]->view);
      cs.push_back(to_camera(cams[v]));
    }
    b2c::EvidenceParams p;
    p.evidence_normal_weight = normal_weight;
    p.export_labels = export_labels != 0;
    b2c::compute_evidence(c->ctx, m->m, vs, cs, p, c->stream);
  });
}

int b2c_download_evidence(const b2c_model* m, float* out) {
  return guarded([&] {
    const std::vector<float> e = b2c::download_evidence(m->m, nullptr);
    std::copy(e.begin(), e.end(), out);
  });
}

int b2c_download_labels(const b2c_model* m, float* out) {
  return guarded([&] {
    const std::vector<float> l = b2c::download_labels(m->m, nullptr);
    std::copy(l.begin(), l.end(), out);
  });
}

int b2c_probe_depth(b2c_ctx* c, float tau, float delta, const float* ref_z, float margin, float* out) {
  return guarded([&] {
    b2c::probe_depth(c->ctx, tau, delta, ref_z, margin, reinterpret_cast<float4*>(out), c->stream);
    HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int b2c_device_download(void* host, const void* dev, size_t bytes) {
  return guarded([&] {
    HIP_CHECK(hipDeviceSynchronize());
    if (bytes) HIP_CHECK(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost));
  });
}

extern "C++" {
namespace {
std::vector<std::string> split_lines(const char* text) {
  std::vector<std::string> out;
  if (!text) return out;
  std::string cur;
  for (const char* p = text; *p; p++) {
    if (*p == '\n') {
      out.push_back(cur);
      cur.clear();
    } else {
      cur += *p;
    }
  }
  if (!cur.empty()) out.push_back(cur);
  return out;
}

void info_of(const b2c::SplatCloud& c, bool binary, b2c_ply_info* out) {
  out->n = (int64_t)c.n;
  out->sh_degree = c.sh_degree;
  out->binary = binary;
  out->has_scales = c.has_scales;
  out->has_evidence = c.has_evidence;
  out->has_labels = c.has_labels;
  out->has_fill = c.has_fill;
  out->has_gate = c.has_gate;
  out->has_gate_s = c.has_gate_s;
  out->has_open = c.has_open;
}

// The optional blocks of a cloud, flagged by desc, copied from host arrays.
void extras_from(const b2c_ply_info* desc, const b2c_ply_arrays* in, b2c::SplatCloud& c) {
  if (!desc || !in) return;
  const auto take = [&](int flag, float* src, bool& has, std::vector<float>& dst, size_t width) {
    has = flag != 0;
    if (!has) return;
    if (!src) throw std::runtime_error("ply: a flagged optional block has no array");
    dst.assign(src, src + c.n * width);
  };
  take(desc->has_evidence, in->evidence, c.has_evidence, c.evidence, 7);
  take(desc->has_labels, in->labels, c.has_labels, c.labels, 2);
  take(desc->has_fill, in->fill, c.has_fill, c.fill, 1);
  take(desc->has_gate, in->gate, c.has_gate, c.gate, 2);
  take(desc->has_gate_s, in->gate_s, c.has_gate_s, c.gate_s, 1);
  take(desc->has_open, in->open, c.has_open, c.open, 4);
}
}  // namespace
}  // extern "C++"

int b2c_ply_info_get(const char* path, b2c_ply_info* out) {
  return guarded([&] { info_of(b2c::read_ply_shape(path), b2c::read_ply_header(path).binary, out); });
}

int b2c_ply_read(const char* path, const b2c_ply_arrays* out) {
  return guarded([&] {
    const b2c::SplatCloud c = b2c::read_ply(path);
    const auto give = [](float* dst, const std::vector<float>& v) {
      if (dst && !v.empty()) std::memcpy(dst, v.data(), v.size() * sizeof(float));
    };
    give(out->pos, c.pos);
    give(out->log_scale, c.log_scale);
    give(out->quat, c.quat);
    give(out->opacity, c.opacity);
    give(out->sh, c.sh);
    give(out->evidence, c.evidence);
    give(out->labels, c.labels);
    give(out->fill, c.fill);
    give(out->gate, c.gate);
    give(out->gate_s, c.gate_s);
    give(out->open, c.open);
  });
}

int b2c_ply_write(const char* path, const b2c_ply_info* desc, const b2c_ply_arrays* in, const char* comments) {
  return guarded([&] {
    if (desc->n < 0 || desc->sh_degree < 0 || desc->sh_degree > 4) throw std::runtime_error("ply_write: bad n or degree");
    b2c::SplatCloud c;
    c.resize((size_t)desc->n, desc->sh_degree);
    const auto copy = [&](std::vector<float>& dst, const float* src) {
      if (!src) throw std::runtime_error("ply_write: missing a base array");
      std::memcpy(dst.data(), src, dst.size() * sizeof(float));
    };
    copy(c.pos, in->pos);
    copy(c.log_scale, in->log_scale);
    copy(c.quat, in->quat);
    copy(c.opacity, in->opacity);
    copy(c.sh, in->sh);
    extras_from(desc, in, c);
    b2c::write_ply(path, c, split_lines(comments));
  });
}

int b2c_ply_is_vertex_only(const char* path) {
  int r = -1;
  const int rc = guarded([&] { r = b2c::ply_is_vertex_only(path) ? 1 : 0; });
  return rc ? -1 : r;
}

int b2c_ply_comments(const char* path, char* buf, size_t cap, size_t* needed) {
  return guarded([&] {
    std::string all;
    for (const std::string& c : b2c::read_ply_comments(path)) {
      if (!all.empty()) all += '\n';
      all += c;
    }
    if (needed) *needed = all.size() + 1;
    if (buf && cap) {
      const size_t k = std::min(cap - 1, all.size());
      std::memcpy(buf, all.data(), k);
      buf[k] = 0;
    }
  });
}

int b2c_png_decode(const char* path, int* w, int* h, int* channels, uint8_t* rgba, size_t rgba_bytes) {
  return guarded([&] {
    const b2c::DecodedImage d = b2c::decode_png(path);
    *w = d.w;
    *h = d.h;
    *channels = d.channels_in_file;
    if (rgba) {
      if (rgba_bytes < d.rgba.size()) throw std::runtime_error("png_decode: output buffer too small");
      std::memcpy(rgba, d.rgba.data(), d.rgba.size());
    }
  });
}

int b2c_image_decode(const char* path, int* w, int* h, int* channels, uint8_t* rgba, size_t rgba_bytes) {
  return guarded([&] {
    const b2c::DecodedImage d = b2c::decode_image(path);
    *w = d.w;
    *h = d.h;
    *channels = d.channels_in_file;
    if (rgba) {
      if (rgba_bytes < d.rgba.size()) throw std::runtime_error("image_decode: output buffer too small");
      std::memcpy(rgba, d.rgba.data(), d.rgba.size());
    }
  });
}

int b2c_image_resample(const uint8_t* src, int w, int h, uint8_t* dst, int nw, int nh, int filter) {
  return guarded([&] {
    if (filter < 0 || filter > 2) throw std::invalid_argument("image_resample: filter must be 0, 1 or 2");
    const std::vector<uint8_t> out = b2c::resample_rgba8(src, w, h, nw, nh, (b2c::ResampleFilter)filter);
    std::memcpy(dst, out.data(), out.size());
  });
}

b2c_dataset* b2c_dataset_load(const b2c_dataset_opts* o) {
  b2c_dataset* d = new b2c_dataset();
  const int rc = guarded([&] {
    b2c::DatasetOptions opt;
    opt.source = o->source ? o->source : "";
    if (o->max_frames >= 0) opt.max_frames = (uint32_t)o->max_frames;
    opt.max_resolution = o->max_resolution;
    if (o->eval_split_every >= 0) opt.eval_split_every = (uint32_t)o->eval_split_every;
    if (o->subsample_frames >= 0) opt.subsample_frames = (uint32_t)o->subsample_frames;
    if (o->alpha_mode >= 0) opt.alpha_mode = o->alpha_mode == 0 ? b2c::AlphaMode::Masked : b2c::AlphaMode::Transparent;
    d->ds = b2c::load_dataset(opt);
  });
  if (rc) {
    delete d;
    return nullptr;
  }
  return d;
}

void b2c_dataset_destroy(b2c_dataset* d) { delete d; }

int b2c_dataset_count(const b2c_dataset* d, int split) {
  return split == 0 ? (int)d->ds.train.size() : split == 1 ? (int)d->ds.eval.size() : -1;
}

extern "C++" {
namespace {
const b2c::View& dataset_view(const b2c_dataset* d, int split, int i) {
  const std::vector<b2c::View>& v = split == 0 ? d->ds.train : d->ds.eval;
  if ((split != 0 && split != 1) || i < 0 || (size_t)i >= v.size()) throw std::runtime_error("dataset: no such view");
  return v[(size_t)i];
}
}  // namespace
}  // extern "C++"

int b2c_dataset_view_info(const b2c_dataset* d, int split, int i, b2c_view_info* out) {
  return guarded([&] {
    const b2c::View& v = dataset_view(d, split, i);
    *out = b2c_view_info{};
    out->w = v.w;
    out->h = v.h;
    out->cam.width = v.cam.width;
    out->cam.height = v.cam.height;
    out->cam.fx = v.cam.fx;
    out->cam.fy = v.cam.fy;
    out->cam.cx = v.cam.cx;
    out->cam.cy = v.cam.cy;
    std::copy(v.cam.R, v.cam.R + 9, out->cam.R);
    std::copy(v.cam.t, v.cam.t + 3, out->cam.t);
    out->has_alpha = v.has_alpha;
    out->masked = v.mode == b2c::AlphaMode::Masked;
    out->has_normals = v.has_normals();
    out->has_weights = v.has_weights();
    out->has_labels = v.has_labels();
    out->alpha_coverage = v.alpha_coverage;
    out->normal_mask_count = v.normal_mask_count;
    std::snprintf(out->name, sizeof out->name, "%s", v.name.c_str());
  });
}

int b2c_dataset_view_read(const b2c_dataset* d, int split, int i, uint32_t* rgba, uint32_t* normals, uint8_t* weights,
                          uint8_t* labels) {
  return guarded([&] {
    const b2c::View& v = dataset_view(d, split, i);
    if (rgba) std::copy(v.rgba.begin(), v.rgba.end(), rgba);
    if (normals) std::copy(v.normals.begin(), v.normals.end(), normals);
    if (weights) std::copy(v.weights.begin(), v.weights.end(), weights);
    if (labels) std::copy(v.labels.begin(), v.labels.end(), labels);
  });
}

b2c_view* b2c_dataset_view_upload(const b2c_dataset* d, int split, int i) {
  b2c_view* out = nullptr;
  const int rc = guarded([&] {
    const b2c::View& v = dataset_view(d, split, i);
    out = b2c_view_create(v.w, v.h, v.rgba.data(), v.has_weights() ? v.weights.data() : nullptr);
    if (!out) throw std::runtime_error(b2c_last_error());
    if (v.has_normals() && b2c_view_set_normals(out, v.normals.data())) throw std::runtime_error(b2c_last_error());
    if (v.has_labels() && b2c_view_set_labels(out, v.labels.data())) throw std::runtime_error(b2c_last_error());
    b2c_view_set_flags(out, v.has_alpha, v.mode == b2c::AlphaMode::Masked, v.alpha_coverage, (float)v.normal_mask_count);
  });
  if (rc && out) {
    b2c_view_destroy(out);
    out = nullptr;
  }
  return out;
}

int b2c_dataset_points(const b2c_dataset* d, float* xyz, uint8_t* rgb, int64_t* count) {
  return guarded([&] {
    const std::vector<b2c::Point3D>& p = d->ds.points;
    if (count) *count = (int64_t)p.size();
    for (size_t k = 0; k < p.size(); k++) {
      if (xyz) {
        xyz[k * 3] = p[k].x;
        xyz[k * 3 + 1] = p[k].y;
        xyz[k * 3 + 2] = p[k].z;
      }
      if (rgb) {
        rgb[k * 3] = p[k].r;
        rgb[k * 3 + 1] = p[k].g;
        rgb[k * 3 + 2] = p[k].b;
      }
    }
  });
}

int b2c_dataset_summary(const b2c_dataset* d, char* buf, size_t cap, int* counts) {
  return guarded([&] {
    const std::string s = d->ds.root + "\n" + d->ds.name + "\n" + d->ds.init_ply;
    if (buf && cap) std::snprintf(buf, cap, "%s", s.c_str());
    if (counts) {
      counts[0] = d->ds.n_masked;
      counts[1] = d->ds.n_transparent;
      counts[2] = d->ds.n_weighted;
      counts[3] = d->ds.n_normals;
      counts[4] = d->ds.n_labels;
    }
  });
}

int b2c_model_load_ply(b2c_model* m, const char* path, int sh_fp16, int* has_scales) {
  return guarded([&] {
    m->m.sh_fp16 = sh_fp16 != 0;
    const bool s = b2c::load_ply(m->m, path, nullptr);
    if (has_scales) *has_scales = s;
  });
}

int b2c_model_save_ply(const b2c_model* m, const char* path, const char* comments, const b2c_ply_info* extras_desc,
                       const b2c_ply_arrays* extras) {
  return guarded([&] {
    b2c::SplatCloud x;
    x.n = (size_t)m->m.n;
    extras_from(extras_desc, extras, x);
    b2c::save_ply(m->m, path, split_lines(comments), extras_desc ? &x : nullptr, nullptr);
  });
}

void* b2c_device_upload(const void* host, size_t bytes) {
  void* d = nullptr;
  const int rc = guarded([&] {
    HIP_CHECK(hipMalloc(&d, bytes ? bytes : 1));
    if (bytes) HIP_CHECK(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
  });
  if (rc && d) {
    (void)hipFree(d);
    d = nullptr;
  }
  return d;
}

void b2c_device_free(void* p) {
  if (p) (void)hipFree(p);
}

int b2c_normal_loss(b2c_ctx* c, const b2c_view* v, const b2c_loss_opts* o) {
  return guarded([&] { b2c::normal_loss(c->ctx, v->view, to_loss(*o), c->stream); });
}

int b2c_hollow_loss(b2c_ctx* c, float lam) {
  return guarded([&] { b2c::hollow_loss(c->ctx, lam, c->stream); });
}

int b2c_eval_metrics(b2c_ctx* c, const b2c_view* v, int mask_weighted) {
  return guarded([&] { b2c::eval_metrics(c->ctx, v->view, mask_weighted != 0, c->stream); });
}

int b2c_render_forward(b2c_ctx* c, const b2c_model* m, const b2c_render_opts* o) {
  return guarded([&] { b2c::render_forward(c->ctx, m->m, to_params(*o), c->stream); });
}

int b2c_project_splats(b2c_ctx* c, const b2c_model* m, const b2c_render_opts* o) {
  return guarded([&] { b2c::project_splats(c->ctx, m->m, to_params(*o), c->stream); });
}

int b2c_bin_and_sort(b2c_ctx* c, const b2c_model* m) {
  return guarded([&] { b2c::bin_and_sort(c->ctx, m->m, c->stream); });
}

int b2c_rasterize_forward(b2c_ctx* c, const b2c_render_opts* o) {
  return guarded([&] { b2c::rasterize_forward(c->ctx, to_params(*o), c->stream); });
}

int b2c_photometric_loss(b2c_ctx* c, const b2c_view* v, const b2c_loss_opts* o) {
  return guarded([&] {
    if (v->view.W != c->ctx.W || v->view.H != c->ctx.H) throw std::runtime_error("photometric_loss: view size != render size");
    b2c::photometric_loss(c->ctx, v->view, to_loss(*o), c->stream);
  });
}

int b2c_accumulate_loss(b2c_ctx* c) {
  return guarded([&] { b2c::accumulate_loss(c->ctx, c->stream); });
}

int b2c_rasterize_backward(b2c_ctx* c, b2c_model* m, const b2c_render_opts* o, int mode, float grad_scale) {
  return guarded([&] {
    if (mode == 0)
      b2c::rasterize_backward(c->ctx, m->m, to_params(*o), c->stream);
    else
      b2c::rasterize_backward_tc(c->ctx, m->m, to_params(*o), grad_scale, c->stream);
  });
}

int b2c_optimizer_grad(b2c_ctx* c, b2c_model* m, const b2c_render_opts* o, int active_deg, int flags) {
  return guarded([&] {
    const size_t per = 11 + 3 * (size_t)m->m.K();
    const size_t need = (size_t)m->m.n * per;
    if (c->grads.count < need || c->degree != m->m.degree) {
      c->grads.free();
      c->grads.reserve(need);
      c->grads.zero(c->stream);
      c->degree = m->m.degree;
    }
    b2c::OptimParams op;
    op.cam = to_params(*o).cam;
    op.active_sh_degree = active_deg;
    op.grad_out = c->grads.ptr;
    op.grad_accumulate = (flags & B2C_GRAD_ACCUMULATE) != 0;
    op.sparse = (flags & B2C_GRAD_SPARSE) != 0;
    b2c::optimizer_step(c->ctx, m->m, op, c->stream);
  });
}

void b2c_adam_defaults(b2c_adam_opts* a) {
  const b2c::OptimParams d{};
  *a = b2c_adam_opts{};
  a->t = 0;
  a->sparse = 0;
  a->beta1 = d.beta1; a->beta2 = d.beta2; a->eps = d.eps;
  a->lr_mean = d.lr_mean; a->lr_rot = d.lr_rot; a->lr_scale = d.lr_scale; a->lr_opac = d.lr_opac;
  a->lr_dc = d.lr_dc; a->lr_sh_rest = d.lr_sh_rest;
  a->noise_weight = d.noise_weight; a->noise_clamp = d.noise_clamp;
  a->seed = d.seed; a->step = d.step;
}

int b2c_optimizer_step(b2c_ctx* c, b2c_model* m, const b2c_render_opts* o, const b2c_adam_opts* a) {
  return guarded([&] {
    b2c::OptimParams op = to_optim(*o, *a, m->m);
    b2c::optimizer_step(c->ctx, m->m, op, c->stream);
  });
}

int b2c_train_step(b2c_ctx* c, b2c_model* m, const b2c_view* v, const b2c_render_opts* ro, const b2c_loss_opts* lo,
                   int mode, int flags, b2c_step_times* times) {
  return train_step(c, m, v, ro, lo, mode, flags, nullptr, times);
}

int b2c_train_step_adam(b2c_ctx* c, b2c_model* m, const b2c_view* v, const b2c_render_opts* ro,
                        const b2c_loss_opts* lo, int mode, const b2c_adam_opts* a, b2c_step_times* times) {
  return train_step(c, m, v, ro, lo, mode, 0, a, times);
}

}  // extern "C"

namespace {

int train_step(b2c_ctx* c, b2c_model* m, const b2c_view* v, const b2c_render_opts* ro, const b2c_loss_opts* lo,
               int mode, int flags, const b2c_adam_opts* adam, b2c_step_times* times) {
  return guarded([&] {
    b2c::RenderParams p = to_params(*ro);
    p.write_proj = mode == 0;  // only the fp32 backward reads proj0..3; the step leaves them unwritten otherwise
    b2c::LossParams lp = to_loss(*lo);
    lp.assign_loss = true;  // the step's loss replaces loss_accum[0..1] (no separate clear)
    lp.running_sum = true;  // and [2..3] become what the trainer's per-step clear + accumulate_loss leave
    hipStream_t s = c->stream;
    auto mark = [&](int k) {
      if (times) HIP_CHECK(hipEventRecord(c->ev[k], s));
    };
    const size_t per = 11 + 3 * (size_t)m->m.K();
    if (!adam && (c->grads.count < (size_t)m->m.n * per || c->degree != m->m.degree)) {
      c->grads.free();
      c->grads.reserve((size_t)m->m.n * per);
      c->grads.zero(s);
      c->degree = m->m.degree;
    }
    // the update's parameters are checked (and the step counter advanced) before any work is queued
    b2c::OptimParams op = adam ? to_optim(*ro, *adam, m->m) : b2c::OptimParams{};
    mark(0);
    b2c::project_splats(c->ctx, m->m, p, s);
    mark(1);
    b2c::bin_and_sort(c->ctx, m->m, s);
    mark(2);
    b2c::rasterize_forward(c->ctx, p, s);
    mark(3);
    // the trainer's loss order (trainer.cpp:502-505): photometric, normal-map, hollow, then the step sums
    const bool normals_on = p.feat == b2c::FeatureMode::Normals && lp.normal_scale > 0.f && v->view.normals;
    const bool hollow_on = p.hollow_z && p.hollow_lam != 0.f;
    lp.running_sum = !(normals_on || hollow_on);
    // the VJP below sums the loss's partials (no launch of its own) when nothing reads loss_accum before it
    lp.defer_sum = lp.running_sum && m->m.n > 0;
    b2c::photometric_loss(c->ctx, v->view, lp, s);
    if (normals_on) b2c::normal_loss(c->ctx, v->view, lp, s);
    if (hollow_on) b2c::hollow_loss(c->ctx, p.hollow_lam, s);
    if (!lp.running_sum) LAUNCH_CHECK(b2c_hip_step_loss_sums(c->ctx.loss_accum.ptr, s));
    mark(4);
    c->ctx.bwd_split_event = (times && mode != 0) ? c->ev[7] : nullptr;
    {
      // the VJP below consumes the pass's visibility, so it may stay in v_splat (reset on every exit)
      struct DeferVis {
        b2c::RenderCtx& x;
        ~DeferVis() { x.defer_vis = false; }
      } scope{c->ctx};
      c->ctx.defer_vis = true;
      if (mode == 0)
        b2c::rasterize_backward(c->ctx, m->m, p, s);
      else
        b2c::rasterize_backward_tc(c->ctx, m->m, p, lp.grad_scale, s);
    }
    c->ctx.bwd_split_event = nullptr;
    mark(5);
    if (!adam) {
      op.cam = p.cam;
      op.active_sh_degree = p.sh_degree;
      op.grad_out = c->grads.ptr;
      op.grad_accumulate = (flags & B2C_GRAD_ACCUMULATE) != 0;
      op.sparse = (flags & B2C_GRAD_SPARSE) != 0;
    }
    b2c::optimizer_step(c->ctx, m->m, op, s);
    mark(6);
    if (times) {
      HIP_CHECK(hipEventSynchronize(c->ev[6]));
      float* out[6] = {&times->project_ms, &times->bin_ms, &times->forward_ms, &times->loss_ms, &times->backward_ms,
                       &times->vjp_ms};
      for (int k = 0; k < 6; k++) HIP_CHECK(hipEventElapsedTime(out[k], c->ev[k], c->ev[k + 1]));
      HIP_CHECK(hipEventElapsedTime(&times->total_ms, c->ev[0], c->ev[6]));
      if (mode != 0) {
        HIP_CHECK(hipEventElapsedTime(&times->raster_bwd_ms, c->ev[4], c->ev[7]));
        HIP_CHECK(hipEventElapsedTime(&times->reduce_ms, c->ev[7], c->ev[5]));
      } else {
        times->raster_bwd_ms = times->backward_ms;
        times->reduce_ms = 0.f;
      }
    }
  });
}

}  // namespace
