// TEST INFRASTRUCTURE ONLY. A C-ABI entry into the reference's own double-precision CPU loss,
// tests/reference.cpp:34-143, compiled unmodified from /root/reference by oracle/Makefile into
// oracle/_ref/. Used to pin the restatement in b2c_oracle.c (orc_ref_loss) and to write the
// fixtures under tests/golden/. This file is this repository's code; no reference source is copied.
#include <cstdint>
#include <vector>

#include "reference.h"

extern "C" double ref_reference_loss_ext(int n, int degree, const float* pos, const float* log_scale,
                                         const float* quat, const float* opacity, const float* sh, int W, int H,
                                         const float* R, const float* t, float fx, float fy, float cx, float cy,
                                         const double* bg, const uint32_t* gt, const uint8_t* wts, int composite,
                                         int mask, int alpha_lane, double l1_w, double ssim_w,
                                         double match_alpha_weight, double scale, const uint32_t* gtn,
                                         double normal_scale, const float* hollow_z, double hollow_lam,
                                         double hollow_margin);

extern "C" double ref_reference_loss(int n, int degree, const float* pos, const float* log_scale, const float* quat,
                                     const float* opacity, const float* sh, int W, int H, const float* R,
                                     const float* t, float fx, float fy, float cx, float cy, const double* bg,
                                     const uint32_t* gt, const uint8_t* wts, int composite, int mask, int alpha_lane,
                                     double l1_w, double ssim_w, double match_alpha_weight, double scale) {
  return ref_reference_loss_ext(n, degree, pos, log_scale, quat, opacity, sh, W, H, R, t, fx, fy, cx, cy, bg, gt, wts,
                                composite, mask, alpha_lane, l1_w, ssim_w, match_alpha_weight, scale, nullptr, 0.0,
                                nullptr, 0.0, 0.05);
}

// The same with the normal-map term (gtn non-NULL: RefParams::normals) and the hollow term (hollow_z non-NULL).
extern "C" double ref_reference_loss_ext(int n, int degree, const float* pos, const float* log_scale,
                                         const float* quat, const float* opacity, const float* sh, int W, int H,
                                         const float* R, const float* t, float fx, float fy, float cx, float cy,
                                         const double* bg, const uint32_t* gt, const uint8_t* wts, int composite,
                                         int mask, int alpha_lane, double l1_w, double ssim_w,
                                         double match_alpha_weight, double scale, const uint32_t* gtn,
                                         double normal_scale, const float* hollow_z, double hollow_lam,
                                         double hollow_margin) {
  b2c::SplatCloud c;
  c.resize((size_t)n, degree);
  const int K = c.K();
  for (int i = 0; i < n * 3; i++) { c.pos[i] = pos[i]; c.log_scale[i] = log_scale[i]; }
  for (int i = 0; i < n * 4; i++) c.quat[i] = quat[i];
  for (int i = 0; i < n; i++) c.opacity[i] = opacity[i];
  for (int i = 0; i < n * K * 3; i++) c.sh[i] = sh[i];
  std::vector<uint32_t> g(gt, gt + (size_t)W * H);
  std::vector<uint8_t> w;
  if (wts) w.assign(wts, wts + (size_t)W * H);
  RefParams p{};
  p.W = W; p.H = H;
  p.cam.width = W; p.cam.height = H;
  p.cam.fx = fx; p.cam.fy = fy; p.cam.cx = cx; p.cam.cy = cy;
  for (int i = 0; i < 9; i++) p.cam.R[i] = R[i];
  for (int i = 0; i < 3; i++) p.cam.t[i] = t[i];
  p.cam.update_pos();
  for (int i = 0; i < 3; i++) p.bg[i] = bg[i];
  p.composite = composite != 0; p.mask = mask != 0; p.alpha_lane = alpha_lane != 0; p.normals = gtn != nullptr;
  p.l1_w = l1_w; p.ssim_w = ssim_w; p.match_alpha_weight = match_alpha_weight; p.scale = scale;
  p.normal_scale = gtn ? normal_scale : 0.0;
  std::vector<uint32_t> gn;
  if (gtn) gn.assign(gtn, gtn + (size_t)W * H);
  std::vector<float> hz;
  if (hollow_z) hz.assign(hollow_z, hollow_z + (size_t)W * H);
  p.gt = &g; p.gtn = gtn ? &gn : nullptr; p.wts = wts ? &w : nullptr;
  if (hollow_z) {
    p.hollow_z = &hz;
    p.hollow_lam = hollow_lam;
    p.hollow_margin = hollow_margin;
  }
  return reference_loss(c, p);
}

// ---- The reference's ply reader and writer (src/ply.cpp), for the ply fixtures under tests/golden/ply/ ----
// Each returns 0, or 1 with the reference's error message in err (cap bytes).
#include <cstring>
#include <stdexcept>
#include <string>

#include "ply.h"

namespace {
int ply_error(const std::exception& e, char* err, size_t cap) {
  if (err && cap) {
    std::strncpy(err, e.what(), cap - 1);
    err[cap - 1] = 0;
  }
  return 1;
}
}  // namespace

// flags: has_scales, has_evidence, has_labels, has_fill, has_gate, has_gate_s, has_open
extern "C" int ref_ply_info(const char* path, long long* n, int* degree, int* flags, char* err, size_t cap) {
  try {
    const b2c::SplatCloud c = b2c::read_ply(path);
    *n = (long long)c.n;
    *degree = c.sh_degree;
    const bool f[7] = {c.has_scales, c.has_evidence, c.has_labels, c.has_fill, c.has_gate, c.has_gate_s, c.has_open};
    for (int k = 0; k < 7; k++) flags[k] = f[k];
    return 0;
  } catch (const std::exception& e) {
    return ply_error(e, err, cap);
  }
}

// arrays: pos, log_scale, quat, opacity, sh, evidence, labels, fill, gate, gate_s, open (NULL = skip)
extern "C" int ref_ply_read(const char* path, float** arrays, char* err, size_t cap) {
  try {
    const b2c::SplatCloud c = b2c::read_ply(path);
    const std::vector<float>* src[11] = {&c.pos, &c.log_scale, &c.quat, &c.opacity, &c.sh, &c.evidence,
                                         &c.labels, &c.fill, &c.gate, &c.gate_s, &c.open};
    for (int k = 0; k < 11; k++)
      if (arrays[k] && !src[k]->empty()) std::memcpy(arrays[k], src[k]->data(), src[k]->size() * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    return ply_error(e, err, cap);
  }
}

// flags as ref_ply_info (has_scales ignored); comments '\n'-separated or NULL
extern "C" int ref_ply_write(const char* path, long long n, int degree, const int* flags, float* const* arrays,
                             const char* comments, char* err, size_t cap) {
  try {
    b2c::SplatCloud c;
    c.has_evidence = flags[1]; c.has_labels = flags[2]; c.has_fill = flags[3]; c.has_gate = flags[4];
    c.has_gate_s = flags[5]; c.has_open = flags[6];
    c.resize((size_t)n, degree);
    std::vector<float>* dst[11] = {&c.pos, &c.log_scale, &c.quat, &c.opacity, &c.sh, &c.evidence,
                                   &c.labels, &c.fill, &c.gate, &c.gate_s, &c.open};
    for (int k = 0; k < 11; k++)
      if (arrays[k] && !dst[k]->empty()) std::memcpy(dst[k]->data(), arrays[k], dst[k]->size() * sizeof(float));
    std::vector<std::string> cm;
    if (comments) {
      std::string cur;
      for (const char* p = comments; *p; p++) {
        if (*p == '\n') { cm.push_back(cur); cur.clear(); } else { cur += *p; }
      }
      if (!cur.empty()) cm.push_back(cur);
    }
    b2c::write_ply(path, c, cm);
    return 0;
  } catch (const std::exception& e) {
    return ply_error(e, err, cap);
  }
}

extern "C" int ref_ply_is_vertex_only(const char* path) { return b2c::ply_is_vertex_only(path) ? 1 : 0; }

extern "C" int ref_ply_comments(const char* path, char* buf, size_t cap) {
  std::string all;
  for (const std::string& s : b2c::read_ply_comments(path)) {
    if (!all.empty()) all += '\n';
    all += s;
  }
  if (cap) {
    const size_t k = std::min(cap - 1, all.size());
    std::memcpy(buf, all.data(), k);
    buf[k] = 0;
  }
  return (int)all.size();
}

// ---- The reference's dataset loader (src/dataset/views.cpp, colmap.cpp), for tests/golden/colmap/ ----
#include "dataset/views.h"

namespace {
b2c::Dataset g_dataset;
const b2c::View& dataset_view(int split, int i) { return split == 0 ? g_dataset.train.at(i) : g_dataset.eval.at(i); }
}  // namespace

// max_frames, eval_every, subsample < 0: unset; alpha_mode -1 unset, 0 masked, 1 transparent
extern "C" int ref_dataset_load(const char* source, int max_frames, unsigned max_res, int eval_every, int subsample,
                                int alpha_mode, char* err, size_t cap) {
  try {
    b2c::Config cfg;
    cfg.source = source;
    if (max_frames >= 0) cfg.max_frames = (uint32_t)max_frames;
    cfg.max_resolution = max_res;
    if (eval_every >= 0) cfg.eval_split_every = (uint32_t)eval_every;
    if (subsample >= 0) cfg.subsample_frames = (uint32_t)subsample;
    if (alpha_mode >= 0) cfg.alpha_mode = alpha_mode == 0 ? b2c::AlphaMode::Masked : b2c::AlphaMode::Transparent;
    g_dataset = b2c::load_dataset(cfg);
    return 0;
  } catch (const std::exception& e) {
    return ply_error(e, err, cap);
  }
}

extern "C" int ref_dataset_count(int split) { return (int)(split == 0 ? g_dataset.train.size() : g_dataset.eval.size()); }

// ints: w, h, cam width, cam height, has_alpha, masked, has_normals, has_weights, has_labels
// floats: fx fy cx cy R[9] t[3] pos[3] alpha_coverage
extern "C" void ref_dataset_view(int split, int i, int* ints, float* floats, double* normal_mask_count, char* name,
                                 size_t cap) {
  const b2c::View& v = dataset_view(split, i);
  const int iv[9] = {v.w, v.h, v.cam.width, v.cam.height, v.has_alpha, v.mode == b2c::AlphaMode::Masked,
                     v.has_normals(), v.has_weights(), v.has_labels()};
  for (int k = 0; k < 9; k++) ints[k] = iv[k];
  floats[0] = v.cam.fx; floats[1] = v.cam.fy; floats[2] = v.cam.cx; floats[3] = v.cam.cy;
  for (int k = 0; k < 9; k++) floats[4 + k] = v.cam.R[k];
  for (int k = 0; k < 3; k++) { floats[13 + k] = v.cam.t[k]; floats[16 + k] = v.cam.pos[k]; }
  floats[19] = v.alpha_coverage;
  *normal_mask_count = v.normal_mask_count;
  std::strncpy(name, v.name.c_str(), cap - 1);
  name[cap - 1] = 0;
}

extern "C" void ref_dataset_view_arrays(int split, int i, uint32_t* rgba, uint32_t* normals, uint8_t* weights,
                                        uint8_t* labels) {
  const b2c::View& v = dataset_view(split, i);
  std::memcpy(rgba, v.rgba.data(), v.rgba.size() * 4);
  if (!v.normals.empty()) std::memcpy(normals, v.normals.data(), v.normals.size() * 4);
  if (!v.weights.empty()) std::memcpy(weights, v.weights.data(), v.weights.size());
  if (!v.labels.empty()) std::memcpy(labels, v.labels.data(), v.labels.size());
}

// counts: masked, transparent, weighted, normals, labels; text: root \n name \n init_ply
extern "C" long long ref_dataset_summary(int* counts, char* text, size_t cap, float* xyz, uint8_t* rgb) {
  const int c[5] = {g_dataset.n_masked, g_dataset.n_transparent, g_dataset.n_weighted, g_dataset.n_normals,
                    g_dataset.n_labels};
  for (int k = 0; k < 5; k++) counts[k] = c[k];
  const std::string s = g_dataset.root + "\n" + g_dataset.name + "\n" + g_dataset.init_ply;
  std::strncpy(text, s.c_str(), cap - 1);
  text[cap - 1] = 0;
  for (size_t k = 0; k < g_dataset.points.size(); k++) {
    const b2c::Point3D& p = g_dataset.points[k];
    if (xyz) { xyz[k * 3] = p.x; xyz[k * 3 + 1] = p.y; xyz[k * 3 + 2] = p.z; }
    if (rgb) { rgb[k * 3] = p.r; rgb[k * 3 + 1] = p.g; rgb[k * 3 + 2] = p.b; }
  }
  return (long long)g_dataset.points.size();
}

// ---- The reference loader's image decoder and resize (stb_image v2.30 / stb_image_resize2 v2.18 as
// src/dataset/views.cpp compiles them), for the image fixtures under tests/golden/images/ ----
#include "stb_image.h"
#include "stb_image_resize2.h"

// stbi_load(path, ..., 4): 0 and the image (rgba: w * h * 4 bytes when not NULL), or 1 with the reason.
extern "C" int ref_image_load(const char* path, int* w, int* h, int* channels, uint8_t* rgba, size_t cap,
                              char* err, size_t err_cap) {
  unsigned char* p = stbi_load(path, w, h, channels, 4);
  if (!p) {
    std::strncpy(err, stbi_failure_reason(), err_cap - 1);
    err[err_cap - 1] = 0;
    return 1;
  }
  const size_t n = (size_t)*w * *h * 4;
  if (rgba && cap >= n) std::memcpy(rgba, p, n);
  stbi_image_free(p);
  return 0;
}

// The loader's resize_rgba (views.cpp:73-78): filter 0 triangle, 1 Mitchell, 2 point sample.
extern "C" int ref_image_resize(const uint8_t* src, int w, int h, uint8_t* dst, int nw, int nh, int filter) {
  const stbir_filter f = filter == 0 ? STBIR_FILTER_TRIANGLE : filter == 1 ? STBIR_FILTER_MITCHELL
                                                                         : STBIR_FILTER_POINT_SAMPLE;
  return stbir_resize(src, w, h, 0, dst, nw, nh, 0, STBIR_4CHANNEL, STBIR_TYPE_UINT8, STBIR_EDGE_CLAMP, f) ? 0 : 1;
}
