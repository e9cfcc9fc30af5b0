/*
 * b2c.h — C ABI over the MI355X splat rasterizer's C++ drop-in API (b2ctrain_amd/csrc/b2c/), for
 * callers that bind through an FFI (ctypes, cgo, JNI, N-API). Opaque handles own the C++ objects; every
 * function returns 0 on success or a nonzero code, with the message in b2c_last_error().
 *
 * The reference (Erant/b2ctrain) has no FFI: its callers use the C++ API directly. Each entry point below
 * cites the C++ function it wraps, which in turn replaces the cited reference function.
 */
#ifndef B2C_H
#define B2C_H

#include <stddef.h>
#include <stdint.h>

#include "b2c_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct b2c_model b2c_model; /* b2c::Model     (src/model.h:14-40) */
typedef struct b2c_ctx b2c_ctx;     /* b2c::RenderCtx (src/gpu/render.h:66-95) + its HIP stream */
typedef struct b2c_view b2c_view;   /* b2c::ViewGPU   (src/gpu/loss.h:7-18) + owned device copies */

/* b2c::Camera (src/dataset/camera.h:8-36); pos is derived (-R^T t). */
typedef struct b2c_camera {
  int width, height;
  float fx, fy, cx, cy;
  float R[9];
  float t[3];
} b2c_camera;

/* The RenderParams fields this build supports (src/gpu/render.h:29-63). */
typedef struct b2c_render_opts {
  b2c_camera cam;
  int W, H; /* render size (CameraGPU::from rescales the intrinsics) */
  float bg[3];
  int sh_degree;
  int bwd_info;
  int feat_mode;            /* FeatureMode: 0 none, 1 normals (camera-space pseudo-normals), 2 buffer */
  const float* feat_buffer; /* device [n][3] with feat_mode 2 (b2c_device_upload) */
  const float* hollow_z;    /* device [W*H] reference surface depth (+inf = none), or NULL: no hollow loss */
  float hollow_margin, hollow_lam;
} b2c_render_opts;

/* LossParams (src/gpu/loss.h:20-30). */
typedef struct b2c_loss_opts {
  float l1_w, ssim_w;
  float bg[3];
  int composite, mask, alpha_lane;
  float match_alpha_weight, scale, grad_scale;
  float normal_scale; /* normal_loss weight */
} b2c_loss_opts;

typedef struct b2c_ctx_info {
  int W, H, tiles_x, tiles_y, n_tiles, tile_bits;
  uint32_t num_isect;
  uint64_t isect_cap;
} b2c_ctx_info;

/* Per-stage GPU times of one training step (hipEvents on the context's stream), milliseconds. backward_ms
 * covers the backward raster kernel (raster_bwd_ms) and the per-splat reduce that follows it (reduce_ms). */
typedef struct b2c_step_times {
  float project_ms, bin_ms, forward_ms, loss_ms, backward_ms, vjp_ms, total_ms;
  float raster_bwd_ms, reduce_ms;
} b2c_step_times;

const char* b2c_last_error(void);
int b2c_get_device_count(int* count);
/* CameraGPU::from (src/gpu/render.h:15-24), host only. */
int b2c_camera_gpu_from(const b2c_camera* cam, int W, int H, b2c_camera_gpu* out);

/* Model::upload (src/model.cu:44-80). floor [n] may be NULL (lscale.w = 0 as the reference uploads). */
b2c_model* b2c_model_create(void);
void b2c_model_destroy(b2c_model* m);
int b2c_model_upload(b2c_model* m, int n, int degree, int sh_fp16, const float* pos, const float* log_scale,
                     const float* quat, const float* opacity, const float* sh, const float* floor_);
/* Copy a model buffer to host: "pos_op", "quat", "lscale", "vis_weight", "vis_count", "refine_norm", "max_screen". */
int b2c_model_read(const b2c_model* m, const char* field, void* host, size_t bytes);
/* Copy host memory into a model buffer (same names as b2c_model_read, plus the Adam state and planar arrays
 * below). Synchronous. For callers that restore a checkpoint's optimizer state, and for tests. */
int b2c_model_write(b2c_model* m, const char* field, const void* host, size_t bytes);
/* Model::zero_optimizer (src/model.cu:104-107): moments, v_sh and last_step to zero, adam_t = 0. */
int b2c_model_zero_optimizer(b2c_model* m);
/* Model::adam_t: the last Adam step taken (0 after upload / zero_optimizer). */
int b2c_model_adam_t(const b2c_model* m, int* t);
/* Field names of the Adam state (src/model.h:19-28): "m_pos_op", "v_pos_op", "m_quat", "v_quat", "m_lscale",
 * "v_lscale" (float4 [n]), "v_sh" (float [n]), "last_step" (uint32 [n]); planar arrays, whole [lanes][cap]:
 * "sh_dc", "m_sh_dc" (fp32, 3 lanes) and "sh_hi" / "m_sh_hi" (binary16) or "sh_hi32" / "m_sh_hi32" (fp32)
 * for the 3K - 3 band lanes, by the model's band storage. */
/* Device address and size of a model buffer (same names), and the planar SH view the kernels take: for
 * FFI callers that launch their own kernels on the model, as the reference's refine / cage code reads
 * Model fields directly (src/model.h:14-40). */
int b2c_model_device_ptr(const b2c_model* m, const char* field, void** ptr, size_t* bytes);
int b2c_model_sh_view(const b2c_model* m, b2c_sh_view* out);

/* RenderCtx and RenderCtx::setup (src/gpu/render.cu:5-21). */
b2c_ctx* b2c_ctx_create(void);
void b2c_ctx_destroy(b2c_ctx* c);
int b2c_ctx_setup(b2c_ctx* c, int W, int H, int n_splats);
int b2c_ctx_info_get(const b2c_ctx* c, b2c_ctx_info* out);
/* Copy a RenderCtx buffer to / from host memory by field name ("proj0", "tile_count", "keys_sorted",
 * "vals_sorted", "tile_ranges", "out_rgba", "v_out", "v_splat", "grads", ...). Synchronous. */
int b2c_ctx_read(b2c_ctx* c, const char* field, void* host, size_t bytes);
/* Device address and size of a RenderCtx buffer by the same names: the reference's evidence / probe /
 * cage code reads ctx.tile_ranges, vals_sorted, proj0..3, last_idx and v_splat directly
 * (src/train/evidence.cu:224-229, src/gpu/probe.cu:52, src/gpu/cage_app.cu:454). */
int b2c_ctx_device_ptr(b2c_ctx* c, const char* field, void** ptr, size_t* bytes);
int b2c_ctx_write(b2c_ctx* c, const char* field, const void* host, size_t bytes);
int b2c_ctx_zero(b2c_ctx* c, const char* field);
int b2c_ctx_synchronize(b2c_ctx* c);
/* The context's HIP stream (hipStream_t) for callers that enqueue their own work around the path. */
void* b2c_ctx_stream(b2c_ctx* c);

/* A view: device copies of packed RGBA8 and optional u8 weights. */
b2c_view* b2c_view_create(int W, int H, const uint32_t* rgba, const uint8_t* weights);
void b2c_view_destroy(b2c_view* v);
/* ViewGPU::normals: a device copy of a packed RGBA8 normal map [W*H] (NULL removes it). */
int b2c_view_set_normals(b2c_view* v, const uint32_t* normals);
/* ViewGPU::labels: a device copy of per-pixel class ids [W*H] (NULL removes them), read by the evidence pass. */
int b2c_view_set_labels(b2c_view* v, const uint8_t* labels);
/* ViewGPU's flags (src/gpu/loss.h:13-15). */
int b2c_view_set_flags(b2c_view* v, int has_alpha, int masked, float alpha_coverage, float normal_count);
/* A device copy of host memory (for RenderParams' device arrays: feat_buffer, hollow_z), a device-to-host
 * copy, and the release. */
void* b2c_device_upload(const void* host, size_t bytes);
int b2c_device_download(void* host, const void* dev, size_t bytes);
void b2c_device_free(void* p);

/* ---- Splat clouds in brush's ply layout (src/ply.h:12-49) ---- */
typedef struct b2c_ply_info {
  int64_t n;
  int sh_degree;
  int binary; /* binary_little_endian (else ascii) */
  int has_scales, has_evidence, has_labels, has_fill, has_gate, has_gate_s, has_open;
} b2c_ply_info;
/* Host arrays of a cloud (SplatCloud's, coefficient-major SH [n][K][3]); NULL skips an array on read and
 * marks an optional block absent on write. */
typedef struct b2c_ply_arrays {
  float *pos, *log_scale, *quat, *opacity, *sh;
  float *evidence, *labels, *fill, *gate, *gate_s, *open;
} b2c_ply_arrays;
/* read_ply's view of a file without reading the rows: count, degree, flags (and its errors). */
int b2c_ply_info_get(const char* path, b2c_ply_info* out);
/* read_ply (src/ply.cpp:85-170) into caller-sized host arrays. */
int b2c_ply_read(const char* path, const b2c_ply_arrays* out);
/* write_ply (src/ply.cpp:180-226): desc gives n, sh_degree and the has_* flags of the optional blocks;
 * comments is '\n'-separated (or NULL). */
int b2c_ply_write(const char* path, const b2c_ply_info* desc, const b2c_ply_arrays* in, const char* comments);
/* ply_is_vertex_only (src/ply.cpp:63-83): 1 or 0 (-1 on an internal error). */
int b2c_ply_is_vertex_only(const char* path);
/* read_ply_comments joined by '\n' into buf (truncated to cap - 1 bytes; *needed = full length + 1). */
int b2c_ply_comments(const char* path, char* buf, size_t cap, size_t* needed);
/* Device-direct ply load into a model (Model::upload of read_ply without the host cloud; the rows are
 * decoded on the GPU) and save (write_ply of the model, rows encoded on the GPU). extras: optional blocks
 * as host arrays, flagged in extras_desc (both may be NULL). */
int b2c_model_load_ply(b2c_model* m, const char* path, int sh_fp16, int* has_scales);
int b2c_model_save_ply(const b2c_model* m, const char* path, const char* comments, const b2c_ply_info* extras_desc,
                       const b2c_ply_arrays* extras);

/* ---- COLMAP datasets (src/dataset/views.h:38, colmap.h:30): PNG frames and sidecars at their own size ---- */
typedef struct b2c_dataset b2c_dataset; /* b2c::Dataset */
typedef struct b2c_dataset_opts {
  const char* source;
  int max_frames;           /* < 0: all */
  unsigned max_resolution;  /* the reference's default is 1920 */
  int eval_split_every;     /* < 0: no eval split */
  int subsample_frames;     /* < 0: every frame */
  int alpha_mode;           /* -1 per view (masks/ sidecar: masked), 0 masked, 1 transparent */
} b2c_dataset_opts;
typedef struct b2c_view_info {
  int w, h;
  b2c_camera cam; /* at the loaded resolution */
  int has_alpha, masked, has_normals, has_weights, has_labels;
  float alpha_coverage;
  double normal_mask_count;
  char name[256];
} b2c_view_info;
/* load_dataset (views.cpp:74-253); NULL on failure (message in b2c_last_error). JPEG frames and frames
 * needing resampling are rejected. */
b2c_dataset* b2c_dataset_load(const b2c_dataset_opts* o);
void b2c_dataset_destroy(b2c_dataset* d);
/* split 0: train, 1: eval. */
int b2c_dataset_count(const b2c_dataset* d, int split);
int b2c_dataset_view_info(const b2c_dataset* d, int split, int i, b2c_view_info* out);
/* The view's packed planes into host arrays of w*h (NULL skips; an absent plane is not written). */
int b2c_dataset_view_read(const b2c_dataset* d, int split, int i, uint32_t* rgba, uint32_t* normals, uint8_t* weights,
                          uint8_t* labels);
/* A device view (ViewGPU) of a dataset view with its planes and flags, ready for the loss and evidence. */
b2c_view* b2c_dataset_view_upload(const b2c_dataset* d, int split, int i);
/* points3D.txt: *count points (xyz float [count][3], rgb uint8 [count][3]; NULL arrays to query the count). */
int b2c_dataset_points(const b2c_dataset* d, float* xyz, uint8_t* rgb, int64_t* count);
/* root, name and the initial ply path ('\n'-separated) into buf; counts[5] = masked, transparent, weighted,
 * normals, labels views. */
int b2c_dataset_summary(const b2c_dataset* d, char* buf, size_t cap, int* counts);

/* The loader's PNG decoder: *w, *h, *channels (in the file) and, when rgba is not NULL, the image as 8-bit
 * RGBA [h][w][4] (rgba_bytes must hold it). */
int b2c_png_decode(const char* path, int* w, int* h, int* channels, uint8_t* rgba, size_t rgba_bytes);

/* The loader's image decoder (the reference's stbi_load(path, &w, &h, &c, 4), views.cpp:63-72): PNG or JPEG
 * (baseline, extended sequential or progressive Huffman, 8-bit) chosen by the file's signature; outputs as
 * b2c_png_decode. */
int b2c_image_decode(const char* path, int* w, int* h, int* channels, uint8_t* rgba, size_t rgba_bytes);

/* The loader's resize (the reference's resize_rgba, views.cpp:73-78: stbir_resize of four independent 8-bit
 * channels, edges clamped): src [h][w][4] to dst [nh][nw][4]; filter 0 triangle, 1 Mitchell, 2 point
 * sample (views.cpp:158,169,191,202,209). */
int b2c_image_resample(const uint8_t* src, int w, int h, uint8_t* dst, int nw, int nh, int filter);

/* compute_evidence / download_evidence / download_labels (src/train/evidence.h:10-22) over nviews views and
 * their cameras: the evidence [n][7] = (w_in, w_all, err, views, dir xyz) and, with export_labels, the label
 * vote [n][2] = (winning class, share). Synchronous; the accumulators are module-level, as the reference's. */
int b2c_compute_evidence(b2c_ctx* c, const b2c_model* m, const b2c_view* const* views, const b2c_camera* cams,
                         int nviews, float normal_weight, int export_labels);
int b2c_download_evidence(const b2c_model* m, float* out);
int b2c_download_labels(const b2c_model* m, float* out);
/* probe_depth (src/gpu/probe.h:6-11) after b2c_project_splats + b2c_bin_and_sort: out is a device array of
 * W*H float4 (b2c_device_upload), ref_z a device array or NULL. Synchronous. */
int b2c_probe_depth(b2c_ctx* c, float tau, float delta, const float* ref_z, float margin, float* out);

/* render_forward / project_splats / bin_and_sort / rasterize_forward (src/gpu/render.h:97-103). */
int b2c_render_forward(b2c_ctx* c, const b2c_model* m, const b2c_render_opts* o);
int b2c_project_splats(b2c_ctx* c, const b2c_model* m, const b2c_render_opts* o);
int b2c_bin_and_sort(b2c_ctx* c, const b2c_model* m);
int b2c_rasterize_forward(b2c_ctx* c, const b2c_render_opts* o);
/* photometric_loss / accumulate_loss (src/gpu/loss.h:33-37). */
int b2c_photometric_loss(b2c_ctx* c, const b2c_view* v, const b2c_loss_opts* o);
int b2c_accumulate_loss(b2c_ctx* c);
/* normal_loss / hollow_loss / eval_metrics (src/gpu/loss.h:35-41): the normal-map loss into loss_accum[1]
 * with its gradient in "v_feat"; lam * sum of "hollow_pen" into loss_accum[0]; squared-error and SSIM
 * sums of the 8-bit render into loss_accum[4] and [5]. */
int b2c_normal_loss(b2c_ctx* c, const b2c_view* v, const b2c_loss_opts* o);
int b2c_hollow_loss(b2c_ctx* c, float lam);
int b2c_eval_metrics(b2c_ctx* c, const b2c_view* v, int mask_weighted);
/* rasterize_backward (mode 0) / rasterize_backward_tc (mode 1, divides by grad_scale) (src/gpu/render.h:105-109). */
int b2c_rasterize_backward(b2c_ctx* c, b2c_model* m, const b2c_render_opts* o, int mode, float grad_scale);
/* Flags of the gradient write: B2C_GRAD_ACCUMULATE sums into the "grads" buffer instead of overwriting it (this
 * build's extension for several views); B2C_GRAD_SPARSE leaves the rows of splats without a gradient this step
 * untouched (OptimParams::sparse, optim.cu:148: the kernel returns before the grad_out write). */
#define B2C_GRAD_ACCUMULATE 1
#define B2C_GRAD_SPARSE 2
/* optimizer_step with grad_out = the context's "grads" buffer [n][11 + 3K] (src/gpu/optim.h:50,
 * optim.cu:292-296); flags as above. */
int b2c_optimizer_grad(b2c_ctx* c, b2c_model* m, const b2c_render_opts* o, int active_deg, int flags);
/* The update half of OptimParams (src/gpu/optim.h:6-20, 36); b2c_adam_defaults fills the reference's
 * defaults. t = 0 takes the model's step counter plus one (op.t = ++model.adam_t, trainer.cpp:512). */
typedef struct b2c_adam_opts {
  int t;
  int sparse; /* lazy sparse Adam: splats without gradient keep their state and catch up when next seen */
  float beta1, beta2, eps;
  float lr_mean, lr_rot, lr_scale, lr_opac, lr_dc, lr_sh_rest;
  float noise_weight, noise_clamp; /* MCMC noise on the means; weight 0 disables */
  uint32_t seed, step;
} b2c_adam_opts;
void b2c_adam_defaults(b2c_adam_opts* a);
/* optimizer_step without grad_out (src/gpu/optim.h:50, optim.cu:99-377): the projection VJP and the fused
 * Adam / lazy sparse Adam / MCMC noise update of the model. The active SH degree is o->sh_degree. */
int b2c_optimizer_step(b2c_ctx* c, b2c_model* m, const b2c_render_opts* o, const b2c_adam_opts* a);
/* One training step as trainer.cpp:487-529 orders it (forward, loss with grad_scale, backward in `mode`,
 * projection VJP with the gradient flags above). The losses follow trainer.cpp:502-505: photometric, then
 * the normal-map loss when ro->feat_mode = 1, lo->normal_scale > 0 and the view has a normal map, then the
 * hollow loss when ro->hollow_z is set and hollow_lam != 0; loss_accum then holds [photometric + hollow,
 * normal, their sum, 1], what the trainer's per-step clear and accumulate_loss leave. times may be NULL
 * (no events recorded). */
int b2c_train_step(b2c_ctx* c, b2c_model* m, const b2c_view* v, const b2c_render_opts* ro, const b2c_loss_opts* lo,
                   int mode, int flags, b2c_step_times* times);
/* The same step ending in the fused update (b2c_optimizer_step) instead of the gradient write: a complete
 * training iteration (trainer.cpp:487-529). times->vjp_ms then covers the VJP with the update. */
int b2c_train_step_adam(b2c_ctx* c, b2c_model* m, const b2c_view* v, const b2c_render_opts* ro,
                        const b2c_loss_opts* lo, int mode, const b2c_adam_opts* a, b2c_step_times* times);

#ifdef __cplusplus
}
#endif
#endif
