/*
 * TEST INFRASTRUCTURE ONLY — the checker, never the product.
 *
 * CPU restatement of Erant/b2ctrain's differentiable splat rasterizer, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg. Nothing in b2ctrain_amd/ may link,
 * load or call it.
 *
 * Two independent paths:
 *   1. fp64 brute force (orc_ref_loss): restates tests/reference.cpp:34-143 — per-pixel compositing
 *      over every depth-sorted splat, full-image L1 + SSIM + alpha lane. No tiles.
 *   2. fp32 tiled (orc_project .. orc_vjp): restates the reference GPU pipeline step by step —
 *      src/gpu/splat_math.cuh, project.cu, binning.cu, raster_fwd.cu, raster_bwd.cu, loss.cu,
 *      optim.cu (grad_out path). Projection and binning are written so that, compiled with
 *      -ffp-contract=off, they are bit-exact with the HIP kernels (same operation order, IEEE
 *      division/sqrt, exp/log from the Cephes single-precision method in both).
 *
 * Every function cites the reference lines it follows. Pinning of each function (how it is checked
 * against something other than itself) is listed in tests/test_oracle_*.py.
 */
#ifndef B2C_ORACLE_H
#define B2C_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* CameraGPU after CameraGPU::from (src/gpu/render.h:8-25). R is world->camera, row major. */
typedef struct {
  float R[9];
  float t[3];
  float pos[3];
  float fx, fy, cx, cy;
  int W, H;
  float lim_pos_x, lim_pos_y, lim_neg_x, lim_neg_y;
} orc_cam_t;

/* Splat parameters in the Model's float4 layout (src/model.h:8-23); SH coefficient-major [n][K][3]
 * (SplatCloud layout, src/ply.h), already fp16-rounded when the model stores bands as fp16. */
typedef struct {
  int n, degree;
  const float* pos_op; /* [n][4] x, y, z, opacity logit */
  const float* quat;   /* [n][4] w, x, y, z (unnormalised) */
  const float* lscale; /* [n][4] log sx, log sy, log sz, floor f */
  const float* sh;     /* [n][K][3] */
} orc_model_t;

/* LossParams (src/gpu/loss.h:20-30). */
typedef struct {
  float l1_w, ssim_w;
  float bg[3];
  int composite, mask, alpha_lane;
  float match_alpha_weight, scale, grad_scale;
} orc_loss_params_t;

/* ---- deterministic single-precision math (Cephes expf / logf, S. L. Moshier) ---- */
float orc_expf(float x);
float orc_logf(float x);

/* Feature lanes and hollow loss of the tiled path (render.h:33-63): feat composites / back-propagates the
 * features in proj2.w and proj3; hollow_z (per pixel, +inf = no surface) adds the hollow penalty. */
typedef struct {
  int feat;
  const float* proj3;     /* [n][2] */
  const float* hollow_z;  /* [P] or NULL */
  float hollow_margin, hollow_lam;
  float* out_feat;        /* forward: [P][3] or NULL */
  float* hollow_pen;      /* forward: [P] or NULL */
  const float* v_feat;    /* backward: [P][4] */
} orc_ext_t;

/* The fp64 brute force's normals and hollow terms (tests/reference.h:8-16). */
typedef struct {
  int normals;
  const uint32_t* gtn;    /* [P] packed normal map */
  double normal_scale;
  const float* hollow_z;  /* [P] or NULL */
  double hollow_lam, hollow_margin;
} orc_ref_ext_t;

/* ---- fp32 tiled path ---- */

/* RenderCtx::setup tile geometry (src/gpu/render.cu:5-8). */
int orc_tile_bits(int n_tiles);

/* project.cu:8-84 with splat_math.cuh:224-293 (mip off, no feature lane, no warp / overrides).
 * Culled splats write only tile_count = 0 (the other outputs are left untouched). */
void orc_project(const orc_model_t* m, const orc_cam_t* cam, int active_deg, int tiles_x, int tiles_y,
                 float* proj0, float* proj1, float* proj2, float* proj3,
                 uint32_t* tile_count, uint32_t* hit_info /* [n][2] */);

/* project.cu:82-83: max_screen[i] = max(max_screen[i], max(ex / W, ey / H)) for every splat that survives
 * the projection's culls. */
void orc_max_screen(const orc_model_t* m, const orc_cam_t* cam, float* max_screen);

/* The same with the feature lanes (feat_mode 1: pseudo-normals, 2: feat_buffer [n][3], project.cu:63-77). */
void orc_project_feat(const orc_model_t* m, const orc_cam_t* cam, int active_deg, int tiles_x, int tiles_y,
                      float* proj0, float* proj1, float* proj2, float* proj3, uint32_t* tile_count, uint32_t* hit_info,
                      int feat_mode, const float* feat_buffer);

/* binning.cu:109-143: depth sort (stable on z bits, culled last), count scan in depth order, emit
 * in depth order, stable sort by tile id, per-tile ranges. Returns M (number of intersections).
 * keys/vals are written only when M <= cap. order/tile_off are [n]; tile_ranges is [n_tiles][2]. */
uint32_t orc_bin(int n, const uint32_t* tile_count, const uint32_t* hit_info, const float* proj0,
                 const float* proj1, int tiles_x, int tiles_y, uint32_t cap,
                 uint32_t* order, uint32_t* tile_off, uint32_t* keys_sorted, uint32_t* vals_sorted,
                 uint32_t* tile_ranges);

/* raster_fwd.cu:8-71 (BWD on, no feature, no hollow). Shrinks tile_ranges[t].y in place.
 * out_rgba [P][4], out_T [P], last_idx [P]. */
void orc_raster_fwd(int W, int H, int tiles_x, int tiles_y, const float bg[3], uint32_t* tile_ranges,
                    const uint32_t* vals_sorted, const float* proj0, const float* proj1, const float* proj2,
                    float* out_rgba, float* out_T, uint32_t* last_idx);

void orc_raster_fwd_ext(int W, int H, int tiles_x, int tiles_y, const float bg[3], uint32_t* tile_ranges,
                        const uint32_t* vals_sorted, const float* proj0, const float* proj1, const float* proj2,
                        float* out_rgba, float* out_T, uint32_t* last_idx, const orc_ext_t* ext);

/* loss.cu:18-195 restated over the whole image in double precision (zero padding, 11-tap
 * Gaussian sigma 1.5 normalised, loss.cu:296-303). pred is [P][4] float (rgb + alpha), gt packed
 * RGBA8, weights u8 or NULL. Returns the loss value; writes v_out [P][4] (scaled by grad_scale)
 * when v_out is not NULL. */
double orc_photometric(int W, int H, const float* pred, const uint32_t* gt, const uint8_t* weights,
                       const orc_loss_params_t* lp, float* v_out);

/* raster_bwd.cu:37-139 (fp32 per-fragment math, double accumulators). v_splat [n][13] and
 * vis_weight [n] are accumulated (caller zeroes them); vis_flag [n] set to 1 for contributors.
 * Every accumulated lane is multiplied by inv_gscale (1 for the fp32 kernel's semantics). */
void orc_raster_bwd(int W, int H, int tiles_x, int tiles_y, const float bg[3], const uint32_t* tile_ranges,
                    const uint32_t* vals_sorted, const float* proj0, const float* proj1, const float* proj2,
                    const float* out_rgba, const float* out_T, const uint32_t* last_idx, const float* v_out,
                    float inv_gscale, double* v_splat, uint32_t* vis_flag, double* vis_weight);

void orc_raster_bwd_ext(int W, int H, int tiles_x, int tiles_y, const float bg[3], const uint32_t* tile_ranges,
                        const uint32_t* vals_sorted, const float* proj0, const float* proj1, const float* proj2,
                        const float* out_rgba, const float* out_T, const uint32_t* last_idx, const float* v_out,
                        float inv_gscale, double* v_splat, uint32_t* vis_flag, double* vis_weight, const orc_ext_t* ext);

/* loss.cu:206-238: returns the normal loss, writes v_feat [P][4]. */
double orc_normal_loss(int W, int H, const float* feat, const uint32_t* normals, const uint8_t* weights, float scale,
                       float grad_scale, float* v_feat);
/* loss.cu:197-204 without lam: the sum of the per-pixel penalties. */
double orc_hollow_sum(int npix, const float* pen);
/* loss.cu:240-286: sums of the squared error and of SSIM over pixels and channels. */
void orc_eval(int W, int H, const float* pred, const uint32_t* gt, int mask_weighted, double* sum_se, double* sum_ssim);

#define ORC_LABEL_BINS 32 /* evidence.cu:38 */
/* evidence_kernel and label_vote_kernel (evidence.cu:47-112, 141-183) of one rendered view, given the forward's
 * tile_ranges, out_rgba [P][4], out_feat [P][3] (read when normals and normal_weight > 0) and last_idx:
 * view_acc [n][3] += (w_in, err, w_all) and, when labels and label_acc are given, label_acc [n][32] += the
 * per-class weight. Caller zeroes. */
void orc_evidence_view(int W, int H, int tiles_x, int tiles_y, const uint32_t* tile_ranges, const uint32_t* vals_sorted,
                       const float* proj0, const float* proj1, const float* out_rgba, const float* out_feat,
                       const uint32_t* last_idx, const uint32_t* gt, const uint32_t* normals, const uint8_t* weights,
                       const uint8_t* labels, int masked_has_alpha, float normal_weight, double* view_acc,
                       double* label_acc);
/* probe_kernel (probe.cu:7-45): out [P][4] = (A, z_first, deep, behind); ref_z may be NULL. */
void orc_probe(int W, int H, int tiles_x, int tiles_y, const uint32_t* tile_ranges, const uint32_t* vals_sorted,
               const float* proj0, const float* proj1, float tau, float delta, const float* ref_z, float margin,
               float* out);

/* optim.cu:99-253 + grad_out (292-296): projection VJP, fp32. grad_out [n][11 + 3K]. */
void orc_vjp(const orc_model_t* m, const orc_cam_t* cam, int active_deg, const float* v_splat,
             const uint32_t* vis_flag, const uint32_t* tile_count, float* grad_out);

/* ---- fp64 brute force (tests/reference.cpp:34-143) ----
 * Parameters in SplatCloud layout, double: pos [n][3], log_scale [n][3], quat [n][4] (w,x,y,z),
 * opacity [n], sh [n][K][3]. floor [n] (may be NULL = 0) and degree 4 extend the reference
 * (which has neither); with floor 0 and degree <= 3 the arithmetic is the reference's.
 * The camera is used as given (fx/fy/cx/cy at the render size; the clamp limits are recomputed in
 * double from W/H as reference.cpp:37-38 does). float_exp = 1 evaluates exp(log scale) and
 * exp(-opacity logit) in single precision, as the reference does (its std::exp receives floats);
 * 0 keeps them in double. out_img [P][4] (rgb + bg, alpha) may be NULL. */
double orc_ref_loss(int n, int degree, const double* pos, const double* log_scale, const double* quat,
                    const double* opacity, const double* sh, const double* floor_, const orc_cam_t* cam,
                    int W, int H, const double bg[3], const uint32_t* gt, const uint8_t* weights,
                    int composite, int mask, int alpha_lane, double l1_w, double ssim_w,
                    double match_alpha_weight, double scale, int float_exp, double* out_img);

double orc_ref_loss_ext(int n, int degree, const double* pos, const double* log_scale, const double* quat,
                        const double* opacity, const double* sh, const double* floor_, const orc_cam_t* cam, int W, int H,
                        const double bg[3], const uint32_t* gt, const uint8_t* weights, int composite, int mask,
                        int alpha_lane, double l1_w, double ssim_w, double match_alpha_weight, double scale, int float_exp,
                        double* out_img, const orc_ref_ext_t* rx);

/* Bounded sample for the CPU baseline: after orc_ref_set_sample(s) with s > 1, orc_ref_loss renders only the
 * pixels whose row-major index is a multiple of s, skips the loss (returns 0) and records the compositing
 * time, read by orc_ref_composite_seconds(); orc_ref_set_sample(1) restores the full loss. */
void orc_ref_set_sample(uint64_t stride);
double orc_ref_composite_seconds(void);

/* Host threads of orc_raster_fwd / orc_raster_bwd (OpenMP over tiles); 1 by default (fixed summation order). */
void orc_set_threads(int n);

/* ---- internal pieces exported for the pinning tests ---- */
/* The raster kernels' fragment sigma of a splat (centre mx, my; conic c00, c01, c11) at a pixel centre
 * (pcx, pcy): the quadratic about the centre of the pixel's 8x8 tile. */
void orc_frag_sigma(int n, const float* mx, const float* my, const float* c00, const float* c01, const float* c11,
                    const float* pcx, const float* pcy, float* out);
void orc_sh_basis_f(int deg, float x, float y, float z, float* out);      /* splat_math.cuh:122-145 */
/* The projection's cull decision for one splat (pr.ok of splat_math.cuh:224-293). */
int orc_project_ok(const float* po, const float* q, const float* ls, const orc_cam_t* cam);
void orc_sh_basis_d(int deg, double x, double y, double z, double* out);  /* reference.cpp:16-30 (+ degree 4) */
void orc_quat_to_mat(const float* q, float* R);                           /* util.cuh:235-243 */
int orc_tile_hit(float rmin_x, float rmin_y, float rmax_x, float rmax_y, float mx, float my, float c00, float c01,
                 float c11, float power);                                 /* splat_math.cuh:27-41 */

/* ---- fused optimizer (optim.cu:104-148, 298-377), restated in oracle/orc_adam.c ---- */
/* One Adam step's constants (b2c_adam_step of include/b2c_kernels.h, field for field). */
typedef struct {
  int t, sparse;
  float beta1, beta2, eps;
  float bc1, bc2, ln_beta1, ln_beta2, ratio, ln_ratio;
  float lr_mean, lr_rot, lr_scale, lr_opac, lr_dc, lr_sh_rest;
  float noise_weight, noise_clamp;
  uint32_t seed, step;
} orc_adam_step_t;

/* bc1 = 1 / (1 - beta1^t), bc2 likewise, ln beta1, ln beta2, ratio = beta1 / sqrt(beta2), ln ratio:
 * formed in double, rounded to float. */
void orc_adam_constants(orc_adam_step_t* s);

/* A model with its Adam state in host arrays: float4 fields [n][4]; SH and their first moments
 * coefficient-major [n][K][3]. sh_half = 1: the band lanes (k >= 1) hold binary16 values (as floats) and
 * are stored back as the model stores them (parameters stochastically rounded, moments to nearest). */
typedef struct {
  int n, degree, sh_half;
  float* pos_op, *quat, *lscale, *sh;
  float* m_pos_op, *v_pos_op, *m_quat, *v_quat, *m_lscale, *v_lscale;
  float* m_sh, *v_sh;
  uint32_t* last_step;
} orc_adam_model_t;

/* The update of every splat from its gradient row grads [n][11 + 3K] (the projection VJP's output for this
 * v_splat), v_splat [n][13], vis_flag and tile_count as the optimizer reads them (optim.cu:104-148). */
void orc_adam_update(orc_adam_model_t* m, const orc_cam_t* cam, int active_deg, const float* v_splat,
                     const uint32_t* vis_flag, const uint32_t* tile_count, const float* grads,
                     const orc_adam_step_t* s);

/* Pieces of the update exported for the pinning tests. */
uint32_t orc_mix32(uint32_t x);                            /* util.cuh:106-110, the chain's finaliser */
float orc_hash_unit(uint32_t a, uint32_t b, uint32_t c);   /* util.cuh:106-112 */
float orc_hash_gauss(uint32_t a, uint32_t b, uint32_t c);  /* util.cuh:114-117 */
float orc_cos_turns(float u);                              /* cos(2 pi u), u in [0, 1) */
uint16_t orc_f16_bits(float v);                            /* binary16, round to nearest even */
float orc_f16_value(uint16_t h);
uint16_t orc_f16_stochastic(float v, float u01);           /* util.cuh:148-162 */

#ifdef __cplusplus
}
#endif
#endif
