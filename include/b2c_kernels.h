/*
 * b2c_kernels.h — the C-ABI launcher layer of the MI355X (gfx950) splat rasterizer.
 *
 * Plain structs of device pointers and sizes; every launcher enqueues its HIP kernels on `stream`
 * and returns a hipError_t as int (0 = success). No allocation happens in any launcher: scratch
 * buffers are passed in by the caller (the C++ RenderCtx owns them). The C++ drop-in API in
 * b2ctrain_amd/csrc/b2c/{render,loss,optim}.h is built on these; the reference's equivalents are
 * the static kernels and launch code cited on each entry point (paths relative to Erant/b2ctrain).
 */
#ifndef B2C_KERNELS_H
#define B2C_KERNELS_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* CameraGPU after CameraGPU::from (src/gpu/render.h:8-25); also the kernels' CamDev (splat_math.cuh:219-221). */
typedef struct b2c_camera_gpu {
  float R[9]; /* world -> camera, row major */
  float t[3];
  float pos[3]; /* camera centre, world */
  float fx, fy, cx, cy;
  int W, H;
  float lim_pos_x, lim_pos_y, lim_neg_x, lim_neg_y; /* EWA Jacobian clamp */
} b2c_camera_gpu;

/* Planar SH view (ShBuf, src/gpu/util.cuh:129-164): DC lanes fp32 in dc[lane*stride + i]; lanes >= 3 in
 * hi32 (fp32) or hi16 (IEEE binary16) at [(lane-3)*stride + i]. Exactly one of hi16/hi32 is used when
 * the degree is > 0 (hi32 wins when both are set). */
typedef struct b2c_sh_view {
  const float* dc;
  const uint16_t* hi16;
  const float* hi32;
  size_t stride;
} b2c_sh_view;

/* ---- projection: replaces project_kernel / project_splats (src/gpu/project.cu:8-126) ---- */
typedef struct b2c_project_args {
  int n, degree, active_deg;
  const float* pos_op; /* [n] float4 (x, y, z, opacity logit) */
  const float* quat;   /* [n] float4 (w, x, y, z) */
  const float* lscale; /* [n] float4 (log s xyz, floor) */
  b2c_sh_view sh;
  b2c_camera_gpu cam;
  int tiles_x, tiles_y;
  float* proj0;        /* [n] float4 (x, y, c00, c01); proj0..3 may all be NULL (not written) */
  float* proj1;        /* [n] float4 (c11, opacity, depth, power) */
  float* proj2;        /* [n] float4 (r, g, b, feat.x) */
  float* proj3;        /* [n] float2 (feat.y, feat.z) */
  uint32_t* tile_count;/* [n] */
  uint32_t* depth_bits;/* [n]: the depth sort key of each splat (b2c_hip_depth_keys' keys, formed here): the bits
                          of its camera depth (proj1.z), or 0xFFFFFFFF for a splat without tiles */
  uint32_t* hit_info;  /* [n] uint2 (hit mask or 0xFFFFFFFF, min_x | min_y << 12 | bw << 24) */
  uint32_t* hit_wide;  /* [n] uint2, written where hit_info's mask word is 0xFFFFFFFF: the 64-bit hit mask
                          (low word first, bits in row-major bbox order) of a bbox of at most 64 tiles, or
                          (0, 0) for a bbox of more than 64 tiles */
  float* max_screen;   /* [n] or NULL: max(., max(ex/W, ey/H)) (project.cu:82-83) */
  float* raster_rec;   /* [n][16]: the raster kernels' per-splat record, one 64-byte line: (mx, my, c00/2, c01),
                          (c11/2, opacity, power, sign bits of r, g, b), (max(r,0), max(g,0), max(b,0), log2 opacity),
                          (feat.x, feat.y, feat.z, camera depth) */
  uint32_t* big_list;  /* [n] scratch: splats whose bbox exceeds 64 tiles */
  uint32_t* big_count; /* [2] scratch counters, 8-byte aligned: [0] big-list entries, [1] big work items */
  uint32_t* big_info;  /* [n][4] scratch: per big-list entry, bbox origin, width, area, chunk length */
  uint32_t* big_chunk; /* [n][B2C_BIG_CHUNKS] scratch: per-chunk hit counts of each entry */
  uint32_t* big_items; /* [n][B2C_BIG_CHUNKS] scratch: work items (entry << 5 | chunk) */
  uint32_t* big_items_count; /* big_count + 1 (both are bumped in one 64-bit atomic) */
  int feat_mode;       /* FeatureMode (render.h:27): 0 none, 1 normals (the camera-space pseudo-normal: the
                          shortest semi-axis, turned to face the camera), 2 buffer (feat_buffer, clamped) */
  const float* feat_buffer; /* [n][3] when feat_mode = 2 */
  uint32_t* clear_next;     /* No reference counterpart: NULL, or a second pair of counters like big_count
                               (8-byte aligned) that the next projection will use. When set, big_count and
                               big_items_count must already be zero (the launcher then queues no clearing
                               launch) and the kernel zeroes clear_next instead: callers alternate two pairs. */
} b2c_project_args;

/* At most this many chunks per big splat (one wave each); and the grid (workgroups of 256) that the
 * chunk kernels stride over. */
#define B2C_BIG_CHUNKS 32
#define B2C_BIG_GRID 8192
int b2c_hip_project(const b2c_project_args* a, hipStream_t stream);

/* ---- binning (src/gpu/binning.cu:10-143) ---- */

/* Radix-sort scratch: bytes needed to sort up to n pairs (LSD, 8-bit digits, reduce-then-scan); monotone in n. */
size_t b2c_radix_sort_temp_bytes(uint32_t n);

/* Stable LSD key-value radix sort of keys_in/vals_in over bits [begin_bit, end_bit) into keys_out/vals_out
 * (replaces cub::DeviceRadixSort::SortPairs, binning.cu:116-118,140-142). keys_alt/vals_alt are ping-pong
 * buffers of n entries; the inputs are not modified. vals_in may be NULL: the values are then the input
 * positions 0 .. n-1 (vals_out receives the sorting permutation). n_dev (may be NULL) points at a device
 * copy of n: the launch covers n entries, the kernels read the live count from n_dev when it is set (n is
 * then the capacity). The key buffers (keys_in, keys_out, keys_alt) must be 16-byte aligned. */
int b2c_hip_radix_sort_pairs(const uint32_t* keys_in, const uint32_t* vals_in, uint32_t* keys_out, uint32_t* vals_out,
                             uint32_t* keys_alt, uint32_t* vals_alt, uint32_t n, const uint32_t* n_dev, int begin_bit,
                             int end_bit, void* temp, size_t temp_bytes, hipStream_t stream);

/* The same sort carrying a second value array (vals2_in -> vals2_out, ping-pong vals2_alt); the tile pass
 * uses it to sort (tile, emit position, splat id) in one go. vals_in may be NULL as above. */
int b2c_hip_radix_sort_kv2(const uint32_t* keys_in, const uint32_t* vals_in, const uint32_t* vals2_in,
                           uint32_t* keys_out, uint32_t* vals_out, uint32_t* vals2_out, uint32_t* keys_alt,
                           uint32_t* vals_alt, uint32_t* vals2_alt, uint32_t n, const uint32_t* n_dev, int begin_bit,
                           int end_bit, void* temp, size_t temp_bytes, hipStream_t stream);

/* depth_keys_kernel (binning.cu:10-15): key = bits of view z if tile_count > 0 else 0xFFFFFFFF, val = index;
 * the depth bits come from b2c_hip_project's depth_bits (keys may be that array: the update is in place). */
int b2c_hip_depth_keys(int n, const uint32_t* tile_count, const uint32_t* depth_bits, uint32_t* keys, uint32_t* vals,
                       hipStream_t stream);

/* Scratch bytes of b2c_hip_scan_counts for n splats. */
size_t b2c_scan_temp_bytes(uint32_t n);

/* permute_counts_kernel + cub::DeviceScan::InclusiveSum (binning.cu:16-19,120-124): tile_off[r] = sum over
 * r' <= r of tile_count[order[r']]; the total is written to *total_dev. */
int b2c_hip_scan_counts(int n, const uint32_t* order, const uint32_t* tile_count, uint32_t* tile_off,
                        uint32_t* total_dev, void* temp, size_t temp_bytes, hipStream_t stream);

/* The same scan, also storing the total into total_host: pinned host memory (hipHostMalloc) given by its
 * device address (hipHostGetDevicePointer). The reference copies the total back with cudaMemcpy
 * (binning.cu:125-126); this delivers it from the scan's last workgroup without a copy launch. The value is
 * visible to the host once the scan has completed (an event recorded after it); n must be positive. */
int b2c_hip_scan_counts_host(int n, const uint32_t* order, const uint32_t* tile_count, uint32_t* tile_off,
                             uint32_t* total_dev, uint32_t* total_host, void* temp, size_t temp_bytes,
                             hipStream_t stream);

/* emit_kernel (binning.cu:25-93): intersections in depth order, key = tile id, val = splat index. Splats of
 * at most 64 bbox tiles (the hit mask of hit_info, or of hit_wide for 33 to 64 tiles and for a full
 * 32-tile mask) are dealt out over the lanes of a wave, each intersection the k-th set bit of its splat's
 * mask; splats with more than 64 bbox tiles are emitted by one wave per chunk of their bbox (the chunks
 * b2c_hip_project counted), in row-major order: the reference's serial re-test of every splat over 32
 * tiles gives the same lists, since the bbox and the tile test are the projection's. Slots a big splat does not fill get key = n_tiles (cannot happen when the counts come
 * from b2c_hip_project; kept as the reference's guard). */
typedef struct b2c_emit_args {
  int n;
  const uint32_t* order, *tile_count, *tile_off, *hit_info;
  const uint32_t* hit_wide;             /* from b2c_hip_project */
  const float* raster_rec;              /* [n][16] from b2c_hip_project: the big splats' centre, conic, power */
  int tiles_x, tiles_y;
  uint32_t cap;
  uint32_t* keys, *vals;
  const uint32_t* big_list, *big_count; /* from b2c_hip_project */
  const uint32_t* big_info, *big_chunk; /* from b2c_hip_project */
  const uint32_t* big_items, *big_items_count; /* from b2c_hip_project */
  uint32_t* big_base;                   /* [n] scratch: first slot of each big splat */
} b2c_emit_args;
int b2c_hip_emit(const b2c_emit_args* a, hipStream_t stream);

/* tile_ranges_kernel (binning.cu:95-105), every tile written (empty tiles [0, 0)): ranges[t] = [first, last) of tile t, and
 * tile_end[t] = last (may be NULL; a copy the forward does not shrink; n_tiles + 1 entries, the last = the
 * position where the sentinel keys of an emit shortfall start, m if there are none). When slot_sorted is set (the
 * permutation from an index sort of the emitted keys), also writes vals_sorted[i] = vals[slot_sorted[i]]:
 * the splat ids in list order, as the reference's key-value sort leaves them. keys_sorted must be 16-byte
 * aligned. */
int b2c_hip_tile_ranges(uint32_t m, const uint32_t* m_dev, const uint32_t* keys_sorted, const uint32_t* slot_sorted,
                        const uint32_t* vals, uint32_t* vals_sorted, uint32_t n_tiles, uint32_t* ranges,
                        uint32_t* tile_end, hipStream_t stream);

/* ---- rasterization ---- */

/* raster_fwd_kernel<FEAT, BWD, HOLLOW> / rasterize_forward (src/gpu/raster_fwd.cu:8-90). With feat the
 * feature lanes are composited into out_feat.xyz (no background term); with hollow_z each pixel's penalty
 * sum of vis * clamp((z - z_ref - margin) / max(margin, 1e-4), 0, 1) goes to hollow_pen. */
typedef struct b2c_raster_fwd_args {
  uint32_t* tile_ranges;      /* [n_tiles] uint2; .y shrunk in place when bwd_info */
  const uint32_t* vals_sorted;
  const float* proj0, *proj1, *proj2;
  const float* raster_rec;    /* [n][16] from b2c_hip_project (the same values, one line per splat) */
  int W, H, tiles_x, tiles_y;
  float bg[3];
  int bwd_info;
  float* out_rgba;            /* [P] float4 */
  float* out_feat;            /* [P] float4 (feat xyz, T) */
  uint32_t* last_idx;         /* [P] */
  int feat;                   /* composite the feature lanes (raster_rec[3].xyz) */
  const float* hollow_z;      /* [P] reference surface depth (+inf = none) or NULL */
  float hollow_margin;
  float* hollow_pen;          /* [P] with hollow_z */
  /* No reference counterpart (read by this build's MFMA backward): with bwd_info and cvals set, the forward
   * also writes each tile's compacted list, the entries of its range that at least one pixel composited, in
   * list order: their splat ids to cvals and their emit positions (from slot_sorted) to cslots at
   * [range.x, cend[tile]), and per pixel clast, one past its last composited entry in that list (range.x when
   * none). The entries left out have alpha = 0 at every pixel of the tile. */
  const uint32_t* slot_sorted;
  uint32_t* cvals, *cslots;   /* [M] */
  uint32_t* clast;            /* [P] */
  uint32_t* cend;             /* [n_tiles] */
} b2c_raster_fwd_args;
int b2c_hip_raster_fwd(const b2c_raster_fwd_args* a, hipStream_t stream);

/* Backward through compositing: raster_bwd_kernel (fp32 reduction, src/gpu/raster_bwd.cu:10-156) when
 * mode = 0, raster_bwd_tc_kernel (src/gpu/raster_bwd_tc.cu:29-225; here MFMA f16 split hi/lo with fp32
 * accumulation) when mode = 1. Gradients are multiplied by inv_gscale (mode 1 semantics; pass 1 for mode 0
 * to match the reference's fp32 kernel).
 *
 * Mode 0 accumulates into v_splat / vis_weight with float atomics, as the reference does. Mode 1 uses no
 * atomics: each (tile, splat) pair writes a 12-float row of raw moments about the tile centre (sum v_sigma
 * * [v, u^2, uv, v^2] | sum v_sigma * [1, u], sum of blend weights, refine sum | sum vis * v_rgb, tile id) to
 * isect_rows[slot_sorted[i]] for the entries of the shrunk ranges, with the tag word row_tag | tile in its
 * last float; the rows of one splat are then a contiguous run in emit order, which a segmented reduction
 * turns into gradient lanes (tile centre from the tag's tile bits), sums in a fixed order and adds to
 * v_splat, vis_weight and vis_flag. A row whose tag bits (outside tile_mask) differ from row_tag was not
 * written by this pass (a pair past its tile's shrunk end, or a sentinel entry) and counts as zero, so
 * those rows are neither written nor cleared. The caller passes a row_tag that no row of the buffer holds
 * unless this pass wrote it (a fresh tag per pass; the buffer cleared before a tag repeats and whenever the
 * row layout or tile_mask changes). The result is deterministic. */
typedef struct b2c_raster_bwd_args {
  const uint32_t* tile_ranges;
  const uint32_t* vals_sorted;
  const float* proj0, *proj1, *proj2;
  const float* raster_rec;    /* [n][16] from b2c_hip_project */
  const float* out_rgba, *out_feat;
  const uint32_t* last_idx;
  const float* v_out;         /* [P] float4 dL/d(rgb, alpha) */
  int W, H, tiles_x, tiles_y;
  float bg[3];
  float inv_gscale;
  int mode;
  float* v_splat;             /* [n][13], accumulated */
  int v_splat_zero;           /* mode 1: the caller knows v_splat is all zero on entry (the invariant of the
                                 reference's training step, optim.cu:111-121): the sums are stored without
                                 reading it */
  uint32_t* vis_flag;         /* [n] */
  float* vis_weight;          /* [n] or NULL */
  /* mode 1 only */
  uint32_t num_isect;         /* M */
  const uint32_t* slot_sorted;/* [M] emit position of list entry i */
  const uint32_t* isect_vals; /* [M] splat id of emit position s (the emit kernel's values) */
  const uint32_t* tile_count; /* [n] intersections per splat (the length of its run of emit positions) */
  float* isect_rows;          /* [M][16] scratch (12 floats a row are used without feat) */
  uint32_t row_tag;           /* this pass's tag bits (none inside tile_mask, not 0) */
  uint32_t tile_mask;         /* tag bits that hold the tile id: 2^tile_bits - 1, tile ids < 2^tile_bits */
  uint32_t* row_live;         /* [M] or NULL: when given, each written row's tag word is also stored here at
                                 the row's emit position, and the reduce reads only the rows whose word here
                                 is this pass's tag (lists shrunk to a small share of their pairs leave most
                                 rows unread). Same tag contract as isect_rows (cleared with it). */
  float* isect_part;          /* [ceil(M / 256)][32] scratch: partial sums of runs crossing 256-row windows */
  uint32_t* isect_part_flags; /* [ceil(M / 256)] scratch */
  void* split_event;          /* optional hipEvent_t recorded between the raster kernel and the reduce */
  /* feature lanes and hollow loss (raster_bwd.cu:84-110, raster_bwd_tc.cu:126-141) */
  int feat;                   /* v_feat back through the composited feature lanes, into v_splat[10..12] */
  const float* v_feat;        /* [P] float4 with feat */
  const float* proj3;         /* [n] float2 (feature y, z): mode 0 with feat */
  const float* hollow_z;      /* [P] or NULL */
  float hollow_margin;
  float hollow_lam;           /* dL / d(penalised weight) per pixel in v_out's units (times grad_scale) */
  /* mode 1, no reference counterpart: when cvals is set, the compacted lists of a forward run with them
   * (b2c_raster_fwd_args) replace vals_sorted / slot_sorted / last_idx and the range end: tile t walks
   * [tile_ranges[t].x, cend[t]) of cvals / cslots, each pixel up to its clast. The entries left out
   * composited nowhere in the tile, so their rows are zero and stay unwritten. */
  const uint32_t* cvals, *cslots, *clast, *cend;
  /* No reference counterpart (set by this build's fused training step only): mode 1 without feat, with
   * v_splat_zero. Each visible splat's blend-weight sum is stored in v_splat lane 10 (a feature lane, unused
   * without feat) and neither vis_flag nor vis_weight is touched; the projection VJP, run with vis_from_row,
   * then derives the flag from that lane and adds it to vis_weight (the same sums as a pass without it). */
  int defer_vis;
} b2c_raster_bwd_args;
int b2c_hip_raster_bwd(const b2c_raster_bwd_args* a, hipStream_t stream);

/* ---- loss: photometric_kernel / photometric_loss (src/gpu/loss.cu:18-195,296-315) ----
 * Images up to 2^28 pixels (16 P bytes of out_rgba must fit 32-bit buffer offsets); larger ones return
 * hipErrorInvalidValue. */
typedef struct b2c_loss_args {
  const float* pred;          /* [P] float4 out_rgba */
  const uint32_t* gt;         /* [P] packed RGBA8 */
  const uint8_t* weights;     /* [P] or NULL */
  int W, H;
  float l1_w, ssim_w, bg[3];
  int composite, mask, alpha_lane;
  float match_alpha_weight, scale, grad_scale;
  float* v_out;               /* [P] float4 */
  float* loss_accum;          /* [0] += loss */
  float* partials;            /* scratch, b2c_loss_partials(W, H) floats: per-workgroup sums, reduced in a
                                 fixed order in double (deterministic); NULL = float atomics as the reference */
  int assign;                 /* with partials: loss_accum[0] = loss and loss_accum[1] = 0 (the second loss
                                 term, absent from this build) instead of adding, so the caller need not clear */
  int running;                /* with assign: also loss_accum[2] += loss_accum[0] + loss_accum[1] and
                                 loss_accum[3] += 1, the accumulate_kernel update (loss.cu:317,324), in the same
                                 launch */
  int* defer_sum_count;       /* No reference counterpart: NULL, or (with partials) a host int that receives the
                                 number of partials; the reduction into loss_accum is then not launched, and the
                                 caller hands it to b2c_hip_vjp (b2c_vjp_args.loss_partials). The allocation-free
                                 variant rejects it. */
} b2c_loss_args;
size_t b2c_loss_partials(int W, int H);
int b2c_hip_photometric(const b2c_loss_args* a, hipStream_t stream);

/* Allocation-free variant of b2c_hip_photometric. It has no counterpart in the reference: it is for callers
 * that cannot allocate device memory or pass a workspace (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). a->partials is ignored; the per-workgroup partial sums live in a
 * fixed device array of B2C_LOSS_STATIC_PARTIALS floats (1 MiB) that each GPU holds for the life of the
 * process, so images with b2c_loss_partials(W, H) above that (about 160 megapixels) are rejected with
 * hipErrorInvalidValue before any work is queued. No hipMalloc, hipFree or allocating routine is called.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller. Results are bit-identical to b2c_hip_photometric
 * called with a partials workspace (assign 0 or 1): that form sums the partials in the same fixed order;
 * b2c_hip_photometric without a workspace adds per-wave float atomics in hardware order instead. */
#define B2C_LOSS_STATIC_PARTIALS (1 << 18)
int b2c_hip_photometric_noalloc(const b2c_loss_args* a, hipStream_t stream);

/* accumulate_kernel (loss.cu:317,324): a[2] += a[0] + a[1]; a[3] += 1. */
int b2c_hip_accumulate_loss(float* loss_accum, hipStream_t stream);
/* a[2] = a[0] + a[1]; a[3] = 1: what the trainer's per-step clear of a[0..3] followed by accumulate_kernel
 * leaves, for a step whose losses were assigned rather than added. */
int b2c_hip_step_loss_sums(float* loss_accum, hipStream_t stream);

/* ---- the other losses (src/gpu/loss.cu:197-293, 317-338) ----
 * Each sums its per-workgroup partials in a fixed order in double precision (deterministic); `partials` is
 * scratch of b2c_aux_partials(W, H) floats. */
size_t b2c_aux_partials(int W, int H);

/* normal_loss_kernel (loss.cu:206-238): for pixels whose normal-map alpha is above 127, scale * w *
 * (|p - g|_1 + 1 - cos(p, g)) with g decoded as [+X, -Y, -Z]; the gradient (times grad_scale) to v_feat
 * (zero elsewhere), the loss added to loss_accum[1]. */
typedef struct b2c_normal_loss_args {
  const float* feat;          /* [P] float4 out_feat */
  const uint32_t* normals;    /* [P] packed RGBA8 normal map */
  const uint8_t* weights;     /* [P] or NULL */
  int W, H;
  float scale, grad_scale;
  float* v_feat;              /* [P] float4 */
  float* loss_accum;
  float* partials;
} b2c_normal_loss_args;
int b2c_hip_normal_loss(const b2c_normal_loss_args* a, hipStream_t stream);

/* hollow_reduce_kernel (loss.cu:197-204): loss_accum[0] += lam * sum(hollow_pen). */
int b2c_hip_hollow_loss(const float* hollow_pen, int W, int H, float lam, float* loss_accum, float* partials,
                        hipStream_t stream);

/* eval_kernel (loss.cu:240-286): prediction quantised to 8 bits (clamped to [0, 1]), per channel the sums of
 * the squared error and of the clamped 11-tap SSIM (zero padding), each weighted by the target alpha when
 * mask_weighted; loss_accum[4] += sum of squares, loss_accum[5] += sum of SSIM. */
typedef struct b2c_eval_args {
  const float* pred;          /* [P] float4 out_rgba */
  const uint32_t* gt;         /* [P] packed RGBA8 */
  int W, H;
  int mask_weighted;
  float* loss_accum;
  float* partials;
} b2c_eval_args;
int b2c_hip_eval_metrics(const b2c_eval_args* a, hipStream_t stream);

/* ---- tile-list consumers: evidence / label vote (src/train/evidence.cu:47-183) and the depth probe
 * (src/gpu/probe.cu:7-53) ---- */
#define B2C_LABEL_BINS 32      /* class ids >= this are ignored (evidence.cu:39) */
#define B2C_EVIDENCE_STRIDE 8  /* floats per splat of the evidence accumulator: w_in, w_all, err, -, dir xyz, sum w_in^2 */

/* One view's replay after a forward with bwd_info (shrunk ranges, last_idx): for each entry of a tile's shrunk
 * range, rows[slot_sorted[i]] = (the sums over the tile's composited fragments of vis * m,
 * vis * m * res, vis * k, row_tag as bits) at the entry's emit position, with m = target alpha * w, res the pixel's mean
 * absolute colour residual (+ normal_weight times the normal residual when normals are given), k = (target
 * alpha if masked_has_alpha else 1) * w; entries past a tile's shrunk end (and the sentinel entries) get no
 * row (b2c_hip_evidence_sum reads rows tagged with another row_tag as zero; the tag contract is the
 * backward's, b2c_raster_bwd_args). With labels, label_acc[i][class] += vis * k for the pixel's class
 * (< B2C_LABEL_BINS), float atomics. */
typedef struct b2c_evidence_args {
  const uint32_t* tile_ranges;
  const uint32_t* vals_sorted;
  const float* raster_rec;    /* [n][16] from b2c_hip_project */
  const float* out_rgba, *out_feat;
  const uint32_t* last_idx;
  const uint32_t* gt;         /* [P] packed RGBA8 */
  const uint32_t* normals;    /* [P] normal map or NULL */
  const uint8_t* weights;     /* [P] or NULL */
  const uint8_t* labels;      /* [P] class ids or NULL */
  int W, H, tiles_x, tiles_y;
  int masked_has_alpha;
  float normal_weight;
  const uint32_t* slot_sorted; /* [M] emit position of list entry i */
  uint32_t num_isect;
  float* rows;                /* [M][4] at emit positions */
  uint32_t row_tag;           /* this pass's tag (see b2c_raster_bwd_args) */
  float* label_acc;           /* [n][B2C_LABEL_BINS] or NULL */
} b2c_evidence_args;
int b2c_hip_evidence_view(const b2c_evidence_args* a, hipStream_t stream);
/* The view's per-splat sums from the rows (view_acc[i] = (w_in, err, w_all): a segmented scan over the emit
 * order, whose splat ids are `ids`, and one float atomic per run piece and value), folded into the evidence
 * as fold_view_kernel does (evidence.cu:114-126): evidence[i] (B2C_EVIDENCE_STRIDE floats) += w_in, w_all,
 * err; [7] += w_in^2; [4..6] += w_in * the unit vector from the splat to cam_pos. view_acc is scratch,
 * cleared here. */
typedef struct b2c_evidence_sum_args {
  int n;
  uint32_t m;                 /* intersections */
  const uint32_t* ids;        /* [M] splat id of emit position s */
  const float* rows;          /* [M][4]: row s counts when its .w bits equal row_tag */
  uint32_t row_tag;
  float* view_acc;            /* [n][3] scratch */
  const float* pos_op;        /* [n] float4 */
  float cam_pos[3];
  float* evidence;            /* [n][B2C_EVIDENCE_STRIDE] */
} b2c_evidence_sum_args;
int b2c_hip_evidence_sum(const b2c_evidence_sum_args* a, hipStream_t stream);

/* probe_kernel (probe.cu:7-53) after projection and binning: out[pix] = (accumulated alpha, the depth where it
 * first reaches tau (tau <= 0: the alpha-weighted mean depth, +inf under 5% coverage), the weight from more
 * than delta behind that depth, the weight from more than margin behind ref_z (NULL: none)). */
typedef struct b2c_probe_args {
  const uint32_t* tile_ranges;
  const uint32_t* vals_sorted;
  const float* raster_rec;
  int W, H, tiles_x, tiles_y;
  float tau, delta, margin;
  const float* ref_z;         /* [P] or NULL */
  float* out;                 /* [P] float4 */
} b2c_probe_args;
int b2c_hip_probe_depth(const b2c_probe_args* a, hipStream_t stream);

/* Writable planar SH arrays (the same layout as b2c_sh_view): parameters or their first moments. */
typedef struct b2c_sh_planes {
  float* dc;
  uint16_t* hi16;
  float* hi32;
  size_t stride;
} b2c_sh_planes;

/* Adam state of a model (src/model.h:19-28): moments beside each parameter array. */
typedef struct b2c_adam_state {
  float* m_pos_op, *v_pos_op, *m_quat, *v_quat, *m_lscale, *v_lscale; /* [n] float4 each */
  b2c_sh_planes m_sh;  /* SH first moments, in the SH's own layout and band precision */
  float* v_sh;         /* [n] one second moment per splat, the mean over its SH lanes */
  uint32_t* last_step; /* [n] Adam step of the splat's last update (sparse mode); 0 = never */
} b2c_adam_state;

/* One Adam step's constants (OptimParams, src/gpu/optim.h:10-20). The step-dependent factors are formed
 * on the host in double precision by b2c_adam_step_constants: bc1 = 1 / (1 - beta1^t), bc2 likewise;
 * ln_beta1 / ln_beta2 = ln beta, ratio = beta1 / sqrt(beta2) and ln_ratio = ln ratio give the lazy
 * catch-up's powers beta^s = e^(s ln beta) per splat. */
typedef struct b2c_adam_step {
  int t;
  int sparse;
  float beta1, beta2, eps;
  float bc1, bc2, ln_beta1, ln_beta2, ratio, ln_ratio;
  float lr_mean, lr_rot, lr_scale, lr_opac, lr_dc, lr_sh_rest;
  float noise_weight, noise_clamp; /* MCMC noise on the means: weight 0 disables */
  uint32_t seed, step;             /* noise and stochastic-rounding streams */
} b2c_adam_step;
void b2c_adam_step_constants(b2c_adam_step* s);

/* ---- projection VJP: optim_kernel's gradient part (src/gpu/optim.cu:99-253) ----
 * Reads and clears v_splat / vis_flag. With grad_out set, writes the parameter gradients
 * (optim.cu:292-296); accumulate = 1 adds into grad_out instead of overwriting (for gradients summed over
 * several views). With grad_out NULL, applies the fused Adam update of optim.cu:298-377 instead: the
 * parameters (pos_op, quat, lscale, sh) are then written, and adam / step must be set. */
typedef struct b2c_vjp_args {
  int n, degree, active_deg;
  float* pos_op, *quat, *lscale;
  b2c_sh_view sh;
  b2c_camera_gpu cam;
  float* v_splat;
  uint32_t* vis_flag;
  const uint32_t* tile_count;
  float* grad_out;            /* [n][11 + 3K] */
  int accumulate;             /* add into grad_out (rows of splats without gradient unchanged) */
  int sparse;                 /* leave the rows of splats without gradient unchanged (optim.cu:148) */
  float* refine_norm;         /* [n] or NULL: max(., clamp(g[9], 0, 1e32)) (optim.cu:175-176) */
  float* vis_count;           /* [n] or NULL: += visible (optim.cu:174) */
  int vis_from_row;           /* after a backward with defer_vis: a splat is flagged iff its v_splat lane 10
                                 (the blend-weight sum) is > 0, vis_flag is neither read nor cleared, and the
                                 lane is added to vis_weight; no reference counterpart */
  float* vis_weight;          /* [n] or NULL, with vis_from_row */
  b2c_sh_planes sh_out;       /* the SH as written by the update (the arrays of sh) */
  /* No reference counterpart: a photometric loss launched with defer_sum_count, reduced into loss_accum by the
   * first workgroup (the same fixed-order sum and stores as the loss's own reduction launch). NULL = none. */
  const float* loss_partials;
  int loss_count, loss_assign, loss_running;
  float* loss_accum;
  b2c_adam_state adam;
  b2c_adam_step step;
} b2c_vjp_args;
int b2c_hip_vjp(const b2c_vjp_args* a, hipStream_t stream);

/* ---- utilities ---- */
int b2c_hip_fill_u32(uint32_t* p, uint32_t value, size_t count, hipStream_t stream);

/* ---- model storage (src/model.cu:8-102 defines the layout these fill and read back) ---- */
/* A splat cloud in device memory, one array per field (brush's SplatCloud layout, src/ply.h:10-42):
 * pos [n][3], log_scale [n][3], quat [n][4] (w, x, y, z), opacity [n] (logit), sh [n][3K]
 * coefficient-major, floor_ [n] or NULL. */
typedef struct b2c_cloud_dev {
  float* pos;
  float* log_scale;
  float* quat;
  float* opacity;
  float* sh;
  float* floor_;
} b2c_cloud_dev;

/* The Model's device layout: float4 pos_op / quat / lscale [cap], planar SH with stride cap: sh_dc
 * [3][cap] fp32, bands [3K - 3][cap] in sh_hi32 (fp32) or sh_hi16 (IEEE binary16). */
typedef struct b2c_model_dev {
  int n, cap, sh_lanes; /* sh_lanes = 3K */
  float* pos_op;
  float* quat;
  float* lscale;
  float* sh_dc;
  float* sh_hi32;
  uint16_t* sh_hi16;
} b2c_model_dev;

/* Cloud -> model (Model::upload, model.cu:41-80): lscale.w = floor_[i] (0 when floor_ is NULL), bands
 * rounded to nearest even when stored as fp16. Model slots n .. cap are left untouched. */
int b2c_hip_model_scatter(const b2c_cloud_dev* src, const b2c_model_dev* dst, hipStream_t stream);
/* Model -> cloud (Model::download, model.cu:82-102); fp16 bands widen exactly. floor_ may be NULL. */
int b2c_hip_model_gather(const b2c_model_dev* src, const b2c_cloud_dev* dst, hipStream_t stream);
/* Planar re-layout for capacity growth: dst[l * new_cap + i] = src[l * old_cap + i] for i < n, 0 for
 * n <= i < new_cap, over `lanes` lanes of elem_bytes (2 or 4) each. */
int b2c_hip_planar_regrow(const void* src, void* dst, int elem_bytes, int lanes, int n, int old_cap, int new_cap,
                          hipStream_t stream);
/* lscale[i].w = floor_[i] for i < n (the frozen Mip-Splatting floor). */
int b2c_hip_model_set_floor(float* lscale, const float* floor_, int n, hipStream_t stream);

/* ---- PLY rows <-> model (replaces the per-row loops of src/ply.cpp:127-160 and 188-224) ----
 * A binary little-endian ply's vertex rows are decoded on the device straight into the model layout, and
 * the model is encoded into the rows write_ply lays out. Targets of the decode, in this order:
 * x y z, scale_0..2, rot_0..3, opacity, f_dc_0..2, the colour fallback (red/r, green/g, blue/b), then
 * f_rest_0 .. f_rest_(3(K-1)-1) (channel-major: every red band, then green, then blue). */
#define B2C_PLY_T_POS 0
#define B2C_PLY_T_SCALE 3
#define B2C_PLY_T_ROT 6
#define B2C_PLY_T_OPACITY 10
#define B2C_PLY_T_DC 11
#define B2C_PLY_T_RGB 14
#define B2C_PLY_T_REST 17
#define B2C_PLY_TARGETS (B2C_PLY_T_REST + 72) /* SH degree 4: 3 x 24 rest coefficients */
/* Property types (src/ply.cpp:27-36). */
enum { B2C_PLY_F32 = 0, B2C_PLY_F64, B2C_PLY_U8, B2C_PLY_I8, B2C_PLY_U16, B2C_PLY_I16, B2C_PLY_U32, B2C_PLY_I32 };

typedef struct b2c_ply_decode_args {
  const uint8_t* rows; /* `count` rows of row_bytes each (readable for 4 bytes past the last row) */
  uint32_t row_bytes;
  int count, first; /* the rows are model splats first .. first + count - 1 */
  int16_t col[B2C_PLY_TARGETS]; /* byte offset of each target within a row, -1 = absent (its default) */
  uint8_t type[B2C_PLY_TARGETS];
  int rgb_dc;        /* 1: no f_dc_*; DC = ((colour * rgb_scale) - 0.5) / SH_C0 in double */
  double rgb_scale;  /* 1/255 for uchar, 1/65535 for ushort, else 1 (the red column's type) */
  b2c_model_dev model; /* n = the whole file's splat count; sh_lanes = 3K */
} b2c_ply_decode_args;
int b2c_hip_ply_decode(const b2c_ply_decode_args* a, hipStream_t stream);

/* Rows of write_ply's layout for model splats first .. first + count - 1: x y z, scale_0..2, opacity,
 * the unit quaternion (identity when its norm is not above 1e-32), f_dc_0..2, f_rest channel-major, then
 * the optional blocks from device arrays (NULL = not written): evidence [n][7], labels [n][2], fill [n],
 * gate [n][2], gate_s [n], open [n][4]. row_floats must equal the count of written columns. */
typedef struct b2c_ply_encode_args {
  b2c_model_dev model;
  int count, first, row_floats;
  const float *evidence, *labels, *fill, *gate, *gate_s, *open;
  float* rows; /* [count][row_floats] */
} b2c_ply_encode_args;
int b2c_hip_ply_encode(const b2c_ply_encode_args* a, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
