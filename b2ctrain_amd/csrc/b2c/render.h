// Rendering API of the drop-in (replaces src/gpu/render.h:1-111 and src/dataset/camera.h:8-36): same
// type names, fields and entry points, hipStream_t in place of cudaStream_t. Features outside this build's
// scope (render-side warp, articulated/cage overrides, pose-dependent appearance, mip filtering) keep their
// RenderParams fields so callers compile, and make the entry points throw std::runtime_error when set.
#pragma once
#include "model.h"

namespace b2c {

// Pinhole camera, world->camera R/t (OpenCV axes), R row major (camera.h:8-36).
struct Camera {
  int width = 0, height = 0;
  float fx = 0, fy = 0, cx = 0, cy = 0;
  float R[9] = {1, 0, 0, 0, 1, 0, 0, 0, 1};
  float t[3] = {0, 0, 0};
  float pos[3] = {0, 0, 0};
  void set_w2c_quat(float qw, float qx, float qy, float qz, float tx, float ty, float tz);
  void update_pos();  // pos = -R^T t
  // Intrinsics for a new image size (camera.h:30-34): fx, cx scaled by new_w / width, fy, cy by new_h / height.
  void rescale(int new_w, int new_h);
  float focal_px() const { return 0.5f * (fx + fy); }
};

struct CameraGPU {
  float R[9];
  float t[3];
  float pos[3];
  float fx, fy, cx, cy;
  int W, H;
  float lim_pos_x, lim_pos_y, lim_neg_x, lim_neg_y;  // EWA Jacobian clamp
  static CameraGPU from(const Camera& c, int W, int H);
  b2c_camera_gpu dev() const;
};

enum class FeatureMode { None, Normals, Buffer };

struct RenderParams {
  CameraGPU cam;
  float bg[3] = {0, 0, 0};
  int sh_degree = 3;  // active degree (<= model degree)
  FeatureMode feat = FeatureMode::None;  // Normals: camera-space pseudo-normals; Buffer: feat_buffer
  const float* feat_buffer = nullptr;    // [n][3] device, FeatureMode::Buffer
  bool mip = false;
  bool bwd_info = true;  // write per-pixel last index / shrink tile ranges
  // Write proj0..3, the reference's projection buffers. The raster, binning and replay kernels read only the
  // 64-byte raster record, so a caller that does not read proj0..3 (the fused training step) can skip them.
  bool write_proj = true;
  const float2* warp = nullptr;
  int warp_w = 0, warp_h = 0;
  const float4* pos_override = nullptr;
  const float4* quat_override = nullptr;
  const float4* lscale_override = nullptr;
  const float4* sh_frame = nullptr;
  const float4* app = nullptr;
  float4* col_base = nullptr;
  bool app_add = false;
  // Hollow loss: per-pixel reference depth of the body surface (camera z, +inf = none) [W*H] device; a
  // fragment at depth z is penalised by clamp((z - z_ref - margin) / margin, 0, 1) times its blend weight,
  // summed per pixel into ctx.hollow_pen; hollow_lam = dL/d(penalised weight) per pixel (before grad_scale).
  const float* hollow_z = nullptr;
  float hollow_margin = 0.05f;
  float hollow_lam = 0.f;
};

// Persistent scratch for rendering one view; grows on demand (render.h:66-95).
struct RenderCtx {
  int W = 0, H = 0, tiles_x = 0, tiles_y = 0, n_tiles = 0, tile_bits = 0, depth_bits = 0;
  // per splat (global index)
  DevBuf<float4> proj0, proj1, proj2;  // (xy, c00, c01) | (c11, opac, depth, power = ln(255 opac)) | (r, g, b, feat_x)
  DevBuf<float2> proj3;                // (feat_y, feat_z)
  DevBuf<float4> raster_rec;           // [n][4]: the raster kernels' 64-byte per-splat record (same values)
  DevBuf<uint32_t> tile_count, tile_off;  // hit count; inclusive scan in depth order
  DevBuf<uint2> hit_info;                 // (hit mask within the bbox or 0xFFFFFFFF, min_x | min_y << 12 | bw << 24)
  DevBuf<uint2> hit_wide;                 // where hit_info's mask word is 0xFFFFFFFF: the 64-bit mask of a bbox
                                          // of at most 64 tiles, or (0, 0) beyond 64 tiles
  DevBuf<uint32_t> depth_keys, depth_keys_sorted, order_in, order;  // depth sort
  DevBuf<uint32_t> count_perm;  // kept for layout compatibility; the count scan gathers in place
  // intersections
  DevBuf<uint32_t> keys, vals, keys_sorted, vals_sorted;
  size_t isect_cap = 0;
  uint32_t num_isect = 0;
  PinnedBuf<uint32_t> h_count;
  uint32_t* h_count_dev = nullptr;  // h_count's device address (the count scan stores the total there)
  // per tile / per pixel
  DevBuf<uint2> tile_ranges;
  DevBuf<float4> out_rgba;  // final rgb (with bg) + alpha
  DevBuf<float4> out_feat;  // feat xyz + final transmittance
  DevBuf<float> hollow_pen;
  DevBuf<uint32_t> last_idx;  // one past the last contributing intersection per pixel
  // backward
  DevBuf<float> v_splat;      // [n][13]: xy(2) conic(3) rgb(3) opac(1) refine(1) feat(3)
  // The MFMA backward stores its sums without reading v_splat when v_splat is known to be all zero:
  // v_splat_zero is set where v_splat is cleared (allocation, a caller's zero, and the projection VJP,
  // which clears every row whose vis_flag the backward set) and cleared by a backward. A caller's write of
  // v_splat or vis_flag may leave rows the VJP does not clear (v_splat_foreign, until the caller zeroes
  // v_splat); a caller holding the device pointer may write at any time (v_splat_shared, for good).
  bool v_splat_zero = true;
  bool v_splat_foreign = false;
  bool v_splat_shared = false;
  bool v_splat_known_zero() const { return v_splat_zero && !v_splat_foreign && !v_splat_shared; }
  // defer_vis (set by the fused training step around its backward): a mode-1 backward without feature
  // lanes that finds v_splat known zero keeps each splat's blend-weight sum in v_splat lane 10 and leaves
  // vis_flag and Model::vis_weight alone; vis_in_rows records that, until the projection VJP takes the flag
  // and the weight from that lane.
  bool defer_vis = false;
  bool vis_in_rows = false;
  // A photometric loss run with defer_sum leaves its partials unreduced: loss_pending of them (with the
  // assign / running flags), summed into loss_accum by the next optimizer_step's VJP.
  int loss_pending = 0;
  int loss_pending_assign = 0, loss_pending_running = 0;
  DevBuf<uint32_t> vis_flag;  // [n]
  DevBuf<float4> v_out;       // dL/d(rgba) per pixel
  DevBuf<float4> v_feat;
  DevBuf<float> loss_accum;   // [16] scalar accumulators
  // MI355X build scratch: big-splat list, sort ping-pong buffers, sort/scan temporaries, device counters
  // counters: [0] big splats, [1] big items, [2] intersections, [4..5] the second big-splat pair: projections
  // alternate between [0..1] and [4..5] (big_slot), each clearing the other for the next
  DevBuf<uint32_t> big_list, big_base, counters;
  int big_slot = 0;
  uint32_t* big_counters() const { return counters.ptr + 4 * big_slot; }
  DevBuf<uint4> big_info;                         // per big-list entry: bbox and chunk length
  DevBuf<uint32_t> big_chunk, big_items;          // per big-list entry and chunk: hit offsets; work items
  DevBuf<uint32_t> depth_alt_k, depth_alt_v, isect_alt_k, isect_alt_v, isect_alt_v2;
  // Intersection bookkeeping of the atomic-free backward: slot_sorted[i] = emit position of list entry i
  // (the tile sort sorts positions; a splat's emit positions are contiguous), tile_end[t] = the tile's
  // list end before the forward shrinks it, isect_rows[slot] = that (tile, splat)'s 12-float gradient row
  // (or the evidence pass's 4-float row), written only for the entries of the shrunk ranges; row_live[slot]
  // = the tag word of a row the backward wrote, when it runs with the live-row index (sparse lists).
  DevBuf<uint32_t> slot_sorted, tile_end;
  // The forward's compacted lists for the MFMA backward (the entries of each tile that some pixel
  // composited: ids, emit positions, each pixel's end, each tile's end); compact_ok while they describe the
  // current lists (set by a forward with bwd_info that wrote them, cleared by the binning). B2C_COMPACT_LISTS=0
  // in the environment turns them off.
  DevBuf<uint32_t> cvals, cslots, clast, cend;
  bool compact_lists = true;
  bool compact_ok = false;
  DevBuf<float4> isect_rows;
  DevBuf<uint32_t> row_live;
  DevBuf<float4> isect_part;          // per 256-row window: partial sums of runs crossing the window's edges
  DevBuf<uint32_t> isect_part_flags;  // per 256-row window
  DevBuf<unsigned char> sort_tmp;
  DevBuf<float> loss_partials;  // per-workgroup loss sums, reduced in a fixed order
  DevBuf<float> aux_partials;   // the same for normal_loss, hollow_loss and eval_metrics
  hipEvent_t bwd_split_event = nullptr;  // if set: recorded between the backward raster kernel and its reduce
  hipEvent_t count_event = nullptr;      // owned: recorded after the intersection count's copy to h_count

  RenderCtx() = default;
  RenderCtx(const RenderCtx&) = delete;
  RenderCtx& operator=(const RenderCtx&) = delete;
  ~RenderCtx();
  void setup(int W, int H, int n_splats, hipStream_t stream);
  void ensure_isect_capacity(size_t m, hipStream_t stream);
  // Row tags. Every row a pass writes carries the pass's tag (generation << tile_bits, or'd with the
  // tile) and the readers take a row as this pass's only when the tag matches, so rows of pairs past a
  // shrunk end are neither written nor cleared. A tag is never handed out twice while rows written under
  // it can remain: the buffer is cleared (fill kernel) when it was reallocated, when the row layout
  // (floats per row) or tile_bits changed, and when the generation field is used up; the generation then
  // restarts at 1. row_live holds the same tags and is cleared with the rows.
  uint32_t next_row_tag(int row_floats, hipStream_t stream);
  // Whether the MFMA backward's reduce reads rows through row_live: when the lists are long against the
  // image (more than 4 intersections per pixel) most pairs lie past their tile's shrunk end, and reading
  // a 4-byte tag per row instead of the 48-byte row saves most of the reduce's traffic. B2C_ROW_LIVE = 0
  // or 1 forces the choice.
  bool use_row_live() const;
  uint32_t row_gen = 0;                 // last generation of the current epoch
  uint32_t row_epoch_key = 0;           // row floats | tile_bits << 8 of the current epoch
  const void* row_epoch_buf = nullptr;  // isect_rows.ptr the epoch's clear covered
};

// Full forward: projection, binning, sort, rasterisation. Leaves outputs in ctx.
void render_forward(RenderCtx& ctx, const Model& m, const RenderParams& p, hipStream_t stream);

// Individual stages.
void project_splats(RenderCtx& ctx, const Model& m, const RenderParams& p, hipStream_t stream);
void bin_and_sort(RenderCtx& ctx, const Model& m, hipStream_t stream);
void rasterize_forward(RenderCtx& ctx, const RenderParams& p, hipStream_t stream);

// Backward through rasterisation: consumes ctx.v_out, produces ctx.v_splat; accumulates Model::vis_weight.
void rasterize_backward(RenderCtx& ctx, const Model& m, const RenderParams& p, hipStream_t stream);
// MFMA variant. ctx.v_out must carry `grad_scale`; the accumulated per-splat gradients are divided by it.
void rasterize_backward_tc(RenderCtx& ctx, const Model& m, const RenderParams& p, float grad_scale, hipStream_t stream);

}  // namespace b2c
