// Rendering entry points (replaces src/gpu/render.cu:5-27, project.cu:104-126, binning.cu:109-145,
// raster_fwd.cu:75-90, raster_bwd.cu:239-248, raster_bwd_tc.cu:210-225).
#include "render.h"

#include <algorithm>
#include <cstdlib>
#include <cmath>

namespace b2c {

void Camera::set_w2c_quat(float qw, float qx, float qy, float qz, float tx, float ty, float tz) {
  float n = std::sqrt(qw * qw + qx * qx + qy * qy + qz * qz);
  qw /= n; qx /= n; qy /= n; qz /= n;
  R[0] = 1 - 2 * (qy * qy + qz * qz); R[1] = 2 * (qx * qy - qz * qw);     R[2] = 2 * (qx * qz + qy * qw);
  R[3] = 2 * (qx * qy + qz * qw);     R[4] = 1 - 2 * (qx * qx + qz * qz); R[5] = 2 * (qy * qz - qx * qw);
  R[6] = 2 * (qx * qz - qy * qw);     R[7] = 2 * (qy * qz + qx * qw);     R[8] = 1 - 2 * (qx * qx + qy * qy);
  t[0] = tx; t[1] = ty; t[2] = tz;
  update_pos();
}

void Camera::update_pos() {
  pos[0] = -(R[0] * t[0] + R[3] * t[1] + R[6] * t[2]);
  pos[1] = -(R[1] * t[0] + R[4] * t[1] + R[7] * t[2]);
  pos[2] = -(R[2] * t[0] + R[5] * t[1] + R[8] * t[2]);
}

void Camera::rescale(int new_w, int new_h) {
  const float sx = (float)new_w / (float)width, sy = (float)new_h / (float)height;
  fx *= sx;
  cx *= sx;
  fy *= sy;
  cy *= sy;
  width = new_w;
  height = new_h;
}

CameraGPU CameraGPU::from(const Camera& c, int W, int H) {
  CameraGPU g;
  for (int i = 0; i < 9; i++) g.R[i] = c.R[i];
  for (int i = 0; i < 3; i++) { g.t[i] = c.t[i]; g.pos[i] = c.pos[i]; }
  const float sx = (float)W / c.width, sy = (float)H / c.height;
  g.fx = c.fx * sx; g.fy = c.fy * sy; g.cx = c.cx * sx; g.cy = c.cy * sy; g.W = W; g.H = H;
  g.lim_pos_x = (1.15f * W - g.cx) / g.fx; g.lim_pos_y = (1.15f * H - g.cy) / g.fy;
  g.lim_neg_x = (-0.15f * W - g.cx) / g.fx; g.lim_neg_y = (-0.15f * H - g.cy) / g.fy;
  return g;
}

b2c_camera_gpu CameraGPU::dev() const {
  b2c_camera_gpu d;
  for (int i = 0; i < 9; i++) d.R[i] = R[i];
  for (int i = 0; i < 3; i++) { d.t[i] = t[i]; d.pos[i] = pos[i]; }
  d.fx = fx; d.fy = fy; d.cx = cx; d.cy = cy; d.W = W; d.H = H;
  d.lim_pos_x = lim_pos_x; d.lim_pos_y = lim_pos_y; d.lim_neg_x = lim_neg_x; d.lim_neg_y = lim_neg_y;
  return d;
}

RenderCtx::~RenderCtx() {
  if (count_event) (void)hipEventDestroy(count_event);
}

void RenderCtx::setup(int w, int h, int n, hipStream_t stream) {
  // no system-scope fence on this event: its writeback of the L2s stalls the queue for ~5 us, and the count
  // lands in coherent pinned memory without it (bin_and_sort checks a sentinel)
  if (!count_event) HIP_CHECK(hipEventCreateWithFlags(&count_event, hipEventDisableTiming | hipEventDisableSystemFence));
  W = w; H = h;
  tiles_x = (W + RT_W - 1) / RT_W; tiles_y = (H + RT_W - 1) / RT_W; n_tiles = tiles_x * tiles_y;
  tile_bits = 1;
  while ((1 << tile_bits) < n_tiles + 1) tile_bits++;
  depth_bits = 32 - tile_bits;
  if (depth_bits > 20) depth_bits = 20;
  const size_t nn = (size_t)(n > 0 ? n : 1);
  proj0.reserve(nn); proj1.reserve(nn); proj2.reserve(nn); proj3.reserve(nn); raster_rec.reserve(nn * 4);
  tile_count.reserve(nn); tile_off.reserve(nn); hit_info.reserve(nn); hit_wide.reserve(nn);
  depth_keys.reserve(nn); depth_keys_sorted.reserve(nn); order_in.reserve(nn); order.reserve(nn);
  depth_alt_k.reserve(nn); depth_alt_v.reserve(nn);
  big_list.reserve(nn); big_base.reserve(nn); big_info.reserve(nn); big_chunk.reserve(nn * B2C_BIG_CHUNKS);
  big_items.reserve(nn * B2C_BIG_CHUNKS);
  if (counters.count < 8) {
    counters.reserve(8);
    counters.zero(stream);  // both big-splat counter pairs start at zero
    big_slot = 0;
  }
  if (v_splat.count < nn * GRAD_LANES) {
    v_splat.reserve(nn * GRAD_LANES);
    v_splat.zero(stream);
    v_splat_zero = true;
    v_splat_foreign = false;
    vis_in_rows = false;
  }
  if (vis_flag.count < nn) { vis_flag.reserve(nn); vis_flag.zero(stream); }
  tile_ranges.reserve((size_t)n_tiles); tile_end.reserve((size_t)n_tiles + 1);
  const size_t npx = (size_t)W * H;
  out_rgba.reserve(npx); out_feat.reserve(npx); last_idx.reserve(npx); v_out.reserve(npx);
  clast.reserve(npx); cend.reserve((size_t)n_tiles);
  compact_ok = false;
  if (const char* e = std::getenv("B2C_COMPACT_LISTS")) compact_lists = std::string(e) != "0";
  hollow_pen.reserve(npx);
  if (v_feat.count < npx) { v_feat.reserve(npx); v_feat.zero(stream); }  // read by a FEAT backward
  loss_accum.reserve(16);
  loss_partials.reserve(b2c_loss_partials(W, H));
  aux_partials.reserve(b2c_aux_partials(W, H));
  h_count.reserve(4);
  HIP_CHECK(hipHostGetDevicePointer(reinterpret_cast<void**>(&h_count_dev), h_count.ptr, 0));
  if (isect_cap == 0) ensure_isect_capacity((size_t)1 << 22, stream);
  const size_t need_tmp = std::max({b2c_radix_sort_temp_bytes((uint32_t)nn), b2c_radix_sort_temp_bytes((uint32_t)isect_cap),
                                    b2c_scan_temp_bytes((uint32_t)nn)});
  sort_tmp.reserve(need_tmp);
}

uint32_t RenderCtx::next_row_tag(int row_floats, hipStream_t stream) {
  uint32_t limit = tile_bits >= 31 ? 1u : (1u << (32 - tile_bits)) - 1u;  // generations that fit the tag
  if (const char* env = getenv("B2C_ROW_GEN_LIMIT")) {  // a shorter epoch, for tests
    const long v = atol(env);
    if (v >= 1 && (uint32_t)v < limit) limit = (uint32_t)v;
  }
  const uint32_t key = (uint32_t)row_floats | ((uint32_t)tile_bits << 8);
  if (row_epoch_buf != isect_rows.ptr || key != row_epoch_key || row_gen >= limit) {
    isect_rows.zero(stream);
    row_live.zero(stream);
    row_gen = 0;
    row_epoch_key = key;
    row_epoch_buf = isect_rows.ptr;
  }
  row_gen++;
  return row_gen << tile_bits;
}

bool RenderCtx::use_row_live() const {
  if (const char* env = getenv("B2C_ROW_LIVE")) {
    if (env[0] == '0') return false;
    if (env[0] == '1') return true;
  }
  return (size_t)num_isect > (size_t)4 * (size_t)W * (size_t)H;
}

void RenderCtx::ensure_isect_capacity(size_t m, hipStream_t stream) {
  if (m <= isect_cap && isect_cap) return;
  size_t ncap = isect_cap ? isect_cap : ((size_t)1 << 22);
  while (ncap < m) ncap *= 2;
  keys.reserve(ncap, false, stream); vals.reserve(ncap, false, stream);
  keys_sorted.reserve(ncap, false, stream); vals_sorted.reserve(ncap, false, stream);
  isect_alt_k.reserve(ncap, false, stream); isect_alt_v.reserve(ncap, false, stream);
  isect_alt_v2.reserve(ncap, false, stream);
  // rows: 3 float4 (4 with feature lanes); window partials: 2 x 3 float4 (2 x 4)
  slot_sorted.reserve(ncap, false, stream); isect_rows.reserve(ncap * 4, false, stream);
  cvals.reserve(ncap, false, stream); cslots.reserve(ncap, false, stream);
  compact_ok = false;
  row_live.reserve(ncap, false, stream);
  isect_part.reserve((ncap / 256 + 1) * 8, false, stream); isect_part_flags.reserve(ncap / 256 + 1, false, stream);
  isect_cap = ncap;
  sort_tmp.reserve(b2c_radix_sort_temp_bytes((uint32_t)ncap));
  // The new row buffers hold uninitialised memory, possibly at the address a previous epoch cleared
  // (the allocator may hand a freed block back): force the next pass to start a new epoch.
  row_epoch_buf = nullptr;
}

namespace {

void check_supported(const RenderParams& p) {
  if (p.feat == FeatureMode::Buffer && !p.feat_buffer) throw std::runtime_error("render: FeatureMode::Buffer needs feat_buffer");
  if (p.mip) throw std::runtime_error("render: mip filtering is not supported (the reference trainer rejects it too)");
  if (p.warp || p.pos_override || p.quat_override || p.lscale_override || p.sh_frame || p.app || p.col_base)
    throw std::runtime_error("render: warp / deformation overrides / appearance are not supported by this build");
}

int feat_mode(const RenderParams& p) {
  return p.feat == FeatureMode::Normals ? 1 : (p.feat == FeatureMode::Buffer ? 2 : 0);
}

}  // namespace

void project_splats(RenderCtx& ctx, const Model& m, const RenderParams& p, hipStream_t stream) {
  if (m.n == 0) return;
  check_supported(p);
  if (m.degree < 0 || m.degree > 4) throw std::runtime_error("unsupported SH degree");
  b2c_project_args a{};
  a.n = m.n; a.degree = m.degree; a.active_deg = p.sh_degree;
  a.pos_op = reinterpret_cast<const float*>(m.pos_op.ptr);
  a.quat = reinterpret_cast<const float*>(m.quat.ptr);
  a.lscale = reinterpret_cast<const float*>(m.lscale.ptr);
  a.sh = m.sh().view();
  a.cam = p.cam.dev();
  a.tiles_x = ctx.tiles_x; a.tiles_y = ctx.tiles_y;
  if (p.write_proj) {
    a.proj0 = reinterpret_cast<float*>(ctx.proj0.ptr); a.proj1 = reinterpret_cast<float*>(ctx.proj1.ptr);
    a.proj2 = reinterpret_cast<float*>(ctx.proj2.ptr); a.proj3 = reinterpret_cast<float*>(ctx.proj3.ptr);
  }
  a.raster_rec = reinterpret_cast<float*>(ctx.raster_rec.ptr);
  a.tile_count = ctx.tile_count.ptr;
  a.depth_bits = ctx.depth_keys.ptr;  // made the depth keys in place by the binning
  a.hit_info = reinterpret_cast<uint32_t*>(ctx.hit_info.ptr);
  a.hit_wide = reinterpret_cast<uint32_t*>(ctx.hit_wide.ptr);
  a.max_screen = m.max_screen.ptr;
  a.big_list = ctx.big_list.ptr;
  ctx.big_slot ^= 1;  // this projection appends to the pair the previous one cleared, and clears the other
  a.big_count = ctx.big_counters();
  a.clear_next = ctx.counters.ptr + 4 * (ctx.big_slot ^ 1);
  a.big_info = reinterpret_cast<uint32_t*>(ctx.big_info.ptr);
  a.big_chunk = ctx.big_chunk.ptr;
  a.big_items = ctx.big_items.ptr;
  a.big_items_count = ctx.big_counters() + 1;
  a.feat_mode = feat_mode(p);
  a.feat_buffer = p.feat_buffer;
  LAUNCH_CHECK(b2c_hip_project(&a, stream));
}

namespace {

// 3. emit in depth order, then a stable sort on the tile id alone keeps each tile's list in depth order;
// 4. tile ranges. Sized for ctx.isect_cap; the live intersection count is read from counters[2].
void emit_and_sort(RenderCtx& ctx, const Model& m, hipStream_t stream) {
  const uint32_t cap = (uint32_t)ctx.isect_cap;
  const uint32_t* total_dev = ctx.counters.ptr + 2;
  b2c_emit_args e{};
  e.n = m.n; e.order = ctx.order; e.tile_count = ctx.tile_count; e.tile_off = ctx.tile_off;
  e.hit_info = reinterpret_cast<const uint32_t*>(ctx.hit_info.ptr);
  e.hit_wide = reinterpret_cast<const uint32_t*>(ctx.hit_wide.ptr);
  e.raster_rec = reinterpret_cast<const float*>(ctx.raster_rec.ptr);
  e.tiles_x = ctx.tiles_x; e.tiles_y = ctx.tiles_y; e.cap = cap;
  e.keys = ctx.keys; e.vals = ctx.vals;
  e.big_list = ctx.big_list; e.big_count = ctx.big_counters(); e.big_base = ctx.big_base;
  e.big_info = reinterpret_cast<const uint32_t*>(ctx.big_info.ptr); e.big_chunk = ctx.big_chunk;
  e.big_items = ctx.big_items; e.big_items_count = ctx.big_counters() + 1;
  LAUNCH_CHECK(b2c_hip_emit(&e, stream));
  // The tile pass carries the emit positions next to the splat ids: the backward writes each (tile, splat)
  // gradient row at its emit position, where a splat's rows are contiguous.
  LAUNCH_CHECK(b2c_hip_radix_sort_kv2(ctx.keys, nullptr, ctx.vals, ctx.keys_sorted, ctx.slot_sorted, ctx.vals_sorted,
                                      ctx.isect_alt_k, ctx.isect_alt_v, ctx.isect_alt_v2, cap, total_dev, 0,
                                      ctx.tile_bits, ctx.sort_tmp.ptr, ctx.sort_tmp.bytes(), stream));
  LAUNCH_CHECK(b2c_hip_tile_ranges(cap, total_dev, ctx.keys_sorted, nullptr, nullptr, nullptr, (uint32_t)ctx.n_tiles,
                                   reinterpret_cast<uint32_t*>(ctx.tile_ranges.ptr), ctx.tile_end, stream));
}

}  // namespace

void bin_and_sort(RenderCtx& ctx, const Model& m, hipStream_t stream) {
  ctx.compact_ok = false;
  if (m.n == 0) {  // no lists: every range and list end is empty, so the raster kernels touch no row
    ctx.num_isect = 0;
    ctx.tile_ranges.zero(stream);
    ctx.tile_end.zero(stream, (size_t)ctx.n_tiles + 1);
    return;
  }
  const int n = m.n;
  // 1. depth sort of the splats (culled ones sort last), stable on the 32 z bits: the projection wrote the
  // keys (depth bits, or 0xFFFFFFFF without tiles), and the sort carries the splat indices itself
  LAUNCH_CHECK(b2c_hip_radix_sort_pairs(ctx.depth_keys, nullptr, ctx.depth_keys_sorted, ctx.order, ctx.depth_alt_k,
                                        ctx.depth_alt_v, (uint32_t)n, nullptr, 0, 32, ctx.sort_tmp.ptr,
                                        ctx.sort_tmp.bytes(), stream));
  // 2. inclusive scan of the tile counts in depth order; the total comes back to the host (binning.cu:125-133)
  constexpr uint32_t NO_COUNT = 0xFFFFFFFFu;  // not a possible total (the emit capacity is far below it)
  volatile uint32_t* h_total = ctx.h_count.ptr;
  *h_total = NO_COUNT;  // the previous store into it completed in the previous call
  // the scan's last workgroup stores the total into the pinned word as well (no copy launch)
  LAUNCH_CHECK(b2c_hip_scan_counts_host(n, ctx.order, ctx.tile_count, ctx.tile_off, ctx.counters.ptr + 2,
                                        ctx.h_count_dev, ctx.sort_tmp.ptr, ctx.sort_tmp.bytes(), stream));
  HIP_CHECK(hipEventRecord(ctx.count_event, stream));
  // 3-4 are queued before the host has the total: they are sized for the current capacity and read the
  // live count on the device (the emit skips splats whose slots would not fit), so the GPU does not idle
  // while the count travels to the host. A total beyond the capacity grows the buffers and runs them again.
  emit_and_sort(ctx, m, stream);
  HIP_CHECK(hipEventSynchronize(ctx.count_event));
  // the scan has completed; without the event's fence its value may reach host memory a little later
  for (int spin = 0; *h_total == NO_COUNT && spin < (1 << 20); spin++) {
  }
  if (*h_total == NO_COUNT) HIP_CHECK(hipStreamSynchronize(stream));  // full fence, then it must be there
  const uint32_t total = *h_total;
  if (total == NO_COUNT) throw std::runtime_error("bin_and_sort: the intersection count did not arrive");
  ctx.num_isect = total;
  if (total > ctx.isect_cap) {
    HIP_CHECK(hipStreamSynchronize(stream));  // the speculative launches still use the old buffers
    ctx.ensure_isect_capacity(total, stream);
    emit_and_sort(ctx, m, stream);
  }
}

void rasterize_forward(RenderCtx& ctx, const RenderParams& p, hipStream_t stream) {
  check_supported(p);
  b2c_raster_fwd_args a{};
  a.tile_ranges = reinterpret_cast<uint32_t*>(ctx.tile_ranges.ptr);
  a.vals_sorted = ctx.vals_sorted;
  a.proj0 = reinterpret_cast<const float*>(ctx.proj0.ptr);
  a.proj1 = reinterpret_cast<const float*>(ctx.proj1.ptr);
  a.proj2 = reinterpret_cast<const float*>(ctx.proj2.ptr);
  a.raster_rec = reinterpret_cast<const float*>(ctx.raster_rec.ptr);
  a.W = ctx.W; a.H = ctx.H; a.tiles_x = ctx.tiles_x; a.tiles_y = ctx.tiles_y;
  for (int k = 0; k < 3; k++) a.bg[k] = p.bg[k];
  a.bwd_info = p.bwd_info ? 1 : 0;
  a.out_rgba = reinterpret_cast<float*>(ctx.out_rgba.ptr);
  a.out_feat = reinterpret_cast<float*>(ctx.out_feat.ptr);
  a.last_idx = ctx.last_idx;
  a.feat = p.feat != FeatureMode::None ? 1 : 0;
  a.hollow_z = p.hollow_z;
  a.hollow_margin = p.hollow_margin;
  a.hollow_pen = ctx.hollow_pen.ptr;
  const bool compact = p.bwd_info && ctx.compact_lists;
  if (compact) {
    a.slot_sorted = ctx.slot_sorted;
    a.cvals = ctx.cvals; a.cslots = ctx.cslots; a.clast = ctx.clast; a.cend = ctx.cend;
  }
  LAUNCH_CHECK(b2c_hip_raster_fwd(&a, stream));
  if (p.bwd_info) ctx.compact_ok = compact;
}

void render_forward(RenderCtx& ctx, const Model& m, const RenderParams& p, hipStream_t stream) {
  project_splats(ctx, m, p, stream);
  bin_and_sort(ctx, m, stream);
  rasterize_forward(ctx, p, stream);
}

namespace {

// grad_scale: the factor v_out carries (1 for mode 0); the hollow term is scaled to match
// (raster_bwd_tc.cu:208).
void backward(RenderCtx& ctx, const Model& m, const RenderParams& p, int mode, float grad_scale, hipStream_t stream) {
  check_supported(p);
  if (ctx.vis_in_rows)
    throw std::logic_error("backward: the previous pass's visibility is still held in v_splat (run the VJP first)");
  b2c_raster_bwd_args a{};
  a.tile_ranges = reinterpret_cast<const uint32_t*>(ctx.tile_ranges.ptr);
  a.vals_sorted = ctx.vals_sorted;
  a.proj0 = reinterpret_cast<const float*>(ctx.proj0.ptr);
  a.proj1 = reinterpret_cast<const float*>(ctx.proj1.ptr);
  a.proj2 = reinterpret_cast<const float*>(ctx.proj2.ptr);
  a.raster_rec = reinterpret_cast<const float*>(ctx.raster_rec.ptr);
  a.out_rgba = reinterpret_cast<const float*>(ctx.out_rgba.ptr);
  a.out_feat = reinterpret_cast<const float*>(ctx.out_feat.ptr);
  a.last_idx = ctx.last_idx;
  a.v_out = reinterpret_cast<const float*>(ctx.v_out.ptr);
  a.W = ctx.W; a.H = ctx.H; a.tiles_x = ctx.tiles_x; a.tiles_y = ctx.tiles_y;
  for (int k = 0; k < 3; k++) a.bg[k] = p.bg[k];
  a.inv_gscale = 1.f / grad_scale;
  a.mode = mode;
  a.v_splat = ctx.v_splat;
  a.v_splat_zero = ctx.v_splat_known_zero() ? 1 : 0;
  a.vis_flag = ctx.vis_flag;
  a.vis_weight = m.vis_weight.ptr;
  a.num_isect = ctx.num_isect;
  a.slot_sorted = ctx.slot_sorted;
  a.isect_vals = ctx.vals;
  a.tile_count = ctx.tile_count;
  a.isect_rows = reinterpret_cast<float*>(ctx.isect_rows.ptr);
  a.tile_mask = (1u << ctx.tile_bits) - 1u;
  if (mode == 1 && ctx.num_isect) {
    a.row_tag = ctx.next_row_tag(p.feat != FeatureMode::None ? 16 : 12, stream);
    if (ctx.use_row_live()) a.row_live = ctx.row_live;
  }
  if (mode == 1 && ctx.compact_ok) {
    a.cvals = ctx.cvals; a.cslots = ctx.cslots; a.clast = ctx.clast; a.cend = ctx.cend;
  }
  a.isect_part = reinterpret_cast<float*>(ctx.isect_part.ptr);
  a.isect_part_flags = ctx.isect_part_flags;
  a.split_event = ctx.bwd_split_event;
  a.feat = p.feat != FeatureMode::None ? 1 : 0;
  a.v_feat = reinterpret_cast<const float*>(ctx.v_feat.ptr);
  a.proj3 = reinterpret_cast<const float*>(ctx.proj3.ptr);
  a.hollow_z = p.hollow_z;
  a.hollow_margin = p.hollow_margin;
  a.hollow_lam = p.hollow_lam * grad_scale;
  a.defer_vis = ctx.defer_vis && mode == 1 && !a.feat && a.v_splat_zero ? 1 : 0;
  LAUNCH_CHECK(b2c_hip_raster_bwd(&a, stream));
  ctx.v_splat_zero = false;
  ctx.vis_in_rows = a.defer_vis != 0;
}

}  // namespace

void rasterize_backward(RenderCtx& ctx, const Model& m, const RenderParams& p, hipStream_t stream) {
  backward(ctx, m, p, 0, 1.f, stream);
}

void rasterize_backward_tc(RenderCtx& ctx, const Model& m, const RenderParams& p, float grad_scale, hipStream_t stream) {
  backward(ctx, m, p, 1, grad_scale, stream);
}

}  // namespace b2c
