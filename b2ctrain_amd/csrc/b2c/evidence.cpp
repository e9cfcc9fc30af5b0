// Evidence pass and depth probe (replaces src/train/evidence.cu:185-266 and src/gpu/probe.cu:47-53): the
// host loop over views and the downloads; the replays are kernels/replay.hip.
#include "evidence.h"

namespace b2c {

namespace {
// Module-level accumulators, as the reference keeps them (evidence.cu:22-23, 38-39).
DevBuf<float> g_evidence;  // [n][B2C_EVIDENCE_STRIDE]
DevBuf<float> g_view_acc;  // [n][3] the current view's (w_in, err, w_all)
DevBuf<float> g_labels;    // [n][B2C_LABEL_BINS]
bool g_labels_valid = false;
}  // namespace

void compute_evidence(RenderCtx& ctx, const Model& m, const std::vector<ViewGPU>& views, const std::vector<Camera>& cams,
                      const EvidenceParams& cfg, hipStream_t stream) {
  if (views.size() != cams.size()) throw std::runtime_error("compute_evidence: one camera per view");
  const size_t n = (size_t)(m.n > 0 ? m.n : 1);
  g_evidence.reserve(n * B2C_EVIDENCE_STRIDE);
  g_evidence.zero(stream);
  g_view_acc.reserve(n * 3);
  g_labels_valid = cfg.export_labels;
  if (g_labels_valid) {
    g_labels.reserve(n * B2C_LABEL_BINS);
    g_labels.zero(stream);
  }
  const bool use_normals = cfg.evidence_normal_weight > 0.f;
  for (size_t v = 0; v < views.size(); v++) {
    const ViewGPU& view = views[v];
    if (view.W != ctx.W || view.H != ctx.H) ctx.setup(view.W, view.H, m.cap, stream);
    RenderParams rp;
    rp.cam = CameraGPU::from(cams[v], view.W, view.H);
    rp.sh_degree = m.degree;
    rp.bwd_info = true;
    rp.feat = (use_normals && view.normals) ? FeatureMode::Normals : FeatureMode::None;
    render_forward(ctx, m, rp, stream);
    if (m.n == 0) continue;
    b2c_evidence_args a{};
    a.tile_ranges = reinterpret_cast<const uint32_t*>(ctx.tile_ranges.ptr);
    a.vals_sorted = ctx.vals_sorted;
    a.raster_rec = reinterpret_cast<const float*>(ctx.raster_rec.ptr);
    a.out_rgba = reinterpret_cast<const float*>(ctx.out_rgba.ptr);
    a.out_feat = reinterpret_cast<const float*>(ctx.out_feat.ptr);
    a.last_idx = ctx.last_idx;
    a.gt = view.rgba;
    a.normals = rp.feat == FeatureMode::Normals ? view.normals : nullptr;
    a.weights = view.weights;
    a.labels = g_labels_valid ? view.labels : nullptr;
    a.W = ctx.W; a.H = ctx.H; a.tiles_x = ctx.tiles_x; a.tiles_y = ctx.tiles_y;
    a.masked_has_alpha = (view.masked && view.has_alpha) ? 1 : 0;
    a.normal_weight = cfg.evidence_normal_weight;
    a.slot_sorted = ctx.slot_sorted;
    a.num_isect = ctx.num_isect;
    a.row_tag = ctx.next_row_tag(4, stream);
    a.rows = reinterpret_cast<float*>(ctx.isect_rows.ptr);  // the backward's row buffer, free between passes
    a.label_acc = g_labels_valid ? g_labels.ptr : nullptr;
    LAUNCH_CHECK(b2c_hip_evidence_view(&a, stream));
    b2c_evidence_sum_args sa{};
    sa.n = m.n;
    sa.m = ctx.num_isect;
    sa.ids = ctx.vals;
    sa.rows = a.rows;
    sa.row_tag = a.row_tag;
    sa.view_acc = g_view_acc.ptr;
    sa.pos_op = reinterpret_cast<const float*>(m.pos_op.ptr);
    for (int k = 0; k < 3; k++) sa.cam_pos[k] = cams[v].pos[k];
    sa.evidence = g_evidence.ptr;
    LAUNCH_CHECK(b2c_hip_evidence_sum(&sa, stream));
  }
  HIP_CHECK(hipStreamSynchronize(stream));
}

const float* evidence_device(int* stride) {
  *stride = B2C_EVIDENCE_STRIDE;
  return g_evidence.ptr;
}

std::vector<float> download_evidence(const Model& m, hipStream_t stream) {
  const size_t n = (size_t)m.n;
  std::vector<float> out(n * 7, 0.f);
  if (g_evidence.count < n * B2C_EVIDENCE_STRIDE || n == 0) return out;
  const std::vector<float> acc = g_evidence.download(n * B2C_EVIDENCE_STRIDE, stream);
  for (size_t i = 0; i < n; i++) {
    const float* a = &acc[i * B2C_EVIDENCE_STRIDE];
    float* e = &out[i * 7];
    e[0] = a[0];
    e[1] = a[1];
    e[2] = a[2];
    e[3] = a[7] > 0.f ? (a[0] * a[0]) / a[7] : 0.f;  // the participation ratio of the views' in-mask mass
    e[4] = a[4];
    e[5] = a[5];
    e[6] = a[6];
  }
  return out;
}

std::vector<float> download_labels(const Model& m, hipStream_t stream) {
  const size_t n = (size_t)m.n;
  std::vector<float> out(n * 2, 0.f);
  if (!g_labels_valid || g_labels.count < n * B2C_LABEL_BINS || n == 0) return out;
  const std::vector<float> acc = g_labels.download(n * B2C_LABEL_BINS, stream);
  for (size_t i = 0; i < n; i++) {
    const float* a = &acc[i * B2C_LABEL_BINS];
    float total = 0.f, best = 0.f;
    int win = 0;
    for (int k = 0; k < B2C_LABEL_BINS; k++) {  // the first class with the largest vote wins
      total += a[k];
      if (a[k] > best) {
        best = a[k];
        win = k;
      }
    }
    if (total > 0.f) {
      out[i * 2] = (float)win;
      out[i * 2 + 1] = best / total;
    }
  }
  return out;
}

void probe_depth(RenderCtx& ctx, float tau, float delta, const float* ref_z, float margin, float4* out, hipStream_t stream) {
  b2c_probe_args a{};
  a.tile_ranges = reinterpret_cast<const uint32_t*>(ctx.tile_ranges.ptr);
  a.vals_sorted = ctx.vals_sorted;
  a.raster_rec = reinterpret_cast<const float*>(ctx.raster_rec.ptr);
  a.W = ctx.W; a.H = ctx.H; a.tiles_x = ctx.tiles_x; a.tiles_y = ctx.tiles_y;
  a.tau = tau; a.delta = delta; a.margin = margin;
  a.ref_z = ref_z;
  a.out = reinterpret_cast<float*>(out);
  LAUNCH_CHECK(b2c_hip_probe_depth(&a, stream));
}

}  // namespace b2c
