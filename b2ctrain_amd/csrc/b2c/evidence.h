// Tile-list consumers of the drop-in (replaces src/train/evidence.h:1-23 and src/gpu/probe.h:1-14): the
// multi-view evidence pass with its label vote, and the per-pixel depth probe. Same entry points and
// accumulator semantics; the body-rig / cage posing of the reference's compute_evidence is outside this build.
#pragma once
#include <vector>

#include "loss.h"

namespace b2c {

// The Config fields compute_evidence reads (src/cli.h): the normal residual's weight in the evidence error
// and whether to accumulate the per-class label vote.
struct EvidenceParams {
  float evidence_normal_weight = 0.f;
  bool export_labels = false;
};

// Per splat over all views (evidence.cu:185-226): [n][7] = (w_in, w_all, err, views, dir xyz). Each view
// is rendered (with pseudo-normals when the normal weight is positive and the view has a normal map) and
// replayed; the accumulator stays in a module-level buffer until the next call.
void compute_evidence(RenderCtx& ctx, const Model& m, const std::vector<ViewGPU>& views, const std::vector<Camera>& cams,
                      const EvidenceParams& cfg, hipStream_t stream);
// The reference's signature takes its Config; any type with the two fields above works here.
template <typename Config>
void compute_evidence(RenderCtx& ctx, const Model& m, const std::vector<ViewGPU>& views, const std::vector<Camera>& cams,
                      const Config& cfg, hipStream_t stream) {
  EvidenceParams p;
  p.evidence_normal_weight = cfg.evidence_normal_weight;
  p.export_labels = cfg.export_labels;
  compute_evidence(ctx, m, views, cams, p, stream);
}
// [n][7]: views = (sum w_in)^2 / sum w_in^2, the effective number of supporting views (evidence.cu:236-249).
std::vector<float> download_evidence(const Model& m, hipStream_t stream);
// The device accumulator of the last compute_evidence: [n][*stride], w_all at offset 1.
const float* evidence_device(int* stride);
// [n][2] = (winning class id, its share of the splat's vote); both 0 for a splat no labelled view rendered.
std::vector<float> download_labels(const Model& m, hipStream_t stream);

// Per-pixel depth distribution of the composited splats after project_splats + bin_and_sort
// (probe.h:6-11): out[pix] = (accumulated alpha, first-surface depth at alpha tau (tau <= 0: the
// alpha-weighted mean depth), weight from more than delta behind it, weight from more than margin behind
// ref_z (+inf or NULL = none)). out is a device array of W*H float4.
void probe_depth(RenderCtx& ctx, float tau, float delta, const float* ref_z, float margin, float4* out, hipStream_t stream);

}  // namespace b2c
