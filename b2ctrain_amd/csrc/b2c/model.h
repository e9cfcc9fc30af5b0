// Splat model and its host cloud (replaces src/model.h:8-40 and the SplatCloud of src/ply.h:10-42, the
// fields the rasterizer uses). The device layout is the reference's, unchanged, because refine / cage /
// evidence code reads it:
//   pos_op : float4 (mean x, y, z, opacity logit)
//   quat   : float4 (w, x, y, z), unnormalised
//   lscale : float4 (log sx, log sy, log sz, floor f), f frozen (0 = none)
//   SH     : planar, lane k*3+ch of splat i; DC lanes in sh_dc[lane*cap + i] (fp32); lanes >= 3 in
//            sh_hi[(lane-3)*cap + i] as IEEE fp16 when sh_fp16, else sh_hi32 (fp32).
#pragma once
#include <vector>

#include "util.h"

namespace b2c {

constexpr float SH_C0 = 0.28209479177387814f;
inline int sh_coeffs_for_degree(int d) { return (d + 1) * (d + 1); }

// Host-side splat cloud in brush's parameterisation (src/ply.h:10-42): the fields the rasterizer uses and
// the optional per-splat blocks a ply carries beside them (the evidence and label exports, the cage
// fields), which the model does not hold.
struct SplatCloud {
  size_t n = 0;
  int sh_degree = 0;
  std::vector<float> pos;        // [n][3]
  std::vector<float> log_scale;  // [n][3]
  std::vector<float> quat;       // [n][4] (w, x, y, z)
  std::vector<float> opacity;    // [n] logit
  std::vector<float> sh;         // [n][K][3] coefficient-major
  bool has_scales = true;        // false: the file had no scale_* (a point cloud; scales to be initialised)
  bool has_evidence = false;
  std::vector<float> evidence;   // [n][7] w_in, w_all, err, views, dir xyz (download_evidence)
  bool has_labels = false;
  std::vector<float> labels;     // [n][2] class id, share (download_labels)
  bool has_fill = false;
  std::vector<float> fill;       // [n] cage_fill
  bool has_gate = false;
  std::vector<float> gate;       // [n][2] cage_gate_a, cage_gate_b (-1 when absent)
  bool has_gate_s = false;
  std::vector<float> gate_s;     // [n] cage_gate_s
  bool has_open = false;
  std::vector<float> open;       // [n][4] open_r, open_g, open_b, open_dopacity
  int K() const { return sh_coeffs_for_degree(sh_degree); }
  // src/ply.cpp:15-22: every array sized for `count` splats and zeroed, identity quaternions, the gate
  // pair -1; the optional blocks sized only when their flag is set.
  void resize(size_t count, int degree);
};

// Planar SH view handed to the kernels (ShBuf, util.cuh:129-164).
struct ShBuf {
  float* dc = nullptr;
  uint16_t* hi = nullptr;  // fp16 bits
  float* hi32 = nullptr;
  size_t stride = 0;
  b2c_sh_view view() const { return b2c_sh_view{dc, hi, hi32, stride}; }
  b2c_sh_planes planes() const { return b2c_sh_planes{dc, hi, hi32, stride}; }
};

struct Model {
  int n = 0, cap = 0, degree = 3;
  bool sh_fp16 = false;  // choose before upload(): fp16 storage for SH bands >= 1
  DevBuf<float4> pos_op, quat, lscale;
  DevBuf<float> sh_dc, sh_hi32;
  DevBuf<uint16_t> sh_hi;
  // statistics updated as side effects of the path (model.h:27-30)
  DevBuf<float> refine_norm, max_screen, vis_count, vis_weight;
  // Adam state (model.h:19-28): first / second moments beside each float4 array; SH first moments in the
  // SH's planar layout and band precision; v_sh one second moment per splat; last_step the Adam step of
  // each splat's last update (lazy sparse Adam, 0 = never); adam_t the step counter the trainer advances.
  DevBuf<float4> m_pos_op, v_pos_op, m_quat, v_quat, m_lscale, v_lscale;
  DevBuf<float> m_sh_dc, m_sh_hi32, v_sh;
  DevBuf<uint16_t> m_sh_hi;
  DevBuf<uint32_t> last_step;
  int adam_t = 0;

  ShBuf sh() const {
    ShBuf b;
    b.dc = sh_dc.ptr; b.hi = sh_hi.ptr; b.hi32 = sh_hi32.ptr; b.stride = (size_t)cap;
    return b;
  }
  ShBuf m_sh() const {
    ShBuf b;
    b.dc = m_sh_dc.ptr; b.hi = m_sh_hi.ptr; b.hi32 = m_sh_hi32.ptr; b.stride = (size_t)cap;
    return b;
  }
  int K() const { return sh_coeffs_for_degree(degree); }
  // Capacity for `want` splats, doubling from 1024 (the reference's growth policy, model.cu:8-42); the
  // first n splats keep their values, planar slots past n read as zero.
  void reserve(int want, hipStream_t stream = nullptr);
  // Drop every array and size the model for `count` splats of SH degree `deg` (contents undefined until
  // written: upload and the ply loader fill them, then zero the statistics and the optimizer state).
  void reset(int count, int deg, hipStream_t stream = nullptr);
  // Replace the model by a cloud (model.cu:44-80): bands rounded to nearest even when stored as fp16,
  // statistics zeroed, lscale.w = floor[i] (0 without a floor, as the reference uploads).
  void upload(const SplatCloud& c, hipStream_t stream = nullptr, const float* floor = nullptr);
  SplatCloud download(hipStream_t stream = nullptr) const;
  // Set the frozen per-splat floor f (lscale.w); not part of the reference's upload.
  void set_floor(const std::vector<float>& f, hipStream_t stream = nullptr);
  void zero_stats(hipStream_t stream = nullptr);
  // Moments, v_sh and last_step to zero, adam_t = 0 (model.cu:104-107).
  void zero_optimizer(hipStream_t stream = nullptr);
  // The Adam state as the fused optimizer kernel takes it.
  b2c_adam_state adam_state() const;
  // The device layout as the launcher layer takes it.
  b2c_model_dev layout() const;
};

// IEEE binary16 encode (round to nearest even) / decode on the host.
uint16_t float_to_half_rne(float f);
float half_to_float(uint16_t h);

}  // namespace b2c
