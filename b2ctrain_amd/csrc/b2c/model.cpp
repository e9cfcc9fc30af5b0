// Model storage (replaces the upload / download / growth / optimizer-reset parts of src/model.cu:8-118).
// The host side only moves whole arrays: an upload copies the cloud's five field arrays into one device
// staging block and a scatter kernel writes the float4 fields and the planar SH lanes (fp16 rounding on
// the device); a download is the inverse gather; growth re-lays the planar lanes out with a kernel
// (kernels/model_io.hip) and starts the new slots' statistics and Adam moments at zero.
#include "model.h"

#include <algorithm>

namespace b2c {

void SplatCloud::resize(size_t count, int degree) {
  n = count;
  sh_degree = degree;
  pos.assign(n * 3, 0.f);
  log_scale.assign(n * 3, 0.f);
  quat.assign(n * 4, 0.f);
  opacity.assign(n, 0.f);
  sh.assign(n * (size_t)K() * 3, 0.f);
  for (size_t i = 0; i < n; i++) quat[i * 4] = 1.f;
  const auto block = [&](bool on, std::vector<float>& v, size_t per, float fill_value) {
    if (on) v.assign(n * per, fill_value);
  };
  block(has_evidence, evidence, 7, 0.f);
  block(has_labels, labels, 2, 0.f);
  block(has_fill, fill, 1, 0.f);
  block(has_gate, gate, 2, -1.f);
  block(has_gate_s, gate_s, 1, 0.f);
  block(has_open, open, 4, 0.f);
}

uint16_t float_to_half_rne(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }
float half_to_float(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

namespace {

// A cloud's field arrays back to back in one device block: pos, log_scale, quat, opacity, sh, floor.
struct CloudStage {
  DevBuf<float> block;
  b2c_cloud_dev fields{};

  CloudStage(size_t n, int K, bool with_floor) {
    const size_t o_ls = 3 * n, o_q = o_ls + 3 * n, o_op = o_q + 4 * n, o_sh = o_op + n, o_fl = o_sh + 3 * (size_t)K * n;
    block.reserve(std::max<size_t>(o_fl + (with_floor ? n : 0), 1));
    float* b = block.ptr;
    fields = b2c_cloud_dev{b, b + o_ls, b + o_q, b + o_op, b + o_sh, with_floor ? b + o_fl : nullptr};
  }
};

template <typename T>
void to_device(float* dst, const std::vector<T>& src, hipStream_t s) {
  if (!src.empty()) HIP_CHECK(hipMemcpyAsync(dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice, s));
}

template <typename T>
void to_host(std::vector<T>& dst, const float* src, hipStream_t s) {
  if (!dst.empty()) HIP_CHECK(hipMemcpyAsync(dst.data(), src, dst.size() * sizeof(T), hipMemcpyDeviceToHost, s));
}

// A planar [lanes][cap] array moved to a larger stride by the re-layout kernel (new slots zero).
template <typename T>
void regrow_planar(DevBuf<T>& buf, int lanes, int n, int old_cap, int new_cap, hipStream_t s) {
  if (lanes <= 0) return;
  DevBuf<T> wider;
  wider.reserve((size_t)lanes * new_cap);
  LAUNCH_CHECK(b2c_hip_planar_regrow(buf.ptr, wider.ptr, (int)sizeof(T), lanes, n, old_cap, new_cap, s));
  HIP_CHECK(hipStreamSynchronize(s));  // the old array is freed on assignment
  buf = std::move(wider);
}

}  // namespace

b2c_model_dev Model::layout() const {
  b2c_model_dev d{};
  d.n = n; d.cap = cap; d.sh_lanes = 3 * K();
  d.pos_op = reinterpret_cast<float*>(pos_op.ptr);
  d.quat = reinterpret_cast<float*>(quat.ptr);
  d.lscale = reinterpret_cast<float*>(lscale.ptr);
  d.sh_dc = sh_dc.ptr;
  d.sh_hi32 = sh_fp16 ? nullptr : sh_hi32.ptr;
  d.sh_hi16 = sh_fp16 ? sh_hi.ptr : nullptr;
  return d;
}

void Model::reserve(int want, hipStream_t stream) {
  if (want <= cap) return;
  int grown = std::max(cap, 1024);
  while (grown < want) grown *= 2;
  for (DevBuf<float4>* f : {&pos_op, &quat, &lscale}) f->reserve((size_t)grown, true, stream);
  const int bands = 3 * (K() - 1);
  regrow_planar(sh_dc, 3, n, cap, grown, stream);
  if (sh_fp16) regrow_planar(sh_hi, bands, n, cap, grown, stream);
  else regrow_planar(sh_hi32, bands, n, cap, grown, stream);
  // Per-splat arrays keep their first cap entries; the new ones start at zero (statistics, moments).
  const size_t fresh = (size_t)(grown - cap);
  for (DevBuf<float>* st : {&refine_norm, &max_screen, &vis_count, &vis_weight, &v_sh}) {
    st->reserve((size_t)grown, true, stream);
    LAUNCH_CHECK(b2c_hip_fill_u32(reinterpret_cast<uint32_t*>(st->ptr + cap), 0u, fresh, stream));
  }
  last_step.reserve((size_t)grown, true, stream);
  LAUNCH_CHECK(b2c_hip_fill_u32(last_step.ptr + cap, 0u, fresh, stream));
  for (DevBuf<float4>* mo : {&m_pos_op, &v_pos_op, &m_quat, &v_quat, &m_lscale, &v_lscale}) {
    mo->reserve((size_t)grown, true, stream);
    LAUNCH_CHECK(b2c_hip_fill_u32(reinterpret_cast<uint32_t*>(mo->ptr + cap), 0u, 4 * fresh, stream));
  }
  regrow_planar(m_sh_dc, 3, n, cap, grown, stream);
  if (sh_fp16) regrow_planar(m_sh_hi, bands, n, cap, grown, stream);
  else regrow_planar(m_sh_hi32, bands, n, cap, grown, stream);
  cap = grown;
}

void Model::reset(int count, int deg, hipStream_t stream) {
  degree = deg;
  n = count;
  cap = 0;
  for (DevBuf<float4>* f : {&pos_op, &quat, &lscale, &m_pos_op, &v_pos_op, &m_quat, &v_quat, &m_lscale, &v_lscale})
    f->free();
  for (DevBuf<float>* f : {&sh_dc, &sh_hi32, &m_sh_dc, &m_sh_hi32}) f->free();
  sh_hi.free(); m_sh_hi.free();
  for (DevBuf<float>* st : {&refine_norm, &max_screen, &vis_count, &vis_weight, &v_sh}) st->free();
  last_step.free();
  reserve(std::max(n, 1), stream);
}

void Model::upload(const SplatCloud& c, hipStream_t stream, const float* floor) {
  reset((int)c.n, c.sh_degree, stream);
  CloudStage stage(c.n, K(), floor != nullptr);
  to_device(stage.fields.pos, c.pos, stream);
  to_device(stage.fields.log_scale, c.log_scale, stream);
  to_device(stage.fields.quat, c.quat, stream);
  to_device(stage.fields.opacity, c.opacity, stream);
  to_device(stage.fields.sh, c.sh, stream);
  if (floor && n) HIP_CHECK(hipMemcpyAsync(stage.fields.floor_, floor, n * sizeof(float), hipMemcpyHostToDevice, stream));
  const b2c_model_dev dst = layout();
  LAUNCH_CHECK(b2c_hip_model_scatter(&stage.fields, &dst, stream));
  zero_optimizer(stream);
  zero_stats(stream);
  HIP_CHECK(hipStreamSynchronize(stream));  // the stage and the caller's arrays may go away now
}

SplatCloud Model::download(hipStream_t stream) const {
  SplatCloud c;
  c.resize((size_t)n, degree);
  CloudStage stage(c.n, K(), false);
  const b2c_model_dev src = layout();
  LAUNCH_CHECK(b2c_hip_model_gather(&src, &stage.fields, stream));
  to_host(c.pos, stage.fields.pos, stream);
  to_host(c.log_scale, stage.fields.log_scale, stream);
  to_host(c.quat, stage.fields.quat, stream);
  to_host(c.opacity, stage.fields.opacity, stream);
  to_host(c.sh, stage.fields.sh, stream);
  HIP_CHECK(hipStreamSynchronize(stream));
  return c;
}

void Model::set_floor(const std::vector<float>& f, hipStream_t stream) {
  if ((int)f.size() != n) throw std::runtime_error("set_floor: expected one floor value per splat");
  DevBuf<float> staged;
  staged.upload(f, stream);
  LAUNCH_CHECK(b2c_hip_model_set_floor(reinterpret_cast<float*>(lscale.ptr), staged.ptr, n, stream));
  HIP_CHECK(hipStreamSynchronize(stream));
}

void Model::zero_stats(hipStream_t stream) {
  for (DevBuf<float>* st : {&refine_norm, &max_screen, &vis_count, &vis_weight}) st->zero(stream);
}

void Model::zero_optimizer(hipStream_t stream) {
  for (DevBuf<float4>* mo : {&m_pos_op, &v_pos_op, &m_quat, &v_quat, &m_lscale, &v_lscale}) mo->zero(stream);
  for (DevBuf<float>* f : {&m_sh_dc, &m_sh_hi32, &v_sh}) f->zero(stream);
  m_sh_hi.zero(stream);
  last_step.zero(stream);
  adam_t = 0;
}

b2c_adam_state Model::adam_state() const {
  b2c_adam_state s{};
  s.m_pos_op = reinterpret_cast<float*>(m_pos_op.ptr);
  s.v_pos_op = reinterpret_cast<float*>(v_pos_op.ptr);
  s.m_quat = reinterpret_cast<float*>(m_quat.ptr);
  s.v_quat = reinterpret_cast<float*>(v_quat.ptr);
  s.m_lscale = reinterpret_cast<float*>(m_lscale.ptr);
  s.v_lscale = reinterpret_cast<float*>(v_lscale.ptr);
  const ShBuf m = m_sh();
  s.m_sh = b2c_sh_planes{m.dc, sh_fp16 ? m.hi : nullptr, sh_fp16 ? nullptr : m.hi32, m.stride};
  s.v_sh = v_sh.ptr;
  s.last_step = last_step.ptr;
  return s;
}

}  // namespace b2c
