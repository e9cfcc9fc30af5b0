// Model upload / download / growth (replaces src/model.cu:8-118, the parts the rasterizer path needs).
#include "model.h"

#include <cmath>
#include <cstring>
#include <type_traits>

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
}

uint16_t float_to_half_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

float half_to_float(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

void Model::reserve(int want, hipStream_t stream) {
  if (want <= cap) return;
  int ncap = cap ? cap : 1024;
  while (ncap < want) ncap *= 2;
  const int hi_lanes = (K() - 1) * 3;
  auto grow_planar = [&](auto& b, int lanes) {
    using T = std::remove_reference_t<decltype(*b.ptr)>;
    if (lanes == 0) return;
    DevBuf<T> nb;
    nb.reserve((size_t)ncap * lanes);
    nb.zero(stream);
    if (b.ptr && n > 0)
      HIP_CHECK(hipMemcpy2DAsync(nb.ptr, (size_t)ncap * sizeof(T), b.ptr, (size_t)cap * sizeof(T), (size_t)n * sizeof(T),
                                 lanes, hipMemcpyDeviceToDevice, stream));
    HIP_CHECK(hipStreamSynchronize(stream));
    b = std::move(nb);
  };
  pos_op.reserve(ncap, true, stream);
  quat.reserve(ncap, true, stream);
  lscale.reserve(ncap, true, stream);
  grow_planar(sh_dc, 3);
  if (sh_fp16) grow_planar(sh_hi, hi_lanes); else grow_planar(sh_hi32, hi_lanes);
  for (DevBuf<float>* b : {&refine_norm, &max_screen, &vis_count, &vis_weight}) {
    b->reserve((size_t)ncap, true, stream);
    LAUNCH_CHECK(b2c_hip_fill_u32(reinterpret_cast<uint32_t*>(b->ptr + cap), 0u, (size_t)(ncap - cap), stream));
  }
  cap = ncap;
}

void Model::upload(const SplatCloud& c, hipStream_t stream) {
  degree = c.sh_degree;
  n = (int)c.n;
  cap = 0;
  pos_op.free(); quat.free(); lscale.free(); sh_dc.free(); sh_hi.free(); sh_hi32.free();
  refine_norm.free(); max_screen.free(); vis_count.free(); vis_weight.free();
  reserve(n > 0 ? n : 1, stream);
  std::vector<float4> p(n), q(n), s(n);
  for (int i = 0; i < n; i++) {
    p[i] = make_float4(c.pos[i * 3], c.pos[i * 3 + 1], c.pos[i * 3 + 2], c.opacity[i]);
    q[i] = make_float4(c.quat[i * 4], c.quat[i * 4 + 1], c.quat[i * 4 + 2], c.quat[i * 4 + 3]);
    s[i] = make_float4(c.log_scale[i * 3], c.log_scale[i * 3 + 1], c.log_scale[i * 3 + 2], 0.f);
  }
  if (n) {
    HIP_CHECK(hipMemcpyAsync(pos_op.ptr, p.data(), n * sizeof(float4), hipMemcpyHostToDevice, stream));
    HIP_CHECK(hipMemcpyAsync(quat.ptr, q.data(), n * sizeof(float4), hipMemcpyHostToDevice, stream));
    HIP_CHECK(hipMemcpyAsync(lscale.ptr, s.data(), n * sizeof(float4), hipMemcpyHostToDevice, stream));
  }
  const int K = this->K(), hi = (K - 1) * 3;
  std::vector<float> dc((size_t)cap * 3, 0.f), rest((size_t)cap * hi, 0.f);
  for (int i = 0; i < n; i++) {
    for (int k = 0; k < 3; k++) dc[(size_t)k * cap + i] = c.sh[(size_t)i * K * 3 + k];
    for (int k = 0; k < hi; k++) rest[(size_t)k * cap + i] = c.sh[(size_t)i * K * 3 + 3 + k];
  }
  HIP_CHECK(hipMemcpyAsync(sh_dc.ptr, dc.data(), dc.size() * sizeof(float), hipMemcpyHostToDevice, stream));
  if (hi > 0) {
    if (sh_fp16) {
      std::vector<uint16_t> h(rest.size());
      for (size_t j = 0; j < rest.size(); j++) h[j] = float_to_half_rne(rest[j]);
      HIP_CHECK(hipMemcpyAsync(sh_hi.ptr, h.data(), h.size() * sizeof(uint16_t), hipMemcpyHostToDevice, stream));
      HIP_CHECK(hipStreamSynchronize(stream));
    } else {
      HIP_CHECK(hipMemcpyAsync(sh_hi32.ptr, rest.data(), rest.size() * sizeof(float), hipMemcpyHostToDevice, stream));
    }
  }
  HIP_CHECK(hipStreamSynchronize(stream));
  zero_stats(stream);
  HIP_CHECK(hipStreamSynchronize(stream));
}

SplatCloud Model::download(hipStream_t stream) const {
  SplatCloud c;
  c.resize((size_t)n, degree);
  auto p = pos_op.download(n, stream);
  auto q = quat.download(n, stream);
  auto s = lscale.download(n, stream);
  const int K = this->K(), hi = (K - 1) * 3;
  auto dc = sh_dc.download((size_t)cap * 3, stream);
  std::vector<float> rest;
  if (hi > 0) {
    if (sh_fp16) {
      auto h = sh_hi.download((size_t)cap * hi, stream);
      rest.resize(h.size());
      for (size_t j = 0; j < h.size(); j++) rest[j] = half_to_float(h[j]);
    } else {
      rest = sh_hi32.download((size_t)cap * hi, stream);
    }
  }
  for (int i = 0; i < n; i++) {
    c.pos[i * 3] = p[i].x; c.pos[i * 3 + 1] = p[i].y; c.pos[i * 3 + 2] = p[i].z; c.opacity[i] = p[i].w;
    c.quat[i * 4] = q[i].x; c.quat[i * 4 + 1] = q[i].y; c.quat[i * 4 + 2] = q[i].z; c.quat[i * 4 + 3] = q[i].w;
    c.log_scale[i * 3] = s[i].x; c.log_scale[i * 3 + 1] = s[i].y; c.log_scale[i * 3 + 2] = s[i].z;
    for (int k = 0; k < 3; k++) c.sh[(size_t)i * K * 3 + k] = dc[(size_t)k * cap + i];
    for (int k = 0; k < hi; k++) c.sh[(size_t)i * K * 3 + 3 + k] = rest[(size_t)k * cap + i];
  }
  return c;
}

void Model::set_floor(const std::vector<float>& f, hipStream_t stream) {
  if ((int)f.size() != n) throw std::runtime_error("set_floor: expected one floor value per splat");
  auto s = lscale.download(n, stream);
  for (int i = 0; i < n; i++) s[i].w = f[i];
  if (n) HIP_CHECK(hipMemcpyAsync(lscale.ptr, s.data(), n * sizeof(float4), hipMemcpyHostToDevice, stream));
  HIP_CHECK(hipStreamSynchronize(stream));
}

void Model::zero_stats(hipStream_t stream) {
  refine_norm.zero(stream); max_screen.zero(stream); vis_count.zero(stream); vis_weight.zero(stream);
}

}  // namespace b2c
