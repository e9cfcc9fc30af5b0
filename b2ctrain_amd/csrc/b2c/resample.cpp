// Separable resampling of RGBA8 images, restating the arithmetic stb_image_resize2 v2.18 performs for a
// 4-channel uint8 -> uint8 resize with clamped edges (the reference's resize_rgba, views.cpp:73-78):
//  * per axis, weights are sampled from the filter at pixel centres in single precision (stretched over
//    the output grid when shrinking), leading tiny weights are dropped, each output's weights are
//    normalised in double and rounded to float, weights that fall outside the image are folded onto the
//    edge pixel, and trailing zeros are trimmed; when the scale is a ratio p/q of small integers the first p
//    outputs' weights are computed and repeated every p outputs, shifted by q input pixels;
//  * the horizontal weight rows are re-based so that no row reads past the end of the scanline;
//  * samples are the byte values as floats (no 1/255 scaling); a horizontal output is the sum of its
//    even-position terms plus the sum of its odd-position terms (one running sum when a row has at most 3
//    weights); a vertical output adds its terms in input-row order; outputs are rounded by +0.5 and
//    truncation after clamping to [0, 255];
//  * the vertical pass runs first or second according to a cost model of the two orders.
#pragma clang fp contract(off)
#include "resample.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>

namespace b2c {

namespace {

constexpr float TINY = 1.0f / (float)(1 << 20) / (float)(1 << 20) / (float)(1 << 20) / (float)(1 << 20) /
                       (float)(1 << 20) / (float)(1 << 20);  // 2^-120

struct Filter {
  float support;  // half-width in the grid it is evaluated in
  float (*kernel)(float x);
};

float tent(float x) {
  if (x < 0.0f) x = -x;
  return x <= 1.0f ? 1.0f - x : 0.0f;
}
float mitchell(float x) {  // (B, C) = (1/3, 1/3), evaluated in the reference's operation order
  if (x < 0.0f) x = -x;
  if (x < 1.0f) return (16.0f + x * x * (21.0f * x - 36.0f)) / 18.0f;
  if (x < 2.0f) return (32.0f + x * (-60.0f + x * (36.0f - 7.0f * x))) / 18.0f;
  return 0.0f;
}
float box(float) { return 1.0f; }

Filter filter_of(ResampleFilter f) {
  switch (f) {
    case ResampleFilter::Triangle: return {1.0f, tent};
    case ResampleFilter::Mitchell: return {2.0f, mitchell};
    default: return {0.5f, box};
  }
}

// The scale as numerator / denominator when a continued-fraction convergent with the bounded term is
// within one float ulp of it (bounds the denominator when enlarging, the numerator when shrinking).
bool as_ratio(double f, uint32_t limit, bool limit_denominator, uint32_t* num, uint32_t* den) {
  uint64_t top = (uint64_t)(f * (double)(1 << 25)), bot = 1 << 25;
  uint64_t n_prev = 0, d_prev = 1, n_cur = 1, d_cur = 0;
  for (;;) {
    if ((limit_denominator ? d_cur : n_cur) >= limit) break;
    if (d_cur) {
      double err = (double)n_cur / (double)d_cur - f;
      if (err < 0.0) err = -err;
      if (err < 1.0 / (double)(1 << 24)) {
        *num = (uint32_t)n_cur;
        *den = (uint32_t)d_cur;
        return true;
      }
    }
    if (bot == 0) break;
    const uint64_t q = top / bot, r = top % bot;
    top = bot;
    bot = r;
    const uint64_t d_next = q * d_cur + d_prev, n_next = q * n_cur + n_prev;
    d_prev = d_cur;
    d_cur = d_next;
    n_prev = n_cur;
    n_cur = n_next;
  }
  if (limit_denominator) {
    n_cur = (uint64_t)(f * (double)limit + 0.5);
    d_cur = limit;
  } else {
    n_cur = limit;
    d_cur = (uint64_t)((double)limit / f + 0.5);
  }
  *num = (uint32_t)n_cur;
  *den = (uint32_t)d_cur;
  double err = d_cur ? (double)(uint32_t)n_cur / (double)(uint32_t)d_cur - f : 1.0;
  if (err < 0.0) err = -err;
  return err < 1.0 / (double)(1 << 24);
}

struct Span {
  int n0, n1;
};

enum Mode { SCATTER = 0, GATHER_UP = 1, GATHER_DOWN = 2 };

struct Axis {
  int in = 0, out = 0;
  float scale = 1.f, inv_scale = 1.f;
  bool ratio = false;
  uint32_t num = 0, den = 0;
  Mode mode = GATHER_UP;
  int pixel_width = 0;  // input pixels that can reach one output
  int margin = 0;
  int width = 0;        // weights stored per output
  std::vector<Span> span;
  std::vector<float> w;  // [out][width]
  int widest = 0;
  Filter f{};

  float* row(int n) { return w.data() + (size_t)n * width; }
};

// Adds weight `c` for input pixel `p` to an output's weight row (the reference's insertion rules: the row
// grows at either end within `cap` weights; a pixel already covered accumulates).
void add_weight(Span& s, float* c, int p, float wgt, int cap) {
  if (s.n1 < s.n0) {
    s.n0 = s.n1 = p;
    c[0] = wgt;
  } else if (p <= s.n1) {
    if (p < s.n0) {
      if (s.n1 - p + 1 <= cap) {
        const int shift = s.n0 - p;
        for (int j = s.n1 - s.n0; j >= 0; j--) c[j + shift] = c[j];
        for (int j = 1; j < shift; j++) c[j] = 0.f;
        c[0] = wgt;
        s.n0 = p;
      }
    } else {
      c[p - s.n0] += wgt;
    }
  } else if (p - s.n0 + 1 <= cap) {
    const int e = p - s.n0;
    for (int j = s.n1 - s.n0 + 1; j < e; j++) c[j] = 0.f;
    c[e] = wgt;
    s.n1 = p;
  }
}

// Input pixels an output centre's window reaches.
void in_range(float centre, float radius, float inv_scale, int* first, int* last) {
  const float lo = (centre - radius) * inv_scale, hi = (centre + radius) * inv_scale;
  *first = (int)std::floor(lo + 0.5f);
  *last = (int)std::floor(hi - 0.5f);
  if (*last < *first) *last = *first;
}

// Output pixels an input centre's window reaches, clipped to the output.
void out_range(float centre, float radius, float scale, int out, int* first, int* last) {
  const float lo = (centre - radius) * scale, hi = (centre + radius) * scale;
  *first = std::max((int)std::floor(lo + 0.5f), 0);
  *last = std::min((int)std::floor(hi - 0.5f), out - 1);
}

void setup_axis(Axis& a, int in, int out, const Filter& f, bool horizontal) {
  a.in = in;
  a.out = out;
  a.f = f;
  const double s = (double)out / (double)in;
  a.scale = (float)s;
  a.inv_scale = (float)(1.0 / s);
  a.ratio = as_ratio(s, s <= 1.0 ? (uint32_t)out : (uint32_t)in, s >= 1.0, &a.num, &a.den);
  const bool up = a.scale >= 1.0f - TINY;
  a.pixel_width = up ? (int)std::ceil(f.support * 2.0f) : (int)std::ceil(f.support * 2.0f / a.scale);
  a.mode = up ? GATHER_UP : ((horizontal || a.pixel_width <= 32) ? GATHER_DOWN : SCATTER);
  // a scatter's weights are built in gather form first, pixel_width per output
  a.width = a.mode == GATHER_UP ? (int)std::ceil(f.support * 2.0f)
                                : (int)std::ceil(f.support * 2.0f / a.scale);
  a.margin = a.pixel_width / 2;
  a.span.assign(out, Span{0, -1});
  a.w.assign((size_t)out * a.width + 3, 0.f);
}

void weights_up(Axis& a) {
  const float radius = a.f.support * a.scale;
  const bool poly = a.ratio && (int)a.num < a.out;
  const int end = poly ? (int)a.num : a.out;
  for (int n = 0; n < end; n++) {
    const float centre = (float)n + 0.5f, src = centre * a.inv_scale;
    int first, last;
    in_range(centre, radius, a.inv_scale, &first, &last);
    if (last - first + 1 > a.width) last = first + a.width - 1;
    float* c = a.row(n);
    int last_nz = -1;
    for (int i = 0; i <= last - first; i++) {
      const float wgt = a.f.kernel(src - ((float)(i + first) + 0.5f));
      if (wgt < TINY && wgt > -TINY) {
        if (i == 0) {  // leading zero weights move the window start
          first++;
          i--;
          continue;
        }
        c[i] = 0.f;
      } else {
        c[i] = wgt;
        last_nz = i;
      }
    }
    a.span[n] = {first, last_nz + first};
  }
}

void weights_down(Axis& a) {
  const float radius = a.f.support * a.inv_scale;
  const bool poly = a.ratio && (int)a.num < a.out;
  int inited = -1;
  for (int p = -a.margin; p < a.in + a.margin; p++) {
    const float centre = (float)p + 0.5f, dst = centre * a.scale;
    int first, last;
    out_range(centre, radius, a.scale, a.out, &first, &last);
    if (first > last) continue;
    if (poly) {
      if (first == (int)a.num) break;
      if (last >= (int)a.num) last = (int)a.num - 1;
    }
    for (int o = first; o <= last; o++) {
      float wgt = a.f.kernel(((float)o + 0.5f) - dst) * a.scale;
      if (wgt < TINY && wgt > -TINY) wgt = 0.f;
      float* c = a.row(o);
      Span& s = a.span[o];
      if (o > inited) {
        inited = o;
        s = {p, p};
        c[0] = wgt;
      } else {
        if (c[0] == 0.0f) s.n0 = p;  // a zero first weight is dropped
        s.n1 = p;
        c[p - s.n0] = wgt;
      }
    }
  }
}

// Normalise, repeat over the period, fold the out-of-image weights onto the edge pixels, trim.
void finish_weights(Axis& a) {
  const bool poly = a.ratio && (int)a.num < a.out;
  const int end = poly ? (int)a.num : a.out;
  for (int n = 0; n < end; n++) {
    Span& s = a.span[n];
    float* c = a.row(n);
    double total = 0.0;
    for (int i = 0; i <= s.n1 - s.n0; i++) total += (double)c[i];
    if (total < TINY && total > -TINY) {
      s.n1 = s.n0;
      c[0] = 0.f;
    } else if (total < 1.0f - TINY || total > 1.0f + TINY) {
      const double k = 1.0 / total;
      for (int i = 0; i <= s.n1 - s.n0; i++) c[i] = (float)(c[i] * k);
    }
  }
  if (poly) {
    for (int n = (int)a.num; n < a.out; n++) {
      a.span[n] = {a.span[n - a.num].n0 + (int)a.den, a.span[n - a.num].n1 + (int)a.den};
      std::memcpy(a.row(n), a.row(n - a.num), sizeof(float) * a.width);
    }
  }
  const int last_px = a.in - 1;
  a.widest = -1;
  for (int n = 0; n < a.out; n++) {
    Span& s = a.span[n];
    float* c = a.row(n);
    if (s.n1 > last_px) {  // right edge: pixels past it add to the last pixel, in increasing order
      const int start = s.n0, stop = s.n1;
      s.n1 = last_px;
      for (int p = a.in; p <= stop; p++) add_weight(s, c, last_px, c[p - start], a.width);
    }
    if (s.n0 < 0) {  // left edge: pixels -1, -2, ... add to pixel 0, then the first one after re-basing
      const float* src = c - (s.n0 + 1);  // weight of pixel -1
      for (int p = -1; p > s.n0; p--) add_weight(s, c, 0, *src--, a.width);
      const int old_n0 = s.n0;
      const float first_w = src[0];
      s.n0 = 0;
      for (int i = 0; i <= s.n1; i++) c[i] = c[i - old_n0];
      add_weight(s, c, 0, first_w, a.width);
    }
    if (s.n0 <= s.n1) {
      int count = s.n1 - s.n0 + 1;
      while (count && c[count - 1] == 0.0f) count--;
      s.n1 = s.n0 + count - 1;
      if (s.n0 <= s.n1) a.widest = std::max(a.widest, count);
      for (int i = count; i < a.width; i++) c[i] = 0.f;
    }
  }
}

void build_weights(Axis& a) {
  if (a.mode == GATHER_UP) weights_up(a);
  else weights_down(a);
  finish_weights(a);
}

// Input columns the horizontal pass decodes: those the first and the last output can reach.
Span decoded_columns(const Axis& a) {
  Span r{0, 0};
  if (a.mode == GATHER_UP) {
    const float radius = a.f.support * a.scale;
    int f, l;
    in_range(0.5f, radius, a.inv_scale, &f, &l);
    r.n0 = f;
    in_range((float)(a.out - 1) + 0.5f, radius, a.inv_scale, &f, &l);
    r.n1 = l;
  } else {
    const float radius = a.f.support * a.inv_scale;
    int f, l;
    in_range(0.f, 0.f, a.inv_scale, &f, &l);
    r.n0 = f;
    in_range((float)a.out, 0.f, a.inv_scale, &f, &l);
    r.n1 = l;
    for (int p = r.n0 + 1; p >= -a.margin; p--) {
      int of, ol;
      out_range((float)p + 0.5f, radius, a.scale, a.out, &of, &ol);
      if (of > ol) break;
      r.n0 = p;
    }
    for (int p = r.n1 - 1, stop = p + 1 + a.margin; p <= stop; p++) {
      int of, ol;
      out_range((float)p + 0.5f, radius, a.scale, a.out, &of, &ol);
      if (of > ol) break;
      r.n1 = p;
    }
  }
  r.n0 = std::max(r.n0, 0);
  r.n1 = std::min(r.n1, a.in - 1);
  return r;
}

// Store the horizontal weights `widest` apart and move the windows of the last outputs back so that
// the fixed-width sums never reach past column row_end - 1 (leading zero weights fill the gap).
void pack_horizontal(Axis& a, int row_end) {
  const int wd = a.widest;
  if (a.width != wd)
    for (int n = 0; n < a.out; n++) std::memmove(a.w.data() + (size_t)n * wd, a.row(n), sizeof(float) * wd);
  a.width = wd;
  const auto reach = [wd](const Span& s) {  // weights a sum walks for this output
    if (wd <= 12) return wd;
    const int mod = wd & 3;
    const int r = (((s.n1 - s.n0 + 1) - mod + 3) & ~3) + mod;
    return std::max(r, 8 + mod);
  };
  for (int n = a.out - 1; n >= 0 && a.span[n].n0 + 2 * wd >= row_end; n--) {
    Span& s = a.span[n];
    if (s.n0 + wd <= row_end) continue;
    const int r = reach(s);
    if (s.n0 + r <= row_end) continue;
    const int n0 = row_end - r, back = s.n0 - n0;
    float* c = a.row(n);
    for (int i = s.n1 - s.n0; i >= 0; i--) c[i + back] = c[i];
    for (int i = 0; i < back; i++) c[i] = 0.f;
    s.n0 = n0;
  }
}

// The reference's cost weights for 4-channel data, by resize class (h filter width, h scale x v filter
// width, v filter width, v scale x h filter width); the cheaper estimate picks the pass order.
constexpr float COST4[8][4] = {{0.00000f, 0.50000f, 0.00000f, 0.71875f}, {0.06250f, 0.84375f, 0.00000f, 0.87500f},
                               {1.00000f, 0.50000f, 0.50000f, 0.96875f}, {1.00000f, 0.09375f, 0.31250f, 0.50000f},
                               {0.00000f, 0.50000f, 0.00000f, 0.71875f}, {1.00000f, 0.03125f, 0.03125f, 0.53125f},
                               {1.00000f, 1.00000f, 0.06250f, 1.00000f}, {0.00000f, 1.00000f, 0.03125f, 0.18750f}};

bool vertical_first(const Axis& h, const Axis& v) {
  int cls;
  const bool gather = v.mode != SCATTER;
  if (v.out <= 4 || h.out <= 4) cls = v.out < h.out ? 6 : 7;
  else if (!gather && (v.out <= 16 || h.out <= 16)) cls = 4;
  else if (v.scale <= 1.0f) cls = gather ? 1 : 0;
  else if (v.scale <= 2.0f) cls = 2;
  else if (v.scale <= 3.0f) cls = 3;
  else cls = 5;
  const float* k = COST4[cls];
  const double h_cost = (float)h.pixel_width * k[0] + h.scale * (float)v.pixel_width * k[1];
  const double v_cost = (float)v.pixel_width * k[2] + v.scale * (float)h.pixel_width * k[3];
  return v_cost <= h_cost;
}

// One horizontal pass: src holds columns [col0, ...) as floats, 4 per pixel.
void horizontal(const Axis& a, const float* src, int col0, float* dst) {
  const int wd = a.width;
  for (int n = 0; n < a.out; n++) {
    const float* c = a.w.data() + (size_t)n * wd;
    const float* p = src + (size_t)(a.span[n].n0 - col0) * 4;
    const int cnt = a.span[n].n1 - a.span[n].n0 + 1;
    float* o = dst + (size_t)n * 4;
    for (int ch = 0; ch < 4; ch++) {
      if (wd <= 3) {
        float t = p[ch] * c[0];
        for (int i = 1; i < cnt; i++) t = t + p[i * 4 + ch] * c[i];
        o[ch] = t;
      } else {  // even and odd positions summed apart (zero weights past cnt add nothing)
        float ev = p[ch] * c[0], od = 0.0f;
        for (int i = 1; i < cnt; i++) {
          if (i & 1) od = od + p[i * 4 + ch] * c[i];
          else ev = ev + p[i * 4 + ch] * c[i];
        }
        o[ch] = ev + od;
      }
    }
  }
}

inline uint8_t to_byte(float f) {
  f = f + 0.5f;
  if (!(f > 0.0f)) return 0;  // negative (and NaN) clamp to 0
  if (f >= 255.0f) return 255;
  return (uint8_t)(int)f;
}

// Decoded rows (floats) by index, kept in a ring sized to the vertical window.
struct RowCache {
  int slots = 0, width = 0;
  std::vector<std::vector<float>> data;
  std::vector<int> index;
  void init(int n, int w) {
    slots = n;
    width = w;
    data.assign(n, std::vector<float>((size_t)w * 4 + 16, 0.f));
    index.assign(n, -1);
  }
};

}  // namespace

std::vector<uint8_t> resample_rgba8(const uint8_t* src, int w, int h, int nw, int nh, ResampleFilter filter) {
  if (w <= 0 || h <= 0 || nw <= 0 || nh <= 0) throw std::invalid_argument("resample_rgba8: empty image");
  const Filter f = filter_of(filter);
  Axis ha, va;
  setup_axis(ha, w, nw, f, true);
  setup_axis(va, h, nh, f, false);
  const Span cols = decoded_columns(ha);
  build_weights(ha);
  pack_horizontal(ha, cols.n1 + 1);
  build_weights(va);
  const bool vfirst = vertical_first(ha, va);

  const int ncols = cols.n1 - cols.n0 + 1;
  const auto decode = [&](int y, float* dst) {
    const uint8_t* s = src + ((size_t)y * w + cols.n0) * 4;
    for (int i = 0; i < ncols * 4; i++) dst[i] = (float)s[i];
    for (int i = ncols * 4; i < ncols * 4 + 16; i++) dst[i] = 0.f;  // read with zero weights past the end
  };
  int span_rows = 1;
  for (int n = 0; n < nh; n++) span_rows = std::max(span_rows, va.span[n].n1 - va.span[n].n0 + 1);
  RowCache cache;
  cache.init(span_rows + 1, vfirst ? ncols : nw);
  const auto fetch = [&](int y) -> const float* {
    const int slot = y % cache.slots;
    if (cache.index[slot] != y) {
      float* d = cache.data[slot].data();
      if (vfirst) {
        decode(y, d);
      } else {
        std::vector<float> tmp((size_t)ncols * 4 + 16);
        decode(y, tmp.data());
        horizontal(ha, tmp.data(), cols.n0, d);
      }
      cache.index[slot] = y;
    }
    return cache.data[slot].data();
  };

  std::vector<uint8_t> out((size_t)nw * nh * 4);
  const int vw = (vfirst ? ncols : nw) * 4;
  std::vector<float> acc((size_t)vw + 16, 0.f), hrow((size_t)nw * 4);
  for (int y = 0; y < nh; y++) {
    const Span s = va.span[y];
    const float* c = va.w.data() + (size_t)y * va.width;
    {
      const float* r = fetch(s.n0);
      for (int i = 0; i < vw; i++) acc[i] = r[i] * c[0];
    }
    for (int k = 1; k <= s.n1 - s.n0; k++) {
      const float* r = fetch(s.n0 + k);
      const float ck = c[k];
      for (int i = 0; i < vw; i++) acc[i] = acc[i] + r[i] * ck;
    }
    const float* res = acc.data();
    if (vfirst) {
      horizontal(ha, acc.data(), cols.n0, hrow.data());
      res = hrow.data();
    }
    uint8_t* o = out.data() + (size_t)y * nw * 4;
    for (int i = 0; i < nw * 4; i++) o[i] = to_byte(res[i]);
  }
  return out;
}

}  // namespace b2c
