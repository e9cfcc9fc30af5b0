// JPEG decoding (ITU-T T.81, Huffman processes, 8-bit samples): marker walk, Huffman decoding of
// sequential and progressive scans into per-component coefficient planes, dequantisation and the
// fixed-point inverse DCT, then chroma upsampling and colour conversion to RGBA8 one output row at a time.
// The arithmetic after entropy decoding reproduces stb_image v2.30 (the reference's decoder) exactly; each
// such choice is marked where it is made.
#include "jpeg.h"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <vector>

namespace b2c {

namespace {

[[noreturn]] void bad(const std::string& name, const char* why) {
  throw std::runtime_error("failed to decode '" + name + "': " + why);
}

// Natural (row-major) index of the k-th coefficient of the zig-zag scan (T.81 figure A.6): the
// anti-diagonals r + c = s in turn, walked upwards (decreasing row) for even s, downwards for odd s.
struct ZigZag {
  uint8_t at[64];
};
constexpr ZigZag make_zigzag() {
  ZigZag z{};
  int k = 0;
  for (int s = 0; s < 15; s++) {
    const int lo = s < 8 ? 0 : s - 7, hi = s < 8 ? s : 7;
    if (s % 2 == 0)
      for (int r = hi; r >= lo; r--) z.at[k++] = (uint8_t)(r * 8 + (s - r));
    else
      for (int r = lo; r <= hi; r++) z.at[k++] = (uint8_t)(r * 8 + (s - r));
  }
  return z;
}
constexpr ZigZag ZZ = make_zigzag();
// A corrupt run can step past coefficient 63; like stb_image, such writes land on coefficient 63.
inline int natural(int k) { return ZZ.at[k < 63 ? k : 63]; }

// ---- Huffman tables (T.81 annex C; decoding per F.2.2.3 with a 9-bit lookahead table) ----
struct Huffman {
  bool defined = false;
  uint8_t values[256] = {};
  int32_t maxcode[18] = {};  // largest code of each length, -1 when there is none
  int32_t offset[18] = {};   // values[] index of a code of that length = code + offset
  uint16_t quick[512] = {};  // next 9 bits -> (length << 8 | value) + 1 for codes of at most 9 bits, else 0
};

void build_huffman(Huffman& h, const int counts[16], const std::string& name) {
  int code = 0, k = 0;
  for (int len = 1; len <= 16; len++) {
    const int c = counts[len - 1];
    h.offset[len] = k - code;
    if (c) {
      code += c;
      k += c;
      if (code - 1 >= (1 << len)) bad(name, "bad Huffman code lengths");
      h.maxcode[len] = code - 1;
    } else {
      h.maxcode[len] = -1;
    }
    code <<= 1;
  }
  h.maxcode[17] = 0x7fffffff;
  std::memset(h.quick, 0, sizeof(h.quick));
  code = 0;
  k = 0;
  for (int len = 1; len <= 9; len++) {
    for (int i = 0; i < counts[len - 1]; i++, k++, code++) {
      const int first = code << (9 - len), n = 1 << (9 - len);
      for (int j = 0; j < n; j++) h.quick[first + j] = (uint16_t)(((len << 8) | h.values[k]) + 1);
    }
    code <<= 1;
  }
  h.defined = true;
}

// ---- entropy-coded segment reader: byte unstuffing; a marker ends the data and zeros follow it ----
struct Bits {
  const uint8_t* p = nullptr;
  const uint8_t* end = nullptr;
  uint32_t buf = 0;  // next bits, most significant first
  int count = 0;
  int marker = -1;  // the marker that ended the segment, -1 while none was met

  void refill() {
    while (count <= 24) {
      uint32_t byte = 0;
      if (marker < 0) {
        byte = p < end ? *p++ : 0u;
        if (byte == 0xFF) {
          int next = p < end ? *p++ : 0;
          while (next == 0xFF) next = p < end ? *p++ : 0;
          if (next != 0) {  // a marker: the segment's data are over
            marker = next;
            return;
          }
        }
      }
      buf |= byte << (24 - count);
      count += 8;
    }
  }
  void reset() {
    buf = 0;
    count = 0;
    marker = -1;
  }
  int bit() {
    if (count < 1) refill();
    if (count < 1) return 0;
    const int b = (int)(buf >> 31);
    buf <<= 1;
    count--;
    return b;
  }
  // The reader runs short only where a marker cut the data off mid-code (the refill that meets the marker
  // adds nothing; later ones add zeros): a corrupt stream, whose fields then read as 0.
  int bits(int n) {  // n in 1..16
    if (count < n) refill();
    if (count < n) return 0;
    const uint32_t v = buf >> (32 - n);
    buf <<= n;
    count -= n;
    return (int)v;
  }
  // RECEIVE then EXTEND (T.81 F.2.2.1): an n-bit field with a leading 0 is negative.
  int signed_bits(int n) {
    if (n == 0) return 0;
    if (count < n) refill();
    if (count < n) return 0;
    const int v = bits(n);
    return v < (1 << (n - 1)) ? v - (1 << n) + 1 : v;
  }
  int decode(const Huffman& h, const std::string& name) {
    if (count < 16) refill();
    const uint16_t q = h.quick[buf >> 23];
    if (q) {
      const int len = (q - 1) >> 8;
      if (len > count) bad(name, "bad Huffman code");
      buf <<= len;
      count -= len;
      return (q - 1) & 0xFF;
    }
    for (int len = 10; len <= 16; len++) {
      const int32_t code = (int32_t)(buf >> (32 - len));
      if (code <= h.maxcode[len]) {
        const int idx = code + h.offset[len];
        if (idx < 0 || idx > 255 || len > count) break;
        buf <<= len;
        count -= len;
        return h.values[idx];
      }
    }
    bad(name, "bad Huffman code");
  }
};

struct Component {
  int id = 0, h = 1, v = 1, tq = 0, td = 0, ta = 0;
  int px = 0, py = 0;          // samples of the component (T.81 A.1.1)
  int bw = 0, bh = 0;          // coefficient blocks per row / column of the MCU-padded grid
  std::vector<int16_t> coef;   // [bh][bw][64], natural order
  std::vector<uint8_t> plane;  // [bh * 8][bw * 8] samples after the inverse DCT
  int dc_pred = 0;
  int16_t* block(int bx, int by) { return coef.data() + ((size_t)by * bw + bx) * 64; }
};

// ---- inverse DCT: the Loeffler-Ligtenberg-Moschytz factorisation (the "islow" method of IJG's jidctint)
// with its rotation constants in 12-bit fixed point, rounded as stb_image rounds them: trunc(c 4096 + 1/2),
// which puts the negative constants one unit nearer zero than their positive counterparts. ----
constexpr int q12(float c) { return (int)(c * 4096.0f + 0.5); }

struct Idct1d {
  int even[4], odd[4];  // output i = even[i] + odd[i], output 7 - i = even[i] - odd[i]
};

inline Idct1d idct8(int s0, int s1, int s2, int s3, int s4, int s5, int s6, int s7) {
  Idct1d r;
  // even half: s0, s4 directly, s2 and s6 through one rotation
  const int rot = (s2 + s6) * q12(0.5411961f);
  const int e2 = rot + s6 * q12(-1.847759065f), e3 = rot + s2 * q12(0.765366865f);
  const int e0 = (s0 + s4) * 4096, e1 = (s0 - s4) * 4096;
  r.even[0] = e0 + e3;
  r.even[3] = e0 - e3;
  r.even[1] = e1 + e2;
  r.even[2] = e1 - e2;
  // odd half: s7, s5, s3, s1 through the shared rotation and four butterflies
  const int a = s7 + s3, b = s5 + s1, c = s7 + s1, d = s5 + s3;
  const int z = (a + b) * q12(1.175875602f);
  const int zc = z + c * q12(-0.899976223f), zd = z + d * q12(-2.562915447f);
  const int za = a * q12(-1.961570560f), zb = b * q12(-0.390180644f);
  r.odd[0] = s1 * q12(1.501321110f) + zc + zb;
  r.odd[1] = s3 * q12(3.072711026f) + zd + za;
  r.odd[2] = s5 * q12(2.053119869f) + zd + zb;
  r.odd[3] = s7 * q12(0.298631336f) + zc + za;
  return r;
}

inline uint8_t clamp_u8(int x) { return (uint8_t)(x < 0 ? 0 : (x > 255 ? 255 : x)); }

// Dequantised coefficients (natural order) -> 8x8 samples. The column pass keeps two fractional bits
// (rounded: + 2^9, >> 10); the row pass removes the remaining 2^17 scale with one rounding, the +128 level
// shift folded into the same addend.
void idct_block(const int16_t* c, const uint16_t* q, uint8_t* out, int stride) {
  int d[64];
  for (int i = 0; i < 64; i++) d[i] = (int16_t)(c[i] * q[i]);  // 16-bit products, as the reference stores them
  int t[64];
  for (int col = 0; col < 8; col++) {
    const int* s = d + col;
    const Idct1d r = idct8(s[0], s[8], s[16], s[24], s[32], s[40], s[48], s[56]);
    for (int i = 0; i < 4; i++) {
      t[i * 8 + col] = (r.even[i] + 512 + r.odd[i]) >> 10;
      t[(7 - i) * 8 + col] = (r.even[i] + 512 - r.odd[i]) >> 10;
    }
  }
  constexpr int BIAS = 65536 + (128 << 17);
  for (int row = 0; row < 8; row++) {
    const int* s = t + row * 8;
    const Idct1d r = idct8(s[0], s[1], s[2], s[3], s[4], s[5], s[6], s[7]);
    uint8_t* o = out + (size_t)row * stride;
    for (int i = 0; i < 4; i++) {
      o[i] = clamp_u8((r.even[i] + BIAS + r.odd[i]) >> 17);
      o[7 - i] = clamp_u8((r.even[i] + BIAS - r.odd[i]) >> 17);
    }
  }
}

struct Decoder {
  const uint8_t* data;
  size_t size;
  const std::string& name;
  size_t pos = 0;

  Huffman dc[4], ac[4];
  uint16_t quant[4][64] = {};
  bool quant_defined[4] = {false, false, false, false};
  int restart_interval = 0;
  bool jfif = false;
  int adobe_transform = -1;

  bool progressive = false;
  int width = 0, height = 0, ncomp = 0;
  int hmax = 1, vmax = 1, mcux = 0, mcuy = 0;
  Component comp[4];

  // current scan
  int ns = 0, order[4] = {0, 0, 0, 0};
  int ss = 0, se = 63, ah = 0, al = 0;
  int eobrun = 0;

  Decoder(const uint8_t* d, size_t n, const std::string& nm) : data(d), size(n), name(nm) {}

  int byte() { return pos < size ? data[pos++] : 0; }
  int be16() {
    const int hi = byte();
    return (hi << 8) | byte();
  }
  // The next marker: 0xFF fill bytes are skipped; -1 when the next byte is not 0xFF.
  int next_marker() {
    if (byte() != 0xFF) return -1;
    int m = 0xFF;
    while (m == 0xFF) m = byte();
    return m;
  }
  // After entropy-coded data without a marker: skip to the next marker (stuffed zeros are data).
  int scan_for_marker() {
    while (pos < size) {
      int x = byte();
      while (x == 0xFF) {
        if (pos >= size) return -1;
        x = byte();
        if (x != 0x00 && x != 0xFF) return x;
      }
    }
    return -1;
  }

  void read_dqt() {
    int len = be16() - 2;
    while (len > 0) {
      const int pq = byte();
      const int prec = pq >> 4, t = pq & 15;
      if (prec > 1) bad(name, "bad DQT precision");
      if (t > 3) bad(name, "bad DQT table");
      for (int k = 0; k < 64; k++) quant[t][ZZ.at[k]] = (uint16_t)(prec ? be16() : byte());
      quant_defined[t] = true;
      len -= prec ? 129 : 65;
    }
    if (len != 0) bad(name, "bad DQT length");
  }

  void read_dht() {
    int len = be16() - 2;
    while (len > 0) {
      const int tc_th = byte();
      const int tc = tc_th >> 4, th = tc_th & 15;
      if (tc > 1 || th > 3) bad(name, "bad DHT header");
      int counts[16], total = 0;
      for (int i = 0; i < 16; i++) total += counts[i] = byte();
      if (total > 256) bad(name, "bad DHT header");
      Huffman& h = tc ? ac[th] : dc[th];
      for (int i = 0; i < total; i++) h.values[i] = (uint8_t)byte();
      build_huffman(h, counts, name);
      len -= 17 + total;
    }
    if (len != 0) bad(name, "bad DHT length");
  }

  void read_app_or_comment(int m) {
    int len = be16();
    if (len < 2) bad(name, m == 0xFE ? "bad COM length" : "bad APP length");
    len -= 2;
    const size_t start = pos;
    if (m == 0xE0 && len >= 5) {  // JFIF APP0
      if (pos + 5 <= size && std::memcmp(data + pos, "JFIF", 5) == 0) jfif = true;
    } else if (m == 0xEE && len >= 12) {  // Adobe APP14: the colour transform byte follows 11 bytes of header
      if (pos + 12 <= size && std::memcmp(data + pos, "Adobe", 6) == 0) adobe_transform = data[pos + 11];
    }
    pos = start + (size_t)len;
  }

  void read_frame(int m) {
    progressive = m == 0xC2;
    const int len = be16();
    if (len < 11) bad(name, "bad SOF length");
    if (byte() != 8) bad(name, "only 8-bit JPEG is supported");
    height = be16();
    width = be16();
    if (height == 0) bad(name, "JPEG with the height in a DNL marker is not supported");
    if (width == 0) bad(name, "zero width");
    if (width > (1 << 24) || height > (1 << 24)) bad(name, "image too large");
    ncomp = byte();
    if (ncomp != 1 && ncomp != 3 && ncomp != 4) bad(name, "bad component count");
    if (len != 8 + 3 * ncomp) bad(name, "bad SOF length");
    for (int i = 0; i < ncomp; i++) {
      Component& c = comp[i];
      c.id = byte();
      const int hv = byte();
      c.h = hv >> 4;
      c.v = hv & 15;
      c.tq = byte();
      if (c.h < 1 || c.h > 4) bad(name, "bad H sampling factor");
      if (c.v < 1 || c.v > 4) bad(name, "bad V sampling factor");
      if (c.tq > 3) bad(name, "bad quantisation table selector");
      hmax = std::max(hmax, c.h);
      vmax = std::max(vmax, c.v);
    }
    for (int i = 0; i < ncomp; i++)
      if (hmax % comp[i].h || vmax % comp[i].v) bad(name, "sampling factors are not integer ratios");
    mcux = (width + 8 * hmax - 1) / (8 * hmax);
    mcuy = (height + 8 * vmax - 1) / (8 * vmax);
    for (int i = 0; i < ncomp; i++) {
      Component& c = comp[i];
      c.px = (width * c.h + hmax - 1) / hmax;
      c.py = (height * c.v + vmax - 1) / vmax;
      c.bw = mcux * c.h;
      c.bh = mcuy * c.v;
      c.coef.assign((size_t)c.bw * c.bh * 64, 0);
    }
  }

  void read_scan_header() {
    const int len = be16();
    ns = byte();
    if (ns < 1 || ns > 4 || ns > ncomp) bad(name, "bad SOS component count");
    if (len != 6 + 2 * ns) bad(name, "bad SOS length");
    for (int i = 0; i < ns; i++) {
      const int id = byte(), tables = byte();
      int which = 0;
      while (which < ncomp && comp[which].id != id) which++;
      if (which == ncomp) bad(name, "scan names an unknown component");
      comp[which].td = tables >> 4;
      comp[which].ta = tables & 15;
      if (comp[which].td > 3 || comp[which].ta > 3) bad(name, "bad Huffman table selector");
      order[i] = which;
    }
    ss = byte();
    se = byte();
    const int a = byte();
    ah = a >> 4;
    al = a & 15;
    if (progressive) {
      if (ss > 63 || se > 63 || ss > se || ah > 13 || al > 13) bad(name, "bad progressive scan parameters");
    } else {
      if (ss != 0 || ah != 0 || al != 0) bad(name, "bad sequential scan parameters");
      se = 63;
    }
  }

  const Huffman& table(const Huffman* set, int i) {
    if (!set[i].defined) bad(name, "scan uses an undefined Huffman table");
    return set[i];
  }

  // ---- per-block decoding (T.81 F.2.2 sequential, G.1.2 progressive) ----
  void block_sequential(Bits& in, Component& c, int16_t* blk) {
    const Huffman& hd = table(dc, c.td);
    const Huffman& ha = table(ac, c.ta);
    const int t = in.decode(hd, name);
    if (t > 15) bad(name, "bad DC magnitude category");
    c.dc_pred += in.signed_bits(t);
    blk[0] = (int16_t)c.dc_pred;
    for (int k = 1; k < 64;) {
      const int rs = in.decode(ha, name);
      const int r = rs >> 4, s = rs & 15;
      if (s == 0) {
        if (r != 15) break;  // end of block
        k += 16;
        continue;
      }
      k += r;
      blk[natural(k)] = (int16_t)in.signed_bits(s);
      k++;
    }
  }

  void block_dc_first(Bits& in, Component& c, int16_t* blk) {
    const int t = in.decode(table(dc, c.td), name);
    if (t > 15) bad(name, "bad DC magnitude category");
    c.dc_pred += in.signed_bits(t);
    blk[0] = (int16_t)(c.dc_pred * (1 << al));
  }

  void block_dc_refine(Bits& in, int16_t* blk) {
    if (in.bit()) blk[0] = (int16_t)(blk[0] + (1 << al));
  }

  void block_ac_first(Bits& in, Component& c, int16_t* blk) {
    if (eobrun > 0) {
      eobrun--;
      return;
    }
    const Huffman& ha = table(ac, c.ta);
    for (int k = ss; k <= se;) {
      const int rs = in.decode(ha, name);
      const int r = rs >> 4, s = rs & 15;
      if (s == 0) {
        if (r < 15) {  // EOB run: this block and (2^r - 1 + r extra bits) more are done
          eobrun = (1 << r) - 1 + (r ? in.bits(r) : 0);
          break;
        }
        k += 16;
        continue;
      }
      k += r;
      blk[natural(k)] = (int16_t)(in.signed_bits(s) * (1 << al));
      k++;
    }
  }

  // A correction bit for an already nonzero coefficient: it joins the magnitude (away from zero).
  void refine(Bits& in, int16_t& coef, int bit) {
    if (in.bit() && (coef & bit) == 0) coef = (int16_t)(coef > 0 ? coef + bit : coef - bit);
  }

  void block_ac_refine(Bits& in, Component& c, int16_t* blk) {
    const int bit = 1 << al;
    if (eobrun > 0) {
      eobrun--;
      for (int k = ss; k <= se; k++)
        if (blk[natural(k)] != 0) refine(in, blk[natural(k)], bit);
      return;
    }
    const Huffman& ha = table(ac, c.ta);
    int k = ss;
    do {
      const int rs = in.decode(ha, name);
      int r = rs >> 4;
      const int s = rs & 15;
      int value = 0;
      if (s == 0) {
        if (r < 15) {  // end of band: the remaining nonzero coefficients still take their correction bits
          eobrun = (1 << r) - 1 + (r ? in.bits(r) : 0);
          r = 64;
        }
      } else {
        if (s != 1) bad(name, "bad progressive refinement code");
        value = in.bit() ? bit : -bit;
      }
      // skip r zero-history coefficients (refining the nonzero ones met), then place the new one
      while (k <= se) {
        int16_t& coef = blk[natural(k++)];
        if (coef != 0) {
          refine(in, coef, bit);
        } else {
          if (r == 0) {
            coef = (int16_t)value;
            break;
          }
          r--;
        }
      }
    } while (k <= se);
  }

  void decode_block(Bits& in, Component& c, int16_t* blk) {
    if (!progressive) return block_sequential(in, c, blk);
    if (ss == 0) {
      if (se != 0) bad(name, "progressive scan mixes DC and AC");
      if (ah == 0) block_dc_first(in, c, blk);
      else block_dc_refine(in, blk);
    } else {
      if (ah == 0) block_ac_first(in, c, blk);
      else block_ac_refine(in, c, blk);
    }
  }

  // Decodes the entropy-coded data of the current scan. Returns the marker that follows it.
  int decode_scan() {
    Bits in;
    in.p = data + pos;
    in.end = data + size;
    for (int i = 0; i < ncomp; i++) comp[i].dc_pred = 0;
    eobrun = 0;
    if (progressive && ss > 0 && ns != 1) bad(name, "progressive AC scan with several components");
    const bool single = ns == 1;
    const int units_x = single ? (comp[order[0]].px + 7) / 8 : mcux;
    const int units_y = single ? (comp[order[0]].py + 7) / 8 : mcuy;
    int todo = restart_interval ? restart_interval : 0x7fffffff;
    bool stopped = false;
    for (int uy = 0; uy < units_y && !stopped; uy++) {
      for (int ux = 0; ux < units_x; ux++) {
        if (single) {
          Component& c = comp[order[0]];
          decode_block(in, c, c.block(ux, uy));
        } else {
          for (int i = 0; i < ns; i++) {
            Component& c = comp[order[i]];
            for (int y = 0; y < c.v; y++)
              for (int x = 0; x < c.h; x++) decode_block(in, c, c.block(ux * c.h + x, uy * c.v + y));
          }
        }
        if (--todo <= 0) {  // a restart interval ends here: the next marker must be RSTn, else the scan stops
          if (in.count < 24) in.refill();
          if (in.marker < 0xD0 || in.marker > 0xD7) {
            stopped = true;
            break;
          }
          in.reset();
          for (int i = 0; i < ncomp; i++) comp[i].dc_pred = 0;
          eobrun = 0;
          todo = restart_interval ? restart_interval : 0x7fffffff;
        }
      }
    }
    pos = (size_t)(in.p - data);
    int m = in.marker >= 0 ? in.marker : scan_for_marker();
    if (m >= 0xD0 && m <= 0xD7) m = next_marker();  // a restart marker after the last interval
    return m;
  }

  void decode_all() {
    if (byte() != 0xFF || byte() != 0xD8) bad(name, "no SOI marker");
    // tables and segments up to the frame header
    int m = next_marker();
    while (!(m == 0xC0 || m == 0xC1 || m == 0xC2)) {
      if (m < 0) {
        if (pos >= size) bad(name, "no SOF marker");
        m = next_marker();
        continue;
      }
      if (!segment(m)) bad(name, m == 0xC3 || (m >= 0xC5 && m <= 0xCF && m != 0xC8 && m != 0xCC)
                                     ? "unsupported JPEG process (lossless, hierarchical or arithmetic coding)"
                                     : "unknown marker");
      m = next_marker();
    }
    read_frame(m);
    m = next_marker();
    while (m != 0xD9) {
      if (m == 0xDA) {
        read_scan_header();
        m = decode_scan();
      } else if (m == 0xDC) {  // DNL
        const int len = be16();
        const int lines = be16();
        if (len != 4) bad(name, "bad DNL length");
        if (lines != height) bad(name, "bad DNL height");
        m = next_marker();
      } else {
        if (m < 0 || !segment(m)) break;  // after the frame, an unreadable segment ends the image
        m = next_marker();
      }
    }
  }

  // Tables and other segments that may appear between the SOI and the EOI. False for unknown markers.
  bool segment(int m) {
    if (m == 0xDB) read_dqt();
    else if (m == 0xC4) read_dht();
    else if (m == 0xDD) {
      if (be16() != 4) bad(name, "bad DRI length");
      restart_interval = be16();
    } else if ((m >= 0xE0 && m <= 0xEF) || m == 0xFE) read_app_or_comment(m);
    else return false;
    return true;
  }

  void inverse_transform() {
    for (int i = 0; i < ncomp; i++) {
      Component& c = comp[i];
      if (!quant_defined[c.tq]) bad(name, "component uses an undefined quantisation table");
      const int stride = c.bw * 8;
      c.plane.assign((size_t)stride * c.bh * 8, 0);
      const int nbx = (c.px + 7) / 8, nby = (c.py + 7) / 8;
      for (int by = 0; by < nby; by++)
        for (int bx = 0; bx < nbx; bx++)
          idct_block(c.block(bx, by), quant[c.tq], c.plane.data() + (size_t)by * 8 * stride + bx * 8, stride);
      std::vector<int16_t>().swap(c.coef);
    }
  }
};

// ---- upsampling of one component row to the full width (stb_image's choices, views.cpp's decoder) ----
// The component's rows that output row y reads: for a vertical factor of 2 the nearer row and the farther
// one (the JFIF-centred 3:1 blend); otherwise only the nearer one.
struct RowPick {
  int near, far;
};
RowPick rows_for(int y, int vs, int rows) {
  if (vs == 2) {
    const int m = y >> 1;
    const int far = (y & 1) ? std::min(m + 1, rows - 1) : std::max(m - 1, 0);
    return {std::min(m, rows - 1), far};
  }
  const int m = std::min(y / vs, rows - 1);
  return {m, m};
}

// out[0 .. count) from the lo-res rows (w_lo samples each).
void upsample_row(uint8_t* out, const uint8_t* nr, const uint8_t* fr, int w_lo, int hs, int vs) {
  if (hs == 1 && vs == 1) {
    std::memcpy(out, nr, (size_t)w_lo);
  } else if (hs == 1 && vs == 2) {
    for (int i = 0; i < w_lo; i++) out[i] = (uint8_t)((3 * nr[i] + fr[i] + 2) >> 2);
  } else if (hs == 2 && vs == 1) {
    if (w_lo == 1) {
      out[0] = out[1] = nr[0];
      return;
    }
    out[0] = nr[0];
    out[1] = (uint8_t)((3 * nr[0] + nr[1] + 2) >> 2);
    for (int i = 1; i < w_lo - 1; i++) {
      out[2 * i] = (uint8_t)((3 * nr[i] + nr[i - 1] + 2) >> 2);
      out[2 * i + 1] = (uint8_t)((3 * nr[i] + nr[i + 1] + 2) >> 2);
    }
    // the reference's last pair weights the second-to-last sample by 3 on the left output
    out[2 * w_lo - 2] = (uint8_t)((3 * nr[w_lo - 2] + nr[w_lo - 1] + 2) >> 2);
    out[2 * w_lo - 1] = nr[w_lo - 1];
  } else if (hs == 2 && vs == 2) {
    // vertical blend first (3 near + far, in quarters), then horizontal 3:1 between neighbours
    if (w_lo == 1) {
      out[0] = out[1] = (uint8_t)((3 * nr[0] + fr[0] + 2) >> 2);
      return;
    }
    int prev = 3 * nr[0] + fr[0];
    out[0] = (uint8_t)((prev + 2) >> 2);
    for (int i = 1; i < w_lo; i++) {
      const int cur = 3 * nr[i] + fr[i];
      out[2 * i - 1] = (uint8_t)((3 * prev + cur + 8) >> 4);
      out[2 * i] = (uint8_t)((3 * cur + prev + 8) >> 4);
      prev = cur;
    }
    out[2 * w_lo - 1] = (uint8_t)((prev + 2) >> 2);
  } else {
    for (int i = 0; i < w_lo; i++)
      for (int j = 0; j < hs; j++) out[i * hs + j] = nr[i];
  }
}

// JFIF YCbCr -> RGB with the coefficients in 12-bit fixed point (1.402, 0.71414, 0.34414, 1.772 -> 5743,
// 2925, 1410, 7258), rounded once; the reference truncates green's Cb term to 1/16 first.
inline void ycc_to_rgb(int y, int cb, int cr, uint8_t* o) {
  cb -= 128;
  cr -= 128;
  const int base = y * 4096 + 2048;
  const int cbg = (-1410 * cb) >> 8;  // green's Cb term floored to 1/16 (floor(-0.34414 cb * 16) / 16)
  o[0] = clamp_u8((base + 5743 * cr) >> 12);
  o[1] = clamp_u8((base - 2925 * cr + 256 * cbg) >> 12);
  o[2] = clamp_u8((base + 7258 * cb) >> 12);
}

// x * y / 255 rounded (the reference's fast form), for CMYK and YCCK.
inline uint8_t mul255(int x, int y) {
  const unsigned t = (unsigned)(x * y) + 128u;
  return (uint8_t)((t + (t >> 8)) >> 8);
}

}  // namespace

bool is_jpeg_bytes(const uint8_t* data, size_t size) {
  return size >= 3 && data[0] == 0xFF && data[1] == 0xD8 && data[2] == 0xFF;
}

DecodedImage decode_jpeg_bytes(const uint8_t* data, size_t size, const std::string& name) {
  Decoder d(data, size, name);
  d.decode_all();
  if (d.ncomp == 0) bad(name, "no frame");
  d.inverse_transform();
  const int W = d.width, H = d.height, n = d.ncomp;
  DecodedImage img;
  img.w = W;
  img.h = H;
  img.channels_in_file = n >= 3 ? 3 : 1;
  img.rgba.resize((size_t)W * H * 4);
  // components named 'R', 'G', 'B' (or, without JFIF, an Adobe transform of 0) hold RGB directly
  const bool rgb = n == 3 && ((d.comp[0].id == 'R' && d.comp[1].id == 'G' && d.comp[2].id == 'B') ||
                              (d.adobe_transform == 0 && !d.jfif));
  std::vector<std::vector<uint8_t>> line(n, std::vector<uint8_t>((size_t)W + 3 * 4 + 4));
  for (int y = 0; y < H; y++) {
    for (int k = 0; k < n; k++) {
      const Component& c = d.comp[k];
      const int hs = d.hmax / c.h, vs = d.vmax / c.v;
      const int w_lo = (W + hs - 1) / hs, stride = c.bw * 8;
      const RowPick rp = rows_for(y, vs, c.py);
      upsample_row(line[k].data(), c.plane.data() + (size_t)rp.near * stride, c.plane.data() + (size_t)rp.far * stride,
                   w_lo, hs, vs);
    }
    uint8_t* o = img.rgba.data() + (size_t)y * W * 4;
    const uint8_t* c0 = line[0].data();
    for (int x = 0; x < W; x++, o += 4) {
      o[3] = 255;
      if (n == 1) {
        o[0] = o[1] = o[2] = c0[x];
      } else if (n == 3) {
        if (rgb) {
          o[0] = c0[x];
          o[1] = line[1][x];
          o[2] = line[2][x];
        } else {
          ycc_to_rgb(c0[x], line[1][x], line[2][x], o);
        }
      } else if (d.adobe_transform == 0) {  // CMYK (Adobe's inverted convention)
        const int k = line[3][x];
        o[0] = mul255(c0[x], k);
        o[1] = mul255(line[1][x], k);
        o[2] = mul255(line[2][x], k);
      } else if (d.adobe_transform == 2) {  // YCCK
        ycc_to_rgb(c0[x], line[1][x], line[2][x], o);
        const int k = line[3][x];
        o[0] = mul255(255 - o[0], k);
        o[1] = mul255(255 - o[1], k);
        o[2] = mul255(255 - o[2], k);
      } else {  // four components without a known transform: YCbCr, the fourth ignored
        ycc_to_rgb(c0[x], line[1][x], line[2][x], o);
      }
    }
  }
  return img;
}

}  // namespace b2c
