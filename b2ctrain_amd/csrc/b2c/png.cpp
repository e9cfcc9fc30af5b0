// PNG decoding (W3C PNG specification): chunk walk, zlib inflate of the concatenated IDAT data, per-row
// unfiltering (None, Sub, Up, Average, Paeth), Adam7 de-interlacing, and expansion of every colour type and
// bit depth to 8-bit RGBA.
#include "png.h"

#include <zlib.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>

namespace b2c {

namespace {

constexpr uint8_t SIGNATURE[8] = {0x89, 'P', 'N', 'G', '\r', '\n', 0x1a, '\n'};

[[noreturn]] void bad(const std::string& name, const char* why) {
  throw std::runtime_error("failed to decode '" + name + "': " + why);
}

uint32_t be32(const uint8_t* p) { return ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | p[3]; }

int paeth(int a, int b, int c) {
  const int p = a + b - c, pa = std::abs(p - a), pb = std::abs(p - b), pc = std::abs(p - c);
  if (pa <= pb && pa <= pc) return a;
  return pb <= pc ? b : c;
}

// Undo the filter of each row in place (the filter byte leads every row). bpp: bytes per complete pixel,
// at least 1.
void unfilter(uint8_t* data, size_t rows, size_t row_bytes, int bpp, const std::string& name) {
  std::vector<uint8_t> zero(row_bytes, 0);
  const uint8_t* prior = zero.data();
  for (size_t y = 0; y < rows; y++) {
    uint8_t* f = data + y * (row_bytes + 1);
    const int type = f[0];
    uint8_t* r = f + 1;
    switch (type) {
      case 0: break;
      case 1:
        for (size_t i = bpp; i < row_bytes; i++) r[i] = (uint8_t)(r[i] + r[i - bpp]);
        break;
      case 2:
        for (size_t i = 0; i < row_bytes; i++) r[i] = (uint8_t)(r[i] + prior[i]);
        break;
      case 3:
        for (size_t i = 0; i < row_bytes; i++) {
          const int left = i >= (size_t)bpp ? r[i - bpp] : 0;
          r[i] = (uint8_t)(r[i] + ((left + prior[i]) >> 1));
        }
        break;
      case 4:
        for (size_t i = 0; i < row_bytes; i++) {
          const int left = i >= (size_t)bpp ? r[i - bpp] : 0, ul = i >= (size_t)bpp ? prior[i - bpp] : 0;
          r[i] = (uint8_t)(r[i] + paeth(left, prior[i], ul));
        }
        break;
      default: bad(name, "invalid filter type");
    }
    prior = r;
  }
}

struct Header {
  uint32_t w = 0, h = 0;
  int depth = 0, colour = 0, interlace = 0;
  int samples() const { return colour == 0 ? 1 : colour == 2 ? 3 : colour == 3 ? 1 : colour == 4 ? 2 : 4; }
};

}  // namespace

bool is_png(const std::string& path) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  uint8_t sig[8] = {};
  const bool ok = fread(sig, 1, 8, f) == 8 && std::memcmp(sig, SIGNATURE, 8) == 0;
  fclose(f);
  return ok;
}

DecodedImage decode_png(const std::string& path) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) bad(path, "can't fopen");
  std::vector<uint8_t> bytes;
  uint8_t buf[1 << 16];
  size_t got;
  while ((got = fread(buf, 1, sizeof buf, f)) > 0) bytes.insert(bytes.end(), buf, buf + got);
  fclose(f);
  return decode_png_bytes(bytes.data(), bytes.size(), path);
}

DecodedImage decode_png_bytes(const uint8_t* data, size_t size, const std::string& name) {
  if (size < 8 || std::memcmp(data, SIGNATURE, 8) != 0) bad(name, "not a PNG file");
  Header hd;
  std::vector<uint8_t> idat, palette;  // palette as RGBA entries
  uint8_t trns_rgb16[6] = {};          // colour key (grey in the first two bytes)
  bool key = false, palette_alpha = false, seen_ihdr = false, seen_end = false;
  size_t pos = 8;
  while (pos + 12 <= size && !seen_end) {
    const uint32_t len = be32(data + pos);
    const uint8_t* type = data + pos + 4;
    const uint8_t* body = data + pos + 8;
    if (len > size - pos - 12) bad(name, "truncated chunk");
    if (!std::memcmp(type, "IHDR", 4)) {
      if (len != 13) bad(name, "bad IHDR");
      hd.w = be32(body);
      hd.h = be32(body + 4);
      hd.depth = body[8];
      hd.colour = body[9];
      hd.interlace = body[12];
      const bool ok_depth = (hd.colour == 0 && (hd.depth == 1 || hd.depth == 2 || hd.depth == 4 || hd.depth == 8 ||
                                                hd.depth == 16)) ||
                            (hd.colour == 3 && (hd.depth == 1 || hd.depth == 2 || hd.depth == 4 || hd.depth == 8)) ||
                            ((hd.colour == 2 || hd.colour == 4 || hd.colour == 6) && (hd.depth == 8 || hd.depth == 16));
      if (!ok_depth) bad(name, "unsupported colour type / bit depth");
      if (body[10] != 0 || body[11] != 0 || hd.interlace > 1) bad(name, "bad compression, filter or interlace method");
      if (hd.w == 0 || hd.h == 0 || hd.w > (1u << 24) || hd.h > (1u << 24)) bad(name, "bad image size");
      seen_ihdr = true;
    } else if (!std::memcmp(type, "PLTE", 4)) {
      if (len % 3 || len > 768) bad(name, "bad PLTE");
      palette.assign(len / 3 * 4, 255);
      for (uint32_t k = 0; k < len / 3; k++)
        for (int c = 0; c < 3; c++) palette[k * 4 + c] = body[k * 3 + c];
    } else if (!std::memcmp(type, "tRNS", 4)) {
      if (hd.colour == 3) {
        if (len > palette.size() / 4) bad(name, "bad tRNS");
        for (uint32_t k = 0; k < len; k++) palette[k * 4 + 3] = body[k];
        palette_alpha = true;
      } else if (hd.colour == 0 || hd.colour == 2) {
        if (len != (hd.colour == 0 ? 2u : 6u)) bad(name, "bad tRNS");
        std::memcpy(trns_rgb16, body, len);
        key = true;
      }
    } else if (!std::memcmp(type, "IDAT", 4)) {
      idat.insert(idat.end(), body, body + len);
    } else if (!std::memcmp(type, "IEND", 4)) {
      seen_end = true;
    } else if (!(type[0] & 0x20)) {
      bad(name, "unknown critical chunk");
    }
    pos += 12 + (size_t)len;
  }
  if (!seen_ihdr || idat.empty()) bad(name, "missing IHDR or IDAT");
  if (hd.colour == 3 && palette.empty()) bad(name, "missing PLTE");

  const int samples = hd.samples();
  const int bits_px = samples * hd.depth;
  const int bpp = std::max(1, bits_px / 8);
  // The passes of the image: one for a plain image, Adam7's seven for an interlaced one.
  struct Pass {
    int x0, y0, dx, dy;
  };
  const Pass plain[1] = {{0, 0, 1, 1}};
  const Pass adam7[7] = {{0, 0, 8, 8}, {4, 0, 8, 8}, {0, 4, 4, 8}, {2, 0, 4, 4}, {0, 2, 2, 4}, {1, 0, 2, 2}, {0, 1, 1, 2}};
  const Pass* passes = hd.interlace ? adam7 : plain;
  const int npass = hd.interlace ? 7 : 1;
  size_t raw_size = 0;
  for (int p = 0; p < npass; p++) {
    const size_t pw = hd.w > (uint32_t)passes[p].x0 ? (hd.w - passes[p].x0 + passes[p].dx - 1) / passes[p].dx : 0;
    const size_t ph = hd.h > (uint32_t)passes[p].y0 ? (hd.h - passes[p].y0 + passes[p].dy - 1) / passes[p].dy : 0;
    if (pw && ph) raw_size += ph * (1 + (pw * bits_px + 7) / 8);
  }
  std::vector<uint8_t> raw(raw_size);
  z_stream zs{};
  if (inflateInit(&zs) != Z_OK) bad(name, "inflate init");
  zs.next_in = idat.data();
  zs.avail_in = (uInt)idat.size();
  zs.next_out = raw.data();
  zs.avail_out = (uInt)raw.size();
  const int zr = inflate(&zs, Z_FINISH);
  const size_t produced = raw.size() - zs.avail_out;
  inflateEnd(&zs);
  if ((zr != Z_STREAM_END && zr != Z_BUF_ERROR && zr != Z_OK) || produced < raw.size()) bad(name, "corrupt image data");

  DecodedImage out;
  out.w = (int)hd.w;
  out.h = (int)hd.h;
  // a tRNS chunk counts as an alpha channel: 4 for a palette, one more than the samples for a colour key
  out.channels_in_file = hd.colour == 3 ? (palette_alpha ? 4 : 3) : samples + (key ? 1 : 0);
  out.rgba.assign((size_t)hd.w * hd.h * 4, 0);
  static const int GREY_SCALE[17] = {0, 255, 85, 0, 17, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 0, 1};
  uint8_t* src = raw.data();
  for (int p = 0; p < npass; p++) {
    const Pass& P = passes[p];
    const size_t pw = hd.w > (uint32_t)P.x0 ? (hd.w - P.x0 + P.dx - 1) / P.dx : 0;
    const size_t ph = hd.h > (uint32_t)P.y0 ? (hd.h - P.y0 + P.dy - 1) / P.dy : 0;
    if (!pw || !ph) continue;
    const size_t row_bytes = (pw * bits_px + 7) / 8;
    unfilter(src, ph, row_bytes, bpp, name);
    for (size_t y = 0; y < ph; y++) {
      const uint8_t* r = src + y * (row_bytes + 1) + 1;
      for (size_t x = 0; x < pw; x++) {
        uint8_t* o = &out.rgba[((size_t)(P.y0 + y * P.dy) * hd.w + (P.x0 + x * P.dx)) * 4];
        // sample k of this pixel: at its bit depth (16-bit samples keep the high byte) and, for the
        // colour key, at full precision
        const auto sample = [&](int k, bool full) -> int {
          if (hd.depth == 16) {
            const uint8_t* q = r + (x * samples + k) * 2;
            return full ? (q[0] << 8 | q[1]) : q[0];
          }
          if (hd.depth == 8) return r[x * samples + k];
          const size_t bit = (x * samples + k) * hd.depth;
          return (r[bit >> 3] >> (8 - hd.depth - (int)(bit & 7))) & ((1 << hd.depth) - 1);
        };
        switch (hd.colour) {
          case 0: {
            const int g = hd.depth == 16 ? sample(0, false) : sample(0, false) * GREY_SCALE[hd.depth];
            o[0] = o[1] = o[2] = (uint8_t)g;
            o[3] = 255;
            if (key) {
              const int kv = (trns_rgb16[0] << 8) | trns_rgb16[1];
              const bool hit = hd.depth == 16 ? sample(0, true) == kv : g == ((kv & 255) * GREY_SCALE[hd.depth]);
              if (hit) o[3] = 0;
            }
            break;
          }
          case 2: {
            for (int c = 0; c < 3; c++) o[c] = (uint8_t)sample(c, false);
            o[3] = 255;
            if (key) {
              bool hit = true;
              for (int c = 0; c < 3; c++) {
                const int kv = (trns_rgb16[2 * c] << 8) | trns_rgb16[2 * c + 1];
                hit = hit && (hd.depth == 16 ? sample(c, true) == kv : sample(c, false) == (kv & 255));
              }
              if (hit) o[3] = 0;
            }
            break;
          }
          case 3: {
            const int idx = sample(0, false);
            if ((size_t)idx >= palette.size() / 4) bad(name, "palette index out of range");
            std::memcpy(o, &palette[(size_t)idx * 4], 4);
            break;
          }
          case 4:
            o[0] = o[1] = o[2] = (uint8_t)sample(0, false);
            o[3] = (uint8_t)sample(1, false);
            break;
          default:
            for (int c = 0; c < 4; c++) o[c] = (uint8_t)sample(c, false);
        }
      }
    }
    src += ph * (row_bytes + 1);
  }
  return out;
}

}  // namespace b2c
