// PNG decoding for the dataset loader (the frames and sidecars the reference decodes with stb_image,
// src/dataset/views.cpp:63-72). Written from the PNG specification (W3C PNG, 2nd edition): all colour types
// and bit depths, palettes with tRNS, colour-key tRNS, Adam7 interlacing; zlib inflates the IDAT stream.
// The output is what the loader consumes: 8-bit RGBA with the channel count of the file.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace b2c {

struct DecodedImage {
  int w = 0, h = 0;
  int channels_in_file = 0;   // 1 grey, 2 grey + alpha, 3 RGB (or palette), 4 RGBA; a tRNS chunk adds one
                              // (palette: 4, grey key: 2, RGB key: 4)
  std::vector<uint8_t> rgba;  // [h][w][4]
};

// Expansion to RGBA8 as stb_image's 4-channel request performs it: grey g -> (g, g, g, 255), grey + alpha
// -> (g, g, g, a), RGB -> (r, g, b, 255), palette -> its entry with the tRNS alpha (255 past the tRNS
// list); a colour-key tRNS turns the matching pixels' alpha to 0; 16-bit samples keep their high byte;
// 1, 2 and 4-bit grey samples are scaled to 0..255 (x 255, x 85, x 17). Throws on a file that is not a
// valid PNG (bad signature, CRC-free structure errors, inflate errors, truncated data).
DecodedImage decode_png(const std::string& path);
DecodedImage decode_png_bytes(const uint8_t* data, size_t size, const std::string& name);

// True when the file starts with the PNG signature.
bool is_png(const std::string& path);

}  // namespace b2c
