// JPEG decoding for the dataset loader: the frames and sidecars the reference decodes with stb_image v2.30
// (src/dataset/views.cpp:63-72, third_party/stb_image.h). Written from ITU-T T.81 (Huffman-coded baseline,
// extended sequential and progressive processes, 8-bit samples); where T.81 leaves the arithmetic open, the
// numbers are the ones stb_image produces, so a loaded view is the reference's byte for byte:
//  * the inverse DCT is the Loeffler-Ligtenberg-Moschytz factorisation with 12-bit fixed-point constants,
//    two fractional bits kept between the column and the row pass, rounded once at the end;
//  * chroma is upsampled with the JFIF-centred triangle filter (3/4, 1/4 taps) for 2x factors, nearest
//    neighbour otherwise;
//  * YCbCr -> RGB uses the JFIF coefficients in 12-bit fixed point.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>

#include "png.h"

namespace b2c {

// True when the buffer starts with a JPEG SOI marker followed by another marker.
bool is_jpeg_bytes(const uint8_t* data, size_t size);

// Decodes to RGBA8 (alpha 255): channels_in_file is 3 for 3- and 4-component files, 1 for greyscale, as
// stb_image reports them. Throws std::runtime_error naming `name` on a file it cannot decode (arithmetic
// coding, lossless or 12-bit processes, structural errors).
DecodedImage decode_jpeg_bytes(const uint8_t* data, size_t size, const std::string& name);

}  // namespace b2c
