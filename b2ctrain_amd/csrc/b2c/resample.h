// Resampling of 8-bit RGBA images for the dataset loader: the long-edge cap of a frame and the sizing of its
// sidecars to the frame (src/dataset/views.cpp:73-78,158,167-171,191,202,209), which the reference performs
// with stb_image_resize2 v2.18 (four independent channels, uint8 in and out, edges clamped). This is a
// separable filter with per-axis normalised weights evaluated in single precision; the weights, the order of
// the two passes and the summation order are the reference's, so results are its bytes.
#pragma once
#include <cstdint>
#include <vector>

namespace b2c {

enum class ResampleFilter {
  Triangle,     // tent of radius 1 (in the output grid when shrinking): masks and weight maps
  Mitchell,     // Mitchell-Netravali cubic, B = C = 1/3: frames over the resolution cap
  PointSample,  // box of width 1, no blending: class labels and normal maps
};

// src: [h][w][4] bytes; returns [nh][nw][4]. Throws std::invalid_argument on an empty size.
std::vector<uint8_t> resample_rgba8(const uint8_t* src, int w, int h, int nw, int nh, ResampleFilter filter);

}  // namespace b2c
