// COLMAP text models and the dataset loader (replaces src/dataset/colmap.h:1-32, views.h:1-39 and the
// Camera helpers of camera.h): cameras.txt / images.txt / points3D.txt, frames with their masks/, weights/,
// normals/ and labels/ sidecars, packed into the RGBA8 views the loss reads. Frames and sidecars are PNG
// (png.h) or JPEG (jpeg.h); frames over max_resolution and sidecars of another size are resampled
// (resample.h) as the reference resamples them.
#pragma once
#include <cstdint>
#include <map>
#include <optional>
#include <string>
#include <type_traits>
#include <vector>

#include "png.h"
#include "render.h"

namespace b2c {

// A frame or sidecar file, PNG or JPEG by its signature, as 8-bit RGBA (the reference's
// stbi_load(path, ..., 4), views.cpp:63-72).
DecodedImage decode_image(const std::string& path);

struct ColmapImage {
  int id = 0, camera_id = 0;
  std::string name;
  float q[4] = {1, 0, 0, 0}, t[3] = {0, 0, 0};  // world to camera
};
struct ColmapCamera {
  int id = 0;
  std::string model;
  int width = 0, height = 0;
  std::vector<double> params;
  // pinhole intrinsics of the model's parameter list (colmap.cpp:10-13)
  float fx() const;
  float fy() const;
  float cx() const;
  float cy() const;
};
struct Point3D {
  float x, y, z;
  unsigned char r, g, b;
};
struct ColmapModel {
  std::map<int, ColmapCamera> cameras;
  std::vector<ColmapImage> images;  // sorted by name
  std::vector<Point3D> points;
};
// colmap.cpp:21-71: PINHOLE and SIMPLE_PINHOLE; SIMPLE_RADIAL, RADIAL and OPENCV with their distortion
// ignored; images with the POINTS2D line after each skipped; points3D.txt optional.
ColmapModel read_colmap_text(const std::string& dir);

enum class AlphaMode { Masked, Transparent };

struct View {
  std::string name;
  Camera cam;  // intrinsics at the loaded resolution
  int w = 0, h = 0;
  bool has_alpha = false;
  AlphaMode mode = AlphaMode::Transparent;
  std::vector<uint32_t> rgba;     // r | g << 8 | b << 16 | a << 24; colour premultiplied (bytes) when transparent
  std::vector<uint32_t> normals;  // packed RGBA8 normal map, empty if none
  std::vector<uint8_t> weights;   // per-pixel loss weight, empty if none
  std::vector<uint8_t> labels;    // per-pixel class id, empty if none
  float alpha_coverage = 1.0f;    // mean a / 255
  double normal_mask_count = 0;   // sum of the pixel weights where the normal map's alpha > 127
  bool has_normals() const { return !normals.empty(); }
  bool has_weights() const { return !weights.empty(); }
  bool has_labels() const { return !labels.empty(); }
};

struct Dataset {
  std::string root, name;
  std::vector<View> train, eval;
  std::vector<Point3D> points;
  std::string init_ply;  // init.ply if present, else the lexicographically last splat ply, else empty
  int n_masked = 0, n_transparent = 0, n_weighted = 0, n_normals = 0, n_labels = 0;
};

// The Config fields load_dataset reads (src/cli.h:14,37-40).
struct DatasetOptions {
  std::string source;
  std::optional<uint32_t> max_frames;
  uint32_t max_resolution = 1920;
  std::optional<uint32_t> eval_split_every, subsample_frames;
  std::optional<AlphaMode> alpha_mode;
};

// views.cpp:74-253.
Dataset load_dataset(const DatasetOptions& opt);
// The reference's signature takes its Config; any type with the fields above works here.
template <typename Config>
Dataset load_dataset(const Config& cfg) {
  DatasetOptions o;
  o.source = cfg.source;
  o.max_frames = cfg.max_frames;
  o.max_resolution = cfg.max_resolution;
  o.eval_split_every = cfg.eval_split_every;
  o.subsample_frames = cfg.subsample_frames;
  if (cfg.alpha_mode) {
    using Mode = std::remove_cvref_t<decltype(*cfg.alpha_mode)>;
    o.alpha_mode = *cfg.alpha_mode == Mode::Masked ? AlphaMode::Masked : AlphaMode::Transparent;
  }
  return load_dataset(o);
}

}  // namespace b2c
