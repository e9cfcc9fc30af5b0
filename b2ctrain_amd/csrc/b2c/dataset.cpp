// COLMAP text models and the dataset loader (replaces src/dataset/colmap.cpp:1-73 and views.cpp:1-255).
//
// The loader works in three steps:
//  1. discover(): the layout of the dataset directory (the COLMAP model directory, the sidecar catalogues,
//     the initial splat ply);
//  2. plan(): the frames to load, after subsampling and the frame cap, each with its frame file and
//     sidecar files;
//  3. make_view() on worker threads (one per hardware thread, at most 16; job i runs on thread i mod T):
//     decode the frame, take a mask's alpha, cap the long edge (Mitchell resample), pack the view, then
//     fit and convert each sidecar (triangle resample for masks and weights, point sampling for labels
//     and normals).
// Frames and sidecars are PNG or JPEG (png.h, jpeg.h), resampled by resample.h; the bytes of every view are
// the reference loader's.
#include "dataset.h"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <exception>
#include <filesystem>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <thread>

#include "jpeg.h"
#include "ply.h"
#include "png.h"
#include "resample.h"

namespace b2c {

namespace fs = std::filesystem;

namespace {

[[noreturn]] void fail_dataset(const std::string& msg) { throw std::runtime_error(msg); }

std::string ascii_lower(std::string s) {
  std::transform(s.begin(), s.end(), s.begin(), [](unsigned char c) { return (char)std::tolower(c); });
  return s;
}

// The part of a file name before its last dot.
std::string stem_of(const std::string& name) { return name.substr(0, std::min(name.size(), name.rfind('.'))); }

// ------------------------------------------------------------------------------------------------- images
DecodedImage read_image(const std::string& path) { return decode_image(path); }

bool carries_alpha(const DecodedImage& img) { return img.channels_in_file == 2 || img.channels_in_file == 4; }

// The image's RGBA bytes at w x h: itself, or resampled with `filter` (views.cpp:73-78).
std::vector<uint8_t> at_size(DecodedImage& img, int w, int h, ResampleFilter filter) {
  if (img.w == w && img.h == h) return std::move(img.rgba);
  return resample_rgba8(img.rgba.data(), img.w, img.h, w, h, filter);
}

// --------------------------------------------------------------------------------------------- text model
// Data lines of a COLMAP text file: blank lines and '#' comments are skipped.
class ModelFile {
 public:
  explicit ModelFile(const fs::path& p) : in_(p) {
    if (!in_) fail_dataset("failed to open '" + p.string() + "'");
  }
  bool next(std::string& line) {
    while (std::getline(in_, line))
      if (!line.empty() && line[0] != '#') return true;
    return false;
  }
  void skip_line() {  // images.txt: the POINTS2D line that follows every image line, empty or not
    std::string ignored;
    std::getline(in_, ignored);
  }

 private:
  std::ifstream in_;
};

bool one_focal(const std::string& model) {
  return model == "SIMPLE_PINHOLE" || model == "SIMPLE_RADIAL" || model == "RADIAL";
}

ColmapCamera parse_camera(const std::string& line) {
  std::istringstream ss(line);
  ColmapCamera c;
  ss >> c.id >> c.model >> c.width >> c.height;
  for (double p; ss >> p;) c.params.push_back(p);
  size_t need = 0;
  if (c.model == "PINHOLE") need = 4;
  else if (c.model == "SIMPLE_PINHOLE") need = 3;
  else if (c.model != "SIMPLE_RADIAL" && c.model != "RADIAL" && c.model != "OPENCV")
    fail_dataset("unsupported camera model '" + c.model + "' (only pinhole models are supported)");
  if (c.params.size() < need)
    fail_dataset("cameras.txt: " + c.model + " needs " + std::to_string(need) + " params");
  if (need == 0)  // radial and OpenCV models keep their pinhole part
    std::fprintf(stderr, "[b2c] camera model %s: distortion is ignored (pinhole intrinsics only)\n", c.model.c_str());
  return c;
}

// ----------------------------------------------------------------------------------------------- layout
enum SidecarKind { MASKS, NORMALS, WEIGHTS, LABELS, SIDECAR_KINDS };
constexpr const char* SIDECAR_DIR[SIDECAR_KINDS] = {"masks", "normals", "weights", "labels"};

// Files under a sidecar directory, looked up by frame name: a file matches when its stem (lower case) is
// the frame's file name or the frame's stem, or for masks the frame's stem + ".mask" (views.cpp:24-41);
// the first match in directory order wins.
struct SidecarCatalogue {
  std::vector<std::pair<std::string, std::string>> stem_path;  // (lower-case stem of the file name, path)

  void add_tree(const fs::path& dir) {
    if (!fs::is_directory(dir)) return;
    for (const auto& e : fs::recursive_directory_iterator(dir))
      if (e.is_regular_file()) stem_path.emplace_back(stem_of(ascii_lower(e.path().filename().string())), e.path().string());
  }
  std::string lookup(const std::string& frame, bool mask_suffix) const {
    const std::string name = ascii_lower(frame), stem = stem_of(name);
    for (const auto& [s, path] : stem_path)
      if (s == name || s == stem || (mask_suffix && s == stem + ".mask")) return path;
    return {};
  }
};

struct Layout {
  fs::path root, model_dir;
  SidecarCatalogue sidecars[SIDECAR_KINDS];
  std::string init_ply;
};

Layout discover(const fs::path& root) {
  Layout L;
  L.root = root;
  // the text model: at the root, sparse/0, sparse or colmap/sparse/0, else anywhere below the root
  for (const fs::path& dir : {root, root / "sparse" / "0", root / "sparse", root / "colmap" / "sparse" / "0"})
    if (L.model_dir.empty() && fs::exists(dir / "cameras.txt")) L.model_dir = dir;
  if (L.model_dir.empty())
    for (fs::recursive_directory_iterator it(root), end; it != end && L.model_dir.empty(); ++it)
      if (it->is_regular_file() && it->path().filename() == "cameras.txt") L.model_dir = it->path().parent_path();
  if (L.model_dir.empty())
    fail_dataset("no cameras.txt found under '" + root.string() + "' (only COLMAP text datasets are supported)");
  // sidecar directories at the root; a kind with none there is looked for beside the model
  for (int k = 0; k < SIDECAR_KINDS; k++) {
    L.sidecars[k].add_tree(root / SIDECAR_DIR[k]);
    if (L.sidecars[k].stem_path.empty() && L.model_dir != root) L.sidecars[k].add_tree(L.model_dir / SIDECAR_DIR[k]);
  }
  // the initial splat cloud: a splat ply named init.ply (the last such by path), else the last splat ply
  std::vector<std::string> plys;
  for (const auto& e : fs::recursive_directory_iterator(root, fs::directory_options::follow_directory_symlink))
    if (e.is_regular_file() && ascii_lower(e.path().extension().string()) == ".ply" &&
        ply_is_vertex_only(e.path().string()))
      plys.push_back(e.path().string());
  std::sort(plys.begin(), plys.end());
  for (auto it = plys.rbegin(); it != plys.rend() && L.init_ply.empty(); ++it)
    if (fs::path(*it).filename() == "init.ply") L.init_ply = *it;
  if (L.init_ply.empty() && !plys.empty()) L.init_ply = plys.back();
  return L;
}

bool under_sidecar_dir(const fs::path& rel) {
  for (const auto& part : rel)
    for (const char* d : SIDECAR_DIR)
      if (part == d) return true;
  return false;
}

// The frame file of an image name: images/<name>, <name> at the root, else the first file below the root
// whose path ends in /<name> and that is not inside a sidecar directory (views.cpp:43-61).
std::string frame_file(const fs::path& root, const std::string& name) {
  if (fs::exists(root / "images" / name)) return (root / "images" / name).string();
  if (fs::exists(root / name)) return (root / name).string();
  const std::string suffix = "/" + name;
  for (const auto& e : fs::recursive_directory_iterator(root)) {
    const std::string p = e.path().string();
    if (e.is_regular_file() && p.size() >= suffix.size() && p.ends_with(suffix) &&
        !under_sidecar_dir(fs::relative(e.path(), root)))
      return p;
  }
  return {};
}

// ----------------------------------------------------------------------------------------------- frames
struct FrameSources {
  ColmapImage image;
  std::string frame;
  std::string sidecar[SIDECAR_KINDS];
};

std::vector<FrameSources> plan(const Layout& L, const ColmapModel& model, const DatasetOptions& opt) {
  std::vector<ColmapImage> chosen;
  const size_t step = opt.subsample_frames && *opt.subsample_frames > 1 ? *opt.subsample_frames : 1;
  for (size_t i = 0; i < model.images.size(); i += step) chosen.push_back(model.images[i]);
  if (opt.max_frames && chosen.size() > *opt.max_frames) chosen.resize(*opt.max_frames);
  std::vector<FrameSources> out;
  for (const ColmapImage& im : chosen) {
    FrameSources f;
    f.image = im;
    f.frame = frame_file(L.root, im.name);
    if (f.frame.empty()) {
      std::fprintf(stderr, "[b2c] skipped '%s': image file not found\n", im.name.c_str());
      continue;
    }
    for (int k = 0; k < SIDECAR_KINDS; k++) f.sidecar[k] = L.sidecars[k].lookup(im.name, k == MASKS);
    out.push_back(std::move(f));
  }
  if (out.empty()) fail_dataset("dataset has no usable views");
  return out;
}

// Frame size after the long-edge cap (views.cpp:164-170).
void capped_size(int w, int h, uint32_t max_resolution, int* nw, int* nh) {
  const int longest = std::max(w, h);
  const float s = (int)max_resolution < longest ? (float)max_resolution / (float)longest : 1.0f;
  *nw = std::max(1, (int)std::lround(w * s));
  *nh = std::max(1, (int)std::lround(h * s));
}

// (r, g, b) * a / 255 rounded to nearest, ties up: the byte-space premultiply of transparent frames.
inline uint32_t premultiplied(uint32_t c, uint32_t a) { return (c * a + 127u) / 255u; }

View make_view(const FrameSources& src, const ColmapModel& model, const DatasetOptions& opt) {
  const ColmapImage& im = src.image;
  const auto cam = model.cameras.find(im.camera_id);
  if (cam == model.cameras.end())
    fail_dataset("images.txt: unknown camera id " + std::to_string(im.camera_id) + " for '" + im.name + "'");
  View v;
  v.name = im.name;
  DecodedImage frame = read_image(src.frame);
  const bool masked = !src.sidecar[MASKS].empty();
  if (masked) {  // the mask, fitted to the frame, supplies the frame's alpha: its own alpha, else its red
    DecodedImage m = read_image(src.sidecar[MASKS]);
    const int ch = carries_alpha(m) ? 3 : 0;
    const std::vector<uint8_t> fitted = at_size(m, frame.w, frame.h, ResampleFilter::Triangle);
    for (size_t p = 0; p < (size_t)frame.w * frame.h; p++) frame.rgba[p * 4 + 3] = fitted[p * 4 + ch];
  }
  v.has_alpha = masked || carries_alpha(frame);
  v.mode = opt.alpha_mode ? *opt.alpha_mode : (masked ? AlphaMode::Masked : AlphaMode::Transparent);
  int w = 0, h = 0;
  capped_size(frame.w, frame.h, opt.max_resolution, &w, &h);
  const std::vector<uint8_t> px = at_size(frame, w, h, ResampleFilter::Mitchell);
  v.w = w;
  v.h = h;
  const ColmapCamera& cc = cam->second;
  v.cam.width = cc.width;
  v.cam.height = cc.height;
  v.cam.fx = cc.fx();
  v.cam.fy = cc.fy();
  v.cam.cx = cc.cx();
  v.cam.cy = cc.cy();
  v.cam.rescale(w, h);
  v.cam.set_w2c_quat(im.q[0], im.q[1], im.q[2], im.q[3], im.t[0], im.t[1], im.t[2]);
  if (!std::isfinite(v.cam.pos[0] + v.cam.pos[1] + v.cam.pos[2]))
    fail_dataset("camera for '" + v.name + "' contains nan or inf");

  const size_t P = (size_t)w * h;
  const bool premultiply = v.has_alpha && v.mode == AlphaMode::Transparent;
  v.rgba.resize(P);
  double coverage = 0.0;
  for (size_t p = 0; p < P; p++) {
    const uint32_t a = v.has_alpha ? px[p * 4 + 3] : 255u;
    uint32_t r = px[p * 4], g = px[p * 4 + 1], b = px[p * 4 + 2];
    if (premultiply) {
      r = premultiplied(r, a);
      g = premultiplied(g, a);
      b = premultiplied(b, a);
    }
    v.rgba[p] = r | (g << 8) | (b << 16) | (a << 24);
    coverage += a;
  }
  v.alpha_coverage = (float)(coverage / (255.0 * (double)P));

  if (!src.sidecar[WEIGHTS].empty()) {  // Rec. 709 luma of an RGB(A) map; a grey map's value
    DecodedImage wm = read_image(src.sidecar[WEIGHTS]);
    const bool colour = wm.channels_in_file >= 3;
    const std::vector<uint8_t> q = at_size(wm, w, h, ResampleFilter::Triangle);
    v.weights.resize(P);
    for (size_t p = 0; p < P; p++)
      v.weights[p] = colour ? (uint8_t)std::lround(0.2126 * q[p * 4] + 0.7152 * q[p * 4 + 1] + 0.0722 * q[p * 4 + 2])
                            : q[p * 4];
  }
  if (!src.sidecar[LABELS].empty()) {  // class ids in red, point-sampled (a blended id is another class)
    DecodedImage lm = read_image(src.sidecar[LABELS]);
    const std::vector<uint8_t> q = at_size(lm, w, h, ResampleFilter::PointSample);
    v.labels.resize(P);
    for (size_t p = 0; p < P; p++) v.labels[p] = q[p * 4];
  }
  if (!src.sidecar[NORMALS].empty()) {
    DecodedImage nm = read_image(src.sidecar[NORMALS]);
    const bool own_alpha = carries_alpha(nm);
    const std::vector<uint8_t> q = at_size(nm, w, h, ResampleFilter::PointSample);
    v.normals.resize(P);
    double marked = 0.0;  // weighted count of the pixels whose normal is valid (alpha > 127)
    for (size_t p = 0; p < P; p++) {
      const uint32_t a = own_alpha ? q[p * 4 + 3] : 255u;
      v.normals[p] = (uint32_t)q[p * 4] | ((uint32_t)q[p * 4 + 1] << 8) | ((uint32_t)q[p * 4 + 2] << 16) | (a << 24);
      if (a > 127) marked += v.has_weights() ? v.weights[p] / 255.0 : 1.0;
    }
    v.normal_mask_count = marked;
  }
  return v;
}

}  // namespace

DecodedImage decode_image(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) fail_dataset("failed to decode '" + path + "': can't fopen");
  const std::vector<uint8_t> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  if (is_jpeg_bytes(bytes.data(), bytes.size())) return decode_jpeg_bytes(bytes.data(), bytes.size(), path);
  if (bytes.size() >= 8 && bytes[0] == 0x89 && bytes[1] == 'P' && bytes[2] == 'N' && bytes[3] == 'G')
    return decode_png_bytes(bytes.data(), bytes.size(), path);
  fail_dataset("failed to decode '" + path + "': unknown image type (PNG and JPEG are read)");
}

float ColmapCamera::fx() const { return (float)params[0]; }
float ColmapCamera::fy() const { return (float)params[one_focal(model) ? 0 : 1]; }
float ColmapCamera::cx() const { return (float)params[one_focal(model) ? 1 : 2]; }
float ColmapCamera::cy() const { return (float)params[one_focal(model) ? 2 : 3]; }

ColmapModel read_colmap_text(const std::string& dir) {
  const fs::path d(dir);
  ColmapModel m;
  std::string line;
  for (ModelFile f(d / "cameras.txt"); f.next(line);) {
    ColmapCamera c = parse_camera(line);
    m.cameras[c.id] = std::move(c);
  }
  for (ModelFile f(d / "images.txt"); f.next(line); f.skip_line()) {
    std::istringstream ss(line);
    ColmapImage im;
    ss >> im.id;
    for (float& q : im.q) ss >> q;
    for (float& t : im.t) ss >> t;
    ss >> im.camera_id >> im.name;
    if (im.name.empty()) fail_dataset("images.txt: malformed line '" + line + "'");
    m.images.push_back(std::move(im));
  }
  std::sort(m.images.begin(), m.images.end(), [](const ColmapImage& a, const ColmapImage& b) { return a.name < b.name; });
  if (fs::exists(d / "points3D.txt"))
    for (ModelFile f(d / "points3D.txt"); f.next(line);) {
      std::istringstream ss(line);
      long id = 0;
      int rgb[3] = {0, 0, 0};
      Point3D p{};
      ss >> id >> p.x >> p.y >> p.z >> rgb[0] >> rgb[1] >> rgb[2];
      p.r = (unsigned char)rgb[0];
      p.g = (unsigned char)rgb[1];
      p.b = (unsigned char)rgb[2];
      m.points.push_back(p);
    }
  return m;
}

Dataset load_dataset(const DatasetOptions& opt) {
  const fs::path root = fs::absolute(opt.source);
  if (!fs::is_directory(root)) fail_dataset("dataset path '" + root.string() + "' is not a directory");
  const Layout L = discover(root);
  const ColmapModel model = read_colmap_text(L.model_dir.string());
  const std::vector<FrameSources> frames = plan(L, model, opt);

  std::vector<View> views(frames.size());
  std::vector<std::exception_ptr> errors(frames.size());
  const size_t T = std::min<size_t>(frames.size(), std::max(1u, std::min(std::thread::hardware_concurrency(), 16u)));
  {
    std::vector<std::jthread> workers;
    for (size_t t = 0; t < T; t++)
      workers.emplace_back([&, t] {
        for (size_t i = t; i < frames.size(); i += T) {
          try {
            views[i] = make_view(frames[i], model, opt);
          } catch (...) {
            errors[i] = std::current_exception();
          }
        }
      });
  }
  for (const std::exception_ptr& e : errors)  // the first failing frame in frame order
    if (e) std::rethrow_exception(e);

  Dataset ds;
  ds.root = root.string();
  ds.name = root.filename().string();
  if (ds.name.empty()) ds.name = root.parent_path().filename().string();
  ds.points = model.points;
  ds.init_ply = L.init_ply;
  const uint32_t every = opt.eval_split_every ? *opt.eval_split_every : 0;
  for (size_t i = 0; i < views.size(); i++) {
    View& v = views[i];
    if (v.has_alpha) ++(v.mode == AlphaMode::Masked ? ds.n_masked : ds.n_transparent);
    ds.n_weighted += v.has_weights() ? 1 : 0;
    ds.n_normals += v.has_normals() ? 1 : 0;
    ds.n_labels += v.has_labels() ? 1 : 0;
    (every > 0 && i % every == 0 ? ds.eval : ds.train).push_back(std::move(v));
  }
  if (ds.train.empty()) fail_dataset("dataset has no training views");
  return ds;
}

}  // namespace b2c
