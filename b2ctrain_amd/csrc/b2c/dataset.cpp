// COLMAP text models and the dataset loader (replaces src/dataset/colmap.cpp:1-73 and views.cpp:1-255).
// Frames decode in parallel on host threads (one per hardware thread, at most 16, as the reference
// loads them); each view is packed in one pass over its pixels.
#include "dataset.h"

#include <algorithm>
#include <atomic>
#include <cctype>
#include <cmath>
#include <exception>
#include <filesystem>
#include <fstream>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <thread>

#include "png.h"
#include "ply.h"

namespace b2c {

namespace fs = std::filesystem;

namespace {

[[noreturn]] void dataset_error(const std::string& msg) { throw std::runtime_error(msg); }

// Models whose first three parameters are (f, cx, cy): one focal length for both axes.
bool single_focal(const std::string& model) {
  return model == "SIMPLE_PINHOLE" || model == "SIMPLE_RADIAL" || model == "RADIAL";
}

std::string lowercase(std::string s) {
  for (char& c : s) c = (char)std::tolower((unsigned char)c);
  return s;
}

std::string without_ext(const std::string& name) {
  const size_t dot = name.rfind('.');
  return dot == std::string::npos ? name : name.substr(0, dot);
}

bool sidecar_component(const std::string& c) { return c == "masks" || c == "normals" || c == "weights" || c == "labels"; }

// Every file under a sidecar directory, matched to a frame by stem (views.cpp:24-41): a candidate's stem
// equals the frame's file name, or its stem, or (masks) its stem + ".mask"; case-insensitive.
struct Sidecars {
  std::vector<std::pair<std::string, std::string>> files;  // (lowercase file name, path)
  void scan(const fs::path& dir) {
    if (!fs::is_directory(dir)) return;
    for (const auto& e : fs::recursive_directory_iterator(dir))
      if (e.is_regular_file()) files.emplace_back(lowercase(e.path().filename().string()), e.path().string());
  }
  std::string match(const std::string& frame, bool mask_suffix) const {
    const std::string full = lowercase(frame), stem = lowercase(without_ext(frame));
    for (const auto& [fname, path] : files) {
      const std::string s = without_ext(fname);
      if (s == full || s == stem || (mask_suffix && s == stem + ".mask")) return path;
    }
    return "";
  }
};

// images/<name>, then <name> at the root, then any file whose path ends in /<name> outside the sidecar
// directories (views.cpp:43-61).
std::string locate_frame(const fs::path& root, const std::string& name) {
  for (const fs::path& p : {root / "images" / name, root / name})
    if (fs::exists(p)) return p.string();
  const std::string tail = "/" + name;
  for (const auto& e : fs::recursive_directory_iterator(root)) {
    if (!e.is_regular_file()) continue;
    const std::string p = e.path().string();
    if (p.size() < tail.size() || p.compare(p.size() - tail.size(), tail.size(), tail) != 0) continue;
    bool in_sidecar = false;
    for (const auto& comp : fs::relative(e.path(), root)) in_sidecar = in_sidecar || sidecar_component(comp.string());
    if (!in_sidecar) return p;
  }
  return "";
}

DecodedImage load_image(const std::string& path) {
  if (!is_png(path))
    dataset_error("failed to decode '" + path + "': only PNG frames and sidecars are supported by this build");
  return decode_png(path);
}

// A sidecar must already have the frame's size: this build does not resample.
void require_size(const DecodedImage& img, int w, int h, const std::string& path) {
  if (img.w != w || img.h != h)
    dataset_error("'" + path + "' is " + std::to_string(img.w) + "x" + std::to_string(img.h) + ", the frame " +
                  std::to_string(w) + "x" + std::to_string(h) + ": resampling is not supported by this build");
}

bool has_alpha_channel(const DecodedImage& d) { return d.channels_in_file == 4 || d.channels_in_file == 2; }

struct Job {
  ColmapImage im;
  std::string frame, mask, normal, weight, label;
};

void build_view(const Job& j, const ColmapModel& model, const DatasetOptions& opt, View& v) {
  v.name = j.im.name;
  const auto cam_it = model.cameras.find(j.im.camera_id);
  if (cam_it == model.cameras.end())
    dataset_error("images.txt: unknown camera id " + std::to_string(j.im.camera_id) + " for '" + j.im.name + "'");
  const ColmapCamera& cc = cam_it->second;
  DecodedImage d = load_image(j.frame);
  const bool embedded_alpha = has_alpha_channel(d);
  if (!j.mask.empty()) {  // the frame's alpha from the mask's alpha, or its red channel
    const DecodedImage m = load_image(j.mask);
    require_size(m, d.w, d.h, j.mask);
    const bool mask_alpha = has_alpha_channel(m);
    for (size_t p = 0; p < (size_t)d.w * d.h; p++) d.rgba[p * 4 + 3] = m.rgba[p * 4 + (mask_alpha ? 3 : 0)];
  }
  v.has_alpha = embedded_alpha || !j.mask.empty();
  v.mode = opt.alpha_mode ? *opt.alpha_mode : (!j.mask.empty() ? AlphaMode::Masked : AlphaMode::Transparent);
  const int longest = std::max(d.w, d.h);
  const float scale = (int)opt.max_resolution < longest ? (float)opt.max_resolution / (float)longest : 1.0f;
  const int nw = std::max(1, (int)std::lround(d.w * scale)), nh = std::max(1, (int)std::lround(d.h * scale));
  if (nw != d.w || nh != d.h)
    dataset_error("'" + j.frame + "' (" + std::to_string(d.w) + "x" + std::to_string(d.h) +
                  ") exceeds max_resolution " + std::to_string(opt.max_resolution) +
                  ": resampling is not supported by this build");
  v.w = nw;
  v.h = nh;
  v.cam.width = cc.width;
  v.cam.height = cc.height;
  v.cam.fx = cc.fx();
  v.cam.fy = cc.fy();
  v.cam.cx = cc.cx();
  v.cam.cy = cc.cy();
  v.cam.rescale(nw, nh);
  v.cam.set_w2c_quat(j.im.q[0], j.im.q[1], j.im.q[2], j.im.q[3], j.im.t[0], j.im.t[1], j.im.t[2]);
  if (!std::isfinite(v.cam.pos[0] + v.cam.pos[1] + v.cam.pos[2]))
    dataset_error("camera for '" + v.name + "' contains nan or inf");
  // pack; a transparent view's colour is premultiplied in byte space, round half up (views.cpp:178-183)
  const size_t P = (size_t)nw * nh;
  const bool premultiply = v.mode == AlphaMode::Transparent && v.has_alpha;
  v.rgba.resize(P);
  double alpha_sum = 0;
  for (size_t p = 0; p < P; p++) {
    const uint8_t* px = &d.rgba[p * 4];
    const uint32_t a = v.has_alpha ? px[3] : 255u;
    uint32_t rgb[3] = {px[0], px[1], px[2]};
    if (premultiply)
      for (uint32_t& c : rgb) c = (c * a + 127u) / 255u;
    v.rgba[p] = rgb[0] | (rgb[1] << 8) | (rgb[2] << 16) | (a << 24);
    alpha_sum += a;
  }
  v.alpha_coverage = (float)(alpha_sum / (255.0 * (double)P));
  if (!j.weight.empty()) {  // Rec. 709 luma of an RGB weight map, else its first channel
    const DecodedImage wm = load_image(j.weight);
    require_size(wm, nw, nh, j.weight);
    v.weights.resize(P);
    for (size_t p = 0; p < P; p++) {
      const uint8_t* px = &wm.rgba[p * 4];
      v.weights[p] = wm.channels_in_file >= 3
                         ? (uint8_t)std::lround(0.2126 * px[0] + 0.7152 * px[1] + 0.0722 * px[2])
                         : px[0];
    }
  }
  if (!j.label.empty()) {  // class ids in the red channel
    const DecodedImage lm = load_image(j.label);
    require_size(lm, nw, nh, j.label);
    v.labels.resize(P);
    for (size_t p = 0; p < P; p++) v.labels[p] = lm.rgba[p * 4];
  }
  if (!j.normal.empty()) {
    const DecodedImage nm = load_image(j.normal);
    require_size(nm, nw, nh, j.normal);
    const bool n_alpha = has_alpha_channel(nm);
    v.normals.resize(P);
    double count = 0;
    for (size_t p = 0; p < P; p++) {
      const uint8_t* px = &nm.rgba[p * 4];
      const uint32_t a = n_alpha ? px[3] : 255u;
      v.normals[p] = (uint32_t)px[0] | ((uint32_t)px[1] << 8) | ((uint32_t)px[2] << 16) | (a << 24);
      if (a > 127) count += v.has_weights() ? v.weights[p] / 255.0 : 1.0;
    }
    v.normal_mask_count = count;
  }
}

}  // namespace

float ColmapCamera::fx() const { return (float)params[0]; }
float ColmapCamera::fy() const { return (float)(single_focal(model) ? params[0] : params[1]); }
float ColmapCamera::cx() const { return (float)(single_focal(model) ? params[1] : params[2]); }
float ColmapCamera::cy() const { return (float)(single_focal(model) ? params[2] : params[3]); }

ColmapModel read_colmap_text(const std::string& dir) {
  const auto open = [&](const char* file) {
    std::ifstream f(fs::path(dir) / file);
    if (!f) dataset_error("failed to open '" + (fs::path(dir) / file).string() + "'");
    return f;
  };
  const auto content = [](const std::string& line) { return !line.empty() && line[0] != '#'; };
  ColmapModel m;
  {
    std::ifstream f = open("cameras.txt");
    for (std::string line; std::getline(f, line);) {
      if (!content(line)) continue;
      std::istringstream ss(line);
      ColmapCamera c;
      ss >> c.id >> c.model >> c.width >> c.height;
      for (double v; ss >> v;) c.params.push_back(v);
      const size_t need = c.model == "PINHOLE" ? 4 : c.model == "SIMPLE_PINHOLE" ? 3 : 0;
      if (c.model == "PINHOLE" || c.model == "SIMPLE_PINHOLE") {
        if (c.params.size() < need)
          dataset_error("cameras.txt: " + c.model + " needs " + std::to_string(need) + " params");
      } else if (c.model != "SIMPLE_RADIAL" && c.model != "RADIAL" && c.model != "OPENCV") {
        dataset_error("unsupported camera model '" + c.model + "' (only pinhole models are supported)");
      }
      m.cameras[c.id] = c;
    }
  }
  {
    std::ifstream f = open("images.txt");
    for (std::string line; std::getline(f, line);) {
      if (!content(line)) continue;
      std::istringstream ss(line);
      ColmapImage im;
      ss >> im.id >> im.q[0] >> im.q[1] >> im.q[2] >> im.q[3] >> im.t[0] >> im.t[1] >> im.t[2] >> im.camera_id >> im.name;
      if (im.name.empty()) dataset_error("images.txt: malformed line '" + line + "'");
      m.images.push_back(im);
      std::getline(f, line);  // its POINTS2D line (possibly empty)
    }
    std::sort(m.images.begin(), m.images.end(), [](const ColmapImage& a, const ColmapImage& b) { return a.name < b.name; });
  }
  const fs::path pts = fs::path(dir) / "points3D.txt";
  if (fs::exists(pts)) {
    std::ifstream f = open("points3D.txt");
    for (std::string line; std::getline(f, line);) {
      if (!content(line)) continue;
      std::istringstream ss(line);
      long id;
      Point3D p{};
      int r = 0, g = 0, b = 0;
      ss >> id >> p.x >> p.y >> p.z >> r >> g >> b;
      p.r = (unsigned char)r;
      p.g = (unsigned char)g;
      p.b = (unsigned char)b;
      m.points.push_back(p);
    }
  }
  return m;
}

Dataset load_dataset(const DatasetOptions& opt) {
  Dataset ds;
  const fs::path root = fs::absolute(opt.source);
  if (!fs::is_directory(root)) dataset_error("dataset path '" + root.string() + "' is not a directory");
  ds.root = root.string();
  ds.name = root.filename().string();
  if (ds.name.empty()) ds.name = root.parent_path().filename().string();

  fs::path model_dir;
  for (const fs::path& c : {root, root / "sparse" / "0", root / "sparse", root / "colmap" / "sparse" / "0"})
    if (fs::exists(c / "cameras.txt")) {
      model_dir = c;
      break;
    }
  if (model_dir.empty())
    for (const auto& e : fs::recursive_directory_iterator(root))
      if (e.is_regular_file() && e.path().filename() == "cameras.txt") {
        model_dir = e.path().parent_path();
        break;
      }
  if (model_dir.empty())
    dataset_error("no cameras.txt found under '" + root.string() + "' (only COLMAP text datasets are supported)");
  const ColmapModel model = read_colmap_text(model_dir.string());
  ds.points = model.points;

  {  // the initial splat cloud: init.ply, else the last splat ply by path (meshes skipped)
    std::vector<std::string> plys;
    for (const auto& e : fs::recursive_directory_iterator(root, fs::directory_options::follow_directory_symlink))
      if (e.is_regular_file() && lowercase(e.path().extension().string()) == ".ply" && ply_is_vertex_only(e.path().string()))
        plys.push_back(e.path().string());
    std::sort(plys.begin(), plys.end());
    for (const std::string& p : plys)
      if (fs::path(p).filename() == "init.ply") ds.init_ply = p;
    if (ds.init_ply.empty() && !plys.empty()) ds.init_ply = plys.back();
  }

  std::vector<ColmapImage> frames = model.images;
  if (opt.subsample_frames && *opt.subsample_frames > 1) {
    std::vector<ColmapImage> kept;
    for (size_t i = 0; i < frames.size(); i += *opt.subsample_frames) kept.push_back(frames[i]);
    frames = kept;
  }
  if (opt.max_frames && frames.size() > *opt.max_frames) frames.resize(*opt.max_frames);

  Sidecars masks, normals, weights, labels;
  Sidecars* all[4] = {&masks, &normals, &weights, &labels};
  const char* dirs[4] = {"masks", "normals", "weights", "labels"};
  for (int k = 0; k < 4; k++) all[k]->scan(root / dirs[k]);
  if (model_dir != root)  // sidecars beside the model instead
    for (int k = 0; k < 4; k++)
      if (all[k]->files.empty()) all[k]->scan(model_dir / dirs[k]);

  std::vector<Job> jobs;
  for (const ColmapImage& im : frames) {
    Job j;
    j.im = im;
    j.frame = locate_frame(root, im.name);
    if (j.frame.empty()) continue;  // the reference warns and skips it
    j.mask = masks.match(im.name, true);
    j.normal = normals.match(im.name, false);
    j.weight = weights.match(im.name, false);
    j.label = labels.match(im.name, false);
    jobs.push_back(j);
  }
  if (jobs.empty()) dataset_error("dataset has no usable views");

  std::vector<View> views(jobs.size());
  std::atomic<size_t> next{0};
  std::exception_ptr failure;
  std::mutex failure_lock;
  const unsigned threads = std::max(1u, std::min(std::thread::hardware_concurrency(), 16u));
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < threads; t++)
    pool.emplace_back([&] {
      try {
        for (size_t i; (i = next.fetch_add(1)) < jobs.size();) build_view(jobs[i], model, opt, views[i]);
      } catch (...) {
        std::lock_guard<std::mutex> hold(failure_lock);
        if (!failure) failure = std::current_exception();
      }
    });
  for (std::thread& t : pool) t.join();
  if (failure) std::rethrow_exception(failure);

  for (size_t i = 0; i < views.size(); i++) {
    View& v = views[i];
    if (v.has_alpha) (v.mode == AlphaMode::Masked ? ds.n_masked : ds.n_transparent)++;
    ds.n_weighted += v.has_weights();
    ds.n_normals += v.has_normals();
    ds.n_labels += v.has_labels();
    const bool to_eval = opt.eval_split_every && *opt.eval_split_every > 0 && i % *opt.eval_split_every == 0;
    (to_eval ? ds.eval : ds.train).push_back(std::move(v));
  }
  if (ds.train.empty()) dataset_error("dataset has no training views");
  return ds;
}

}  // namespace b2c
