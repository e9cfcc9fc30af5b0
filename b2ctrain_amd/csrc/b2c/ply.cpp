// Splat clouds in brush's ply layout (replaces src/ply.cpp:1-228). The header parse and the mapping from
// properties to cloud fields are shared by the host reader and the device-direct loader, so both accept
// and reject the same files; the row decode and encode of the device-direct pair run in
// kernels/ply_io.hip.
#include "ply.h"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>

namespace b2c {

const char* const EVIDENCE_FIELDS[7] = {"ev_w_in", "ev_w_all", "ev_err", "ev_views", "ev_dir_0", "ev_dir_1", "ev_dir_2"};
const char* const LABEL_FIELDS[2] = {"seg_label", "seg_conf"};

namespace {

[[noreturn]] void ply_error(const char* fmt, ...) {
  char msg[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  throw std::runtime_error(msg);
}

std::string field(const char* stem, int k) { return std::string(stem) + std::to_string(k); }

struct TypeName {
  const char* a;
  const char* b;
  int type;
  uint32_t bytes;
};
constexpr TypeName TYPES[] = {{"float", "float32", B2C_PLY_F32, 4}, {"double", "float64", B2C_PLY_F64, 8},
                              {"uchar", "uint8", B2C_PLY_U8, 1},    {"char", "int8", B2C_PLY_I8, 1},
                              {"ushort", "uint16", B2C_PLY_U16, 2}, {"short", "int16", B2C_PLY_I16, 2},
                              {"uint", "uint32", B2C_PLY_U32, 4},   {"int", "int32", B2C_PLY_I32, 4}};

const TypeName& type_named(const std::string& s) {
  for (const TypeName& t : TYPES)
    if (s == t.a || s == t.b) return t;
  ply_error("ply: unsupported property type '%s'", s.c_str());
}

// A little-endian binary value as double (the reference reader's representation of every value).
double value_at(const unsigned char* p, int type) {
  const auto load = [p](auto v) {
    std::memcpy(&v, p, sizeof v);
    return v;
  };
  switch (type) {
    case B2C_PLY_F32: return load(0.f);
    case B2C_PLY_F64: return load(0.0);
    case B2C_PLY_U8: return load(uint8_t{0});
    case B2C_PLY_I8: return load(int8_t{0});
    case B2C_PLY_U16: return load(uint16_t{0});
    case B2C_PLY_I16: return load(int16_t{0});
    case B2C_PLY_U32: return load(uint32_t{0});
    default: return load(int32_t{0});
  }
}

// Which property feeds which cloud field, with read_ply's rules and error order (ply.cpp:127-147).
struct PlyLayout {
  int degree = 0;
  bool has_scales = false, rgb = false;
  double rgb_scale = 1.0;
  int pos[3], scale[3], rot[4], opacity, dc[3], colour[3];
  std::vector<int> rest;  // f_rest_0 .. f_rest_(3(K-1)-1)
  int evidence[7], label, conf, fill, gate[2], gate_s, open[4];
  bool has_evidence = false, has_labels = false, has_fill = false, has_gate = false, has_gate_s = false,
       has_open = false;
};

PlyLayout layout_of(const PlyHeader& h) {
  PlyLayout L;
  // read_ply looks a group's other members up row by row (ply.cpp:150-166): a missing one is an error only
  // for a file that has rows.
  const auto need = [&](const std::string& name) {
    const int c = h.find(name.c_str());
    if (c < 0 && h.vertices > 0) ply_error("ply: missing property '%s'", name.c_str());
    return c;
  };
  const auto group = [&](int* out, const char* const* names, int count) {  // all or none
    if (h.find(names[0]) < 0) {
      for (int k = 0; k < count; k++) out[k] = -1;
      return false;
    }
    for (int k = 0; k < count; k++) out[k] = need(names[k]);
    return true;
  };
  int n_rest = 0;
  while (h.find(field("f_rest_", n_rest).c_str()) >= 0) n_rest++;
  const int K = 1 + n_rest / 3;
  L.degree = (int)std::lround(std::sqrt((double)K)) - 1;
  if (sh_coeffs_for_degree(L.degree) != K) ply_error("ply: %d f_rest properties is not a valid SH layout", n_rest);
  static const char* const XYZ[3] = {"x", "y", "z"};
  static const char* const SCALE[3] = {"scale_0", "scale_1", "scale_2"};
  static const char* const ROT[4] = {"rot_0", "rot_1", "rot_2", "rot_3"};
  static const char* const DC[3] = {"f_dc_0", "f_dc_1", "f_dc_2"};
  static const char* const GATE[2] = {"cage_gate_a", "cage_gate_b"};
  static const char* const OPEN[4] = {"open_r", "open_g", "open_b", "open_dopacity"};
  for (int k = 0; k < 3; k++) L.pos[k] = h.find(XYZ[k]);
  L.has_scales = group(L.scale, SCALE, 3);
  group(L.rot, ROT, 4);
  L.opacity = h.find("opacity");
  const bool dc = group(L.dc, DC, 3);
  const bool red = h.find("red") >= 0;
  L.colour[0] = h.find(red ? "red" : "r");
  L.colour[1] = h.find(h.find("green") >= 0 ? "green" : "g");
  L.colour[2] = h.find(h.find("blue") >= 0 ? "blue" : "b");
  L.rgb = !dc && L.colour[0] >= 0;
  if (L.colour[0] >= 0) {
    const int t = h.props[L.colour[0]].type;
    L.rgb_scale = t == B2C_PLY_U8 ? 1.0 / 255.0 : t == B2C_PLY_U16 ? 1.0 / 65535.0 : 1.0;
  }
  if (L.rgb && (L.colour[1] < 0 || L.colour[2] < 0) && h.vertices > 0)
    ply_error("ply: colour properties need all three channels");
  for (int j = 0; j < 3 * (K - 1); j++) L.rest.push_back(need(field("f_rest_", j)));
  L.has_evidence = group(L.evidence, EVIDENCE_FIELDS, 7);
  L.label = h.find("seg_label");
  L.conf = h.find("seg_conf");
  L.has_labels = L.label >= 0;
  L.fill = h.find("cage_fill");
  L.has_fill = L.fill >= 0;
  L.has_gate = h.find(GATE[0]) >= 0 && h.find(GATE[1]) >= 0;
  L.gate[0] = h.find(GATE[0]);
  L.gate[1] = h.find(GATE[1]);
  L.gate_s = h.find("cage_gate_s");
  L.has_gate_s = L.has_gate && L.gate_s >= 0;
  L.has_open = true;
  for (int k = 0; k < 4; k++) {
    L.open[k] = h.find(OPEN[k]);
    L.has_open = L.has_open && L.open[k] >= 0;
  }
  if (L.pos[0] < 0 || L.pos[1] < 0 || L.pos[2] < 0) ply_error("ply: missing x/y/z");
  return L;
}

// One parsed row (doubles by property index) into splat i of the cloud (ply.cpp:148-168).
template <typename Get>
void fill_splat(SplatCloud& c, const PlyLayout& L, size_t i, Get v) {
  const int K = c.K();
  for (int k = 0; k < 3; k++) c.pos[i * 3 + k] = (float)v(L.pos[k]);
  if (L.has_scales)
    for (int k = 0; k < 3; k++) c.log_scale[i * 3 + k] = (float)v(L.scale[k]);
  if (L.rot[0] >= 0)
    for (int k = 0; k < 4; k++) c.quat[i * 4 + k] = (float)v(L.rot[k]);
  if (L.opacity >= 0) c.opacity[i] = (float)v(L.opacity);
  float* sh = &c.sh[i * (size_t)K * 3];
  for (int ch = 0; ch < 3; ch++) {
    if (L.dc[0] >= 0) sh[ch] = (float)v(L.dc[ch]);
    else if (L.rgb) sh[ch] = (float)((v(L.colour[ch]) * L.rgb_scale - 0.5) / (double)SH_C0);
  }
  for (int ch = 0; ch < 3; ch++)
    for (int k = 1; k < K; k++) sh[k * 3 + ch] = (float)v(L.rest[ch * (K - 1) + (k - 1)]);
  if (L.has_evidence)
    for (int k = 0; k < 7; k++) c.evidence[i * 7 + k] = (float)v(L.evidence[k]);
  if (L.has_labels) {
    c.labels[i * 2] = (float)v(L.label);
    c.labels[i * 2 + 1] = L.conf >= 0 ? (float)v(L.conf) : 1.f;
  }
  if (L.has_fill) c.fill[i] = (float)v(L.fill);
  if (L.has_gate)
    for (int k = 0; k < 2; k++) c.gate[i * 2 + k] = (float)v(L.gate[k]);
  if (L.has_gate_s) c.gate_s[i] = (float)v(L.gate_s);
  if (L.has_open)
    for (int k = 0; k < 4; k++) c.open[i * 4 + k] = (float)v(L.open[k]);
}

SplatCloud empty_cloud(const PlyLayout& L, size_t n) {
  SplatCloud c;
  c.has_evidence = L.has_evidence;
  c.has_labels = L.has_labels;
  c.has_fill = L.has_fill;
  c.has_gate = L.has_gate;
  c.has_gate_s = L.has_gate_s;
  c.has_open = L.has_open;
  c.resize(n, L.degree);
  c.has_scales = L.has_scales;
  return c;
}

struct File {
  FILE* f = nullptr;
  explicit File(const std::string& path, const char* mode) : f(fopen(path.c_str(), mode)) {}
  ~File() {
    if (f) fclose(f);
  }
};

// The header write_ply emits and the number of floats per row (ply.cpp:181-200).
std::string header_text(const SplatCloud& c, const std::vector<std::string>& comments, int* row_floats) {
  std::string h = "ply\nformat binary_little_endian 1.0\n";
  for (const std::string& cm : comments) h += "comment " + cm + "\n";
  h += "element vertex " + std::to_string(c.n) + "\n";
  int cols = 0;
  const auto prop = [&](const std::string& name) {
    h += "property float " + name + "\n";
    cols++;
  };
  for (const char* b : {"x", "y", "z", "scale_0", "scale_1", "scale_2", "opacity", "rot_0", "rot_1", "rot_2", "rot_3",
                        "f_dc_0", "f_dc_1", "f_dc_2"})
    prop(b);
  for (int j = 0; j < 3 * (c.K() - 1); j++) prop(field("f_rest_", j));
  if (c.has_evidence)
    for (const char* e : EVIDENCE_FIELDS) prop(e);
  if (c.has_labels)
    for (const char* e : LABEL_FIELDS) prop(e);
  if (c.has_fill) prop("cage_fill");
  if (c.has_gate) {
    prop("cage_gate_a");
    prop("cage_gate_b");
  }
  if (c.has_gate_s) prop("cage_gate_s");
  if (c.has_open)
    for (const char* e : {"open_r", "open_g", "open_b", "open_dopacity"}) prop(e);
  h += "end_header\n";
  *row_floats = cols;
  return h;
}

constexpr size_t CHUNK_BYTES = (size_t)32 << 20;  // staging per chunk of a streamed load or save
constexpr size_t DEC_ROWS_ALIGN = 64;             // chunks of whole decode workgroups

}  // namespace

// A repeated property name resolves to its last occurrence, as read_ply's name -> column map does
// (ply.cpp:96-97).
int PlyHeader::find(const char* name) const {
  for (size_t k = props.size(); k-- > 0;)
    if (props[k].name == name) return (int)k;
  return -1;
}

PlyHeader read_ply_header(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) ply_error("failed to open ply '%s'", path.c_str());
  std::string line;
  std::getline(f, line);
  if (line.rfind("ply", 0) != 0) ply_error("'%s' is not a ply file", path.c_str());
  PlyHeader h;
  bool big_endian = false, in_vertex = false;
  while (std::getline(f, line)) {
    if (!line.empty() && line.back() == '\r') line.pop_back();
    std::istringstream ss(line);
    std::string word;
    ss >> word;
    if (word == "format") {
      std::string fmt;
      ss >> fmt;
      h.binary = fmt != "ascii";
      big_endian = fmt == "binary_big_endian";
    } else if (word == "element") {
      std::string name;
      size_t count = 0;
      ss >> name >> count;
      in_vertex = name == "vertex";
      if (in_vertex) h.vertices = count;
      else if (count > 0) ply_error("ply: unsupported non-vertex element '%s'", name.c_str());
    } else if (word == "property" && in_vertex) {
      std::string type, name;
      ss >> type;
      if (type == "list") ply_error("ply: list properties are not supported on vertices");
      const TypeName& t = type_named(type);
      ss >> name;
      h.props.push_back({name, t.type, h.row_bytes});
      h.row_bytes += t.bytes;
    } else if (word == "comment") {
      h.comments.push_back(line.size() > 8 ? line.substr(8) : std::string());
    } else if (word == "end_header") {
      break;
    }
  }
  if (big_endian) ply_error("ply: big-endian files are not supported");
  h.data_offset = (size_t)f.tellg();
  return h;
}

bool ply_is_vertex_only(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::string line;
  std::getline(f, line);
  if (line.rfind("ply", 0) != 0) return false;
  bool vertices = false;
  while (std::getline(f, line)) {
    if (!line.empty() && line.back() == '\r') line.pop_back();
    std::istringstream ss(line);
    std::string word;
    ss >> word;
    if (word == "end_header") break;
    if (word != "element") continue;
    std::string name;
    size_t count = 0;
    ss >> name >> count;
    if (name == "vertex") vertices = count > 0;
    else if (count > 0) return false;
  }
  return vertices;
}

SplatCloud read_ply(const std::string& path) {
  const PlyHeader h = read_ply_header(path);
  const PlyLayout L = layout_of(h);
  const size_t n = h.vertices, P = h.props.size();
  SplatCloud c = empty_cloud(L, n);
  std::ifstream f(path, std::ios::binary);
  f.seekg((std::streamoff)h.data_offset);
  if (h.binary) {
    const size_t rows_per = std::max<size_t>(1, CHUNK_BYTES / std::max<uint32_t>(h.row_bytes, 1));
    std::vector<unsigned char> buf(rows_per * h.row_bytes);
    for (size_t done = 0; done < n;) {
      const size_t rows = std::min(rows_per, n - done);
      f.read(reinterpret_cast<char*>(buf.data()), (std::streamsize)(rows * h.row_bytes));
      const size_t got = (size_t)f.gcount();
      if (got != rows * h.row_bytes)
        ply_error("ply: truncated file '%s' (got %zu of %zu vertices)", path.c_str(), done + got / h.row_bytes, n);
      for (size_t r = 0; r < rows; r++) {
        const unsigned char* row = buf.data() + r * h.row_bytes;
        fill_splat(c, L, done + r, [&](int k) { return value_at(row + h.props[k].offset, h.props[k].type); });
      }
      done += rows;
    }
  } else {
    std::vector<double> row(P);
    for (size_t i = 0; i < n; i++) {
      for (size_t k = 0; k < P; k++)
        if (!(f >> row[k])) ply_error("ply: truncated ascii file '%s'", path.c_str());
      fill_splat(c, L, i, [&](int k) { return row[k]; });
    }
  }
  return c;
}

SplatCloud read_ply_shape(const std::string& path) {
  const PlyHeader h = read_ply_header(path);
  SplatCloud c = empty_cloud(layout_of(h), 0);
  c.n = h.vertices;
  return c;
}

std::vector<std::string> read_ply_comments(const std::string& path) {
  std::vector<std::string> out;
  std::ifstream f(path, std::ios::binary);
  std::string line;
  while (std::getline(f, line) && line != "end_header")
    if (line.rfind("comment ", 0) == 0) out.push_back(line.substr(8));
  return out;
}

void write_ply(const std::string& path, const SplatCloud& c, const std::vector<std::string>& comments) {
#pragma clang fp contract(off)
  File f(path, "wb");
  if (!f.f) ply_error("failed to open '%s' for writing", path.c_str());
  int row_floats = 0;
  const std::string head = header_text(c, comments, &row_floats);
  bool ok = fwrite(head.data(), 1, head.size(), f.f) == head.size();
  const int K = c.K();
  const size_t rows_per = std::max<size_t>(1, CHUNK_BYTES / (4 * (size_t)row_floats));
  std::vector<float> buf;
  buf.reserve(rows_per * row_floats);
  const auto put = [&](const float* v, int count) { buf.insert(buf.end(), v, v + count); };
  for (size_t i = 0; i < c.n && ok; i++) {
    put(&c.pos[i * 3], 3);
    put(&c.log_scale[i * 3], 3);
    put(&c.opacity[i], 1);
    float q[4] = {c.quat[i * 4], c.quat[i * 4 + 1], c.quat[i * 4 + 2], c.quat[i * 4 + 3]};
    float qn = std::sqrt(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]);
    if (!(qn > 1e-32f)) {
      qn = 1.f;
      q[0] = 1.f;
      q[1] = q[2] = q[3] = 0.f;
    }
    for (float& x : q) x = x / qn;
    put(q, 4);
    const float* sh = &c.sh[i * (size_t)K * 3];
    put(sh, 3);
    for (int ch = 0; ch < 3; ch++)
      for (int k = 1; k < K; k++) buf.push_back(sh[k * 3 + ch]);
    if (c.has_evidence) put(&c.evidence[i * 7], 7);
    if (c.has_labels) put(&c.labels[i * 2], 2);
    if (c.has_fill) put(&c.fill[i], 1);
    if (c.has_gate) put(&c.gate[i * 2], 2);
    if (c.has_gate_s) put(&c.gate_s[i], 1);
    if (c.has_open) put(&c.open[i * 4], 4);
    if (buf.size() >= rows_per * row_floats || i + 1 == c.n) {
      ok = fwrite(buf.data(), sizeof(float), buf.size(), f.f) == buf.size();
      buf.clear();
    }
  }
  if (!ok || fflush(f.f) != 0) ply_error("failed writing '%s'", path.c_str());
}

bool load_ply(Model& m, const std::string& path, hipStream_t stream) {
  const PlyHeader h = read_ply_header(path);
  const PlyLayout L = layout_of(h);
  if (L.degree > 4) ply_error("ply: SH degree %d exceeds the model's maximum of 4", L.degree);
  if (!h.binary) {
    const SplatCloud c = read_ply(path);
    m.upload(c, stream);
    return c.has_scales;
  }
  const size_t n = h.vertices;
  if (n > (size_t)INT32_MAX) ply_error("ply: %zu vertices exceed the model's capacity", n);
  b2c_ply_decode_args a{};
  for (int t = 0; t < B2C_PLY_TARGETS; t++) a.col[t] = -1;
  const auto map = [&](int target, int prop) {
    if (prop < 0) return;
    if (h.props[prop].offset > 32767u) ply_error("ply: row of %u bytes is not a splat layout", h.row_bytes);
    a.col[target] = (int16_t)h.props[prop].offset;
    a.type[target] = (uint8_t)h.props[prop].type;
  };
  for (int k = 0; k < 3; k++) map(B2C_PLY_T_POS + k, L.pos[k]);
  for (int k = 0; k < 3; k++) map(B2C_PLY_T_SCALE + k, L.has_scales ? L.scale[k] : -1);
  for (int k = 0; k < 4; k++) map(B2C_PLY_T_ROT + k, L.rot[k]);
  map(B2C_PLY_T_OPACITY, L.opacity);
  for (int k = 0; k < 3; k++) map(B2C_PLY_T_DC + k, L.dc[k]);
  for (int k = 0; k < 3; k++) map(B2C_PLY_T_RGB + k, L.rgb ? L.colour[k] : -1);
  for (size_t j = 0; j < L.rest.size(); j++) map(B2C_PLY_T_REST + (int)j, L.rest[j]);
  a.rgb_dc = L.rgb ? 1 : 0;
  a.rgb_scale = L.rgb_scale;
  a.row_bytes = h.row_bytes;

  m.reset((int)n, L.degree, stream);
  a.model = m.layout();
  File f(path, "rb");
  if (!f.f || fseeko(f.f, (off_t)h.data_offset, SEEK_SET) != 0) ply_error("failed to open ply '%s'", path.c_str());
  // Two pinned chunks and two device staging chunks: the disk read of chunk k + 1 overlaps the copy and
  // decode of chunk k; a pinned chunk is refilled once the copy that read it has completed.
  const size_t rows_per = std::max<size_t>(DEC_ROWS_ALIGN, CHUNK_BYTES / h.row_bytes / DEC_ROWS_ALIGN * DEC_ROWS_ALIGN);
  const size_t chunk_bytes = rows_per * h.row_bytes;
  PinnedBuf<unsigned char> host[2];
  DevBuf<unsigned char> staging[2];
  hipEvent_t copied[2] = {nullptr, nullptr};
  struct Events {
    hipEvent_t* e;
    ~Events() {
      for (int k = 0; k < 2; k++)
        if (e[k]) (void)hipEventDestroy(e[k]);
    }
  } events{copied};
  for (int k = 0; k < 2; k++) {
    host[k].reserve(std::min(chunk_bytes, n * h.row_bytes) + 8);
    staging[k].reserve(std::min(chunk_bytes, n * h.row_bytes) + 8);
    HIP_CHECK(hipEventCreateWithFlags(&copied[k], hipEventDisableTiming));
  }
  size_t done = 0;
  for (int k = 0; done < n; k ^= 1) {
    const size_t rows = std::min(rows_per, n - done);
    HIP_CHECK(hipEventSynchronize(copied[k]));  // the copy out of this pinned chunk (two chunks ago) is done
    const size_t got = fread(host[k].ptr, 1, rows * h.row_bytes, f.f);
    if (got != rows * h.row_bytes) {
      HIP_CHECK(hipStreamSynchronize(stream));
      ply_error("ply: truncated file '%s' (got %zu of %zu vertices)", path.c_str(), done + got / h.row_bytes, n);
    }
    HIP_CHECK(hipMemcpyAsync(staging[k].ptr, host[k].ptr, rows * h.row_bytes, hipMemcpyHostToDevice, stream));
    HIP_CHECK(hipEventRecord(copied[k], stream));
    a.rows = staging[k].ptr;
    a.count = (int)rows;
    a.first = (int)done;
    LAUNCH_CHECK(b2c_hip_ply_decode(&a, stream));
    done += rows;
  }
  m.zero_optimizer(stream);
  m.zero_stats(stream);
  HIP_CHECK(hipStreamSynchronize(stream));
  return L.has_scales;
}

void save_ply(const Model& m, const std::string& path, const std::vector<std::string>& comments,
              const SplatCloud* extras, hipStream_t stream) {
  SplatCloud shape;  // the header's description: size, degree and which optional blocks follow
  shape.n = (size_t)m.n;
  shape.sh_degree = m.degree;
  b2c_ply_encode_args a{};
  a.model = m.layout();
  DevBuf<float> blocks[6];
  if (extras) {
    const std::pair<bool, const std::vector<float>*> src[6] = {
        {extras->has_evidence, &extras->evidence}, {extras->has_labels, &extras->labels},
        {extras->has_fill, &extras->fill},         {extras->has_gate, &extras->gate},
        {extras->has_gate_s, &extras->gate_s},     {extras->has_open, &extras->open}};
    const size_t widths[6] = {7, 2, 1, 2, 1, 4};
    const float** dst[6] = {&a.evidence, &a.labels, &a.fill, &a.gate, &a.gate_s, &a.open};
    for (int b = 0; b < 6; b++) {
      if (!src[b].first) continue;
      if (src[b].second->size() != shape.n * widths[b]) ply_error("save_ply: an optional block does not have one row per splat");
      blocks[b].upload(*src[b].second, stream);
      *dst[b] = blocks[b].ptr;
    }
    shape.has_evidence = extras->has_evidence;
    shape.has_labels = extras->has_labels;
    shape.has_fill = extras->has_fill;
    shape.has_gate = extras->has_gate;
    shape.has_gate_s = extras->has_gate_s;
    shape.has_open = extras->has_open;
  }
  int row_floats = 0;
  const std::string head = header_text(shape, comments, &row_floats);
  a.row_floats = row_floats;
  File f(path, "wb");
  if (!f.f) ply_error("failed to open '%s' for writing", path.c_str());
  bool ok = fwrite(head.data(), 1, head.size(), f.f) == head.size();
  const size_t n = shape.n, row_bytes = 4 * (size_t)row_floats;
  const size_t rows_per = std::max<size_t>(1, CHUNK_BYTES / row_bytes);
  PinnedBuf<float> host[2];
  DevBuf<float> rows_dev[2];
  hipEvent_t ready[2] = {nullptr, nullptr};
  struct Events {
    hipEvent_t* e;
    ~Events() {
      for (int k = 0; k < 2; k++)
        if (e[k]) (void)hipEventDestroy(e[k]);
    }
  } events{ready};
  for (int k = 0; k < 2; k++) {
    host[k].reserve(std::max<size_t>(1, std::min(rows_per, n) * row_floats));
    rows_dev[k].reserve(std::max<size_t>(1, std::min(rows_per, n) * row_floats));
    HIP_CHECK(hipEventCreateWithFlags(&ready[k], hipEventDisableTiming));
  }
  // Chunk k + 1 is encoded and copied while the host writes chunk k.
  const auto queue = [&](size_t first, int k) {
    a.first = (int)first;
    a.count = (int)std::min(rows_per, n - first);
    a.rows = rows_dev[k].ptr;
    LAUNCH_CHECK(b2c_hip_ply_encode(&a, stream));
    HIP_CHECK(hipMemcpyAsync(host[k].ptr, rows_dev[k].ptr, (size_t)a.count * row_bytes, hipMemcpyDeviceToHost, stream));
    HIP_CHECK(hipEventRecord(ready[k], stream));
  };
  if (n) queue(0, 0);
  for (size_t first = 0; first < n && ok; first += rows_per) {
    const int k = (int)((first / rows_per) & 1);
    if (first + rows_per < n) queue(first + rows_per, k ^ 1);
    HIP_CHECK(hipEventSynchronize(ready[k]));
    const size_t count = std::min(rows_per, n - first);
    ok = fwrite(host[k].ptr, row_bytes, count, f.f) == count;
  }
  HIP_CHECK(hipStreamSynchronize(stream));
  if (!ok || fflush(f.f) != 0) ply_error("failed writing '%s'", path.c_str());
}

}  // namespace b2c
