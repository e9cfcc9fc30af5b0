// Splat clouds in brush's ply layout (replaces src/ply.h:1-51): the header probe, the host reader and
// writer with the reference's semantics, and the device-direct pair this build adds, which move a file's
// rows between the disk and the model's device layout without a host-side re-layout.
#pragma once
#include <string>
#include <vector>

#include "model.h"

namespace b2c {

extern const char* const EVIDENCE_FIELDS[7];  // ev_w_in ev_w_all ev_err ev_views ev_dir_0 ev_dir_1 ev_dir_2
extern const char* const LABEL_FIELDS[2];     // seg_label seg_conf

// The vertex element of a ply header: every property with its type and byte offset in a binary row.
struct PlyHeader {
  bool binary = false;  // binary_little_endian; false: ascii
  size_t vertices = 0;
  struct Property {
    std::string name;
    int type;         // B2C_PLY_* (include/b2c_kernels.h)
    uint32_t offset;  // byte offset within a binary row
  };
  std::vector<Property> props;
  uint32_t row_bytes = 0;
  size_t data_offset = 0;  // file offset of the first row
  std::vector<std::string> comments;
  int find(const char* name) const;  // property index, or -1
};
// Parses and checks the header as read_ply does (ply.cpp:88-110): a vertex element with scalar properties
// of the eight types, no other non-empty element, not big-endian. Throws on anything else.
PlyHeader read_ply_header(const std::string& path);

// True when the file is a ply read_ply can load: its only non-empty element is `vertex` (ply.cpp:63-83).
bool ply_is_vertex_only(const std::string& path);

// ply.cpp:85-170: values are read as double and stored as float; the SH degree follows from the count of
// f_rest_* properties; without f_dc_* the DC comes from red/green/blue (or r/g/b), scaled by the red
// column's type; rot_* absent gives the identity, scale_* absent clears has_scales. The optional blocks
// (ev_*, seg_*, cage_*, open_*) are read when present.
SplatCloud read_ply(const std::string& path);
// What read_ply would return, without the arrays: the vertex count, SH degree and the flags.
SplatCloud read_ply_shape(const std::string& path);
// The header's comment lines without the "comment " prefix (ply.cpp:172-178).
std::vector<std::string> read_ply_comments(const std::string& path);
// ply.cpp:180-226: binary little-endian, float properties in brush's order, unit quaternions, f_rest
// channel-major, then the optional blocks. The bytes are the reference writer's for the same cloud.
void write_ply(const std::string& path, const SplatCloud& c, const std::vector<std::string>& comments);

// Device-direct load: Model::upload(read_ply(path)) without the host cloud. Binary files stream through
// pinned chunks into a device staging buffer and are decoded into the model's layout by a kernel; ascii
// files are read on the host. The model's sh_fp16 choice is kept. Returns the file's has_scales.
bool load_ply(Model& m, const std::string& path, hipStream_t stream);
// Device-direct save: write_ply(path, download + the optional blocks of `extras`) with the rows encoded on
// the device. `extras` (may be null) supplies has_evidence / has_labels / ... and their arrays, [n] rows.
void save_ply(const Model& m, const std::string& path, const std::vector<std::string>& comments,
              const SplatCloud* extras, hipStream_t stream);

}  // namespace b2c
