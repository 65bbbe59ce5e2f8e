// Reader for .safetensors files and their compressed-tensors quantization
// metadata.  Pure host C++ (no HIP): the checkpoint entry points of the C ABI
// (checkpoint.cpp) use it, and a sanitizer build links it on its own.
//
// File layout (the safetensors format): an 8-byte little-endian header
// length L, L bytes of UTF-8 JSON, then the tensor bytes.  The JSON maps each
// tensor name to {"dtype", "shape", "data_offsets": [begin, end]} (offsets
// relative to the end of the header) and may hold a "__metadata__" object of
// string values.  teeny-quant stores its scheme there under
// "quantization_config" as a JSON string, and names a quantized weight's
// companions foo.weight_scale / foo.weight_zero_point
// (utilities/teeny-quant/src/format.rs:16-35, :118-126).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace teeny {
namespace st {

// ── a small JSON value and parser (objects, arrays, strings, numbers, bools, null) ──
struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  bool integral = false;  // a number written without fraction or exponent
  int64_t i = 0;          // its value when integral (exact up to 2^63)
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;  // insertion order kept
  const Json *get(const std::string &key) const;
};

// Parses `text` (exactly one value, surrounding whitespace allowed).  On
// failure returns false and sets *err.  Nesting is limited to 64 levels.
bool parse_json(const char *text, size_t len, Json *out, std::string *err);

enum class DType { F64, F32, F16, BF16, I64, I32, I16, I8, U8, BOOL, F8_E4M3, F8_E5M2, Unknown };
DType dtype_from_name(const std::string &name);
size_t dtype_size(DType d);  // bytes per element; 0 for Unknown

struct TensorEntry {
  std::string name;
  std::string dtype_name;
  DType dtype = DType::Unknown;
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;  // byte offsets into the data section
  int64_t numel() const;
};

// The scheme of a compressed-tensors checkpoint (format.rs:52-126): one
// config group's "weights" block plus the file-level fields.
struct QuantConfig {
  bool present = false;
  std::string quant_method, format;
  int num_bits = 0;
  std::string type;  // "int" or "float"
  bool symmetric = true;  // required in the file: parse fails without it
  std::string strategy;  // "tensor", "channel" or "group"
  int64_t axis = -1;     // -1 when absent
  int64_t group_size = 0;
  std::vector<std::string> ignore;
  int n_groups = 0;  // config groups in the file
};

class File {
 public:
  ~File();
  // Maps `path` read-only and parses its header; false with *err on any
  // malformed or inconsistent content (bounds, dtypes, offsets, metadata).
  bool open(const std::string &path, std::string *err);
  // The same over a caller-owned byte image (not copied; must outlive this).
  bool open_image(const uint8_t *data, size_t size, std::string *err);

  const std::vector<TensorEntry> &tensors() const { return tensors_; }
  const TensorEntry *find(const std::string &name) const;
  const std::map<std::string, std::string> &metadata() const { return metadata_; }
  const QuantConfig &quant_config() const { return qcfg_; }
  const uint8_t *data(const TensorEntry &t) const { return base_ + data_start_ + t.begin; }

 private:
  bool parse(std::string *err);
  const uint8_t *base_ = nullptr;
  size_t size_ = 0;
  size_t data_start_ = 0;
  void *mapping_ = nullptr;  // mmap'd region owned by this object
  std::vector<TensorEntry> tensors_;
  std::map<std::string, size_t> index_;
  std::map<std::string, std::string> metadata_;
  QuantConfig qcfg_;
};

}  // namespace st
}  // namespace teeny
