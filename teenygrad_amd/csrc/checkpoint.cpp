// Compressed-tensors int8 checkpoints: the C ABI over the safetensors reader.
//
// Reference: teeny-quant's output convention (utilities/teeny-quant/src/
// format.rs:16-35): for a quantized weight foo.weight, the file holds
// foo.weight (I8, the tensor's own shape), foo.weight_scale (F32, one per
// group), foo.weight_zero_point (I32, asymmetric schemes only) and the
// scheme as JSON under __metadata__["quantization_config"] (:52-126), read
// back by dequantize_tensor (:249-289).  These entry points open such a file
// (mmap'd, header validated), describe its tensors and scheme, and copy a
// tensor's bytes, or a W8A16 layer's int8 weights and per-channel scales,
// straight into caller-owned device buffers that teeny_w8a16_linear_forward
// and teeny_w8a16_conv2d_forward consume.
#include <cstring>
#include <memory>
#include <vector>

#include "common.hpp"
#include "safetensors.hpp"

namespace teeny {

struct Checkpoint {
  st::File file;
};

static void copy_str(char *dst, size_t cap, const std::string &s) {
  std::strncpy(dst, s.c_str(), cap - 1);
  dst[cap - 1] = '\0';
}

static teeny_status checkpoint_of(teeny_checkpoint h, Checkpoint **out, const char *what) {
  TEENY_REQUIRE(h != nullptr, TEENY_ERR_NULL_POINTER, std::string(what) + ": checkpoint");
  *out = static_cast<Checkpoint *>(h);
  return TEENY_OK;
}

static int granularity_code(const std::string &strategy) {
  if (strategy == "tensor") return TEENY_PER_TENSOR;
  if (strategy == "channel") return TEENY_PER_CHANNEL;
  if (strategy == "group") return TEENY_GROUP;
  return -1;
}

static teeny_status copy_out(const void *src, void *dst, size_t bytes, int32_t to_device, hipStream_t s) {
  if (bytes == 0) return TEENY_OK;
  if (!to_device) {
    std::memcpy(dst, src, bytes);
    return TEENY_OK;
  }
  TEENY_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
  // the source is the file mapping: finish before the caller may close it
  TEENY_CHECK_HIP(hipStreamSynchronize(s));
  return TEENY_OK;
}

}  // namespace teeny

using namespace teeny;

extern "C" {

teeny_status teeny_checkpoint_open(const char *path, teeny_checkpoint *ckpt) {
  TEENY_REQUIRE(path != nullptr && ckpt != nullptr, TEENY_ERR_NULL_POINTER, "checkpoint_open: path/ckpt");
  *ckpt = nullptr;
  auto c = std::make_unique<Checkpoint>();
  std::string err;
  if (!c->file.open(path, &err)) return fail(TEENY_ERR_INVALID_ARGUMENT, "checkpoint_open: " + err);
  *ckpt = c.release();
  return TEENY_OK;
}

teeny_status teeny_checkpoint_open_image(const void *data, size_t size, teeny_checkpoint *ckpt) {
  TEENY_REQUIRE(data != nullptr && ckpt != nullptr, TEENY_ERR_NULL_POINTER, "checkpoint_open_image: data/ckpt");
  *ckpt = nullptr;
  auto c = std::make_unique<Checkpoint>();
  std::string err;
  if (!c->file.open_image(static_cast<const uint8_t *>(data), size, &err))
    return fail(TEENY_ERR_INVALID_ARGUMENT, "checkpoint_open_image: " + err);
  *ckpt = c.release();
  return TEENY_OK;
}

teeny_status teeny_checkpoint_close(teeny_checkpoint ckpt) {
  delete static_cast<Checkpoint *>(ckpt);
  return TEENY_OK;
}

teeny_status teeny_checkpoint_num_tensors(teeny_checkpoint ckpt, int64_t *n) {
  Checkpoint *c;
  teeny_status st = checkpoint_of(ckpt, &c, "checkpoint_num_tensors");
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(n != nullptr, TEENY_ERR_NULL_POINTER, "checkpoint_num_tensors: n");
  *n = static_cast<int64_t>(c->file.tensors().size());
  return TEENY_OK;
}

teeny_status teeny_checkpoint_tensor_info(teeny_checkpoint ckpt, int64_t index, teeny_tensor_info *info) {
  Checkpoint *c;
  teeny_status st = checkpoint_of(ckpt, &c, "checkpoint_tensor_info");
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(info != nullptr, TEENY_ERR_NULL_POINTER, "checkpoint_tensor_info: info");
  const auto &ts = c->file.tensors();
  TEENY_REQUIRE(index >= 0 && index < static_cast<int64_t>(ts.size()), TEENY_ERR_INVALID_ARGUMENT,
                "checkpoint_tensor_info: index out of range");
  const st::TensorEntry &t = ts[static_cast<size_t>(index)];
  TEENY_REQUIRE(t.name.size() < sizeof(info->name), TEENY_ERR_UNSUPPORTED,
                "checkpoint_tensor_info: tensor name longer than 255 bytes");
  std::memset(info, 0, sizeof(*info));
  copy_str(info->name, sizeof(info->name), t.name);
  copy_str(info->dtype, sizeof(info->dtype), t.dtype_name);
  info->ndim = static_cast<int32_t>(t.shape.size());
  for (size_t d = 0; d < t.shape.size(); ++d) info->shape[d] = t.shape[d];
  info->nbytes = t.end - t.begin;
  return TEENY_OK;
}

teeny_status teeny_checkpoint_find(teeny_checkpoint ckpt, const char *name, int64_t *index) {
  Checkpoint *c;
  teeny_status st = checkpoint_of(ckpt, &c, "checkpoint_find");
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(name != nullptr && index != nullptr, TEENY_ERR_NULL_POINTER, "checkpoint_find: name/index");
  const st::TensorEntry *t = c->file.find(name);
  if (t == nullptr) return fail(TEENY_ERR_NOT_FOUND, std::string("checkpoint_find: no tensor ") + name);
  *index = t - c->file.tensors().data();
  return TEENY_OK;
}

teeny_status teeny_checkpoint_quant_scheme(teeny_checkpoint ckpt, teeny_quant_scheme *scheme) {
  Checkpoint *c;
  teeny_status st = checkpoint_of(ckpt, &c, "checkpoint_quant_scheme");
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(scheme != nullptr, TEENY_ERR_NULL_POINTER, "checkpoint_quant_scheme: scheme");
  const st::QuantConfig &q = c->file.quant_config();
  std::memset(scheme, 0, sizeof(*scheme));
  scheme->present = q.present ? 1 : 0;
  scheme->num_bits = q.num_bits;
  scheme->symmetric = q.symmetric ? 1 : 0;
  scheme->granularity = granularity_code(q.strategy);
  scheme->axis = q.axis;
  scheme->group_size = q.group_size;
  scheme->n_config_groups = q.n_groups;
  copy_str(scheme->quant_method, sizeof(scheme->quant_method), q.quant_method);
  copy_str(scheme->format, sizeof(scheme->format), q.format);
  copy_str(scheme->type, sizeof(scheme->type), q.type);
  return TEENY_OK;
}

teeny_status teeny_checkpoint_read(teeny_checkpoint ckpt, int64_t index, void *dst, size_t bytes, int32_t to_device,
                                   teeny_stream stream) {
  Checkpoint *c;
  teeny_status st = checkpoint_of(ckpt, &c, "checkpoint_read");
  if (st != TEENY_OK) return st;
  const auto &ts = c->file.tensors();
  TEENY_REQUIRE(index >= 0 && index < static_cast<int64_t>(ts.size()), TEENY_ERR_INVALID_ARGUMENT,
                "checkpoint_read: index out of range");
  const st::TensorEntry &t = ts[static_cast<size_t>(index)];
  TEENY_REQUIRE(bytes == t.end - t.begin, TEENY_ERR_SHAPE_MISMATCH,
                "checkpoint_read: tensor " + t.name + " holds " + std::to_string(t.end - t.begin) + " bytes, " +
                    std::to_string(bytes) + " requested");
  TEENY_REQUIRE(bytes == 0 || dst != nullptr, TEENY_ERR_NULL_POINTER, "checkpoint_read: dst");
  return copy_out(c->file.data(t), dst, bytes, to_device, static_cast<hipStream_t>(stream));
}

// The layer `weight_name` as W8A16 operands: int8 [N, K] plus N fp32 scales,
// from a symmetric 8-bit integer scheme that is per output channel (axis 0)
// or per tensor (its one scale repeated N times).
static teeny_status w8a16_layer(Checkpoint *c, const char *weight_name, const st::TensorEntry **w,
                                const st::TensorEntry **s, const char *what) {
  const std::string nm(what), wn(weight_name);
  const st::QuantConfig &q = c->file.quant_config();
  TEENY_REQUIRE(q.present, TEENY_ERR_UNSUPPORTED, nm + ": the file has no quantization_config");
  TEENY_REQUIRE(q.quant_method == "compressed-tensors", TEENY_ERR_UNSUPPORTED,
                nm + ": quant_method '" + q.quant_method + "' is not compressed-tensors");
  TEENY_REQUIRE(q.n_groups == 1, TEENY_ERR_UNSUPPORTED, nm + ": more than one config group");
  TEENY_REQUIRE(q.type == "int" && q.num_bits == 8 && q.format == "int-quantized", TEENY_ERR_UNSUPPORTED,
                nm + ": scheme is " + q.type + std::to_string(q.num_bits) + " '" + q.format +
                    "'; W8A16 needs 8-bit int-quantized");
  TEENY_REQUIRE(q.symmetric, TEENY_ERR_UNSUPPORTED, nm + ": asymmetric scheme (zero points): dequantize instead");
  // a channel or group strategy names its axis (validate.rs:94-103)
  TEENY_REQUIRE(q.strategy == "tensor" || q.axis >= 0, TEENY_ERR_INVALID_ARGUMENT,
                nm + ": strategy '" + q.strategy + "' without an axis is ambiguous");
  TEENY_REQUIRE(q.strategy == "tensor" || (q.strategy == "channel" && q.axis == 0), TEENY_ERR_UNSUPPORTED,
                nm + ": strategy '" + q.strategy + "' (axis " + std::to_string(q.axis) +
                    "): W8A16 takes per-output-channel (axis 0) or per-tensor scales; dequantize instead");
  for (const std::string &ig : q.ignore)
    TEENY_REQUIRE(ig != wn, TEENY_ERR_INVALID_ARGUMENT, nm + ": " + wn + " is listed as unquantized");
  *w = c->file.find(wn);
  *s = c->file.find(wn + "_scale");
  TEENY_REQUIRE(*w != nullptr, TEENY_ERR_NOT_FOUND, nm + ": no tensor " + wn);
  // a symmetric scheme has an implicit zero point of 0 and omits the tensor
  // (format.rs:25-26); one present contradicts the scheme
  TEENY_REQUIRE(c->file.find(wn + "_zero_point") == nullptr, TEENY_ERR_INVALID_ARGUMENT,
                nm + ": " + wn + "_zero_point present under a symmetric scheme");
  TEENY_REQUIRE(*s != nullptr, TEENY_ERR_NOT_FOUND, nm + ": no tensor " + wn + "_scale");
  TEENY_REQUIRE((*w)->dtype == st::DType::I8 && (*w)->shape.size() >= 2, TEENY_ERR_UNSUPPORTED_DTYPE,
                nm + ": " + wn + " must be I8 of rank >= 2, is " + (*w)->dtype_name);
  TEENY_REQUIRE((*s)->dtype == st::DType::F32, TEENY_ERR_UNSUPPORTED_DTYPE, nm + ": " + wn + "_scale must be F32");
  const int64_t n = (*w)->shape[0];
  const int64_t want = q.strategy == "tensor" ? 1 : n;
  TEENY_REQUIRE((*s)->numel() == want, TEENY_ERR_SHAPE_MISMATCH,
                nm + ": " + wn + "_scale has " + std::to_string((*s)->numel()) + " entries, expected " +
                    std::to_string(want));
  return TEENY_OK;
}

teeny_status teeny_checkpoint_w8a16_shape(teeny_checkpoint ckpt, const char *weight_name, int64_t *N, int64_t *K) {
  Checkpoint *c;
  teeny_status st = checkpoint_of(ckpt, &c, "checkpoint_w8a16_shape");
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(weight_name != nullptr && N != nullptr && K != nullptr, TEENY_ERR_NULL_POINTER,
                "checkpoint_w8a16_shape: weight_name/N/K");
  const st::TensorEntry *w, *s;
  st = w8a16_layer(c, weight_name, &w, &s, "checkpoint_w8a16_shape");
  if (st != TEENY_OK) return st;
  *N = w->shape[0];
  *K = w->numel() / (w->shape[0] == 0 ? 1 : w->shape[0]);
  return TEENY_OK;
}

teeny_status teeny_checkpoint_load_w8a16(teeny_checkpoint ckpt, const char *weight_name, int8_t *qweight,
                                         float *scale, int64_t N, int64_t K, teeny_stream stream) {
  Checkpoint *c;
  teeny_status st = checkpoint_of(ckpt, &c, "checkpoint_load_w8a16");
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(weight_name != nullptr, TEENY_ERR_NULL_POINTER, "checkpoint_load_w8a16: weight_name");
  const st::TensorEntry *w, *s;
  st = w8a16_layer(c, weight_name, &w, &s, "checkpoint_load_w8a16");
  if (st != TEENY_OK) return st;
  const int64_t n = w->shape[0], k = w->numel() / (n == 0 ? 1 : n);
  TEENY_REQUIRE(N == n && K == k, TEENY_ERR_SHAPE_MISMATCH,
                "checkpoint_load_w8a16: " + std::string(weight_name) + " is [" + std::to_string(n) + ", " +
                    std::to_string(k) + "], buffers are for [" + std::to_string(N) + ", " + std::to_string(K) + "]");
  if (N == 0) return TEENY_OK;
  TEENY_REQUIRE(qweight != nullptr && scale != nullptr, TEENY_ERR_NULL_POINTER, "checkpoint_load_w8a16: qweight/scale");
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (w->shape.size() == 4) {
    // A conv weight: teeny-quant stores the tensor in the reference's own
    // order [C_OUT, C_IN/G, KH, KW] (conv2d.rs:43-156); the W8A16 conv takes
    // [C_OUT, KH, KW, C_IN/G] (K = (kh, kw, ci) contiguous per channel).  The
    // per-output-channel scales are unaffected by the repack.
    const int64_t ci = w->shape[1], kh = w->shape[2], kw = w->shape[3];
    const int8_t *src = reinterpret_cast<const int8_t *>(c->file.data(*w));
    std::vector<int8_t> packed(static_cast<size_t>(N * K));
    for (int64_t o = 0; o < N; ++o)
      for (int64_t c_ = 0; c_ < ci; ++c_)
        for (int64_t y = 0; y < kh; ++y)
          for (int64_t x = 0; x < kw; ++x)
            packed[static_cast<size_t>(((o * kh + y) * kw + x) * ci + c_)] =
                src[((o * ci + c_) * kh + y) * kw + x];
    st = copy_out(packed.data(), qweight, packed.size(), 1, hs);
  } else {
    st = copy_out(c->file.data(*w), qweight, static_cast<size_t>(w->end - w->begin), 1, hs);
  }
  if (st != TEENY_OK) return st;
  if (s->numel() == N) return copy_out(c->file.data(*s), scale, static_cast<size_t>(N) * 4, 1, hs);
  // per-tensor: the one scale for every output channel
  float one;
  std::memcpy(&one, c->file.data(*s), 4);
  std::vector<float> rep(static_cast<size_t>(N), one);
  return copy_out(rep.data(), scale, rep.size() * 4, 1, hs);
}

}  // extern "C"
