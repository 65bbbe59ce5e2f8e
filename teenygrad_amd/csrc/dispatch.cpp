// teeny_dispatch: runs an operator from the reference's packed argument list.
//
// The reference executor packs each node's kernel arguments through
// RuntimeOp::pack_args into an ArgVisitor (core/teeny-core/src/model/mod.rs
// :78-331, core/teeny-core/src/device/program.rs:22-46) and launches the
// kernel "{name}_entry_point" with RuntimeOp::grid (drivers/teeny-cuda/src/
// model/mod.rs:524-700).  This translation unit accepts that same list —
// argument kinds and order exactly as each reference RuntimeOp visits them —
// plus the kernel's const generics, and forwards to the matching teeny_*
// entry point.  Argument kinds are checked; a mismatch is an error, never a
// reinterpretation.
#include <algorithm>
#include <cstring>
#include <string>

#include "common.hpp"

namespace teeny {

struct ArgReader {
  const teeny_arg *args;
  int n;
  int i = 0;
  const char *op;
  teeny_status st = TEENY_OK;

  bool take(int kind, const char *what) {
    if (st != TEENY_OK) return false;
    if (i >= n) {
      st = fail(TEENY_ERR_INVALID_ARGUMENT, std::string(op) + ": missing argument " + what);
      return false;
    }
    if (args[i].kind != kind) {
      st = fail(TEENY_ERR_INVALID_ARGUMENT, std::string(op) + ": argument " + std::to_string(i) +
                                                " (" + what + ") has the wrong kind");
      return false;
    }
    return true;
  }
  void *ptr(const char *what) { return take(TEENY_ARG_PTR, what) ? args[i++].v.ptr : nullptr; }
  int64_t i32(const char *what) { return take(TEENY_ARG_I32, what) ? args[i++].v.i32 : 0; }
  float f32(const char *what) { return take(TEENY_ARG_F32, what) ? args[i++].v.f32 : 0.0f; }
  teeny_status done() {
    if (st == TEENY_OK && i != n)
      st = fail(TEENY_ERR_INVALID_ARGUMENT, std::string(op) + ": " + std::to_string(n - i) +
                                                " unexpected trailing argument(s)");
    return st;
  }
};

static bool name_is(const char *ep, const char *base) {
  const size_t lb = std::strlen(base);
  return std::strncmp(ep, base, lb) == 0 &&
         (ep[lb] == '\0' || std::strcmp(ep + lb, "_entry_point") == 0);
}

}  // namespace teeny

using namespace teeny;

extern "C" teeny_status teeny_dispatch(const char *entry_point, const int64_t *cg, int32_t n_cg,
                                       const teeny_arg *args, int32_t n_args,
                                       const uint32_t grid[3], teeny_dtype dtype,
                                       teeny_stream stream) {
  TEENY_REQUIRE(entry_point != nullptr, TEENY_ERR_NULL_POINTER, "dispatch: entry_point");
  TEENY_REQUIRE(n_args == 0 || args != nullptr, TEENY_ERR_NULL_POINTER, "dispatch: args");
  TEENY_REQUIRE(n_cg == 0 || cg != nullptr, TEENY_ERR_NULL_POINTER, "dispatch: const generics");
  ArgReader r{args, n_args, 0, entry_point};

  // relu/gelu/silu_forward<BLOCK_SIZE>(x, y, n_elements)   relu.rs:143-159 etc.
  const char *acts[3] = {"relu_forward", "gelu_forward", "silu_forward"};
  for (int a = 0; a < 3; ++a) {
    if (!name_is(entry_point, acts[a])) continue;
    TEENY_REQUIRE(n_cg == 1, TEENY_ERR_INVALID_ARGUMENT,
                  std::string(acts[a]) + ": expects const generic BLOCK_SIZE");
    void *x = r.ptr("x_ptr");
    void *y = r.ptr("y_ptr");
    int64_t n = r.i32("n_elements");
    if (r.done() != TEENY_OK) return r.st;
    return a == 0 ? teeny_relu_forward(x, y, n, dtype, stream)
           : a == 1 ? teeny_gelu_forward(x, y, n, dtype, stream)
                    : teeny_silu_forward(x, y, n, dtype, stream);
  }

  // relu/gelu/silu_backward<BLOCK_SIZE>(dy, y | x, dx, n_elements)
  //   relu.rs:156-172, gelu.rs:293-309, sigmoid.rs:424-440
  const char *grads[3] = {"relu_backward", "gelu_backward", "silu_backward"};
  for (int a = 0; a < 3; ++a) {
    if (!name_is(entry_point, grads[a])) continue;
    TEENY_REQUIRE(n_cg == 1, TEENY_ERR_INVALID_ARGUMENT,
                  std::string(grads[a]) + ": expects const generic BLOCK_SIZE");
    void *dy = r.ptr("dy_ptr");
    void *saved = r.ptr(a == 0 ? "y_ptr" : "x_ptr");
    void *dx = r.ptr("dx_ptr");
    int64_t n = r.i32("n_elements");
    if (r.done() != TEENY_OK) return r.st;
    return a == 0 ? teeny_relu_backward(dy, saved, dx, n, dtype, stream)
           : a == 1 ? teeny_gelu_backward(dy, saved, dx, n, dtype, stream)
                    : teeny_silu_backward(dy, saved, dx, n, dtype, stream);
  }

  // layer_norm_forward_inference<BLOCK_N>(x, y, weight, bias, M, N, eps)   layernorm.rs:539-548
  if (name_is(entry_point, "layer_norm_forward_inference")) {
    TEENY_REQUIRE(n_cg == 1, TEENY_ERR_INVALID_ARGUMENT, "layer_norm: expects const generic BLOCK_N");
    void *x = r.ptr("x"), *y = r.ptr("y"), *w = r.ptr("weight"), *b = r.ptr("bias");
    int64_t M = r.i32("M"), N = r.i32("N");
    float eps = r.f32("eps");
    if (r.done() != TEENY_OK) return r.st;
    return teeny_layer_norm_forward_inference(x, y, w, b, M, N, eps, dtype, stream);
  }

  // rms_norm_forward<BLOCK_N>(x, y, weight, rrms, M, N, eps)   rmsnorm.rs:39-47
  if (name_is(entry_point, "rms_norm_forward")) {
    TEENY_REQUIRE(n_cg == 1, TEENY_ERR_INVALID_ARGUMENT, "rms_norm: expects const generic BLOCK_N");
    void *x = r.ptr("x"), *y = r.ptr("y"), *w = r.ptr("weight"), *rr = r.ptr("rrms");
    int64_t M = r.i32("M"), N = r.i32("N");
    float eps = r.f32("eps");
    if (r.done() != TEENY_OK) return r.st;
    return teeny_rms_norm_forward(x, y, w, static_cast<float *>(rr), M, N, eps, dtype, stream);
  }

  // conv2d_forward<KH,KW,SH,SW,PH,PW,G,BLOCK_OW>(x, w, y, B, C_IN, C_OUT, H, W, OH, OW)
  // conv2d_bias_forward<...>(x, w, bias, y, ...)      conv2d.rs:543-562, :794-810
  const bool conv = name_is(entry_point, "conv2d_forward");
  const bool conv_bias = name_is(entry_point, "conv2d_bias_forward");
  if (conv || conv_bias) {
    TEENY_REQUIRE(n_cg == 8, TEENY_ERR_INVALID_ARGUMENT,
                  "conv2d: expects const generics KH,KW,STRIDE_H,STRIDE_W,PAD_H,PAD_W,G,BLOCK_OW");
    teeny_conv2d_params p;
    p.KH = static_cast<int32_t>(cg[0]);
    p.KW = static_cast<int32_t>(cg[1]);
    p.stride_h = static_cast<int32_t>(cg[2]);
    p.stride_w = static_cast<int32_t>(cg[3]);
    p.pad_h = static_cast<int32_t>(cg[4]);
    p.pad_w = static_cast<int32_t>(cg[5]);
    p.groups = static_cast<int32_t>(cg[6]);
    p.act = TEENY_ACT_NONE;
    void *x = r.ptr("x_ptr"), *w = r.ptr("w_ptr");
    void *bias = conv_bias ? r.ptr("bias_ptr") : nullptr;
    void *y = r.ptr("y_ptr");
    int64_t B = r.i32("B"), Ci = r.i32("C_IN"), Co = r.i32("C_OUT"), H = r.i32("H"),
            W = r.i32("W"), OH = r.i32("OH"), OW = r.i32("OW");
    if (r.done() != TEENY_OK) return r.st;
    if (conv_bias)
      return teeny_conv2d_bias_forward(x, w, bias, y, B, Ci, Co, H, W, OH, OW, &p, dtype,
                                       TEENY_NCHW, stream);
    return teeny_conv2d_forward(x, w, y, B, Ci, Co, H, W, OH, OW, &p, dtype, TEENY_NCHW, stream);
  }

  // flash_attention2_forward<HEAD_DIM[, CAUSAL]>(q, k, v, o, l, n_ctx_q, n_ctx_k, scale, neg_inf)
  // grid (N_CTX_Q, BH, 1)                                flash_attn2.rs:48-63
  // The reference kernel is non-causal; an optional second const generic
  // CAUSAL != 0 masks key j > query i.
  // multi_head_attention_forward<HEAD_DIM, CAUSAL, Q_HEADS, KV_HEADS>(same
  // arguments), grid (N_CTX_Q, BATCH * Q_HEADS, 1): the lowering target of
  // Op::MultiHeadAttention{q_num_heads, kv_num_heads} (core/teeny-core/src/
  // graph/mod.rs:1240-1246), a TODO arm of the reference's lowering
  // (kernels/teeny-kernels/src/graph/mod.rs:2477-2481); K/V carry KV_HEADS
  // heads per batch, shared by Q_HEADS / KV_HEADS query heads each.
  const bool fa = name_is(entry_point, "flash_attention2_forward");
  const bool mha = name_is(entry_point, "multi_head_attention_forward");
  if (fa || mha) {
    if (fa)
      TEENY_REQUIRE(n_cg == 1 || n_cg == 2, TEENY_ERR_INVALID_ARGUMENT,
                    "flash_attention2: expects const generics HEAD_DIM[, CAUSAL]");
    else
      TEENY_REQUIRE(n_cg == 4, TEENY_ERR_INVALID_ARGUMENT,
                    "multi_head_attention: expects const generics HEAD_DIM, CAUSAL, Q_HEADS, KV_HEADS");
    TEENY_REQUIRE(grid != nullptr, TEENY_ERR_NULL_POINTER, "attention: grid (BH = grid[1])");
    void *q = r.ptr("q_ptr"), *k = r.ptr("k_ptr"), *v = r.ptr("v_ptr"), *o = r.ptr("o_ptr"),
         *l = r.ptr("l_ptr");
    int64_t nq = r.i32("n_ctx_q"), nk = r.i32("n_ctx_k");
    float scale = r.f32("softmax_scale");
    r.f32("neg_inf");
    if (r.done() != TEENY_OK) return r.st;
    TEENY_REQUIRE(grid[0] == static_cast<uint32_t>(nq), TEENY_ERR_SHAPE_MISMATCH,
                  "attention: grid[0] must equal n_ctx_q");
    const int32_t causal = n_cg >= 2 && cg[1] != 0 ? 1 : 0;
    if (fa)
      return teeny_flash_attention2_forward(q, k, v, o, static_cast<float *>(l), nq, nk, scale,
                                            grid[1], cg[0], causal, dtype, stream);
    TEENY_REQUIRE(cg[2] > 0 && grid[1] % cg[2] == 0, TEENY_ERR_SHAPE_MISMATCH,
                  "multi_head_attention: grid[1] must be BATCH * Q_HEADS");
    return teeny_attention_forward(q, k, v, o, static_cast<float *>(l), grid[1] / cg[2], cg[2], cg[3], nq, nk,
                                   cg[0], scale, causal, dtype, stream);
  }

  // w8a16_linear_forward<USE_BIAS, ACT>(x, qweight, scale, bias, y, M, N, K): the
  // lowering target of Op::QLinearMatMul / Op::MatMulInteger with teeny-quant
  // per-output-channel int8 weights (TODO arms, graph/mod.rs:2595-2601); x bf16
  // [M, K], qweight int8 [N, K], scale / bias fp32 [N], y bf16 [M, N].
  if (name_is(entry_point, "w8a16_linear_forward")) {
    TEENY_REQUIRE(n_cg == 2, TEENY_ERR_INVALID_ARGUMENT, "w8a16_linear_forward: expects const generics USE_BIAS, ACT");
    void *x = r.ptr("x_ptr"), *q = r.ptr("qweight_ptr"), *sc = r.ptr("scale_ptr"), *b = r.ptr("bias_ptr"),
         *y = r.ptr("y_ptr");
    int64_t M = r.i32("M"), N = r.i32("N"), K = r.i32("K");
    if (r.done() != TEENY_OK) return r.st;
    TEENY_REQUIRE(dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE, "w8a16_linear_forward: dtype must be BF16");
    return teeny_w8a16_linear_forward(x, static_cast<const int8_t *>(q), static_cast<const float *>(sc),
                                      cg[0] ? static_cast<const float *>(b) : nullptr, y, M, N, K,
                                      static_cast<teeny_activation>(cg[1]), stream);
  }

  // w8a16_conv2d_forward<KH,KW,SH,SW,PH,PW,G,BLOCK_OW,USE_BIAS,ACT>(x, qweight,
  // scale, bias, y, B, C_IN, C_OUT, H, W, OH, OW): Op::QLinearConv /
  // Op::ConvInteger (TODO arms, graph/mod.rs:2595-2601) on NHWC bf16
  // activations and int8 weights [C_OUT, KH, KW, C_IN/G].
  if (name_is(entry_point, "w8a16_conv2d_forward")) {
    TEENY_REQUIRE(n_cg == 10, TEENY_ERR_INVALID_ARGUMENT,
                  "w8a16_conv2d_forward: expects const generics KH,KW,STRIDE_H,STRIDE_W,PAD_H,PAD_W,G,"
                  "BLOCK_OW,USE_BIAS,ACT");
    teeny_conv2d_params p;
    p.KH = static_cast<int32_t>(cg[0]);
    p.KW = static_cast<int32_t>(cg[1]);
    p.stride_h = static_cast<int32_t>(cg[2]);
    p.stride_w = static_cast<int32_t>(cg[3]);
    p.pad_h = static_cast<int32_t>(cg[4]);
    p.pad_w = static_cast<int32_t>(cg[5]);
    p.groups = static_cast<int32_t>(cg[6]);
    p.act = static_cast<int32_t>(cg[9]);
    void *x = r.ptr("x_ptr"), *q = r.ptr("qweight_ptr"), *sc = r.ptr("scale_ptr"), *b = r.ptr("bias_ptr"),
         *y = r.ptr("y_ptr");
    int64_t B = r.i32("B"), Ci = r.i32("C_IN"), Co = r.i32("C_OUT"), H = r.i32("H"), W = r.i32("W"),
            OH = r.i32("OH"), OW = r.i32("OW");
    if (r.done() != TEENY_OK) return r.st;
    TEENY_REQUIRE(dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE, "w8a16_conv2d_forward: dtype must be BF16");
    return teeny_w8a16_conv2d_forward(x, static_cast<const int8_t *>(q), static_cast<const float *>(sc),
                                      cg[8] ? static_cast<const float *>(b) : nullptr, y, B, Ci, Co, H, W, OH,
                                      OW, &p, stream);
  }

  // quantize_affine<GRANULARITY, AXIS, GROUP_SIZE, SYMMETRIC, BITS>(data, qvalues,
  // scales, zero_points, groups, ndim, dim_0 .. dim_{ndim-1}) and
  // dequantize_affine<GRANULARITY, AXIS, GROUP_SIZE>(qvalues, scales,
  // zero_points, out, ndim, dims...): teeny-quant's quantize_affine /
  // dequantize_affine (utilities/teeny-quant/src/quant/affine.rs:55-161), the
  // lowering targets of Op::QuantizeLinear / Op::DequantizeLinear (TODO arms,
  // graph/mod.rs:2691-2697).  Dims are i64 arguments.
  const bool quant = name_is(entry_point, "quantize_affine");
  const bool dequant = name_is(entry_point, "dequantize_affine");
  if (quant || dequant) {
    TEENY_REQUIRE(n_cg == (quant ? 5 : 3), TEENY_ERR_INVALID_ARGUMENT,
                  quant ? "quantize_affine: expects const generics GRANULARITY, AXIS, GROUP_SIZE, SYMMETRIC, BITS"
                        : "dequantize_affine: expects const generics GRANULARITY, AXIS, GROUP_SIZE");
    void *a0 = r.ptr(quant ? "data_ptr" : "qvalues_ptr");
    void *a1 = r.ptr(quant ? "qvalues_ptr" : "scales_ptr");
    void *a2 = r.ptr(quant ? "scales_ptr" : "zero_points_ptr");
    void *a3 = r.ptr(quant ? "zero_points_ptr" : "out_ptr");
    void *groups = quant ? r.ptr("groups_ptr") : nullptr;
    const int64_t ndim = r.i32("ndim");
    if (r.st != TEENY_OK) return r.st;
    TEENY_REQUIRE(ndim >= 0 && ndim <= 16, TEENY_ERR_INVALID_ARGUMENT, std::string(entry_point) + ": ndim in [0, 16]");
    int64_t shape[16];
    for (int64_t d = 0; d < ndim; ++d) shape[d] = r.take(TEENY_ARG_I64, "dim") ? args[r.i++].v.i64 : 0;
    if (r.done() != TEENY_OK) return r.st;
    if (quant) {
      TEENY_REQUIRE(dtype == TEENY_F32, TEENY_ERR_UNSUPPORTED_DTYPE, "quantize_affine: dtype is the input's, F32");
      return teeny_quantize_affine(static_cast<const float *>(a0), shape, static_cast<int32_t>(ndim),
                                   static_cast<teeny_granularity>(cg[0]), static_cast<int32_t>(cg[1]), cg[2],
                                   static_cast<int32_t>(cg[3]), static_cast<int32_t>(cg[4]),
                                   static_cast<int8_t *>(a1), static_cast<float *>(a2),
                                   static_cast<int32_t *>(a3), static_cast<uint32_t *>(groups), stream);
    }
    TEENY_REQUIRE(dtype == TEENY_F32, TEENY_ERR_UNSUPPORTED_DTYPE, "dequantize_affine: dtype is the output's, F32");
    return teeny_dequantize_affine(static_cast<const int8_t *>(a0), static_cast<const float *>(a1),
                                   static_cast<const int32_t *>(a2), shape, static_cast<int32_t>(ndim),
                                   static_cast<teeny_granularity>(cg[0]), static_cast<int32_t>(cg[1]), cg[2],
                                   static_cast<float *>(a3), stream);
  }

  // linear_forward<USE_BIAS,BLOCK_M,BLOCK_N,BLOCK_K,GROUP_M>(x, w, b, y, M, N, K,
  //   stride_xm, stride_xk, stride_wn, stride_wk, stride_ym, stride_yn)   linear.rs:297-311
  if (name_is(entry_point, "linear_forward")) {
    TEENY_REQUIRE(n_cg == 5, TEENY_ERR_INVALID_ARGUMENT,
                  "linear_forward: expects const generics USE_BIAS,BLOCK_M,BLOCK_N,BLOCK_K,GROUP_M");
    void *x = r.ptr("x_ptr"), *w = r.ptr("w_ptr"), *b = r.ptr("b_ptr"), *y = r.ptr("y_ptr");
    int64_t M = r.i32("M"), N = r.i32("N"), K = r.i32("K");
    int64_t sxm = r.i32("stride_xm"), sxk = r.i32("stride_xk"), swn = r.i32("stride_wn"),
            swk = r.i32("stride_wk"), sym = r.i32("stride_ym"), syn = r.i32("stride_yn");
    if (r.done() != TEENY_OK) return r.st;
    return teeny_linear_forward(x, w, cg[0] ? b : nullptr, y, M, N, K, sxm, sxk, swn, swk, sym,
                                syn, dtype, stream);
  }

  // linear_backward<USE_BIAS,BLOCK_M,BLOCK_N,BLOCK_K,GROUP_M>(x, w, dy, dx, dw, db, M, N, K,
  //   stride_xm, stride_xk, stride_wk, stride_wn, stride_dym, stride_dyn, stride_dxm, stride_dxk,
  //   stride_dwk, stride_dwn, stride_dbn)                                   linear.rs:118-150, :341-384
  if (name_is(entry_point, "linear_backward")) {
    TEENY_REQUIRE(n_cg == 5, TEENY_ERR_INVALID_ARGUMENT,
                  "linear_backward: expects const generics USE_BIAS,BLOCK_M,BLOCK_N,BLOCK_K,GROUP_M");
    void *x = r.ptr("x_ptr"), *w = r.ptr("w_ptr"), *dy = r.ptr("dy_ptr"), *dx = r.ptr("dx_ptr"),
         *dw = r.ptr("dw_ptr"), *db = r.ptr("db_ptr");
    int64_t M = r.i32("M"), N = r.i32("N"), K = r.i32("K");
    int64_t sxm = r.i32("stride_xm"), sxk = r.i32("stride_xk"), swk = r.i32("stride_wk"),
            swn = r.i32("stride_wn"), sdym = r.i32("stride_dym"), sdyn = r.i32("stride_dyn"),
            sdxm = r.i32("stride_dxm"), sdxk = r.i32("stride_dxk"), sdwk = r.i32("stride_dwk"),
            sdwn = r.i32("stride_dwn"), sdbn = r.i32("stride_dbn");
    if (r.done() != TEENY_OK) return r.st;
    return teeny_linear_backward(x, w, dy, dx, dw, cg[0] ? db : nullptr, M, N, K, sxm, sxk, swk, swn, sdym, sdyn,
                                 sdxm, sdxk, sdwk, sdwn, sdbn, dtype, stream);
  }

  // Conv + BatchNorm (folded scale / shift) + SiLU, the reference's three fused variants
  // (nn/fused/): fp32 NCHW, the activation fixed to SiLU.
  //   conv2d_bn_silu_forward<KH,KW,SH,SW,PH,PW,G,BLOCK_OW>(x, w, bn_scale, bn_shift, y,
  //     B, C_IN, C_OUT, H, W, OH, OW)                               conv2d_bn_silu.rs:40-64
  //   conv2d_bn_silu_gemm_forward<BLOCK_M,BLOCK_N,BLOCK_K,GROUP_M>(x, w, bn_scale, bn_shift,
  //     y, B, C_IN, C_OUT, M, y_row_stride): 1x1 stride 1, output rows of y_row_stride
  //                                                                 conv2d_bn_silu_gemm.rs:61-80
  //   conv2d_bn_silu_tiled_forward<KH,KW,SH,SW,PH,PW,BLOCK_OW,BLOCK_N>(x, w, bn_scale,
  //     bn_shift, y, B, C_IN, C_OUT, H, W, OH, OW, y_col_stride): groups 1, each oh row
  //     y_col_stride wide                                           conv2d_bn_silu_tiled.rs:49-78
  const bool bn_plain = name_is(entry_point, "conv2d_bn_silu_forward");
  const bool bn_gemm = name_is(entry_point, "conv2d_bn_silu_gemm_forward");
  const bool bn_tiled = name_is(entry_point, "conv2d_bn_silu_tiled_forward");
  if (bn_plain || bn_gemm || bn_tiled) {
    TEENY_REQUIRE(n_cg == (bn_gemm ? 4 : 8), TEENY_ERR_INVALID_ARGUMENT,
                  std::string(entry_point) + (bn_gemm ? ": expects const generics BLOCK_M,BLOCK_N,BLOCK_K,GROUP_M"
                                                      : ": expects 8 const generics"));
    teeny_conv2d_params p{1, 1, 1, 1, 0, 0, 1, TEENY_ACT_SILU};
    if (!bn_gemm) {
      p.KH = static_cast<int32_t>(cg[0]);
      p.KW = static_cast<int32_t>(cg[1]);
      p.stride_h = static_cast<int32_t>(cg[2]);
      p.stride_w = static_cast<int32_t>(cg[3]);
      p.pad_h = static_cast<int32_t>(cg[4]);
      p.pad_w = static_cast<int32_t>(cg[5]);
      p.groups = bn_plain ? static_cast<int32_t>(cg[6]) : 1;
    }
    void *x = r.ptr("x_ptr"), *w = r.ptr("w_ptr"), *sc = r.ptr("bn_scale_ptr"), *sh = r.ptr("bn_shift_ptr"),
         *y = r.ptr("y_ptr");
    int64_t B = r.i32("B"), Ci = r.i32("C_IN"), Co = r.i32("C_OUT");
    int64_t H, W, OH, OW, ys[4];
    if (bn_gemm) {
      const int64_t M = r.i32("M"), rs = r.i32("y_row_stride");
      H = OH = 1;
      W = OW = M;
      ys[0] = Co * rs;
      ys[1] = rs;
      ys[2] = rs;
      ys[3] = 1;
    } else {
      H = r.i32("H");
      W = r.i32("W");
      OH = r.i32("OH");
      OW = r.i32("OW");
      if (bn_tiled) {
        const int64_t cs = r.i32("y_col_stride");
        ys[0] = Co * OH * cs;
        ys[1] = OH * cs;
        ys[2] = cs;
        ys[3] = 1;
      }
    }
    if (r.done() != TEENY_OK) return r.st;
    return teeny_conv2d_bn_act_forward(x, w, static_cast<const float *>(sc), static_cast<const float *>(sh), y, B, Ci,
                                       Co, H, W, OH, OW, bn_plain ? nullptr : ys, &p, dtype, TEENY_NCHW, stream);
  }

  // ── training kernels ──
  // layer_norm_forward<BLOCK_N>(x, y, weight, bias, mean, rstd, M, N, eps)        layernorm.rs:163-172
  // layer_norm_backward<BLOCK_N>(dy, x, dx, weight, dweight, dbias, mean, rstd, M, N)  :301-311
  // rms_norm_backward<BLOCK_N>(dy, x, dx, weight, dweight, rrms, M, N)            rmsnorm.rs:136-144
  // The statistics and parameter gradients are fp32 buffers for every dtype.
  if (name_is(entry_point, "layer_norm_forward")) {
    TEENY_REQUIRE(n_cg == 1, TEENY_ERR_INVALID_ARGUMENT, "layer_norm_forward: expects const generic BLOCK_N");
    void *x = r.ptr("x"), *y = r.ptr("y"), *w = r.ptr("weight"), *b = r.ptr("bias"), *mean = r.ptr("mean"),
         *rstd = r.ptr("rstd");
    int64_t M = r.i32("M"), N = r.i32("N");
    float eps = r.f32("eps");
    if (r.done() != TEENY_OK) return r.st;
    return teeny_layer_norm_forward(x, y, w, b, static_cast<float *>(mean), static_cast<float *>(rstd), M, N, eps,
                                    dtype, stream);
  }
  if (name_is(entry_point, "layer_norm_backward")) {
    TEENY_REQUIRE(n_cg == 1, TEENY_ERR_INVALID_ARGUMENT, "layer_norm_backward: expects const generic BLOCK_N");
    void *dy = r.ptr("dy"), *x = r.ptr("x"), *dx = r.ptr("dx"), *w = r.ptr("weight"), *dw = r.ptr("dweight"),
         *db = r.ptr("dbias"), *mean = r.ptr("mean"), *rstd = r.ptr("rstd");
    int64_t M = r.i32("M"), N = r.i32("N");
    if (r.done() != TEENY_OK) return r.st;
    return teeny_layer_norm_backward(dy, x, dx, w, static_cast<float *>(dw), static_cast<float *>(db),
                                     static_cast<const float *>(mean), static_cast<const float *>(rstd), M, N, dtype,
                                     stream);
  }
  if (name_is(entry_point, "rms_norm_backward")) {
    TEENY_REQUIRE(n_cg == 1, TEENY_ERR_INVALID_ARGUMENT, "rms_norm_backward: expects const generic BLOCK_N");
    void *dy = r.ptr("dy"), *x = r.ptr("x"), *dx = r.ptr("dx"), *w = r.ptr("weight"), *dw = r.ptr("dweight"),
         *rr = r.ptr("rrms");
    int64_t M = r.i32("M"), N = r.i32("N");
    if (r.done() != TEENY_OK) return r.st;
    return teeny_rms_norm_backward(dy, x, dx, w, static_cast<float *>(dw), static_cast<const float *>(rr), M, N,
                                   dtype, stream);
  }

  // conv2d_backward_dx<KH,KW,SH,SW,PH,PW,G,BLOCK_OW>(dy, w, dx, B, C_IN, C_OUT, H, W, OH, OW)  conv2d.rs:172-196
  // conv2d_backward_dw<...>(dy, x, dw, B, C_IN, C_OUT, H, W, OH, OW)                         :287-311
  // conv2d_backward<...>(dy, x, w, dx, dw, B, C_IN, C_OUT, H, W, OH, OW)  (the Conv2d RuntimeOp's
  //   backward kernel, :400-425, :574-617); NCHW as conv2d_forward.
  const bool cbx = name_is(entry_point, "conv2d_backward_dx");
  const bool cbw = name_is(entry_point, "conv2d_backward_dw");
  const bool cb = name_is(entry_point, "conv2d_backward");
  if (cbx || cbw || cb) {
    TEENY_REQUIRE(n_cg == 8, TEENY_ERR_INVALID_ARGUMENT,
                  std::string(entry_point) + ": expects const generics KH,KW,STRIDE_H,STRIDE_W,PAD_H,PAD_W,G,BLOCK_OW");
    teeny_conv2d_params p;
    p.KH = static_cast<int32_t>(cg[0]);
    p.KW = static_cast<int32_t>(cg[1]);
    p.stride_h = static_cast<int32_t>(cg[2]);
    p.stride_w = static_cast<int32_t>(cg[3]);
    p.pad_h = static_cast<int32_t>(cg[4]);
    p.pad_w = static_cast<int32_t>(cg[5]);
    p.groups = static_cast<int32_t>(cg[6]);
    p.act = TEENY_ACT_NONE;
    void *dy = r.ptr("dy_ptr");
    void *x = cbx ? nullptr : r.ptr("x_ptr");
    void *w = cbw ? nullptr : r.ptr("w_ptr");
    void *dx = cbw ? nullptr : r.ptr("dx_ptr");
    void *dw = cbx ? nullptr : r.ptr("dw_ptr");
    int64_t B = r.i32("B"), Ci = r.i32("C_IN"), Co = r.i32("C_OUT"), H = r.i32("H"), W = r.i32("W"),
            OH = r.i32("OH"), OW = r.i32("OW");
    if (r.done() != TEENY_OK) return r.st;
    if (cbx) return teeny_conv2d_backward_dx(dy, w, dx, B, Ci, Co, H, W, OH, OW, &p, dtype, TEENY_NCHW, stream);
    if (cbw) return teeny_conv2d_backward_dw(dy, x, dw, B, Ci, Co, H, W, OH, OW, &p, dtype, TEENY_NCHW, stream);
    return teeny_conv2d_backward(dy, x, w, dx, dw, B, Ci, Co, H, W, OH, OW, &p, dtype, TEENY_NCHW, stream);
  }

  // flash_attention2_backward_dq<HEAD_DIM[, CAUSAL]>(q, k, v, o, do, l, dq, n_ctx_q, n_ctx_k,
  //   softmax_scale), grid (n_ctx_q, BH, 1)                           flash_attn2.rs:174-185
  // flash_attention2_backward_dkv<HEAD_DIM[, CAUSAL]>(q, k, v, o, do, l, dk, dv, n_ctx_q,
  //   n_ctx_k, softmax_scale), grid (n_ctx_k, BH, 1)                   :312-324
  const bool fdq = name_is(entry_point, "flash_attention2_backward_dq");
  const bool fdkv = name_is(entry_point, "flash_attention2_backward_dkv");
  if (fdq || fdkv) {
    TEENY_REQUIRE(n_cg == 1 || n_cg == 2, TEENY_ERR_INVALID_ARGUMENT,
                  std::string(entry_point) + ": expects const generics HEAD_DIM[, CAUSAL]");
    TEENY_REQUIRE(grid != nullptr, TEENY_ERR_NULL_POINTER, std::string(entry_point) + ": grid (BH = grid[1])");
    void *q = r.ptr("q_ptr"), *k = r.ptr("k_ptr"), *v = r.ptr("v_ptr"), *o = r.ptr("o_ptr"), *d_o = r.ptr("do_ptr"),
         *l = r.ptr("l_ptr");
    void *g0 = r.ptr(fdq ? "dq_ptr" : "dk_ptr");
    void *g1 = fdkv ? r.ptr("dv_ptr") : nullptr;
    int64_t nq = r.i32("n_ctx_q"), nk = r.i32("n_ctx_k");
    float scale = r.f32("softmax_scale");
    if (r.done() != TEENY_OK) return r.st;
    TEENY_REQUIRE(grid[0] == static_cast<uint32_t>(fdq ? nq : nk), TEENY_ERR_SHAPE_MISMATCH,
                  std::string(entry_point) + (fdq ? ": grid[0] must equal n_ctx_q" : ": grid[0] must equal n_ctx_k"));
    const int32_t causal = n_cg == 2 && cg[1] != 0 ? 1 : 0;
    if (fdq)
      return teeny_flash_attention2_backward_dq(q, k, v, o, d_o, static_cast<const float *>(l), g0, nq, nk, scale,
                                                grid[1], cg[0], causal, dtype, stream);
    return teeny_flash_attention2_backward_dkv(q, k, v, o, d_o, static_cast<const float *>(l), g0, g1, nq, nk, scale,
                                               grid[1], cg[0], causal, dtype, stream);
  }

  // pointwise_fuse_<m0>_<m1>..._entry_point(x, y, scratch_0 .. scratch_{n-2}, n_elements) and
  // pointwise_fuse_<tag>_backward_entry_point(dy, y, dx, scratch_0 .., n_elements): the
  // PointwiseFuse custom op's runtime ABI (graph/optimizer/ops/pointwise_fuse.rs:155-268);
  // the tag joins the members' kernel names without "_forward" (:315-321).
  {
    const char *pre = "pointwise_fuse_";
    const size_t lp = std::strlen(pre);
    if (std::strncmp(entry_point, pre, lp) == 0) {
      std::string tag(entry_point + lp);
      const std::string ep_suffix = "_entry_point";
      if (tag.size() > ep_suffix.size() && tag.compare(tag.size() - ep_suffix.size(), ep_suffix.size(), ep_suffix) == 0)
        tag.resize(tag.size() - ep_suffix.size());
      const std::string bwd_suffix = "_backward";
      const bool bwd =
          tag.size() > bwd_suffix.size() && tag.compare(tag.size() - bwd_suffix.size(), bwd_suffix.size(), bwd_suffix) == 0;
      if (bwd) tag.resize(tag.size() - bwd_suffix.size());
      int32_t ops[8];
      int32_t n_ops = 0;
      size_t at = 0;
      while (at <= tag.size()) {
        const size_t end = std::min(tag.find('_', at), tag.size());
        const std::string m = tag.substr(at, end - at);
        int32_t op = m == "relu" ? TEENY_PW_RELU : m == "gelu" ? TEENY_PW_GELU_TANH : m == "silu" ? TEENY_PW_SILU
                     : m == "sigmoid" ? TEENY_PW_SIGMOID : m == "tanh" ? TEENY_PW_TANH : 0;
        TEENY_REQUIRE(op != 0, TEENY_ERR_NOT_FOUND,
                      std::string("dispatch: pointwise_fuse member '") + m + "' has no fused kernel");
        TEENY_REQUIRE(n_ops < 8, TEENY_ERR_INVALID_ARGUMENT, "dispatch: pointwise_fuse: at most 8 members");
        ops[n_ops++] = op;
        at = end + 1;
      }
      TEENY_REQUIRE(n_ops >= 2, TEENY_ERR_INVALID_ARGUMENT, "dispatch: pointwise_fuse needs at least 2 members");
      void *a = r.ptr(bwd ? "dy_ptr" : "x_ptr");
      void *b = r.ptr("y_ptr");
      void *dx = bwd ? r.ptr("dx_ptr") : nullptr;
      void *scratch[8] = {nullptr};
      for (int32_t m = 0; m + 1 < n_ops; ++m) scratch[m] = r.ptr("scratch");
      const int64_t n = r.i32("n_elements");
      if (r.done() != TEENY_OK) return r.st;
      if (bwd) return teeny_pointwise_chain_backward(a, b, dx, scratch, ops, n_ops, n, dtype, stream);
      return teeny_pointwise_chain_forward(a, b, scratch, ops, n_ops, n, dtype, stream);
    }
  }

  return fail(TEENY_ERR_NOT_FOUND, std::string("dispatch: no operator for ") + entry_point);
}
