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
#include <cstring>

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

  // flash_attention2_forward<HEAD_DIM>(q, k, v, o, l, n_ctx_q, n_ctx_k, scale, neg_inf)
  // grid (N_CTX_Q, BH, 1)                                flash_attn2.rs:48-63
  if (name_is(entry_point, "flash_attention2_forward")) {
    TEENY_REQUIRE(n_cg == 1, TEENY_ERR_INVALID_ARGUMENT, "flash_attention2: expects const generic HEAD_DIM");
    TEENY_REQUIRE(grid != nullptr, TEENY_ERR_NULL_POINTER, "flash_attention2: grid (BH = grid[1])");
    void *q = r.ptr("q_ptr"), *k = r.ptr("k_ptr"), *v = r.ptr("v_ptr"), *o = r.ptr("o_ptr"),
         *l = r.ptr("l_ptr");
    int64_t nq = r.i32("n_ctx_q"), nk = r.i32("n_ctx_k");
    float scale = r.f32("softmax_scale");
    r.f32("neg_inf");
    if (r.done() != TEENY_OK) return r.st;
    TEENY_REQUIRE(grid[0] == static_cast<uint32_t>(nq), TEENY_ERR_SHAPE_MISMATCH,
                  "flash_attention2: grid[0] must equal n_ctx_q");
    return teeny_flash_attention2_forward(q, k, v, o, static_cast<float *>(l), nq, nk, scale,
                                          grid[1], cg[0], 0, dtype, stream);
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

  return fail(TEENY_ERR_NOT_FOUND, std::string("dispatch: no operator for ") + entry_point);
}
