/*
 * teeny_hip.h — C ABI of the MI355X (gfx950) teeny-kernels operator library.
 *
 * This header is the whole boundary between a host executor and the HIP
 * kernels.  It replaces two pieces of the reference:
 *
 *   1. the CUDA driver crate's device/buffer/stream/module/launch surface
 *      (drivers/teeny-cuda/src/device/mod.rs:212-490,
 *       drivers/teeny-cuda/src/device/buffer.rs:37-62), and
 *   2. the per-kernel C-ABI entry points that the #[kernel] macro generates as
 *      "{name}_entry_point" (macros/teeny-macros/src/macros/kernel.rs:781-803)
 *      for the hot-path operators in kernels/teeny-kernels/src/nn/ and the
 *      host-side int8 quantizer in utilities/teeny-quant/src/quant/affine.rs.
 *
 * Conventions (all functions):
 *   - Every function returns a teeny_status; 0 is success.  On failure the
 *     thread-local message behind teeny_hip_last_error() says what was wrong.
 *   - Operator entry points keep the reference kernel's argument order and
 *     meaning.  Compile-time generics of the reference (KH, KW, HEAD_DIM, ...)
 *     become trailing arguments, followed by a dtype (and layout where the op
 *     has one) and a stream.  Element counts and dimensions are int64_t where
 *     the reference used i32, so tensors beyond 2^31 elements are addressable.
 *   - Operators never allocate and never synchronize: work is enqueued on the
 *     given stream (NULL = the device's null stream).  Scratch, where a
 *     faster path wants it, is a caller-owned buffer attached to the stream
 *     (teeny_hip_stream_set_workspace).  Setting the
 *     environment variable TEENY_HIP_SYNC=1 makes every operator synchronize
 *     the stream after its launch, reproducing the reference executor's
 *     synchronize-after-every-launch behaviour
 *     (drivers/teeny-cuda/src/device/mod.rs:366-388).
 *   - Argument validation (null pointers, shapes, dtypes, alignment) happens
 *     on the host before any HIP call, so a rejected call has no effect on
 *     the device.
 *   - The caller owns every buffer (reference: LoadedModel owns params and
 *     intermediates, drivers/teeny-cuda/src/model/mod.rs:680-691).
 *   - Handles are plain HIP handles (hipStream_t, hipEvent_t, hipModule_t,
 *     hipFunction_t) passed as void*, so callers that already hold HIP
 *     objects can pass them directly.
 */
#ifndef TEENY_HIP_H
#define TEENY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ── status codes ─────────────────────────────────────────────────────────
 * Reference: anyhow::Result with Error::CudaError{code,message}
 * (drivers/teeny-cuda/src/errors.rs) for device failures, lowering errors for
 * unsupported dtypes (kernels/teeny-kernels/src/graph/mod.rs:164,194,208) and
 * teeny-quant's Error::{ShapeMismatch,InvalidAxis,InvalidGroupSize}
 * (utilities/teeny-quant/src/quant/affine.rs:62-87). */
typedef int32_t teeny_status;
#define TEENY_OK 0
#define TEENY_ERR_INVALID_ARGUMENT 1
#define TEENY_ERR_NULL_POINTER 2
#define TEENY_ERR_UNSUPPORTED_DTYPE 3
#define TEENY_ERR_SHAPE_MISMATCH 4
#define TEENY_ERR_MISALIGNED 5
#define TEENY_ERR_INVALID_AXIS 6
#define TEENY_ERR_INVALID_GROUP_SIZE 7
#define TEENY_ERR_NO_DEVICE 8
#define TEENY_ERR_HIP 9
#define TEENY_ERR_NOT_FOUND 10
#define TEENY_ERR_UNSUPPORTED 11

/* Element types.  TEENY_F32 is the reference's D = f32; TEENY_BF16 stores
 * IEEE bfloat16 (round-to-nearest-even on store, fp32 arithmetic inside every
 * kernel); TEENY_I8 is the int8 output of teeny-quant. */
typedef enum teeny_dtype {
  TEENY_F32 = 0,
  TEENY_BF16 = 1,
  TEENY_I8 = 2
} teeny_dtype;

/* Activation layouts for conv2d.  NCHW is the reference's only layout
 * (kernels/teeny-kernels/src/nn/conv/conv2d.rs:28-42): x [B,C_IN,H,W],
 * w [C_OUT,C_IN/G,KH,KW], y [B,C_OUT,OH,OW].  NHWC is this library's
 * MFMA layout: x [B,H,W,C_IN], w [C_OUT,KH,KW,C_IN/G], y [B,OH,OW,C_OUT]. */
typedef enum teeny_layout {
  TEENY_NCHW = 0,
  TEENY_NHWC = 1
} teeny_layout;

/* Elementwise epilogues that conv/norm entry points can fuse. */
typedef enum teeny_activation {
  TEENY_ACT_NONE = 0,
  TEENY_ACT_RELU = 1,
  TEENY_ACT_GELU_TANH = 2,
  TEENY_ACT_SILU = 3
} teeny_activation;

typedef void *teeny_stream;   /* hipStream_t */
typedef void *teeny_event;    /* hipEvent_t */
typedef void *teeny_module;   /* hipModule_t */
typedef void *teeny_function; /* hipFunction_t */
typedef void *teeny_graph;    /* hipGraphExec_t */

/* Message for the last failure on the calling thread ("" if none). */
const char *teeny_hip_last_error(void);
/* Static name of a status code. */
const char *teeny_status_string(teeny_status status);
/* Library version string. */
const char *teeny_hip_version(void);

/* ── device ───────────────────────────────────────────────────────────────
 * Reference: CudaDevice::try_new (cuDeviceGet, cuCtxCreate_v4),
 * drivers/teeny-cuda/src/device/mod.rs:225-262; teeny-runtime open(),
 * runtime/teeny-runtime/src/lib.rs:250-259. */
typedef struct teeny_device_info {
  char name[256];
  char arch[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;
  int32_t wavefront_size;
  int32_t clock_khz;
  int32_t memory_clock_khz;
  int32_t memory_bus_width;
  int32_t l2_cache_bytes;
  int64_t total_global_mem;
  int64_t shared_mem_per_block;
} teeny_device_info;

teeny_status teeny_hip_init(void);
teeny_status teeny_hip_device_count(int32_t *count);
/* Makes `ordinal` the calling thread's current device. */
teeny_status teeny_hip_device_open(int32_t ordinal);
teeny_status teeny_hip_device_info(int32_t ordinal, teeny_device_info *info);
teeny_status teeny_hip_device_synchronize(void);
teeny_status teeny_hip_device_close(int32_t ordinal);

/* ── device buffers ───────────────────────────────────────────────────────
 * Reference: device.buffer::<T>(n), to_device, to_host
 * (drivers/teeny-cuda/src/device/buffer.rs:37-62). */
teeny_status teeny_hip_malloc(void **ptr, size_t bytes);
teeny_status teeny_hip_free(void *ptr);
teeny_status teeny_hip_memcpy_h2d(void *dst, const void *src, size_t bytes, teeny_stream stream);
teeny_status teeny_hip_memcpy_d2h(void *dst, const void *src, size_t bytes, teeny_stream stream);
teeny_status teeny_hip_memcpy_d2d(void *dst, const void *src, size_t bytes, teeny_stream stream);
teeny_status teeny_hip_memset(void *dst, int32_t value, size_t bytes, teeny_stream stream);

/* ── streams and events ───────────────────────────────────────────────────
 * Reference: synchronous launches on the null stream plus CUDA-event timing in
 * CudaGraphModel::run_timed (drivers/teeny-cuda/src/model/mod.rs:1729-1797).
 * Streams are always created at the default priority. */
teeny_status teeny_hip_stream_create(teeny_stream *stream);
teeny_status teeny_hip_stream_destroy(teeny_stream stream);
teeny_status teeny_hip_stream_sync(teeny_stream stream);
/* Attaches a caller-owned device buffer (256-byte aligned) to a stream as
 * operator scratch; ptr NULL or bytes 0 detaches.  Operators never allocate:
 * the paths that need scratch -- split-K partial sums for GEMM and conv grids
 * too small to fill the device, the space-to-depth copy of stride-2 NHWC
 * convs whose C_IN is not a multiple of 8, and the bf16 copy of the int8
 * weights of W8A16 3x3 convs that run on the band-tiled kernel -- run only
 * when the stream's
 * workspace is large enough (sizes from teeny_linear_workspace_size and
 * teeny_conv2d_workspace_size), and otherwise the operator takes a path that
 * needs none.  Work on one stream runs in order, so every operator on it may
 * share the buffer; the buffer must outlive the work enqueued while it is
 * attached.  Destroying the stream detaches it.  Reference counterpart: none
 * (the reference's ops use no scratch; this mirrors cublasSetWorkspace). */
teeny_status teeny_hip_stream_set_workspace(teeny_stream stream, void *ptr, size_t bytes);
teeny_status teeny_hip_event_create(teeny_event *event);
teeny_status teeny_hip_event_destroy(teeny_event event);
teeny_status teeny_hip_event_record(teeny_event event, teeny_stream stream);
teeny_status teeny_hip_event_sync(teeny_event event);
teeny_status teeny_hip_event_elapsed_ms(float *ms, teeny_event start, teeny_event stop);

/* Graph capture of a stream's work: everything enqueued on `stream` between
 * begin and end (operators, raw launches, device-to-device copies) is
 * recorded instead of run, and end instantiates it as one executable graph
 * that teeny_hip_graph_launch replays with a single submission.  Operators
 * keep their buffers and plans from capture time.  Reference: the CUDA-graph
 * executor, cuStreamBeginCapture_v2 / cuStreamEndCapture /
 * cuGraphInstantiateWithFlags / cuGraphLaunch in LoadedModel::capture_graph
 * and CudaGraphModel::run (drivers/teeny-cuda/src/model/mod.rs:1245-1640,
 * :1693-1797).  The null stream cannot be captured. */
teeny_status teeny_hip_stream_begin_capture(teeny_stream stream);
teeny_status teeny_hip_stream_end_capture(teeny_stream stream, teeny_graph *graph);
teeny_status teeny_hip_graph_launch(teeny_graph graph, teeny_stream stream);
teeny_status teeny_hip_graph_destroy(teeny_graph graph);

/* ── code objects and raw launch ──────────────────────────────────────────
 * Reference: CudaProgram::try_from_ptx (cuModuleLoadDataEx) and
 * CudaDevice::launch_with_packer (cuLaunchKernel with a void** argument
 * array), drivers/teeny-cuda/src/device/program.rs:327-390 and
 * drivers/teeny-cuda/src/device/mod.rs:430-490.  Here the image is a gfx950
 * code object (.hsaco); no trailing Triton scratch pointers are appended. */
teeny_status teeny_hip_module_load(teeny_module *module, const char *path);
teeny_status teeny_hip_module_load_data(teeny_module *module, const void *image);
teeny_status teeny_hip_module_get_function(teeny_function *function, teeny_module module,
                                           const char *name);
teeny_status teeny_hip_module_unload(teeny_module module);
teeny_status teeny_hip_launch(teeny_function function, const uint32_t grid[3],
                              const uint32_t block[3], uint32_t shared_mem_bytes,
                              teeny_stream stream, void **args);

/* ── elementwise activations ──────────────────────────────────────────────
 * y[i] = f(x[i]) for i < n_elements; x and y may alias (in-place).
 *   relu:  max(x, 0)                      nn/activation/relu.rs:27-64
 *   gelu:  x / (1 + exp(-2c(x + 0.044715 x^3))), c = sqrt(2/pi)
 *                                         nn/activation/gelu.rs:31-78
 *   silu:  x * 1/(1 + exp(-x))            nn/activation/sigmoid.rs:119-158
 * Reference arguments: (x_ptr, y_ptr, n_elements).  dtype: F32 or BF16. */
teeny_status teeny_relu_forward(const void *x, void *y, int64_t n_elements, teeny_dtype dtype,
                                teeny_stream stream);
teeny_status teeny_gelu_forward(const void *x, void *y, int64_t n_elements, teeny_dtype dtype,
                                teeny_stream stream);
teeny_status teeny_silu_forward(const void *x, void *y, int64_t n_elements, teeny_dtype dtype,
                                teeny_stream stream);

/* ── activation gradients ─────────────────────────────────────────────────
 * dx[i] = dy[i] * f'(.) for i < n_elements; dx may alias dy or the saved tensor.
 *   relu:  dx = y > 0 ? dy : 0, y = the forward OUTPUT   nn/activation/relu.rs:67-117
 *   gelu:  inner = x + 0.044715 x^3, t = 2/(1 + exp(-2c inner)) - 1,
 *          dx = dy (0.5 (1 + t) + x 0.5 (1 - t^2) c (1 + 3*0.044715 x^2))
 *                                                        nn/activation/gelu.rs:81-139
 *   silu:  s = 1/(1 + exp(-x)), y = x s, dx = dy (s + y - y s)
 *                                                        nn/activation/sigmoid.rs:161-210
 * Reference arguments: (dy_ptr, y_ptr | x_ptr, dx_ptr, n_elements), as the RuntimeOps'
 * pack_backward_args visit them (relu.rs:156-172, gelu.rs:293-309, sigmoid.rs:424-440).
 * dtype: F32 or BF16. */
teeny_status teeny_relu_backward(const void *dy, const void *y, void *dx, int64_t n_elements,
                                 teeny_dtype dtype, teeny_stream stream);
teeny_status teeny_gelu_backward(const void *dy, const void *x, void *dx, int64_t n_elements,
                                 teeny_dtype dtype, teeny_stream stream);
teeny_status teeny_silu_backward(const void *dy, const void *x, void *dx, int64_t n_elements,
                                 teeny_dtype dtype, teeny_stream stream);

/* ── normalisation ────────────────────────────────────────────────────────
 * LayerNorm over the last dimension of a row-major [M, N] tensor:
 *   y = (x - mean) * rsqrt(var + eps) * weight + bias   (biased variance)
 * Reference: layer_norm_forward_inference(x, y, weight, bias, M, N, eps),
 * kernels/teeny-kernels/src/nn/norm/layernorm.rs:42-157, RuntimeOp :486-561.
 * x, y, weight, bias share `dtype` (F32 or BF16); statistics are fp32. */
teeny_status teeny_layer_norm_forward_inference(const void *x, void *y, const void *weight,
                                                const void *bias, int64_t M, int64_t N,
                                                float eps, teeny_dtype dtype,
                                                teeny_stream stream);

/* RMSNorm: rrms[m] = rsqrt(mean(x[m,:]^2) + eps), y = x * rrms * weight.
 * Reference: rms_norm_forward(x, y, weight, rrms, M, N, eps),
 * kernels/teeny-kernels/src/nn/norm/rmsnorm.rs:39-119.  rrms is always fp32
 * (for dtype F32 this is the reference's D); it may be NULL to skip it. */
teeny_status teeny_rms_norm_forward(const void *x, void *y, const void *weight, float *rrms,
                                    int64_t M, int64_t N, float eps, teeny_dtype dtype,
                                    teeny_stream stream);

/* LayerNorm training forward: the inference result plus the per-row
 * statistics the backward pass reads, mean[m] and rstd[m] =
 * rsqrt(var + eps) (fp32 for every dtype).  Reference: layer_norm_forward(x,
 * y, weight, bias, mean, rstd, M, N, eps), layernorm.rs:162-298. */
teeny_status teeny_layer_norm_forward(const void *x, void *y, const void *weight, const void *bias,
                                      float *mean, float *rstd, int64_t M, int64_t N, float eps,
                                      teeny_dtype dtype, teeny_stream stream);

/* LayerNorm backward.  Reference: layer_norm_backward(dy, x, dx, weight,
 * dweight, dbias, mean, rstd, M, N), layernorm.rs:300-482:
 *   xhat = (x - mean) * rstd, c1 = sum_n(dy * weight) / N,
 *   c2 = sum_n(dy * weight * xhat) / N,
 *   dx = rstd * weight * (dy - c1 - xhat * c2)       (the reference's formula,
 *        which is the gradient of the forward when weight == 1),
 *   dweight[n] += sum_m dy * xhat, dbias[n] += sum_m dy  (accumulated into
 *        the existing values, deterministically).
 * dy, x, dx, weight share `dtype` (F32 or BF16); mean, rstd, dweight, dbias
 * are fp32; dweight and/or dbias may be NULL to skip them.  With a stream
 * workspace of teeny_norm_backward_workspace_size bytes the parameter
 * gradients come from per-workgroup partials; without it from a second pass
 * over x and dy. */
teeny_status teeny_layer_norm_backward(const void *dy, const void *x, void *dx, const void *weight,
                                       float *dweight, float *dbias, const float *mean, const float *rstd,
                                       int64_t M, int64_t N, teeny_dtype dtype, teeny_stream stream);

/* RMSNorm backward.  Reference: rms_norm_backward(dy, x, dx, weight, dweight,
 * rrms, M, N), rmsnorm.rs:135-277:
 *   s = sum_n(dy * weight * x) / N, dx = rrms * weight * (dy - x * rrms^2 * s),
 *   dweight[n] += sum_m dy * x * rrms.   Types and workspace as above. */
teeny_status teeny_rms_norm_backward(const void *dy, const void *x, void *dx, const void *weight, float *dweight,
                                     const float *rrms, int64_t M, int64_t N, teeny_dtype dtype,
                                     teeny_stream stream);

/* Stream workspace that lets the norm backward ops take their fastest plan. */
teeny_status teeny_norm_backward_workspace_size(int64_t M, int64_t N, int32_t is_rms, teeny_dtype dtype,
                                                size_t *bytes);

/* ── fused pointwise chains ───────────────────────────────────────────────
 * The reference's PointwiseFuse custom op (kernels/teeny-kernels/src/graph/
 * optimizer/ops/pointwise_fuse.rs:73-233), built by the Anduin pass
 * (graph/optimizer/anduin.rs:27-60): members ops[0 .. n_ops-1] applied in
 * order in one pass, member i < n_ops-1 writing its output to scratch[i]
 * (the reference's scratch_i, kept for the backward walk; in the forward a
 * NULL scratch array or entry skips that store), the last member to y.
 * Values are rounded to `dtype` between members, so the chain equals the
 * members run as separate kernels.  Member arithmetic: relu.rs, gelu.rs,
 * sigmoid.rs (sigmoid, silu), tanh.rs forward kernels.  1 <= n_ops <= 8. */
typedef enum {
  TEENY_PW_RELU = 1,
  TEENY_PW_GELU_TANH = 2,
  TEENY_PW_SILU = 3,
  TEENY_PW_SIGMOID = 4,
  TEENY_PW_TANH = 5
} teeny_pointwise_op;

teeny_status teeny_pointwise_chain_forward(const void *x, void *y, void *const *scratch, const int32_t *ops,
                                           int32_t n_ops, int64_t n, teeny_dtype dtype, teeny_stream stream);
/* Reverse-mode walk of a chain whose members all have a y-style gradient
 * (relu, sigmoid, tanh; pointwise_fuse.rs:276-279, the reference's
 * lower_pointwise_fuse_backward): dx = dy, then for i = n_ops-1 .. 0
 * dx = grad_i(dx, y_i) with y_i = y (last member) or scratch[i]; dx may
 * alias dy. */
teeny_status teeny_pointwise_chain_backward(const void *dy, const void *y, void *dx, const void *const *scratch,
                                            const int32_t *ops, int32_t n_ops, int64_t n, teeny_dtype dtype,
                                            teeny_stream stream);

/* Fused norm + activation: one pass computing act(norm(x)).  No reference
 * counterpart as a single kernel: it is the composition of the two kernels
 * above with the activation kernels (the Anduin pointwise-fusion idea,
 * kernels/teeny-kernels/src/graph/optimizer/anduin.rs:27-60, applied to a
 * norm epilogue).  is_rms = 0: LayerNorm (bias used), 1: RMSNorm (bias
 * ignored, may be NULL). */
teeny_status teeny_norm_act_forward(const void *x, void *y, const void *weight, const void *bias,
                                    int64_t M, int64_t N, float eps, int32_t is_rms,
                                    teeny_activation act, teeny_dtype dtype, teeny_stream stream);

/* ── conv2d ───────────────────────────────────────────────────────────────
 * y[b,co,oh,ow] = sum_{ci in group(co), kh, kw} x[b,ci,oh*SH-PH+kh, ow*SW-PW+kw]
 *                 * w[co, ci - g*C_IN/G, kh, kw]  (+ bias[co])
 * with zero padding.  Reference: conv2d_forward / conv2d_bias_forward
 * (x, w, [bias,] y, B, C_IN, C_OUT, H, W, OH, OW) with const generics
 * KH, KW, STRIDE_H, STRIDE_W, PAD_H, PAD_W, G,
 * kernels/teeny-kernels/src/nn/conv/conv2d.rs:43-156 and :642-764.
 * BLOCK_OW is a reference tiling choice and has no counterpart here.
 * `act` fuses an activation after the bias (TEENY_ACT_NONE = reference).
 * Layout NCHW: any dtype (F32, BF16).  Layout NHWC: BF16 runs the MFMA
 * implicit-GEMM kernels (weights [C_OUT,KH,KW,C_IN/G]; grouped convs with
 * at least 16 output channels per group too, all groups in one launch);
 * F32 also accepted. */
typedef struct teeny_conv2d_params {
  int32_t KH, KW;
  int32_t stride_h, stride_w;
  int32_t pad_h, pad_w;
  int32_t groups;
  int32_t act; /* teeny_activation */
} teeny_conv2d_params;

teeny_status teeny_conv2d_forward(const void *x, const void *w, void *y, int64_t B, int64_t C_IN,
                                  int64_t C_OUT, int64_t H, int64_t W, int64_t OH, int64_t OW,
                                  const teeny_conv2d_params *params, teeny_dtype dtype,
                                  teeny_layout layout, teeny_stream stream);
teeny_status teeny_conv2d_bias_forward(const void *x, const void *w, const void *bias, void *y,
                                       int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H,
                                       int64_t W, int64_t OH, int64_t OW,
                                       const teeny_conv2d_params *params, teeny_dtype dtype,
                                       teeny_layout layout, teeny_stream stream);

/* conv2d_bias_forward with no allocation and no stream workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, results and plans as
 * teeny_conv2d_bias_forward given a large enough stream workspace, except
 * that the scratch of those plans (split-K partial sums, the space-to-depth
 * copy of stride-2 convs over few channels) is a fixed 32 MiB device array
 * inside the library, one per GPU, held until the process ends.  A shape
 * whose plan needs more than 32 MiB of scratch is rejected with
 * TEENY_ERR_UNSUPPORTED before anything is enqueued (no ResNet-50 layer at
 * batch 64 needs scratch at all).  Every call on one GPU shares that GPU's
 * array: calls that overlap in time on one GPU (different streams, or other
 * host threads) race on it, so serialize them.  Calls no hipMalloc/hipFree. */
teeny_status teeny_conv2d_bias_forward_noalloc(const void *x, const void *w, const void *bias, void *y,
                                               int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H,
                                               int64_t W, int64_t OH, int64_t OW,
                                               const teeny_conv2d_params *params, teeny_dtype dtype,
                                               teeny_layout layout, teeny_stream stream);

/* Conv + BatchNorm (inference) + activation, fused in the conv's epilogue:
 *   y[b,c,...] = act(bn_scale[c] * conv(x, w)[b,c,...] + bn_shift[c])
 * with the BatchNorm folded by the caller to bn_scale = gamma / sqrt(var +
 * eps), bn_shift = beta - bn_scale * mean (fp32 [C_OUT]), and act =
 * params->act.  Reference: conv2d_bn_silu_forward(x, w, bn_scale, bn_shift, y,
 * B, C_IN, C_OUT, H, W, OH, OW) (act SiLU), kernels/teeny-kernels/src/nn/
 * fused/conv2d_bn_silu.rs:26-199, and its GEMM (1x1) and tiled variants
 * conv2d_bn_silu_gemm.rs:61-260, conv2d_bn_silu_tiled.rs:49-293, whose
 * padded output rows are expressed here by `y_strides` (NCHW only: element
 * strides between consecutive b, c, oh, ow; NULL = tight).  Any dtype,
 * layout and groups, as teeny_conv2d_forward; bf16 NHWC (groups == 1, or
 * at least 16 output channels per group) runs on the MFMA implicit GEMM
 * with the affine and activation applied to the fp32 accumulator. */
teeny_status teeny_conv2d_bn_act_forward(const void *x, const void *w, const float *bn_scale, const float *bn_shift,
                                        void *y, int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H, int64_t W,
                                        int64_t OH, int64_t OW, const int64_t *y_strides,
                                        const teeny_conv2d_params *params, teeny_dtype dtype, teeny_layout layout,
                                        teeny_stream stream);

/* conv2d backward.  Reference: conv2d_backward_dx(dy, w, dx, B, C_IN, C_OUT,
 * H, W, OH, OW), conv2d_backward_dw(dy, x, dw, ...) and the combined
 * conv2d_backward(dy, x, w, dx, dw, ...) with conv2d_forward's const
 * generics, conv2d.rs:171-521 (the Conv2d RuntimeOp's backward kernel,
 * :575-617):
 *   dx[b,ci,ih,iw] = sum dy[b,co,oh,ow] * w[co,ci_local,kh,kw] over the
 *                    (co, kh, kw) with oh*SH - PH + kh = ih, ow*SW - PW + kw = iw
 *   dw[co,ci_local,kh,kw] = sum over (b, oh, ow) of dy * x at those positions.
 * The reference atomically adds into zero-initialised dx/dw; these write the
 * sums (same values for zero-initialised buffers, fixed summation order).
 * Any dtype (F32, BF16), layout, stride, padding and groups; dy has y's
 * layout, dw the weight layout of `layout`.  bf16 NHWC dx with groups == 1
 * runs on the MFMA implicit GEMM given a stream workspace of
 * teeny_conv2d_backward_workspace_size bytes (flipped weights and, for a
 * strided conv, dy spread to the stride). */
teeny_status teeny_conv2d_backward_dx(const void *dy, const void *w, void *dx, int64_t B, int64_t C_IN,
                                      int64_t C_OUT, int64_t H, int64_t W, int64_t OH, int64_t OW,
                                      const teeny_conv2d_params *params, teeny_dtype dtype, teeny_layout layout,
                                      teeny_stream stream);
teeny_status teeny_conv2d_backward_dw(const void *dy, const void *x, void *dw, int64_t B, int64_t C_IN,
                                      int64_t C_OUT, int64_t H, int64_t W, int64_t OH, int64_t OW,
                                      const teeny_conv2d_params *params, teeny_dtype dtype, teeny_layout layout,
                                      teeny_stream stream);
teeny_status teeny_conv2d_backward(const void *dy, const void *x, const void *w, void *dx, void *dw, int64_t B,
                                   int64_t C_IN, int64_t C_OUT, int64_t H, int64_t W, int64_t OH, int64_t OW,
                                   const teeny_conv2d_params *params, teeny_dtype dtype, teeny_layout layout,
                                   teeny_stream stream);
teeny_status teeny_conv2d_backward_workspace_size(int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H, int64_t W,
                                                  int64_t OH, int64_t OW, const teeny_conv2d_params *params,
                                                  teeny_dtype dtype, teeny_layout layout, size_t *bytes);

/* ── attention ────────────────────────────────────────────────────────────
 * O = softmax(Q K^T * softmax_scale) V per (batch*head), L = logsumexp of the
 * scaled scores (natural log).  Layout [BH, n_ctx, head_dim] row-major.
 * Reference: flash_attention2_forward(q, k, v, o, l, n_ctx_q, n_ctx_k,
 * softmax_scale, neg_inf) with const HEAD_DIM and grid (n_ctx_q, BH, 1),
 * kernels/teeny-kernels/src/nn/attention/flash_attn2.rs:52-158.  Here BH and
 * head_dim are arguments, neg_inf is internal, and `causal` != 0 masks key j
 * from query i when j > i (top-left aligned, as torch's is_causal).
 * l is fp32 for every dtype and may be NULL.  head_dim 16, 32, 64, 128 or
 * 256 for both dtypes.  dtype BF16 at head_dim 64 and 128 runs the MFMA flash
 * kernel, which needs 16-byte aligned q/k/v/o and one head's K (and V) below
 * 2 GiB (n_ctx_k * head_dim * 2 bytes; TEENY_ERR_SHAPE_MISMATCH otherwise);
 * the other bf16 head sizes and fp32 run the reference's per-query-row
 * structure (fp32 arithmetic on bf16 operands). */
teeny_status teeny_flash_attention2_forward(const void *q, const void *k, const void *v, void *o,
                                            float *l, int64_t n_ctx_q, int64_t n_ctx_k,
                                            float softmax_scale, int64_t BH, int64_t head_dim,
                                            int32_t causal, teeny_dtype dtype,
                                            teeny_stream stream);

/* Multi-head attention with grouped K/V heads: the lowering target of the
 * reference's Op::MultiHeadAttention{q_num_heads, kv_num_heads}
 * (core/teeny-core/src/graph/mod.rs:1240-1246), a TODO arm of its lowering
 * (kernels/teeny-kernels/src/graph/mod.rs:2477-2481).  q/o are
 * [batch * q_heads, n_ctx_q, head_dim], k/v [batch * kv_heads, n_ctx_k,
 * head_dim]; query head h of a batch attends with K/V head
 * h / (q_heads / kv_heads) (q_heads a multiple of kv_heads; equal counts are
 * ordinary multi-head attention).  Otherwise as
 * teeny_flash_attention2_forward, which is this function with batch = BH and
 * q_heads = kv_heads = 1. */
teeny_status teeny_attention_forward(const void *q, const void *k, const void *v, void *o, float *l,
                                     int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t n_ctx_q,
                                     int64_t n_ctx_k, int64_t head_dim, float softmax_scale,
                                     int32_t causal, teeny_dtype dtype, teeny_stream stream);

/* Attention backward.  Reference: flash_attention2_backward_dq(q, k, v, o,
 * do, l, dq, n_ctx_q, n_ctx_k, softmax_scale) with grid (n_ctx_q, BH, 1) and
 * flash_attention2_backward_dkv(q, k, v, o, do, l, dk, dv, n_ctx_q, n_ctx_k,
 * softmax_scale) with grid (n_ctx_k, BH, 1), kernels/teeny-kernels/src/nn/
 * attention/flash_attn2.rs:173-447:
 *   D_m = sum_d o[m,d] do[m,d],  p_mn = exp(scale q_m . k_n - l_m),
 *   ds_mn = p_mn (do_m . v_n - D_m),
 *   dq_m = scale sum_n ds_mn k_n,  dk_n = scale sum_m ds_mn q_m,
 *   dv_n = sum_m p_mn do_m.
 * Shapes and dtypes as the forward (l is the forward's fp32 logsumexp, `dout`
 * the reference's do); `causal` as the forward (the reference is
 * non-causal).  No atomics: each output row is written once.  bf16 with
 * head_dim 64 / 128 and 16-byte aligned tensors runs on the MFMA kernels
 * (dkv needs a stream workspace of teeny_attention_backward_workspace_size
 * bytes for its D_m pre-pass, else it takes the per-row kernel); fp32 and
 * any other head_dim in {16, 32, 64, 128, 256} run the reference's per-row
 * structure. */
teeny_status teeny_flash_attention2_backward_dq(const void *q, const void *k, const void *v, const void *o,
                                                const void *dout, const float *l, void *dq, int64_t n_ctx_q,
                                                int64_t n_ctx_k, float softmax_scale, int64_t BH, int64_t head_dim,
                                                int32_t causal, teeny_dtype dtype, teeny_stream stream);
teeny_status teeny_flash_attention2_backward_dkv(const void *q, const void *k, const void *v, const void *o,
                                                 const void *dout, const float *l, void *dk, void *dv,
                                                 int64_t n_ctx_q, int64_t n_ctx_k, float softmax_scale, int64_t BH,
                                                 int64_t head_dim, int32_t causal, teeny_dtype dtype,
                                                 teeny_stream stream);
/* dq, dk and dv in one call, with grouped K/V heads as teeny_attention_forward
 * (dk/dv of a K/V head sum over the query heads that share it).  It needs no
 * workspace: without one, D_m is parked in dq's memory until the dq kernel
 * overwrites it. */
teeny_status teeny_attention_backward(const void *q, const void *k, const void *v, const void *o, const void *dout,
                                      const float *l, void *dq, void *dk, void *dv, int64_t batch, int64_t q_heads,
                                      int64_t kv_heads, int64_t n_ctx_q, int64_t n_ctx_k, int64_t head_dim,
                                      float softmax_scale, int32_t causal, teeny_dtype dtype, teeny_stream stream);
/* batch * q_heads * n_ctx_q fp32 values (the D_m of every query row). */
teeny_status teeny_attention_backward_workspace_size(int64_t batch, int64_t q_heads, int64_t n_ctx_q,
                                                     size_t *bytes);

/* ── int8 affine quantization (teeny-quant) ───────────────────────────────
 * Reference: quantize_affine(tensor, data, shape, granularity, symmetric,
 * bits) and dequantize_affine, utilities/teeny-quant/src/quant/affine.rs
 * :55-161, groups from assign_groups (quant/groups.rs:78-100).
 *   q = clamp(round_half_away(x / scale) + zero_point, qmin, qmax)
 *   symmetric:  scale = amax == 0 ? 1 : amax / qmax, zero_point = 0
 *   asymmetric: scale = hi == lo ? 1 : (hi - lo) / (qmax - qmin),
 *               zero_point = clamp(round_half_away(qmin - lo / scale))
 * with lo = min(min(x), 0), hi = max(max(x), 0) per group, qmax = 2^(bits-1)-1,
 * qmin = -qmax (symmetric) or -qmax-1.  Bit-exact with the reference. */
typedef enum teeny_granularity {
  TEENY_PER_TENSOR = 0,
  TEENY_PER_CHANNEL = 1, /* one group per index along `axis` */
  TEENY_GROUP = 2        /* group_size-runs along `axis`, other axes independent */
} teeny_granularity;

/* Number of groups for a shape/granularity (reference assign_groups). */
teeny_status teeny_quant_num_groups(const int64_t *shape, int32_t ndim,
                                    teeny_granularity granularity, int32_t axis,
                                    int64_t group_size, int64_t *num_groups);

/* data: fp32 [prod(shape)] on device.  Outputs on device: qvalues int8
 * [prod(shape)], scales fp32 [num_groups], zero_points int32 [num_groups]
 * (all three required; scales and zero_points also serve as the min/max
 * reduction space), groups uint32 [prod(shape)] optional (NULL = skip).
 * bits in [2, 8]. */
teeny_status teeny_quantize_affine(const float *data, const int64_t *shape, int32_t ndim,
                                   teeny_granularity granularity, int32_t axis,
                                   int64_t group_size, int32_t symmetric, int32_t bits,
                                   int8_t *qvalues, float *scales, int32_t *zero_points,
                                   uint32_t *groups, teeny_stream stream);

/* out[i] = (q[i] - zero_point[g(i)]) * scale[g(i)] in fp32; zero_points may
 * be NULL for symmetric tensors. */
teeny_status teeny_dequantize_affine(const int8_t *qvalues, const float *scales,
                                     const int32_t *zero_points, const int64_t *shape,
                                     int32_t ndim, teeny_granularity granularity, int32_t axis,
                                     int64_t group_size, float *out, teeny_stream stream);

/* ── linear / W8A16 ───────────────────────────────────────────────────────
 * y[m,n] = sum_k x[m,k] * w[n,k] (+ b[n]).  Reference: linear_forward(x, w,
 * b, y, M, N, K, stride_xm, stride_xk, stride_wn, stride_wk, stride_ym,
 * stride_yn), kernels/teeny-kernels/src/nn/mlp/linear.rs:20-116; b may be
 * NULL (USE_BIAS = false).  dtype F32 or BF16 (x, w, b, y share it). */
teeny_status teeny_linear_forward(const void *x, const void *w, const void *b, void *y,
                                  int64_t M, int64_t N, int64_t K, int64_t stride_xm,
                                  int64_t stride_xk, int64_t stride_wn, int64_t stride_wk,
                                  int64_t stride_ym, int64_t stride_yn, teeny_dtype dtype,
                                  teeny_stream stream);

/* Gradients of linear_forward.  Reference: linear_backward(x, w, dy, dx, dw,
 * db, M, N, K, stride_xm, stride_xk, stride_wk, stride_wn, stride_dym,
 * stride_dyn, stride_dxm, stride_dxk, stride_dwk, stride_dwn, stride_dbn),
 * kernels/teeny-kernels/src/nn/mlp/linear.rs:118-250 (RuntimeOp hooks
 * :324-385): dx [M,K] = dy W, dw [N,K] = dy^T x, db [N] = sum over m of dy
 * (db NULL: USE_BIAS = false).  All three are written, not accumulated.
 * dtype F32 or BF16 (every tensor shares it), fp32 accumulation.  Contiguous
 * bf16 operands with N and K multiples of 8 run on the matrix cores (as the
 * gradients of a 1x1 convolution; faster with a stream workspace of
 * teeny_linear_backward_workspace_size bytes); any strides take a tiled
 * fp32-accumulating kernel. */
teeny_status teeny_linear_backward(const void *x, const void *w, const void *dy, void *dx, void *dw, void *db,
                                   int64_t M, int64_t N, int64_t K, int64_t stride_xm, int64_t stride_xk,
                                   int64_t stride_wk, int64_t stride_wn, int64_t stride_dym, int64_t stride_dyn,
                                   int64_t stride_dxm, int64_t stride_dxk, int64_t stride_dwk, int64_t stride_dwn,
                                   int64_t stride_dbn, teeny_dtype dtype, teeny_stream stream);
teeny_status teeny_linear_backward_workspace_size(int64_t M, int64_t N, int64_t K, teeny_dtype dtype,
                                                  size_t *bytes);

/* Stream workspace (teeny_hip_stream_set_workspace) that lets linear_forward
 * (dtype F32/BF16, contiguous operands) or w8a16_linear_forward (dtype I8)
 * take its fastest plan at this shape; 0 if it uses none. */
teeny_status teeny_linear_workspace_size(int64_t M, int64_t N, int64_t K, teeny_dtype dtype,
                                         size_t *bytes);

/* W8A16 linear: y[m,n] = scale[n] * sum_k x[m,k] * q[n,k] (+ bias[n]).
 * x bf16 [M,K] row-major, q int8 [N,K] row-major (teeny-quant per-channel
 * axis-0 symmetric output), scale fp32 [N], bias fp32 [N] or NULL, y bf16
 * [M,N].  Equals linear_forward on dequantize_affine's weights
 * (utilities/teeny-quant/src/quant/affine.rs:151-161): int8 is exact in bf16,
 * so the dequant is q -> bf16 in registers and the scale is applied to the
 * fp32 accumulator.  act: fused epilogue activation. */
teeny_status teeny_w8a16_linear_forward(const void *x, const int8_t *qweight, const float *scale,
                                        const float *bias, void *y, int64_t M, int64_t N,
                                        int64_t K, teeny_activation act, teeny_stream stream);

/* W8A16 conv2d, NHWC bf16 activations, int8 weights [C_OUT,KH,KW,C_IN/G]
 * with per-output-channel fp32 scale, fp32 bias or NULL, bf16 output:
 * conv2d_bias_forward (conv2d.rs:642-764) on dequantize_affine's weights.
 * With the workspace teeny_conv2d_workspace_size reports (dtype I8), the
 * 3x3 shapes of the band-tiled kernel run on a bf16 copy of the int8 values
 * made there (exact; the scale multiplies the accumulator either way);
 * without it they take the int8 implicit GEMM. */
teeny_status teeny_w8a16_conv2d_forward(const void *x, const int8_t *qweight, const float *scale,
                                        const float *bias, void *y, int64_t B, int64_t C_IN,
                                        int64_t C_OUT, int64_t H, int64_t W, int64_t OH,
                                        int64_t OW, const teeny_conv2d_params *params,
                                        teeny_stream stream);

/* Stream workspace that lets conv2d_forward / conv2d_bias_forward (dtype
 * F32/BF16) or w8a16_conv2d_forward (dtype I8, layout NHWC) take its fastest
 * plan at this shape; 0 if it uses none. */
teeny_status teeny_conv2d_workspace_size(int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H, int64_t W,
                                         int64_t OH, int64_t OW, const teeny_conv2d_params *params,
                                         teeny_dtype dtype, teeny_layout layout, size_t *bytes);

/* ── compressed-tensors int8 checkpoints ──────────────────────────────────
 * Reference: teeny-quant's checkpoint convention, utilities/teeny-quant/src/
 * format.rs:16-35 (foo.weight I8 in the tensor's shape, foo.weight_scale F32
 * per group, foo.weight_zero_point I32 for asymmetric schemes), the
 * quantization_config JSON in the safetensors __metadata__ (:52-126) and
 * its reader dequantize_tensor (:249-289).  A checkpoint is opened read-only
 * (memory-mapped) and its whole header is validated on open: every offset,
 * shape and dtype is checked against the file before any tensor is touched,
 * so a malformed file fails with TEENY_ERR_INVALID_ARGUMENT.  Handles are
 * not thread-safe for concurrent close. */
typedef void *teeny_checkpoint;

typedef struct teeny_tensor_info {
  char name[256];
  char dtype[16];       /* safetensors dtype name: "I8", "F32", "BF16", ... */
  int32_t ndim;
  int32_t pad_;
  int64_t shape[8];
  uint64_t nbytes;
} teeny_tensor_info;

typedef struct teeny_quant_scheme {
  int32_t present;      /* 0: the file has no quantization_config */
  int32_t num_bits;
  int32_t symmetric;
  int32_t granularity;  /* teeny_granularity of "strategy", -1 if unknown */
  int64_t axis;         /* -1 when absent */
  int64_t group_size;   /* 0 when absent */
  int32_t n_config_groups;
  char quant_method[64];
  char format[64];      /* "int-quantized", "pack-quantized", "float-quantized" */
  char type[16];        /* "int" or "float" */
} teeny_quant_scheme;

teeny_status teeny_checkpoint_open(const char *path, teeny_checkpoint *ckpt);
/* The same over a caller-owned in-memory image, which must outlive the handle. */
teeny_status teeny_checkpoint_open_image(const void *data, size_t size, teeny_checkpoint *ckpt);
teeny_status teeny_checkpoint_close(teeny_checkpoint ckpt);
teeny_status teeny_checkpoint_num_tensors(teeny_checkpoint ckpt, int64_t *n);
teeny_status teeny_checkpoint_tensor_info(teeny_checkpoint ckpt, int64_t index, teeny_tensor_info *info);
/* Index of tensor `name`; TEENY_ERR_NOT_FOUND if absent. */
teeny_status teeny_checkpoint_find(teeny_checkpoint ckpt, const char *name, int64_t *index);
teeny_status teeny_checkpoint_quant_scheme(teeny_checkpoint ckpt, teeny_quant_scheme *scheme);
/* Copies tensor `index`'s raw little-endian bytes (exactly its nbytes) to
 * host memory (to_device = 0) or device memory (1, completed before return). */
teeny_status teeny_checkpoint_read(teeny_checkpoint ckpt, int64_t index, void *dst, size_t bytes,
                                   int32_t to_device, teeny_stream stream);
/* W8A16 operands of layer `weight_name` ("foo.weight"): requires an 8-bit
 * symmetric int-quantized compressed-tensors scheme with per-output-channel
 * (axis 0) or per-tensor scales, foo.weight I8 of rank >= 2 (flattened to
 * [N, K] with N its first dimension) and foo.weight_scale F32 with N (or 1)
 * entries.  Other schemes are TEENY_ERR_UNSUPPORTED (read the tensors and use
 * teeny_dequantize_affine).  _shape reports N and K; _load copies the int8
 * weights to qweight [N, K] and N fp32 scales (a per-tensor scale repeated)
 * to scale, both device buffers, ready for teeny_w8a16_linear_forward.  A
 * rank-4 weight is a conv weight stored in the reference's order [C_OUT,
 * C_IN/G, KH, KW] (conv2d.rs:43-156); _load repacks it to [C_OUT, KH, KW,
 * C_IN/G], the layout teeny_w8a16_conv2d_forward reads. */
teeny_status teeny_checkpoint_w8a16_shape(teeny_checkpoint ckpt, const char *weight_name, int64_t *N,
                                          int64_t *K);
teeny_status teeny_checkpoint_load_w8a16(teeny_checkpoint ckpt, const char *weight_name, int8_t *qweight,
                                         float *scale, int64_t N, int64_t K, teeny_stream stream);

/* ── reference-shaped dispatch ────────────────────────────────────────────
 * Runs an operator from exactly the argument list that the reference's
 * RuntimeOp::pack_args visits (core/teeny-core/src/model/mod.rs:78-331,
 * ArgVisitor core/teeny-core/src/device/program.rs:22-46), the kernel's
 * const generics in declaration order, and the launch grid from
 * RuntimeOp::grid.  This lets an executor written against the reference
 * contract (LoadedModel::forward, drivers/teeny-cuda/src/model/mod.rs:524-700)
 * call this library in place of cuLaunchKernel.  Entry point names are the
 * reference's "{name}_entry_point" symbols, e.g.
 * "conv2d_bias_forward_entry_point".  Names served (argument lists as the
 * matching RuntimeOp packs them): relu/gelu/silu_forward and _backward,
 * layer_norm_forward_inference, rms_norm_forward, conv2d_forward,
 * conv2d_bias_forward, flash_attention2_forward (HEAD_DIM[, CAUSAL]),
 * linear_forward, and for the reference's TODO lowering arms
 * multi_head_attention_forward, w8a16_linear_forward, w8a16_conv2d_forward,
 * quantize_affine and dequantize_affine (dims as TEENY_ARG_I64). */
typedef enum teeny_arg_kind {
  TEENY_ARG_PTR = 0,
  TEENY_ARG_I32 = 1,
  TEENY_ARG_I64 = 2,
  TEENY_ARG_F32 = 3,
  TEENY_ARG_F64 = 4,
  TEENY_ARG_U32 = 5,
  TEENY_ARG_BOOL = 6
} teeny_arg_kind;

typedef struct teeny_arg {
  int32_t kind; /* teeny_arg_kind */
  int32_t pad_;
  union {
    void *ptr;
    int32_t i32;
    int64_t i64;
    float f32;
    double f64;
    uint32_t u32;
    int32_t b;
  } v;
} teeny_arg;

teeny_status teeny_dispatch(const char *entry_point, const int64_t *const_generics,
                            int32_t n_const_generics, const teeny_arg *args, int32_t n_args,
                            const uint32_t grid[3], teeny_dtype dtype, teeny_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* TEENY_HIP_H */
