/*
 * teeny_oracle.c — CPU restatement of the reference's teeny-kernels hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  No product code path calls it.
 *
 * Each function restates one reference kernel in plain C, fp32, following
 * that kernel's program-id decomposition and per-program loop, so that its
 * arithmetic (operation order, accumulation type, masking) is the
 * reference's.  Programs are spread over host threads the way the
 * reference's CPU launcher spreads them (drivers/teeny-riscv/src/native.rs
 * :305-374): threads = TEENY_CPU_THREADS or all online cores; program ids
 * are taken from an atomic counter in chunks of max(total / (threads*8), 1).
 *
 * Every function takes a program range [pid_begin, pid_end) so that a caller
 * can run a prefix (CPU-baseline sampling) or the full grid (pid_end < 0).
 * Status codes match include/teeny_hip.h.
 */
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define OK 0
#define ERR_INVALID_ARGUMENT 1
#define ERR_SHAPE_MISMATCH 4
#define ERR_INVALID_AXIS 6
#define ERR_INVALID_GROUP_SIZE 7

/* ── threaded launcher (native.rs:305-374) ─────────────────────────────── */

typedef void (*program_fn)(const void *ctx, int64_t pid);

typedef struct {
  program_fn fn;
  const void *ctx;
  int64_t begin, end, chunk;
  atomic_llong next;
} launch_t;

static int g_threads_override = 0;

int oracle_set_threads(int n) {
  g_threads_override = n > 0 ? n : 0;
  return OK;
}

int oracle_threads(void) {
  if (g_threads_override > 0) return g_threads_override;
  const char *v = getenv("TEENY_CPU_THREADS");
  if (v != NULL && atoi(v) > 0) return atoi(v);
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

static void *worker(void *arg) {
  launch_t *L = (launch_t *)arg;
  for (;;) {
    int64_t start = atomic_fetch_add(&L->next, L->chunk);
    if (start >= L->end) break;
    int64_t stop = start + L->chunk < L->end ? start + L->chunk : L->end;
    for (int64_t pid = start; pid < stop; ++pid) L->fn(L->ctx, pid);
  }
  return NULL;
}

static void launch(program_fn fn, const void *ctx, int64_t total, int64_t begin, int64_t end) {
  if (end < 0 || end > total) end = total;
  if (begin < 0) begin = 0;
  if (begin >= end) return;
  int64_t n = end - begin;
  int64_t threads = oracle_threads();
  if (threads > n) threads = n;
  if (threads < 1) threads = 1;
  launch_t L;
  L.fn = fn;
  L.ctx = ctx;
  L.begin = begin;
  L.end = end;
  L.chunk = n / (threads * 8) > 1 ? n / (threads * 8) : 1;
  atomic_init(&L.next, begin);
  if (threads == 1) {
    worker(&L);
    return;
  }
  pthread_t *tids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  for (int64_t t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, worker, &L);
  for (int64_t t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
  free(tids);
}

/* ── activations ─────────────────────────────────────────────────────────
 * relu.rs:27-64, gelu.rs:31-78, sigmoid.rs:119-158: program pid covers
 * offsets [pid*BLOCK_SIZE, pid*BLOCK_SIZE + BLOCK_SIZE) masked by n. */

typedef struct {
  const float *x;
  float *y;
  int64_t n;
  int64_t block;
  int kind;
} act_ctx;

static float gelu_ref(float x) {
  /* gelu.rs:53-64: one = 1, neg2c = -2*0.7978845608028654, coeff = 0.044715
   * inner = x + coeff*x*x*x ; y = x / (one + exp(neg2c * inner)) */
  const float one = 1.0f;
  const float neg2c = (float)(-2.0 * 0.7978845608028654);
  const float coeff = 0.044715f;
  float inner = x + coeff * x * x * x;
  return x / (one + expf(neg2c * inner));
}

static float silu_ref(float x) {
  /* sigmoid.rs:144-148: s = one / (one + exp(neg1 * x)); y = x * s */
  const float one = 1.0f, neg1 = -1.0f;
  float s = one / (one + expf(neg1 * x));
  return x * s;
}

static float relu_ref(float x) {
  /* relu.rs:52-53: maximum(x, zeros_like(x)); NaN propagates. */
  return x < 0.0f ? 0.0f : x;
}

static float sigmoid_ref(float x) {
  /* sigmoid.rs (sigmoid_forward): y = one / (one + exp(neg1 * x)) */
  const float one = 1.0f, neg1 = -1.0f;
  return one / (one + expf(neg1 * x));
}

static float tanh_ref(float x) {
  /* tanh.rs (tanh_forward): s2x = one / (one + exp(neg2 * x)); y = two * s2x - one */
  const float one = 1.0f, two = 2.0f, neg2 = -2.0f;
  float s2x = one / (one + expf(neg2 * x));
  return two * s2x - one;
}

static float act_ref(int kind, float v) {
  switch (kind) {
    case 0: return relu_ref(v);
    case 1: return gelu_ref(v);
    case 2: return silu_ref(v);
    case 3: return sigmoid_ref(v);
    default: return tanh_ref(v);
  }
}

static void act_program(const void *c, int64_t pid) {
  const act_ctx *a = (const act_ctx *)c;
  int64_t start = pid * a->block;
  for (int64_t i = start; i < start + a->block && i < a->n; ++i) a->y[i] = act_ref(a->kind, a->x[i]);
}

static int act_run(const float *x, float *y, int64_t n, int64_t block, int kind, int64_t pb,
                   int64_t pe) {
  if (n < 0 || block <= 0) return ERR_SHAPE_MISMATCH;
  act_ctx a = {x, y, n, block, kind};
  launch(act_program, &a, (n + block - 1) / block, pb, pe);
  return OK;
}

int oracle_relu_forward(const float *x, float *y, int64_t n, int64_t block_size, int64_t pb,
                        int64_t pe) {
  return act_run(x, y, n, block_size, 0, pb, pe);
}
int oracle_gelu_forward(const float *x, float *y, int64_t n, int64_t block_size, int64_t pb,
                        int64_t pe) {
  return act_run(x, y, n, block_size, 1, pb, pe);
}
int oracle_silu_forward(const float *x, float *y, int64_t n, int64_t block_size, int64_t pb,
                        int64_t pe) {
  return act_run(x, y, n, block_size, 2, pb, pe);
}
int oracle_sigmoid_forward(const float *x, float *y, int64_t n, int64_t block_size, int64_t pb,
                           int64_t pe) {
  return act_run(x, y, n, block_size, 3, pb, pe);
}
int oracle_tanh_forward(const float *x, float *y, int64_t n, int64_t block_size, int64_t pb,
                        int64_t pe) {
  return act_run(x, y, n, block_size, 4, pb, pe);
}

/* ── activation gradients ────────────────────────────────────────────────
 * relu.rs:67-117, gelu.rs:81-139, sigmoid.rs:161-210: program pid covers the
 * same masked BLOCK_SIZE tile as the forward kernels; v is the forward output
 * y for relu and the forward input x for gelu and silu. */

typedef struct {
  const float *dy;
  const float *v;
  float *dx;
  int64_t n;
  int64_t block;
  int kind;
} act_grad_ctx;

static float relu_grad_ref(float dy, float y) {
  /* relu.rs:105-107: where(y > 0, grad_y, 0); a NaN y selects 0 */
  return y > 0.0f ? dy : 0.0f;
}

static float gelu_grad_ref(float dy, float x) {
  /* gelu.rs:117-130, in the reference's operation order:
   * inner = x + coeff*x*x*x ; s = one / (one + exp(neg2c * inner)) ;
   * t = two*s - one ; sech2 = one - t*t ; dinner = c * (one + three*coeff*x*x) ;
   * dx = dy * (half*(one + t) + x*half*sech2*dinner) */
  const float one = 1.0f, half = 0.5f, two = 2.0f, three = 3.0f;
  const float c = (float)0.7978845608028654;
  const float neg2c = (float)(-2.0 * 0.7978845608028654);
  const float coeff = 0.044715f;
  float inner = x + coeff * x * x * x;
  float s = one / (one + expf(neg2c * inner));
  float t = two * s - one;
  float sech2 = one - t * t;
  float dinner = c * (one + three * coeff * x * x);
  return dy * (half * (one + t) + x * half * sech2 * dinner);
}

static float silu_grad_ref(float dy, float x) {
  /* sigmoid.rs:196-201: s = one / (one + exp(neg1 * x)) ; y = x * s ;
   * dx = dy * (s + y - y * s) */
  const float one = 1.0f, neg1 = -1.0f;
  float s = one / (one + expf(neg1 * x));
  float y = x * s;
  return dy * (s + y - y * s);
}

static float sigmoid_grad_ref(float dy, float y) {
  /* sigmoid.rs (sigmoid_backward): dx = dy * (y - y * y), y the forward output */
  return dy * (y - y * y);
}

static float tanh_grad_ref(float dy, float y) {
  /* tanh.rs (tanh_backward): dx = dy * (one - y * y), y the forward output */
  const float one = 1.0f;
  return dy * (one - y * y);
}

static void act_grad_program(const void *c, int64_t pid) {
  const act_grad_ctx *a = (const act_grad_ctx *)c;
  int64_t start = pid * a->block;
  for (int64_t i = start; i < start + a->block && i < a->n; ++i) {
    float d = a->dy[i], v = a->v[i];
    switch (a->kind) {
      case 0: a->dx[i] = relu_grad_ref(d, v); break;
      case 1: a->dx[i] = gelu_grad_ref(d, v); break;
      case 2: a->dx[i] = silu_grad_ref(d, v); break;
      case 3: a->dx[i] = sigmoid_grad_ref(d, v); break;
      default: a->dx[i] = tanh_grad_ref(d, v); break;
    }
  }
}

static int act_grad_run(const float *dy, const float *v, float *dx, int64_t n, int64_t block,
                        int kind, int64_t pb, int64_t pe) {
  if (n < 0 || block <= 0) return ERR_SHAPE_MISMATCH;
  act_grad_ctx a = {dy, v, dx, n, block, kind};
  launch(act_grad_program, &a, (n + block - 1) / block, pb, pe);
  return OK;
}

int oracle_relu_backward(const float *dy, const float *y, float *dx, int64_t n,
                         int64_t block_size, int64_t pb, int64_t pe) {
  return act_grad_run(dy, y, dx, n, block_size, 0, pb, pe);
}
int oracle_gelu_backward(const float *dy, const float *x, float *dx, int64_t n,
                         int64_t block_size, int64_t pb, int64_t pe) {
  return act_grad_run(dy, x, dx, n, block_size, 1, pb, pe);
}
int oracle_silu_backward(const float *dy, const float *x, float *dx, int64_t n,
                         int64_t block_size, int64_t pb, int64_t pe) {
  return act_grad_run(dy, x, dx, n, block_size, 2, pb, pe);
}
int oracle_sigmoid_backward(const float *dy, const float *y, float *dx, int64_t n,
                            int64_t block_size, int64_t pb, int64_t pe) {
  return act_grad_run(dy, y, dx, n, block_size, 3, pb, pe);
}
int oracle_tanh_backward(const float *dy, const float *y, float *dx, int64_t n,
                         int64_t block_size, int64_t pb, int64_t pe) {
  return act_grad_run(dy, y, dx, n, block_size, 4, pb, pe);
}

/* ── LayerNorm / RMSNorm ─────────────────────────────────────────────────
 * layernorm.rs:42-157 and rmsnorm.rs:39-119: program = row; the row is
 * visited in BLOCK_N tiles; each tile is reduced (T::sum) and the tile sums
 * are accumulated in D = f32. */

typedef struct {
  const float *x;
  float *y;
  const float *w;
  const float *b;
  float *rrms;
  int64_t N;
  float eps;
  int64_t block;
} norm_ctx;

static float tile_sum(const float *v, int64_t n) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s += v[i];
  return s;
}

static void layernorm_program(const void *c, int64_t row) {
  const norm_ctx *a = (const norm_ctx *)c;
  const float *x = a->x + row * a->N;
  float *y = a->y + row * a->N;
  const int64_t N = a->N, B = a->block;
  float *tile = (float *)malloc(sizeof(float) * (size_t)B);
  /* pass 1: mean (layernorm.rs:61-79) */
  float sum = 0.0f;
  for (int64_t s = 0; s < N; s += B) {
    int64_t m = N - s < B ? N - s : B;
    sum = sum + tile_sum(x + s, m);
  }
  const float n_inv = 1.0f / (float)N;
  const float mean = sum * n_inv;
  /* pass 2: variance of (x - mean), masked (layernorm.rs:81-100) */
  float var_sum = 0.0f;
  for (int64_t s = 0; s < N; s += B) {
    int64_t m = N - s < B ? N - s : B;
    for (int64_t i = 0; i < m; ++i) {
      float d = x[s + i] - mean;
      tile[i] = d * d;
    }
    var_sum = var_sum + tile_sum(tile, m);
  }
  const float rstd = 1.0f / sqrtf(var_sum * n_inv + a->eps);
  /* pass 3: y = (x - mean) * rstd * gamma + beta (layernorm.rs:102-156) */
  for (int64_t i = 0; i < N; ++i) y[i] = (x[i] - mean) * rstd * a->w[i] + a->b[i];
  free(tile);
}

static void rmsnorm_program(const void *c, int64_t row) {
  const norm_ctx *a = (const norm_ctx *)c;
  const float *x = a->x + row * a->N;
  float *y = a->y + row * a->N;
  const int64_t N = a->N, B = a->block;
  float *tile = (float *)malloc(sizeof(float) * (size_t)B);
  const float n_inv = 1.0f / (float)N;
  /* pass 1: sum of squares (rmsnorm.rs:58-79) */
  float sq_sum = 0.0f;
  for (int64_t s = 0; s < N; s += B) {
    int64_t m = N - s < B ? N - s : B;
    for (int64_t i = 0; i < m; ++i) tile[i] = x[s + i] * x[s + i];
    sq_sum = sq_sum + tile_sum(tile, m);
  }
  const float rrms = 1.0f / sqrtf(sq_sum * n_inv + a->eps);
  if (a->rrms != NULL) a->rrms[row] = rrms; /* rmsnorm.rs:83 */
  /* pass 2: y = x * rrms * gamma (rmsnorm.rs:85-118) */
  for (int64_t i = 0; i < N; ++i) y[i] = x[i] * rrms * a->w[i];
  free(tile);
}

int oracle_layer_norm_forward_inference(const float *x, float *y, const float *w, const float *b,
                                        int64_t M, int64_t N, float eps, int64_t block_n,
                                        int64_t pb, int64_t pe) {
  if (M < 0 || N <= 0 || block_n <= 0) return ERR_SHAPE_MISMATCH;
  norm_ctx a = {x, y, w, b, NULL, N, eps, block_n};
  launch(layernorm_program, &a, M, pb, pe);
  return OK;
}

int oracle_rms_norm_forward(const float *x, float *y, const float *w, float *rrms, int64_t M,
                            int64_t N, float eps, int64_t block_n, int64_t pb, int64_t pe) {
  if (M < 0 || N <= 0 || block_n <= 0) return ERR_SHAPE_MISMATCH;
  norm_ctx a = {x, y, w, NULL, rrms, N, eps, block_n};
  launch(rmsnorm_program, &a, M, pb, pe);
  return OK;
}

/* ── conv2d ──────────────────────────────────────────────────────────────
 * conv2d.rs:43-156 (conv2d_forward) and :642-764 (conv2d_bias_forward):
 * pid = ((b*C_OUT + c_out)*OH + oh)*num_ow_tiles + ow_tile; each program
 * accumulates a BLOCK_OW strip over the flat (c_in_local, kh, kw) loop with
 * zero padding by masking, then adds bias[c_out] (bias variant). */

typedef struct {
  const float *x, *w, *bias;
  float *y;
  int64_t B, Cin, Cout, H, W, OH, OW;
  int64_t KH, KW, SH, SW, PH, PW, G, block_ow;
  /* conv2d_bn_silu_forward only (NULL otherwise) */
  const float *bn_scale, *bn_shift;
} conv_ctx;

static void conv_program(const void *c, int64_t pid) {
  const conv_ctx *a = (const conv_ctx *)c;
  const int64_t tiles = (a->OW + a->block_ow - 1) / a->block_ow;
  const int64_t ow_tile = pid % tiles;
  const int64_t bco = pid / tiles;
  const int64_t oh = bco % a->OH;
  const int64_t bc = bco / a->OH;
  const int64_t c_out = bc % a->Cout;
  const int64_t b = bc / a->Cout;
  const int64_t ow_start = ow_tile * a->block_ow;
  const int64_t cin_g = a->Cin / a->G;
  const int64_t g_idx = c_out / (a->Cout / a->G);
  const int64_t c_in_start = g_idx * cin_g;
  float acc[512];
  const int64_t BO = a->block_ow;
  for (int64_t t = 0; t < BO; ++t) acc[t] = 0.0f;
  const int64_t loop = cin_g * a->KH * a->KW;
  for (int64_t idx = 0; idx < loop; ++idx) {
    const int64_t kw = idx % a->KW;
    const int64_t kh_cin = idx / a->KW;
    const int64_t kh = kh_cin % a->KH;
    const int64_t cl = kh_cin / a->KH;
    const int64_t ci = c_in_start + cl;
    const int64_t ih = oh * a->SH + kh - a->PH;
    const float wv = a->w[((c_out * cin_g + cl) * a->KH + kh) * a->KW + kw];
    for (int64_t t = 0; t < BO; ++t) {
      const int64_t ow = ow_start + t;
      const int64_t iw = ow * a->SW + kw - a->PW;
      const int in_b = ow < a->OW && ih >= 0 && ih < a->H && iw >= 0 && iw < a->W;
      const float xv = in_b ? a->x[((b * a->Cin + ci) * a->H + ih) * a->W + iw] : 0.0f;
      acc[t] = acc[t] + xv * wv;
    }
  }
  float bias = a->bias != NULL ? a->bias[c_out] : 0.0f;
  for (int64_t t = 0; t < BO; ++t) {
    const int64_t ow = ow_start + t;
    if (ow < a->OW) {
      float v = a->bias != NULL ? acc[t] + bias : acc[t];
      if (a->bn_scale != NULL) {
        /* conv2d_bn_silu.rs:153-180: bn_out = scale * acc + shift, then
         * y = bn_out * (one / (one + exp(neg1 * bn_out))) */
        const float bn_out = a->bn_scale[c_out] * acc[t] + a->bn_shift[c_out];
        v = silu_ref(bn_out);
      }
      a->y[((b * a->Cout + c_out) * a->OH + oh) * a->OW + ow] = v;
    }
  }
}

int oracle_conv2d_forward(const float *x, const float *w, const float *bias, float *y, int64_t B,
                          int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t OH, int64_t OW,
                          int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW,
                          int64_t G, int64_t block_ow, int64_t pb, int64_t pe) {
  if (G <= 0 || Cin % G != 0 || Cout % G != 0) return ERR_SHAPE_MISMATCH;
  if (block_ow <= 0 || block_ow > 512 || KH <= 0 || KW <= 0 || SH <= 0 || SW <= 0)
    return ERR_INVALID_ARGUMENT;
  if (OH != (H + 2 * PH - KH) / SH + 1 || OW != (W + 2 * PW - KW) / SW + 1)
    return ERR_SHAPE_MISMATCH;
  conv_ctx a = {x, w, bias, y, B, Cin, Cout, H, W, OH, OW, KH, KW, SH, SW, PH, PW, G, block_ow, NULL, NULL};
  const int64_t tiles = (OW + block_ow - 1) / block_ow;
  launch(conv_program, &a, B * Cout * OH * tiles, pb, pe);
  return OK;
}

/* conv2d_bn_silu_forward (nn/fused/conv2d_bn_silu.rs:40-199): the programs of
 * conv2d_forward with the BatchNorm affine and SiLU applied before the store. */
int oracle_conv2d_bn_silu_forward(const float *x, const float *w, const float *bn_scale, const float *bn_shift,
                                  float *y, int64_t B, int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t OH,
                                  int64_t OW, int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW,
                                  int64_t G, int64_t block_ow, int64_t pb, int64_t pe) {
  if (G <= 0 || Cin % G != 0 || Cout % G != 0) return ERR_SHAPE_MISMATCH;
  if (block_ow <= 0 || block_ow > 512 || KH <= 0 || KW <= 0 || SH <= 0 || SW <= 0)
    return ERR_INVALID_ARGUMENT;
  if (OH != (H + 2 * PH - KH) / SH + 1 || OW != (W + 2 * PW - KW) / SW + 1)
    return ERR_SHAPE_MISMATCH;
  if (bn_scale == NULL || bn_shift == NULL) return ERR_INVALID_ARGUMENT;
  conv_ctx a = {x, w, NULL, y, B, Cin, Cout, H, W, OH, OW, KH, KW, SH, SW, PH, PW, G, block_ow, bn_scale, bn_shift};
  const int64_t tiles = (OW + block_ow - 1) / block_ow;
  launch(conv_program, &a, B * Cout * OH * tiles, pb, pe);
  return OK;
}

/* The same programs as oracle_conv2d_forward, but only the program ids listed
 * in `pids` (each in [0, B*Cout*OH*ceil(OW/block_ow))): a sampled check of a
 * large conv touches every output tile without running the whole grid. */
typedef struct {
  conv_ctx conv;
  const int64_t *pids;
} conv_list_ctx;

static void conv_list_program(const void *c, int64_t i) {
  const conv_list_ctx *a = (const conv_list_ctx *)c;
  conv_program(&a->conv, a->pids[i]);
}

int oracle_conv2d_programs(const float *x, const float *w, const float *bias, float *y, int64_t B,
                           int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t OH, int64_t OW,
                           int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW,
                           int64_t G, int64_t block_ow, const int64_t *pids, int64_t n_pids) {
  if (G <= 0 || Cin % G != 0 || Cout % G != 0) return ERR_SHAPE_MISMATCH;
  if (block_ow <= 0 || block_ow > 512 || KH <= 0 || KW <= 0 || SH <= 0 || SW <= 0)
    return ERR_INVALID_ARGUMENT;
  if (OH != (H + 2 * PH - KH) / SH + 1 || OW != (W + 2 * PW - KW) / SW + 1)
    return ERR_SHAPE_MISMATCH;
  const int64_t total = B * Cout * OH * ((OW + block_ow - 1) / block_ow);
  for (int64_t i = 0; i < n_pids; ++i)
    if (pids[i] < 0 || pids[i] >= total) return ERR_SHAPE_MISMATCH;
  conv_list_ctx a = {{x, w, bias, y, B, Cin, Cout, H, W, OH, OW, KH, KW, SH, SW, PH, PW, G, block_ow, NULL, NULL},
                     pids};
  launch(conv_list_program, &a, n_pids, 0, -1);
  return OK;
}

/* ── flash attention 2 forward ───────────────────────────────────────────
 * flash_attn2.rs:52-158: program (pid_m, pid_bh); q row in registers;
 * sequential loop over key rows with the online-softmax recurrence
 *   qk = sum(q*k) * scale; m_new = max(m, qk); a = exp(m - m_new);
 *   p = exp(qk - m_new); l = a*l + p; acc = a*acc + p*v; m = m_new
 * then o = acc / l and L = m + log(l).  Causal (an extension: the reference
 * kernel is non-causal) stops the key loop at k_row = pid_m (top-left
 * aligned).  Program id = pid_bh * n_ctx_q + pid_m. */

typedef struct {
  const float *q, *k, *v;
  float *o, *l;
  int64_t nq, nk, D;
  float scale;
  int causal;
  const int64_t *rows; /* optional explicit program list */
} fa_ctx;

static void fa_program_id(const fa_ctx *a, int64_t id) {
  const int64_t pid_bh = id / a->nq, pid_m = id % a->nq;
  const int64_t D = a->D;
  const float *q = a->q + (pid_bh * a->nq + pid_m) * D;
  const float *kb = a->k + pid_bh * a->nk * D;
  const float *vb = a->v + pid_bh * a->nk * D;
  float acc[1024];
  float m_i = -INFINITY, l_i = 0.0f;
  for (int64_t d = 0; d < D; ++d) acc[d] = 0.0f;
  int64_t kend = a->nk;
  if (a->causal && pid_m + 1 < kend) kend = pid_m + 1;
  for (int64_t kr = 0; kr < kend; ++kr) {
    const float *k = kb + kr * D, *v = vb + kr * D;
    float dot = 0.0f;
    for (int64_t d = 0; d < D; ++d) dot += q[d] * k[d];
    const float qk = dot * a->scale;
    const float m_new = m_i > qk ? m_i : qk;
    const float ed = expf(m_i - m_new);
    const float p = expf(qk - m_new);
    l_i = ed * l_i + p;
    for (int64_t d = 0; d < D; ++d) acc[d] = ed * acc[d] + p * v[d];
    m_i = m_new;
  }
  float *o = a->o + (pid_bh * a->nq + pid_m) * D;
  for (int64_t d = 0; d < D; ++d) o[d] = acc[d] / l_i;
  if (a->l != NULL) a->l[pid_bh * a->nq + pid_m] = m_i + logf(l_i);
}

static void fa_program(const void *c, int64_t id) {
  const fa_ctx *a = (const fa_ctx *)c;
  fa_program_id(a, a->rows != NULL ? a->rows[id] : id);
}

int oracle_flash_attention2_forward(const float *q, const float *k, const float *v, float *o,
                                    float *l, int64_t BH, int64_t nq, int64_t nk, int64_t D,
                                    float scale, int causal, int64_t pb, int64_t pe) {
  if (D <= 0 || D > 1024 || nq < 0 || nk <= 0 || BH < 0) return ERR_SHAPE_MISMATCH;
  fa_ctx a = {q, k, v, o, l, nq, nk, D, scale, causal, NULL};
  launch(fa_program, &a, BH * nq, pb, pe);
  return OK;
}

/* Runs only the listed program ids (pid_bh * nq + pid_m); o and l are
 * written at those rows only.  Used to check full-size outputs on a sample. */
int oracle_flash_attention2_rows(const float *q, const float *k, const float *v, float *o,
                                 float *l, int64_t BH, int64_t nq, int64_t nk, int64_t D,
                                 float scale, int causal, const int64_t *rows, int64_t n_rows) {
  if (D <= 0 || D > 1024 || nq < 0 || nk <= 0 || BH < 0) return ERR_SHAPE_MISMATCH;
  for (int64_t i = 0; i < n_rows; ++i)
    if (rows[i] < 0 || rows[i] >= BH * nq) return ERR_SHAPE_MISMATCH;
  fa_ctx a = {q, k, v, o, l, nq, nk, D, scale, causal, rows};
  launch(fa_program, &a, n_rows, 0, -1);
  return OK;
}

/* ── linear ──────────────────────────────────────────────────────────────
 * linear.rs:20-116: y[m,n] = sum_k x[m,k] * w[n,k] (+ b[n]) with fp32
 * accumulation in k order.  Program = output row m. */

typedef struct {
  const float *x, *w, *b;
  float *y;
  int64_t N, K, sxm, sxk, swn, swk, sym, syn;
} lin_ctx;

static void linear_program(const void *c, int64_t m) {
  const lin_ctx *a = (const lin_ctx *)c;
  for (int64_t n = 0; n < a->N; ++n) {
    float acc = 0.0f;
    for (int64_t k = 0; k < a->K; ++k)
      acc += a->x[m * a->sxm + k * a->sxk] * a->w[n * a->swn + k * a->swk];
    if (a->b != NULL) acc = acc + a->b[n];
    a->y[m * a->sym + n * a->syn] = acc;
  }
}

int oracle_linear_forward(const float *x, const float *w, const float *b, float *y, int64_t M,
                          int64_t N, int64_t K, int64_t sxm, int64_t sxk, int64_t swn,
                          int64_t swk, int64_t sym, int64_t syn, int64_t pb, int64_t pe) {
  if (M < 0 || N < 0 || K < 0) return ERR_SHAPE_MISMATCH;
  lin_ctx a = {x, w, b, y, N, K, sxm, sxk, swn, swk, sym, syn};
  launch(linear_program, &a, M, pb, pe);
  return OK;
}

/* linear.rs:118-250 (linear_backward): dx = dy W ([M, K], reduction over n),
 * dw = dy^T x ([N, K], reduction over m), db[n] = sum_m dy[m, n], all
 * written (not accumulated), fp32 accumulation in reduction order.  The
 * reference's programs are (m, n, k) tiles of which the pid_n == 0 ones write
 * dx and the pid_m == 0 ones write dw and db; here program p < M is dx row p
 * and program M + n is dw row n (with db[n]): the same sums per element. */

typedef struct {
  const float *x, *w, *dy;
  float *dx, *dw, *db;
  int64_t M, N, K, sxm, sxk, swk, swn, sdym, sdyn, sdxm, sdxk, sdwk, sdwn, sdbn;
} linb_ctx;

static void linear_bwd_program(const void *c, int64_t p) {
  const linb_ctx *a = (const linb_ctx *)c;
  if (p < a->M) {
    const int64_t m = p;
    for (int64_t k = 0; k < a->K; ++k) {
      float acc = 0.0f;
      for (int64_t n = 0; n < a->N; ++n) acc += a->dy[m * a->sdym + n * a->sdyn] * a->w[n * a->swn + k * a->swk];
      a->dx[m * a->sdxm + k * a->sdxk] = acc;
    }
    return;
  }
  const int64_t n = p - a->M;
  for (int64_t k = 0; k < a->K; ++k) {
    float acc = 0.0f;
    for (int64_t m = 0; m < a->M; ++m) acc += a->dy[m * a->sdym + n * a->sdyn] * a->x[m * a->sxm + k * a->sxk];
    a->dw[n * a->sdwn + k * a->sdwk] = acc;
  }
  if (a->db != NULL) {
    float acc = 0.0f;
    for (int64_t m = 0; m < a->M; ++m) acc += a->dy[m * a->sdym + n * a->sdyn];
    a->db[n * a->sdbn] = acc;
  }
}

int oracle_linear_backward(const float *x, const float *w, const float *dy, float *dx, float *dw, float *db,
                           int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t sxk, int64_t swk, int64_t swn,
                           int64_t sdym, int64_t sdyn, int64_t sdxm, int64_t sdxk, int64_t sdwk, int64_t sdwn,
                           int64_t sdbn) {
  if (M < 0 || N < 0 || K < 0) return ERR_SHAPE_MISMATCH;
  linb_ctx a = {x, w, dy, dx, dw, db, M, N, K, sxm, sxk, swk, swn, sdym, sdyn, sdxm, sdxk, sdwk, sdwn, sdbn};
  launch(linear_bwd_program, &a, M + N, 0, -1);
  return OK;
}

/* ── teeny-quant affine quantization ─────────────────────────────────────
 * utilities/teeny-quant/src/quant/affine.rs:47-161 and groups.rs:20-100.
 * Rust semantics restated: f32::round rounds half away from zero; `as i32`
 * saturates and maps NaN to 0; min/max of f32 via `<`/`>` comparisons. */

enum { PER_TENSOR = 0, PER_CHANNEL = 1, GROUP = 2 };

static int32_t rust_f32_as_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483648.0f) return INT32_MAX;
  if (v <= -2147483648.0f) return INT32_MIN;
  return (int32_t)v;
}

static float rust_round(float v) { return roundf(v); /* C roundf: half away from zero */ }

static void row_major_strides(const int64_t *shape, int ndim, int64_t *strides) {
  if (ndim == 0) return;
  strides[ndim - 1] = 1;
  for (int i = ndim - 2; i >= 0; --i) strides[i] = strides[i + 1] * shape[i + 1];
}

/* groups.rs:78-100 (assign_groups) restated per element. */
static int64_t group_of(int64_t flat, const int64_t *shape, const int64_t *strides, int ndim,
                        int gran, int axis, int64_t group_size) {
  if (gran == PER_TENSOR) return 0;
  int64_t idx_axis = (flat / strides[axis]) % shape[axis];
  if (gran == PER_CHANNEL) return idx_axis;
  /* group_wise_id (groups.rs:51-63): outer id over the other axes, last axis fastest. */
  int64_t outer = 0, mult = 1;
  for (int d = ndim - 1; d >= 0; --d) {
    if (d == axis) continue;
    int64_t idx_d = (flat / strides[d]) % shape[d];
    outer += idx_d * mult;
    mult *= shape[d];
  }
  int64_t along = (shape[axis] + group_size - 1) / group_size;
  return outer * along + idx_axis / group_size;
}

int oracle_quant_num_groups(const int64_t *shape, int ndim, int gran, int axis,
                            int64_t group_size, int64_t *ngroups) {
  if (gran == PER_TENSOR) {
    *ngroups = 1;
    return OK;
  }
  if (axis < 0 || axis >= ndim) return ERR_INVALID_AXIS;
  if (gran == PER_CHANNEL) {
    *ngroups = shape[axis];
    return OK;
  }
  if (group_size == 0) return ERR_INVALID_GROUP_SIZE;
  int64_t outer = 1;
  for (int d = 0; d < ndim; ++d)
    if (d != axis) outer *= shape[d];
  *ngroups = outer * ((shape[axis] + group_size - 1) / group_size);
  return OK;
}

int oracle_quantize_affine(const float *data, int64_t n_data, const int64_t *shape, int ndim,
                           int gran, int axis, int64_t group_size, int symmetric, int bits,
                           int8_t *qvalues, float *scales, int32_t *zero_points,
                           uint32_t *groups) {
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) n *= shape[d];
  if (n_data != n) return ERR_SHAPE_MISMATCH; /* affine.rs:63-70 */
  if (gran != PER_TENSOR) {
    if (axis < 0 || axis >= ndim) return ERR_INVALID_AXIS;                /* :73-80 */
    if (gran == GROUP && group_size == 0) return ERR_INVALID_GROUP_SIZE; /* :81-83 */
  }
  if (bits < 2 || bits > 8) return ERR_INVALID_ARGUMENT;
  const int32_t qmax = (1 << (bits - 1)) - 1;           /* qrange, :47-51 */
  const int32_t qmin = symmetric ? -qmax : -qmax - 1;
  int64_t ngroups = 0;
  int rc = oracle_quant_num_groups(shape, ndim, gran, axis, gran == PER_CHANNEL ? 1 : group_size,
                                   &ngroups);
  if (rc != OK) return rc;
  int64_t strides[16];
  if (ndim > 16) return ERR_INVALID_ARGUMENT;
  row_major_strides(shape, ndim, strides);
  float *vmin = (float *)malloc(sizeof(float) * (size_t)(ngroups > 0 ? ngroups : 1));
  float *vmax = (float *)malloc(sizeof(float) * (size_t)(ngroups > 0 ? ngroups : 1));
  for (int64_t g = 0; g < ngroups; ++g) {
    vmin[g] = INFINITY;
    vmax[g] = -INFINITY;
  }
  /* pass 1: per-group min/max (:90-101) */
  for (int64_t i = 0; i < n; ++i) {
    int64_t g = group_of(i, shape, strides, ndim, gran, axis, group_size);
    if (groups != NULL) groups[i] = (uint32_t)g;
    float x = data[i];
    if (x < vmin[g]) vmin[g] = x;
    if (x > vmax[g]) vmax[g] = x;
  }
  /* params (:103-132) */
  for (int64_t g = 0; g < ngroups; ++g) {
    float lo, hi;
    if (isfinite(vmin[g])) {
      lo = fminf(vmin[g], 0.0f);
      hi = fmaxf(vmax[g], 0.0f);
    } else {
      lo = 0.0f;
      hi = 0.0f;
    }
    if (symmetric) {
      float amax = fmaxf(fabsf(lo), fabsf(hi));
      scales[g] = amax == 0.0f ? 1.0f : amax / (float)qmax;
      zero_points[g] = 0;
    } else {
      float scale = hi == lo ? 1.0f : (hi - lo) / (float)(qmax - qmin);
      int32_t zp = rust_f32_as_i32(rust_round((float)qmin - lo / scale));
      scales[g] = scale;
      zero_points[g] = zp < qmin ? qmin : zp > qmax ? qmax : zp;
    }
  }
  /* pass 2: q = clamp(round(x / scale) as i32 + zp, qmin, qmax) (:134-142) */
  for (int64_t i = 0; i < n; ++i) {
    int64_t g = group_of(i, shape, strides, ndim, gran, axis, group_size);
    int64_t q = (int64_t)rust_f32_as_i32(rust_round(data[i] / scales[g])) + zero_points[g];
    /* i32 add in Rust: wrapping is impossible here because |zp| <= 128 and
     * the saturated value is at most i32::MAX; widen to keep C defined. */
    if (q > INT32_MAX) q = INT32_MAX; /* unreachable for finite scales */
    qvalues[i] = (int8_t)(q < qmin ? qmin : q > qmax ? qmax : q);
  }
  free(vmin);
  free(vmax);
  return OK;
}

/* dequantize_affine (affine.rs:151-161): (v as i32 - zp) as f32 * scale. */
int oracle_dequantize_affine(const int8_t *q, const float *scales, const int32_t *zero_points,
                             const int64_t *shape, int ndim, int gran, int axis,
                             int64_t group_size, float *out) {
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) n *= shape[d];
  if (gran != PER_TENSOR && (axis < 0 || axis >= ndim)) return ERR_INVALID_AXIS;
  if (gran == GROUP && group_size == 0) return ERR_INVALID_GROUP_SIZE;
  int64_t strides[16];
  if (ndim > 16) return ERR_INVALID_ARGUMENT;
  row_major_strides(shape, ndim, strides);
  for (int64_t i = 0; i < n; ++i) {
    int64_t g = group_of(i, shape, strides, ndim, gran, axis, group_size);
    int32_t zp = zero_points != NULL ? zero_points[g] : 0;
    out[i] = (float)((int32_t)q[i] - zp) * scales[g];
  }
  return OK;
}

/* ══ training: norm forward with saved statistics, and the backward kernels ══ */

/* ── LayerNorm training forward ──────────────────────────────────────────
 * layernorm.rs:162-298 (layer_norm_forward): the inference kernel's three
 * passes, plus mean[row] and rstd[row] stored for the backward pass. */

typedef struct {
  const float *x, *w, *b;
  float *y, *mean, *rstd;
  int64_t N, block;
  float eps;
} lnf_ctx;

static void layernorm_train_program(const void *c, int64_t row) {
  const lnf_ctx *a = (const lnf_ctx *)c;
  const float *x = a->x + row * a->N;
  float *y = a->y + row * a->N;
  const int64_t N = a->N, B = a->block;
  float *tile = (float *)malloc(sizeof(float) * (size_t)B);
  float sum = 0.0f;
  for (int64_t s = 0; s < N; s += B) {
    int64_t m = N - s < B ? N - s : B;
    sum = sum + tile_sum(x + s, m);
  }
  const float n_inv = 1.0f / (float)N;
  const float mean = sum * n_inv;
  float var_sum = 0.0f;
  for (int64_t s = 0; s < N; s += B) {
    int64_t m = N - s < B ? N - s : B;
    for (int64_t i = 0; i < m; ++i) {
      float d = x[s + i] - mean;
      tile[i] = d * d;
    }
    var_sum = var_sum + tile_sum(tile, m);
  }
  const float rstd = 1.0f / sqrtf(var_sum * n_inv + a->eps);
  a->mean[row] = mean; /* layernorm.rs:229-230 */
  a->rstd[row] = rstd;
  for (int64_t i = 0; i < N; ++i) y[i] = (x[i] - mean) * rstd * a->w[i] + a->b[i];
  free(tile);
}

int oracle_layer_norm_forward(const float *x, float *y, const float *w, const float *b, float *mean,
                              float *rstd, int64_t M, int64_t N, float eps, int64_t block_n, int64_t pb,
                              int64_t pe) {
  if (M < 0 || N <= 0 || block_n <= 0) return ERR_SHAPE_MISMATCH;
  lnf_ctx a = {x, w, b, y, mean, rstd, N, block_n, eps};
  launch(layernorm_train_program, &a, M, pb, pe);
  return OK;
}

/* ── LayerNorm backward ──────────────────────────────────────────────────
 * layernorm.rs:300-482 (layer_norm_backward): program = row.
 *   pass 1: sum_dy_gamma = sum dy*gamma, sum_dy_gamma_xhat = sum dy*gamma*xhat
 *           (BLOCK_N tiles, tile sums accumulated), c1 = sum_dy_gamma / N,
 *           c2 = sum_dy_gamma_xhat / N, xhat = (x - mean) * rstd;
 *   pass 2: dx = rstd * gamma * (dy - c1 - xhat * c2),
 *           dweight[n] = dweight[n] + dy * xhat, dbias[n] = dbias[n] + dy.
 * The reference updates dweight/dbias by a load-add-store per program; here
 * the programs compute dx in parallel and the parameter gradients are then
 * accumulated in program (row) order, the order a one-program-at-a-time
 * launch gives. */

typedef struct {
  const float *dy, *x, *w, *mean, *rstd;
  float *dx;
  int64_t N, block;
} lnb_ctx;

static void layernorm_bwd_program(const void *c, int64_t row) {
  const lnb_ctx *a = (const lnb_ctx *)c;
  const int64_t N = a->N, B = a->block;
  const float *x = a->x + row * N, *dy = a->dy + row * N;
  float *dx = a->dx + row * N;
  const float mean = a->mean[row], rstd = a->rstd[row];
  const float n_inv = 1.0f / (float)N;
  float *t1 = (float *)malloc(sizeof(float) * (size_t)B);
  float *t2 = (float *)malloc(sizeof(float) * (size_t)B);
  float s1 = 0.0f, s2 = 0.0f;
  for (int64_t s = 0; s < N; s += B) {
    int64_t m = N - s < B ? N - s : B;
    for (int64_t i = 0; i < m; ++i) {
      const float xhat = (x[s + i] - mean) * rstd;
      t1[i] = dy[s + i] * a->w[s + i];
      t2[i] = dy[s + i] * a->w[s + i] * xhat;
    }
    s1 = s1 + tile_sum(t1, m);
    s2 = s2 + tile_sum(t2, m);
  }
  const float c1 = s1 * n_inv, c2 = s2 * n_inv;
  for (int64_t i = 0; i < N; ++i) {
    const float xhat = (x[i] - mean) * rstd;
    dx[i] = rstd * a->w[i] * (dy[i] - c1 - xhat * c2);
  }
  free(t1);
  free(t2);
}

int oracle_layer_norm_backward(const float *dy, const float *x, float *dx, const float *w, float *dweight,
                               float *dbias, const float *mean, const float *rstd, int64_t M, int64_t N,
                               int64_t block_n) {
  if (M < 0 || N <= 0 || block_n <= 0) return ERR_SHAPE_MISMATCH;
  lnb_ctx a = {dy, x, w, mean, rstd, dx, N, block_n};
  launch(layernorm_bwd_program, &a, M, 0, -1);
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      const float xhat = (x[m * N + n] - mean[m]) * rstd[m];
      if (dweight != NULL) dweight[n] = dweight[n] + dy[m * N + n] * xhat;
      if (dbias != NULL) dbias[n] = dbias[n] + dy[m * N + n];
    }
  return OK;
}

/* ── RMSNorm backward ────────────────────────────────────────────────────
 * rmsnorm.rs:135-277 (rms_norm_backward): program = row.
 *   pass 1: dot = sum dy*gamma*x; scale = dot / N;
 *   pass 2: dx = rrms * gamma * (dy - x * rrms^2 * scale),
 *           dweight[n] = dweight[n] + dy * x * rrms  (row order, as above). */

typedef struct {
  const float *dy, *x, *w, *rrms;
  float *dx;
  int64_t N, block;
} rmsb_ctx;

static void rmsnorm_bwd_program(const void *c, int64_t row) {
  const rmsb_ctx *a = (const rmsb_ctx *)c;
  const int64_t N = a->N, B = a->block;
  const float *x = a->x + row * N, *dy = a->dy + row * N;
  float *dx = a->dx + row * N;
  const float r = a->rrms[row];
  float *t = (float *)malloc(sizeof(float) * (size_t)B);
  float dot = 0.0f;
  for (int64_t s = 0; s < N; s += B) {
    int64_t m = N - s < B ? N - s : B;
    for (int64_t i = 0; i < m; ++i) t[i] = dy[s + i] * a->w[s + i] * x[s + i];
    dot = dot + tile_sum(t, m);
  }
  const float rsq = r * r;
  const float scale = dot * (1.0f / (float)N);
  for (int64_t i = 0; i < N; ++i) dx[i] = r * a->w[i] * (dy[i] - x[i] * rsq * scale);
  free(t);
}

int oracle_rms_norm_backward(const float *dy, const float *x, float *dx, const float *w, float *dweight,
                             const float *rrms, int64_t M, int64_t N, int64_t block_n) {
  if (M < 0 || N <= 0 || block_n <= 0) return ERR_SHAPE_MISMATCH;
  rmsb_ctx a = {dy, x, w, rrms, dx, N, block_n};
  launch(rmsnorm_bwd_program, &a, M, 0, -1);
  if (dweight != NULL)
    for (int64_t m = 0; m < M; ++m)
      for (int64_t n = 0; n < N; ++n) dweight[n] = dweight[n] + dy[m * N + n] * x[m * N + n] * rrms[m];
  return OK;
}

/* ── conv2d backward ─────────────────────────────────────────────────────
 * conv2d.rs:171-284 (conv2d_backward_dx) scatters dy[b,co,oh,ow] * w into
 * dx[b, ci, oh*SH - PH + kh, ow*SW - PW + kw] with atomic adds (summation
 * order set by the atomics); :286-397 (conv2d_backward_dw) adds, per
 * program (b, co, oh, ow-tile) and tap, the tile sum of dy * x into
 * dw[co, ci_local, kh, kw].  Restated deterministically: dx as a gather per
 * input element, taps in (co, kh, kw) order; dw as the reference's
 * per-program tile sums added in program order (b, oh, ow-tile).  Both
 * compute exactly the reference's sums of products, in a fixed order. */

typedef struct {
  const float *dy, *w, *x;
  float *out;
  int64_t B, Cin, Cout, H, W, OH, OW, KH, KW, SH, SW, PH, PW, G, block_ow;
} convb_ctx;

static void conv_dx_program(const void *c, int64_t pid) {
  /* pid = (b * Cin + ci) * H + ih: one input row */
  const convb_ctx *a = (const convb_ctx *)c;
  const int64_t ih = pid % a->H, bc = pid / a->H, ci = bc % a->Cin, b = bc / a->Cin;
  const int64_t cin_g = a->Cin / a->G, cout_g = a->Cout / a->G;
  const int64_t g = ci / cin_g, cl = ci % cin_g;
  for (int64_t iw = 0; iw < a->W; ++iw) {
    float acc = 0.0f;
    for (int64_t co = g * cout_g; co < (g + 1) * cout_g; ++co)
      for (int64_t kh = 0; kh < a->KH; ++kh) {
        const int64_t th = ih + a->PH - kh;
        if (th < 0 || th % a->SH != 0 || th / a->SH >= a->OH) continue;
        const int64_t oh = th / a->SH;
        for (int64_t kw = 0; kw < a->KW; ++kw) {
          const int64_t tw = iw + a->PW - kw;
          if (tw < 0 || tw % a->SW != 0 || tw / a->SW >= a->OW) continue;
          const int64_t ow = tw / a->SW;
          acc += a->dy[((b * a->Cout + co) * a->OH + oh) * a->OW + ow] *
                 a->w[((co * cin_g + cl) * a->KH + kh) * a->KW + kw];
        }
      }
    a->out[((b * a->Cin + ci) * a->H + ih) * a->W + iw] = acc;
  }
}

static void conv_dw_program(const void *c, int64_t pid) {
  /* pid = co * (Cin/G) * KH * KW + tap: one weight element */
  const convb_ctx *a = (const convb_ctx *)c;
  const int64_t cin_g = a->Cin / a->G, cout_g = a->Cout / a->G;
  const int64_t kw = pid % a->KW, t1 = pid / a->KW, kh = t1 % a->KH, t2 = t1 / a->KH, cl = t2 % cin_g,
                co = t2 / cin_g;
  const int64_t ci = (co / cout_g) * cin_g + cl;
  const int64_t tiles = (a->OW + a->block_ow - 1) / a->block_ow;
  float acc = 0.0f;
  for (int64_t b = 0; b < a->B; ++b)
    for (int64_t oh = 0; oh < a->OH; ++oh) {
      const int64_t ih = oh * a->SH - a->PH + kh;
      for (int64_t t = 0; t < tiles; ++t) {
        float part = 0.0f; /* T::sum over the ow tile (conv2d.rs:384-386) */
        for (int64_t j = 0; j < a->block_ow; ++j) {
          const int64_t ow = t * a->block_ow + j, iw = ow * a->SW - a->PW + kw;
          if (ow >= a->OW || ih < 0 || ih >= a->H || iw < 0 || iw >= a->W) continue;
          part += a->dy[((b * a->Cout + co) * a->OH + oh) * a->OW + ow] *
                  a->x[((b * a->Cin + ci) * a->H + ih) * a->W + iw];
        }
        acc += part;
      }
    }
  a->out[pid] = acc;
}

static int convb_check(int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t OH, int64_t OW, int64_t KH,
                       int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW, int64_t G) {
  if (G <= 0 || Cin % G != 0 || Cout % G != 0 || KH <= 0 || KW <= 0 || SH <= 0 || SW <= 0) return ERR_SHAPE_MISMATCH;
  if (OH != (H + 2 * PH - KH) / SH + 1 || OW != (W + 2 * PW - KW) / SW + 1) return ERR_SHAPE_MISMATCH;
  return OK;
}

int oracle_conv2d_backward_dx(const float *dy, const float *w, float *dx, int64_t B, int64_t Cin, int64_t Cout,
                              int64_t H, int64_t W, int64_t OH, int64_t OW, int64_t KH, int64_t KW, int64_t SH,
                              int64_t SW, int64_t PH, int64_t PW, int64_t G) {
  int rc = convb_check(Cin, Cout, H, W, OH, OW, KH, KW, SH, SW, PH, PW, G);
  if (rc != OK) return rc;
  convb_ctx a = {dy, w, NULL, dx, B, Cin, Cout, H, W, OH, OW, KH, KW, SH, SW, PH, PW, G, 16};
  launch(conv_dx_program, &a, B * Cin * H, 0, -1);
  return OK;
}

int oracle_conv2d_backward_dw(const float *dy, const float *x, float *dw, int64_t B, int64_t Cin, int64_t Cout,
                              int64_t H, int64_t W, int64_t OH, int64_t OW, int64_t KH, int64_t KW, int64_t SH,
                              int64_t SW, int64_t PH, int64_t PW, int64_t G, int64_t block_ow) {
  int rc = convb_check(Cin, Cout, H, W, OH, OW, KH, KW, SH, SW, PH, PW, G);
  if (rc != OK) return rc;
  if (block_ow <= 0) return ERR_INVALID_ARGUMENT;
  convb_ctx a = {dy, NULL, x, dw, B, Cin, Cout, H, W, OH, OW, KH, KW, SH, SW, PH, PW, G, block_ow};
  launch(conv_dw_program, &a, Cout * (Cin / G) * KH * KW, 0, -1);
  return OK;
}

/* ── flash attention 2 backward ──────────────────────────────────────────
 * flash_attn2.rs:173-309 (backward_dq): program (q_row, bh):
 *   D_q = sum(O_q * dO_q); for each key row k: p = exp(Q_q.K_k * scale - L_q),
 *   dS = p * (dO_q.V_k - D_q), dQ += dS * K_k * scale.
 * flash_attn2.rs:311-447 (backward_dkv): program (k_row, bh): for each query
 *   row m: p = exp(Q_m.K_n * scale - L_m), dV += p * dO_m,
 *   dS = p * (dO_m.V_n - D_m), dK += dS * Q_m * scale.
 * Causal (an extension, as in the forward): only pairs with k_row <= q_row. */

typedef struct {
  const float *q, *k, *v, *o, *dO, *l;
  float *d1, *d2;
  int64_t nq, nk, D;
  float scale;
  int causal;
} fab_ctx;

static float dotf(const float *a, const float *b, int64_t n) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s += a[i] * b[i];
  return s;
}

static void fa_dq_program(const void *c, int64_t id) {
  const fab_ctx *a = (const fab_ctx *)c;
  const int64_t bh = id / a->nq, qr = id % a->nq, D = a->D;
  const float *q = a->q + (bh * a->nq + qr) * D, *o = a->o + (bh * a->nq + qr) * D, *dO = a->dO + (bh * a->nq + qr) * D;
  const float dq_ = dotf(o, dO, D), lq = a->l[bh * a->nq + qr];
  float acc[1024];
  for (int64_t d = 0; d < D; ++d) acc[d] = 0.0f;
  const int64_t kend = a->causal && qr + 1 < a->nk ? qr + 1 : a->nk;
  for (int64_t kr = 0; kr < kend; ++kr) {
    const float *k = a->k + (bh * a->nk + kr) * D, *v = a->v + (bh * a->nk + kr) * D;
    const float p = expf(dotf(q, k, D) * a->scale - lq);
    const float ds = p * (dotf(dO, v, D) - dq_);
    for (int64_t d = 0; d < D; ++d) acc[d] = acc[d] + ds * k[d] * a->scale;
  }
  float *dq = a->d1 + (bh * a->nq + qr) * D;
  for (int64_t d = 0; d < D; ++d) dq[d] = acc[d];
}

static void fa_dkv_program(const void *c, int64_t id) {
  const fab_ctx *a = (const fab_ctx *)c;
  const int64_t bh = id / a->nk, kr = id % a->nk, D = a->D;
  const float *k = a->k + (bh * a->nk + kr) * D, *v = a->v + (bh * a->nk + kr) * D;
  float dk[1024], dv[1024];
  for (int64_t d = 0; d < D; ++d) dk[d] = dv[d] = 0.0f;
  for (int64_t qr = a->causal ? kr : 0; qr < a->nq; ++qr) {
    const float *q = a->q + (bh * a->nq + qr) * D, *o = a->o + (bh * a->nq + qr) * D,
                *dO = a->dO + (bh * a->nq + qr) * D;
    const float lm = a->l[bh * a->nq + qr], dm = dotf(o, dO, D);
    const float p = expf(dotf(q, k, D) * a->scale - lm);
    for (int64_t d = 0; d < D; ++d) dv[d] = dv[d] + p * dO[d];
    const float ds = p * (dotf(dO, v, D) - dm);
    for (int64_t d = 0; d < D; ++d) dk[d] = dk[d] + ds * q[d] * a->scale;
  }
  float *dko = a->d1 + (bh * a->nk + kr) * D, *dvo = a->d2 + (bh * a->nk + kr) * D;
  for (int64_t d = 0; d < D; ++d) {
    dko[d] = dk[d];
    dvo[d] = dv[d];
  }
}

int oracle_flash_attention2_backward(const float *q, const float *k, const float *v, const float *o,
                                     const float *dO, const float *l, float *dq, float *dk, float *dv, int64_t BH,
                                     int64_t nq, int64_t nk, int64_t D, float scale, int causal) {
  if (D <= 0 || D > 1024 || nq < 0 || nk <= 0 || BH < 0) return ERR_SHAPE_MISMATCH;
  fab_ctx a = {q, k, v, o, dO, l, dq, NULL, nq, nk, D, scale, causal};
  launch(fa_dq_program, &a, BH * nq, 0, -1);
  fab_ctx b = {q, k, v, o, dO, l, dk, dv, nq, nk, D, scale, causal};
  launch(fa_dkv_program, &b, BH * nk, 0, -1);
  return OK;
}
