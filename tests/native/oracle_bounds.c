/* Host sanitizer check of the oracle at its limits: the largest head_dim the
 * attention restatement takes (1024, its per-program accumulator), the
 * largest BLOCK_OW of the conv restatement (512), and the argument checks
 * just past them; built with the oracle under ASan/UBSan by a CPU test. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

int oracle_set_threads(int n);
int oracle_conv2d_forward(const float *x, const float *w, const float *bias, float *y, int64_t B, int64_t Cin,
                          int64_t Cout, int64_t H, int64_t W, int64_t OH, int64_t OW, int64_t KH, int64_t KW,
                          int64_t SH, int64_t SW, int64_t PH, int64_t PW, int64_t G, int64_t block_ow, int64_t pb,
                          int64_t pe);
int oracle_flash_attention2_forward(const float *q, const float *k, const float *v, float *o, float *l, int64_t BH,
                                    int64_t nq, int64_t nk, int64_t D, float scale, int causal, int64_t pb,
                                    int64_t pe);
int oracle_layer_norm_forward_inference(const float *x, float *y, const float *w, const float *b, int64_t M,
                                        int64_t N, float eps, int64_t block_n, int64_t pb, int64_t pe);

static float *buf(size_t n) {
  float *p = (float *)malloc(n * sizeof(float));
  for (size_t i = 0; i < n; ++i) p[i] = (float)((i * 37) % 17) / 17.0f - 0.5f;
  return p;
}

int main(void) {
  oracle_set_threads(3);
  int bad = 0;
  /* attention: D = 1024 accepted, 1025 rejected */
  {
    const int64_t BH = 2, nq = 3, nk = 5, D = 1024;
    float *q = buf(BH * nq * D), *k = buf(BH * nk * D), *v = buf(BH * nk * D), *o = buf(BH * nq * D), *l = buf(BH * nq);
    bad |= oracle_flash_attention2_forward(q, k, v, o, l, BH, nq, nk, D, 0.03f, 1, 0, -1) != 0;
    bad |= oracle_flash_attention2_forward(q, k, v, o, l, BH, nq, nk, D + 1, 0.03f, 1, 0, -1) == 0;
    free(q); free(k); free(v); free(o); free(l);
  }
  /* conv: BLOCK_OW = 512 with OW = 700 (a ragged last tile), 513 rejected */
  {
    const int64_t B = 1, C = 2, H = 3, W = 700, K = 3;
    float *x = buf(B * C * H * W), *w = buf(C * C * K * K), *b = buf(C), *y = buf(B * C * H * W);
    bad |= oracle_conv2d_forward(x, w, b, y, B, C, C, H, W, H, W, K, K, 1, 1, 1, 1, 1, 512, 0, -1) != 0;
    bad |= oracle_conv2d_forward(x, w, b, y, B, C, C, H, W, H, W, K, K, 1, 1, 1, 1, 1, 513, 0, -1) == 0;
    free(x); free(w); free(b); free(y);
  }
  /* layernorm with a ragged last BLOCK_N tile */
  {
    const int64_t M = 3, N = 1000;
    float *x = buf(M * N), *y = buf(M * N), *w = buf(N), *b = buf(N);
    bad |= oracle_layer_norm_forward_inference(x, y, w, b, M, N, 1e-5f, 256, 0, -1) != 0;
    free(x); free(y); free(w); free(b);
  }
  printf("oracle bounds: %s\n", bad ? "FAILED" : "ok");
  return bad;
}
