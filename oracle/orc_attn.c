/*
 * orc_attn.c - one decode-attention layer as the reference runs it, and the
 * batched CPU baseline.  TEST INFRASTRUCTURE ONLY (see orc.h).
 *
 * Follows /root/reference/src/l5_model.c:461-474 (pos check), :513-516
 * (RoPE, append), :518-557 (__AVX2__ scores / softmax / V) and :558-577
 * (scalar branch).  The AVX2 order is reproduced with scalar fmaf() over the
 * same lanes: four 8-lane accumulators s0..s3 over 32-element steps, reduced
 * as ((s0+s1)+(s2+s3)), then 128-bit halves, then movehl, then lane 1, then
 * a non-fused scalar tail for head_dim % 32.  fmaf() is exact fused
 * multiply-add, which is what _mm256_fmadd_ps computes lane by lane.
 */
#include "orc.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* kv_key_row / kv_val_row (l5_model.c:248-265): full row -> nkv floats. */
static void orc_fetch_row(const orc_shape *s, const uint8_t *cache, int32_t ctx_cap,
                          int32_t layer, int32_t t, float *row) {
  int32_t nkv = s->n_kv_heads * s->head_dim;
  const uint8_t *p = cache + orc_kv_offset(s, ctx_cap, layer, t);
  if (s->kv_q8) orc_q8_dequant_row(p, row, nkv);
  else memcpy(row, p, (size_t)nkv * 4u);
}

/* dot product in the lane order of l5_model.c:524-536 */
static float orc_dot_avx2_order(const float *a, const float *b, int32_t n) {
  float acc[4][8];
  memset(acc, 0, sizeof acc);
  int32_t jj = 0;
  for (; jj + 31 < n; jj += 32)
    for (int r = 0; r < 4; r++)
      for (int l = 0; l < 8; l++)
        acc[r][l] = fmaf(a[jj + 8 * r + l], b[jj + 8 * r + l], acc[r][l]);
  float ss[8], lo[4];
  for (int l = 0; l < 8; l++) ss[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
  for (int l = 0; l < 4; l++) lo[l] = ss[l] + ss[l + 4];
  float m0 = lo[0] + lo[2], m1 = lo[1] + lo[3]; /* add with movehl */
  float s = m0 + m1;                            /* add_ss with lane 1 */
  for (; jj < n; jj++) s += a[jj] * b[jj];
  return s;
}

static float orc_dot_scalar_order(const float *a, const float *b, int32_t n) {
  float s = 0.f;
  for (int32_t j = 0; j < n; j++) s += a[j] * b[j];
  return s;
}

int orc_attn_layer(const orc_shape *s, int32_t ctx_cap, int32_t layer, int32_t pos,
                   uint8_t *kcache, uint8_t *vcache, float *q_inout,
                   const float *k_in, const float *v_in, float *att, int avx2_order) {
  if (pos < 0 || pos >= ctx_cap || layer < 0 || layer >= s->n_layers) return -1;
  const int32_t hd = s->head_dim, nh = s->n_heads;
  const int32_t nkv = s->n_kv_heads * hd, nq = nh * hd;
  int32_t group = s->n_kv_heads > 0 ? nh / s->n_kv_heads : 1; /* l5_model.c:465-466 */
  if (group < 1) group = 1;

  float *row = (float *)malloc((size_t)nkv * sizeof(float));
  if (!row) return -1;

  orc_rope(s->arch, q_inout, nq, pos, hd, s->rope_theta);
  orc_kv_append(s, ctx_cap, layer, pos, kcache, vcache, k_in, v_in);

  const float scale = 1.f / sqrtf((float)hd); /* l5_model.c:518 */
  for (int32_t t = 0; t <= pos; t++) {
    orc_fetch_row(s, kcache, ctx_cap, layer, t, row);
    for (int32_t h = 0; h < nh; h++) {
      const float *qh = q_inout + (size_t)h * hd;
      const float *kt = row + (size_t)(h / group) * hd;
      float d = avx2_order ? orc_dot_avx2_order(qh, kt, hd) : orc_dot_scalar_order(qh, kt, hd);
      att[(size_t)h * ctx_cap + t] = d * scale;
    }
  }
  for (int32_t h = 0; h < nh; h++) orc_softmax(att + (size_t)h * ctx_cap, pos + 1);
  for (int32_t j = 0; j < nq; j++) q_inout[j] = 0.f;
  for (int32_t t = 0; t <= pos; t++) {
    orc_fetch_row(s, vcache, ctx_cap, layer, t, row);
    for (int32_t h = 0; h < nh; h++) {
      float w = att[(size_t)h * ctx_cap + t];
      const float *vh = row + (size_t)(h / group) * hd;
      float *oh = q_inout + (size_t)h * hd;
      int32_t jj = 0;
      if (avx2_order)
        for (; jj + 31 < hd; jj += 32)
          for (int l = 0; l < 32; l++) oh[jj + l] = fmaf(w, vh[jj + l], oh[jj + l]);
      for (; jj < hd; jj++) oh[jj] += w * vh[jj];
    }
  }
  free(row);
  return 0;
}

int orc_attn_batch(const orc_shape *s, int32_t layer0, int32_t n_layers, int32_t n_seq,
                   const int32_t *pos, const int32_t *ctx_cap,
                   uint8_t *const *kcache, uint8_t *const *vcache,
                   float *q_inout, const float *k_in, const float *v_in,
                   int n_threads) {
  const int32_t nq = s->n_heads * s->head_dim, nkv = s->n_kv_heads * s->head_dim;
  int failures = 0;
  int32_t max_cap = 1;
  for (int32_t i = 0; i < n_seq; i++)
    if (ctx_cap[i] > max_cap) max_cap = ctx_cap[i];
#ifdef _OPENMP
  int nt = n_threads > 1 ? n_threads : 1;
#pragma omp parallel num_threads(nt) reduction(+ : failures)
#endif
  {
    float *att = (float *)malloc((size_t)s->n_heads * (size_t)max_cap * sizeof(float));
    if (!att) failures += 1;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int32_t i = 0; i < n_seq; i++) {
      if (!att) continue;
      for (int32_t l = 0; l < n_layers; l++) {
        size_t slot = (size_t)l * (size_t)n_seq + (size_t)i;
        int rc = orc_attn_layer(s, ctx_cap[i], layer0 + l, pos[i], kcache[i], vcache[i],
                                q_inout + slot * (size_t)nq, k_in + slot * (size_t)nkv,
                                v_in + slot * (size_t)nkv, att, 1);
        if (rc) failures += 1;
      }
    }
    free(att);
  }
  return failures;
}
