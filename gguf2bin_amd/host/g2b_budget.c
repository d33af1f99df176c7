/*
 * g2b_budget.c - HBM budgeting of the KV caches, C99, host only.
 *
 * The reference sizes its runtime for a RAM budget:
 *   - model_kv_bytes (/root/reference/src/l5_model.c:195-203): K+V bytes at
 *     the model's full seq_len in a given KV mode;
 *   - est_for (:174-187): the resident runtime, KV plus host buffers and the
 *     tokenizer;
 *   - model_auto_budget (:218-230): first switch the KV to Q8_0 if F32 at the
 *     starting context does not fit, then halve ctx (integer halving, not
 *     below 256) while the estimate exceeds the budget, then model_set_ctx,
 *     whose clamp (:166-169) maps ctx <= 0 to 256 and caps it at seq_len.
 * Here the same decision is taken against an HBM budget for n_seq sequences
 * of one shape (one Model each).  What lives in HBM is their KV caches and
 * the decode path's scratch (g2b_hbm_bytes); the reference's host buffers,
 * tokenizer and weights are not part of it.
 */
#include "g2b_attn.h"
#include "../csrc/g2b_limits.h"

/* kv_q8_rowsize (l5_model.c:47) or nkv*4, for the given mode. */
static uint64_t row_bytes_mode(const g2b_shape *s, int32_t kv_q8) {
  const uint64_t nkv = (uint64_t)s->n_kv_heads * (uint64_t)s->head_dim;
  return kv_q8 ? (nkv + 31u) / 32u * 34u : nkv * 4u;
}

static int shape_ok(const g2b_shape *s) {
  return s && s->n_layers > 0 && s->n_heads > 0 && s->n_kv_heads > 0 && s->head_dim > 0;
}

uint64_t g2b_model_kv_bytes(const g2b_shape *s, int32_t seq_len, int32_t kv_q8) {
  if (!shape_ok(s) || seq_len <= 0) return 0;
  return 2u * (uint64_t)s->n_layers * (uint64_t)seq_len * row_bytes_mode(s, kv_q8);
}

int32_t g2b_clamp_ctx(int32_t ctx, int32_t seq_len) {
  if (ctx <= 0) ctx = 256;
  if (seq_len > 0 && ctx > seq_len) ctx = seq_len;
  return ctx;
}

static uint64_t grain(uint64_t b) {
  return (b + G2B_ALLOC_GRAIN - 1u) / G2B_ALLOC_GRAIN * G2B_ALLOC_GRAIN;
}

/* The context's own buffers for n_seq sequences at context ctx, for any call
 * form (one layer per call up to all layers in one call), each allocation
 * rounded up to the allocation grain - what g2b_api.hip allocates:
 *   RoPE table: grown by doubling, so at most max(2*ctx, 256) positions of
 *     head_dim floats;
 *   split partials: n_layers x g2b_splits_per_layer_cap(n_seq) splits x
 *     n_heads x (4 + head_dim) floats (a call over fewer layers needs less);
 *   rotated q of the generic path: n_layers x n_seq x nq floats;
 *   work-queue counters: two sets of max(n_layers*n_seq + 1, 256) lines;
 *   batch descriptors: max(n_seq, 64) of them;
 *   QK-RMSNorm weights and flags: n_layers x (2*head_dim + 1) words;
 *   the spanned short kernel's counters: n_layers x n_seq x n_kv_heads words;
 *   the work queue's home units: G2B_HOME_ENTRIES words;
 *   the host entry point's staging: nq + 2*nkv + n_heads*ctx floats. */
static uint64_t ctx_bytes(const g2b_shape *s, int32_t ctx, int32_t n_seq) {
  const uint64_t L = (uint64_t)s->n_layers, nh = (uint64_t)s->n_heads;
  const uint64_t hd = (uint64_t)s->head_dim, ns = (uint64_t)n_seq;
  const uint64_t nq = nh * hd, nkv = (uint64_t)s->n_kv_heads * hd;
  uint64_t rope_pos = 2u * (uint64_t)ctx;
  if (rope_pos < 256u) rope_pos = 256u;
  uint64_t wq_lines = L * ns + 1u;
  if (wq_lines < G2B_WQ_MIN_LINES) wq_lines = G2B_WQ_MIN_LINES;
  const uint64_t descs = ns > G2B_SEQ_DESC_MIN ? ns : G2B_SEQ_DESC_MIN;
  uint64_t span_ctrs = L * ns * (uint64_t)s->n_kv_heads;
  if (span_ctrs < G2B_SPAN_CTR_MIN) span_ctrs = G2B_SPAN_CTR_MIN;
  return grain(rope_pos * hd * 4u) +
         grain(L * g2b_splits_per_layer_cap(n_seq) * nh * (G2B_PART_HEAD + hd) * 4u) +
         grain(L * ns * nq * 4u) +
         grain(2u * wq_lines * G2B_WQ_LINE_BYTES) +
         grain(descs * G2B_SEQ_DESC_BYTES) +
         grain(L * 2u * hd * 4u) + grain(L * 4u) + grain(span_ctrs * 4u) +
         grain((uint64_t)G2B_HOME_ENTRIES * 4u) +
         grain((nq + 2u * nkv + nh * (uint64_t)ctx) * 4u);
}

uint64_t g2b_hbm_bytes(const g2b_shape *s, int32_t ctx, int32_t kv_q8, int32_t n_seq) {
  if (!shape_ok(s) || ctx <= 0 || n_seq < 1) return 0;
  /* alloc_rt's two caches per sequence, with their read slack */
  const uint64_t cache = grain((uint64_t)s->n_layers * (uint64_t)ctx * row_bytes_mode(s, kv_q8) +
                               G2B_KV_SLACK);
  return (uint64_t)n_seq * 2u * cache + ctx_bytes(s, ctx, n_seq);
}

int g2b_auto_budget(const g2b_shape *s, int32_t seq_len, int32_t n_seq, uint64_t budget,
                    int32_t *kv_q8, int32_t *ctx_out) {
  if (!shape_ok(s) || !budget || n_seq < 1 || !kv_q8 || !ctx_out) return G2B_EINVAL;
  int32_t q8 = s->kv_q8 ? 1 : 0;
  int32_t ctx = seq_len > 0 ? seq_len : 2048;
  if (!q8 && g2b_hbm_bytes(s, ctx, 0, n_seq) > budget) q8 = 1;
  while (ctx > 256 && g2b_hbm_bytes(s, ctx, q8, n_seq) > budget) ctx /= 2;
  const int fits = g2b_hbm_bytes(s, ctx, q8, n_seq) <= budget;
  *kv_q8 = q8;
  *ctx_out = g2b_clamp_ctx(ctx, seq_len);
  return fits ? G2B_OK : G2B_ENOMEM;
}
