/*
 * g2b_attn.h - C ABI of the MI355X (gfx950) decode-attention path for
 * gguf2bin2.  Plain C99 types and pointers only; implemented in HIP by
 * gguf2bin_amd/libg2b_attn.so.
 *
 * The reference has no plugin API: the path is inline in model_forward.  Each
 * entry point below replaces one piece of it, cited as file:line into the
 * reference (AnonymoDGH/gguf2bin):
 *   - KV sizing / allocation / release ....... src/l5_model.c:47,120-149,113-119,197-203
 *   - RoPE(q,k) + kv_store + scores + softmax + V-accumulate, output over q
 *                                             .. src/l5_model.c:513-578
 *   - the pos check that aborts a forward ..... src/l5_model.c:469-474
 *
 * Layout contract (unchanged from the reference, src/l5_model.c:131-147,
 * :232-247): per sequence, K and V are two separate buffers laid out
 * [n_layers][ctx_cap][row], row = ceil(nkv/32)*34 bytes for Q8_0 (34-byte
 * blocks: little-endian fp16 scale, then 32 x int8) and nkv*4 bytes for F32,
 * nkv = n_kv_heads*head_dim.  The layer stride uses the effective context
 * ctx_cap (Model.ctx), not seq_len.
 *
 * Caches are 16-byte aligned device buffers (g2b_kv_alloc's are; the decode
 * kernels read them in 16-byte pieces): a misaligned cache is G2B_EINVAL.
 *
 * Conventions: 0 on success, a negative G2B_E* code on error; nothing
 * aborts or exits (the reference's model_set_ctx/alloc_rt return -1,
 * model_forward returns early).  Device pointers are HIP device addresses on
 * the context's device.  Calls are ordered on the context's stream; the
 * device-pointer entry points are asynchronous (g2b_sync waits), the *_host
 * entry points are synchronous like the reference.  One context serves one
 * Model (the reference model_forward is single-threaded per Model); distinct
 * contexts share no mutable state.
 */
#ifndef G2B_ATTN_H
#define G2B_ATTN_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  G2B_OK = 0,
  G2B_EINVAL = -1,  /* bad argument or shape (model_set_ctx: -1, l5_model.c:167)   */
  G2B_EPOS = -2,    /* pos outside [0, ctx_cap) (model_forward, l5_model.c:469-474) */
  G2B_ENOKV = -3,   /* KV buffers missing (model_forward, l5_model.c:481-483)       */
  G2B_ENOMEM = -4,  /* device allocation failed (alloc_rt, l5_model.c:129,143,146) */
  G2B_EDEVICE = -5, /* HIP runtime or launch failure                                */
  G2B_ESWAP = -6,   /* file-backed KV (model_enable_swap, l5_model.c:153-163) cannot
                       live in HBM: the caller keeps the CPU path for it            */
  G2B_EUNSUP = -7   /* shape outside what this build implements                     */
};

/* Reference arch ids (include/g2b.h:17): ARCH_LLAMA rotates interleaved
 * pairs, every other arch rotates NEOX half-split pairs (l5_model.c:448-452). */
enum { G2B_ARCH_LLAMA = 0, G2B_ARCH_QWEN2 = 1, G2B_ARCH_QWEN3 = 2 };

/* The ModelCfg fields and Model flag the path reads (include/g2b.h:51-55,
 * :77-78, F_KV_Q8 :18). */
typedef struct {
  int32_t n_layers, n_heads, n_kv_heads, head_dim;
  float rope_theta;
  int32_t arch;  /* G2B_ARCH_* */
  int32_t kv_q8; /* nonzero: Q8_0 KV cache (m->flags & F_KV_Q8) */
} g2b_shape;

/* One sequence of a batch: its own Model's KV and position. */
typedef struct {
  int32_t pos;     /* position of the new token; attends to t <= pos   */
  int32_t ctx_cap; /* capacity of this sequence's KV (its Model.ctx)   */
  void *kcache;    /* device, [n_layers][ctx_cap][row]                 */
  void *vcache;    /* device, [n_layers][ctx_cap][row]                 */
} g2b_seq;

typedef struct g2b_ctx g2b_ctx;

/* Context on `device` for one model shape.  Validates the shape: n_heads a
 * multiple of n_kv_heads (group = n_heads/n_kv_heads, l5_model.c:465),
 * head_dim even (RoPE pairs), nkv >= 1.  head_dim > 1024 is accepted and, as
 * in the reference (l3_math.c:67,86), leaves q and k unrotated. */
int g2b_ctx_create(g2b_ctx **out, int32_t device, const g2b_shape *shape);
int g2b_ctx_destroy(g2b_ctx *ctx);
/* Launch on `hip_stream` (a hipStream_t; NULL restores the context's own
 * stream).  Streams must have the default priority. */
int g2b_ctx_set_stream(g2b_ctx *ctx, void *hip_stream);
void *g2b_ctx_stream(g2b_ctx *ctx);
const char *g2b_strerror(int32_t code);
/* Text of the last error this context recorded ("" if none). */
const char *g2b_ctx_last_error(g2b_ctx *ctx);

/* kv_q8_rowsize(nkv) for Q8_0 or nkv*4 for F32 (l5_model.c:47,131-132). */
size_t g2b_kv_row_bytes(const g2b_shape *shape);
/* Bytes of ONE of the two caches (alloc_rt's `half`, l5_model.c:131-132). */
uint64_t g2b_kv_bytes(const g2b_shape *shape, int32_t ctx_cap);
/* Byte offset of (layer, pos) inside one cache (l5_model.c:232-234,239-240). */
uint64_t g2b_kv_offset(const g2b_shape *shape, int32_t ctx_cap, int32_t layer, int32_t pos);

/* HBM budgeting (host arithmetic; no device needed).
 * g2b_model_kv_bytes: model_kv_bytes (l5_model.c:195-203), K+V bytes of one
 *   sequence at the full seq_len in the given mode (0 when seq_len <= 0).
 * g2b_clamp_ctx: model_set_ctx's clamp (l5_model.c:166-169): ctx <= 0 -> 256,
 *   then at most seq_len when seq_len > 0.
 * g2b_hbm_bytes: an upper bound of the HBM that one context serving n_seq
 *   sequences of the shape at context ctx allocates - their K and V caches
 *   and the context's buffers for any call form, g2b_attn_layers over all
 *   layers in one call included: the RoPE table (up to max(2*ctx, 256)
 *   positions), the split partials (at most max(2048, 64*n_seq) splits per
 *   layer of a call, n_heads x (4+head_dim) floats each), the generic path's
 *   rotated q, the work-queue counters, the batch descriptors, the
 *   QK-RMSNorm weights and the host entry point's staging, each allocation
 *   rounded up to 2 MiB.  Takes the place of est_for (l5_model.c:174-187),
 *   whose host buffers and tokenizer are not in HBM.  0 for a bad shape,
 *   ctx <= 0 or n_seq < 1.
 * g2b_auto_budget: model_auto_budget (l5_model.c:218-230) against an HBM
 *   budget for n_seq sequences: starting from kv_q8 = shape->kv_q8 and
 *   ctx = seq_len (2048 when seq_len <= 0), switch to Q8_0 if F32 does not
 *   fit, halve ctx (integer halving) while ctx > 256 and it does not fit, and
 *   clamp as g2b_clamp_ctx.  Writes the chosen mode and context; returns
 *   G2B_OK when g2b_hbm_bytes fits the budget, G2B_ENOMEM when even the
 *   smallest context tried does not (where the reference prints a warning and
 *   goes on), G2B_EINVAL for a bad shape, budget 0, n_seq < 1 or null outputs
 *   (the reference returns -1 for budget 0 or no layers). */
uint64_t g2b_model_kv_bytes(const g2b_shape *shape, int32_t seq_len, int32_t kv_q8);
int32_t g2b_clamp_ctx(int32_t ctx, int32_t seq_len);
uint64_t g2b_hbm_bytes(const g2b_shape *shape, int32_t ctx, int32_t kv_q8, int32_t n_seq);
int g2b_auto_budget(const g2b_shape *shape, int32_t seq_len, int32_t n_seq, uint64_t budget,
                    int32_t *kv_q8, int32_t *ctx);
/* Free and total HBM of the context's device (hipMemGetInfo), e.g. as the
 * budget of g2b_auto_budget. */
int g2b_hbm_info(g2b_ctx *ctx, uint64_t *free_bytes, uint64_t *total_bytes);

/* alloc_rt's KV half (l5_model.c:141-147) in HBM: two zeroed device buffers
 * of g2b_kv_bytes(ctx_cap) each.  Also extends the context's RoPE table to
 * ctx_cap positions.  ctx_cap must be >= 1 (model_set_ctx clamps before
 * calling alloc_rt, l5_model.c:168-169). */
int g2b_kv_alloc(g2b_ctx *ctx, int32_t ctx_cap, void **kcache, void **vcache);
/* free_rt's KV part (l5_model.c:117-118). */
int g2b_kv_free(g2b_ctx *ctx, void *kcache, void *vcache);
/* Copy nbytes of a device cache from byte offset `offset` into host memory
 * and wait: what reading Model.kcache/kcq directly does on the host (e.g.
 * kv_key_row, l5_model.c:248-265, or a tool comparing caches). */
int g2b_kv_read(g2b_ctx *ctx, const void *cache, uint64_t offset, uint64_t nbytes, void *host);

/* QK-RMSNorm of one layer: with F_QK_NORM set, model_forward runs
 * qk_rmsnorm (l3_math.c:107-114) on q with attn_q_norm and on the new k with
 * attn_k_norm before RoPE, each when the layer has that slot
 * (l5_model.c:505-511).  q_norm, k_norm: host arrays of head_dim floats
 * (copied), or NULL for none; NULL for both turns the layer's norm off.
 * eps is ModelCfg.eps, one value per model: a different eps while another
 * layer has weights set is G2B_EINVAL.  Applies to every later call that
 * touches the layer, the prefill append included.  Waits for the context's
 * stream. */
int g2b_set_qk_norm(g2b_ctx *ctx, int32_t layer, const float *q_norm, const float *k_norm,
                    float eps);

/* Prefill append: for t in [pos0, pos0+n_rows), [QK-RMSNorm and] RoPE k_t at
 * position t and store k_t, v_t at (layer, t) - the kv_store of
 * l5_model.c:505-516 applied row by row.  k, v: device, [n_rows][nkv] fp32,
 * pre-norm and pre-RoPE. */
int g2b_kv_append_rows(g2b_ctx *ctx, void *kcache, void *vcache, int32_t ctx_cap,
                       int32_t layer, int32_t pos0, int32_t n_rows,
                       const float *k, const float *v);

/* Stage a batch of n_seq sequences (host array).  Each pos must be in
 * [0, ctx_cap) (G2B_EPOS otherwise) and each cache non-null (G2B_ENOKV).
 * The batch stays current until the next g2b_batch_begin. */
int g2b_batch_begin(g2b_ctx *ctx, int32_t n_seq, const g2b_seq *seqs);

/* The decode-attention path (l5_model.c:505-578) for every sequence of the
 * current batch and layers [layer0, layer0+n_layers):
 *   [QK-RMSNorm of q and k where g2b_set_qk_norm gave the layer weights]
 *   RoPE(q), RoPE(k) -> store k, v at (layer, pos) -> scores over t <= pos
 *   scaled by 1/sqrt(head_dim) -> softmax -> q := sum_t w_t v_t.
 * q: device [n_layers][n_seq][n_heads*head_dim], overwritten by the output
 * exactly as the reference overwrites q (l5_model.c:541-557).
 * k, v: device [n_layers][n_seq][n_kv_heads*head_dim], pre-norm and pre-RoPE;
 * not written.
 * att: NULL, or device [n_layers][n_seq][n_heads][att_stride] receiving the
 * softmax weights of t <= pos in the reference att[h*ctx+t] layout
 * (l5_model.c:486,537,540); att_stride >= max pos+1 of the batch.
 * Asynchronous on the context's stream. */
int g2b_attn_layers(g2b_ctx *ctx, int32_t layer0, int32_t n_layers,
                    float *q, const float *k, const float *v,
                    float *att, int32_t att_stride);

/* Single-sequence, single-layer form of the two calls above: the literal
 * replacement of l5_model.c:513-578 inside the layer loop of model_forward.
 * att: NULL or device [n_heads][ctx_cap] (the reference layout). */
int g2b_attn_forward(g2b_ctx *ctx, int32_t layer, int32_t pos, int32_t ctx_cap,
                     void *kcache, void *vcache, float *q, const float *k,
                     const float *v, float *att);

/* The same call, allocating nothing: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Its scratch (the
 * split partials, and the rotated q of shapes without a specialised kernel)
 * is a fixed 2 MiB array in the library's device memory, one per GPU, held
 * until the process ends; every call on a GPU shares that GPU's array, so
 * calls that overlap on one GPU race.  It never uses the work-queue schedule
 * (whose counters need clearing) and lengthens its splits until the partials
 * fit; a shape whose one split does not fit is G2B_EUNSUP.  The RoPE table
 * must already cover pos (g2b_kv_alloc of the cache extends it): G2B_EINVAL
 * otherwise.  No weights output.  Asynchronous like g2b_attn_forward. */
int g2b_attn_forward_noalloc(g2b_ctx *ctx, int32_t layer, int32_t pos, int32_t ctx_cap,
                             void *kcache, void *vcache, float *q, const float *k,
                             const float *v);

/* Same, with q/k/v/att in HOST memory (the reference keeps them in m->buf):
 * copies in, runs, copies the output back over q, and returns when done. */
int g2b_attn_forward_host(g2b_ctx *ctx, int32_t layer, int32_t pos, int32_t ctx_cap,
                          void *kcache, void *vcache, float *q, const float *k,
                          const float *v, float *att);

/* RoPE angle table on the host (C99, this process's C library, as the
 * reference computes it in rope_th_llama/rope_th_neox, l3_math.c:68-73,87-92):
 * freq_0 = 1, freq_{j+1} = freq_j * powf(theta, -2/head_dim) serially,
 * cs[i*head_dim + 2j] = cosf((float)(pos0+i) * freq_j), cs[... + 2j+1] = sinf(..).
 * G2B_EUNSUP when head_dim/2 > 512, G2B_EINVAL for odd head_dim. */
int g2b_rope_table(int32_t pos0, int32_t n_pos, int32_t head_dim, float theta, float *cs);

/* Wait for all work queued on the context's stream. */
int g2b_sync(g2b_ctx *ctx);

#ifdef __cplusplus
}
#endif
#endif
