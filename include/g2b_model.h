/*
 * g2b_model.h - a whole decode step of gguf2bin2 on the device: the G2BX
 * container parsed on the host, its weights resident in HBM, and
 * model_forward (src/l5_model.c:461-606) run as device kernels (C ABI,
 * implemented by gguf2bin_amd/libg2b_attn.so next to g2b_attn.h and
 * g2b_matmul.h).
 *
 * The container (G2BX, written by g2bx_pack / exp_synth_qwen_tiny,
 * l5_model.c:634-681; read by load_header_body, :286-391): "G2BX", u16
 * version, u8 arch, u8 flags, the packed 40-byte ModelCfg
 * (include/g2b.h:51-54), u32 n_slots, n_slots packed 16-byte Slots (u8 role,
 * u16 layer (0xFFFF = global), u8 GGML type, u32 nbytes, u64 offset into the
 * blob), then the weight blob (data_size = max(offset + nbytes) rounded up to
 * 64), then the tokenizer section (not read here).
 */
#ifndef G2B_MODEL_H
#define G2B_MODEL_H
#include <stddef.h>
#include <stdint.h>

#include "g2b_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Slot roles (include/g2b.h:20-24). */
enum {
  G2B_R_TOK_EMBD = 0, G2B_R_OUT_NORM, G2B_R_OUTPUT,
  G2B_R_ATTN_NORM, G2B_R_ATTN_Q, G2B_R_ATTN_K, G2B_R_ATTN_V, G2B_R_ATTN_O, G2B_R_ATTN_Q_NORM,
  G2B_R_ATTN_K_NORM, G2B_R_FFN_NORM, G2B_R_FFN_GATE, G2B_R_FFN_UP, G2B_R_FFN_DOWN, G2B_R_COUNT
};
/* Model flags (include/g2b.h:18). */
enum { G2B_F_TIE_EMBD = 1, G2B_F_QK_NORM = 2 };

/* ModelCfg (include/g2b.h:51-54). */
typedef struct {
  int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab, seq_len, head_dim;
  float eps, rope_theta;
} g2b_model_cfg;

typedef struct {
  uint8_t role;
  uint16_t layer; /* 0xFFFF: a global slot */
  uint8_t type;   /* GGML type id */
  uint32_t nbytes;
  uint64_t off;   /* into the weight blob */
} g2b_slot;

/* A parsed container: header, slot table and the weight blob in host memory. */
typedef struct {
  uint16_t version;
  uint8_t arch, flags;
  g2b_model_cfg cfg; /* seq_len <= 0 in the file becomes 2048 (l5_model.c:375) */
  uint32_t n_slots;
  g2b_slot *slots;
  uint8_t *data;
  uint64_t data_size;
} g2b_g2bx;

/* load_header_body's parse (l5_model.c:286-301, :368-375): G2B_EINVAL for a
 * missing file, a bad magic, a short header or slot table, or a blob shorter
 * than the slots need ("truncado"); G2B_ENOMEM when the host allocations fail.
 * The blob is read into host memory (the reference maps it). */
int g2b_g2bx_open(const char *path, g2b_g2bx *out);
void g2b_g2bx_close(g2b_g2bx *g);
/* slot_get over the parsed table (l5_model.c:27-31, index of build_index
 * :34-45: a later slot with the same role and layer wins; roles >= R_COUNT and
 * layers >= n_layers are ignored).  layer < 0: the global slot.  NULL if none. */
const g2b_slot *g2b_g2bx_slot(const g2b_g2bx *g, int32_t role, int32_t layer);

typedef struct g2b_model g2b_model;

/* model_load_g2bx (l5_model.c:393-408) onto `device`: parse, upload the blob
 * to HBM, build the attention context for the model's shape and allocate the
 * KV for `ctx` positions (ctx <= 0: seq_len, as model_set_ctx's clamp) in F32
 * or Q8_0 (kv_q8).  The device forward supports matrices and token
 * embeddings in F32, F16, Q8_0, Q4_0 or Q4_1 and norm vectors in F32; other
 * slot types (the K-quants, whose gguf_dequant output the reference leaves
 * undefined, as include/g2b_matmul.h says) are G2B_EUNSUP at load. */
int g2b_model_load_g2bx(g2b_model **out, int32_t device, const char *path, int32_t kv_q8,
                        int32_t ctx);
int g2b_model_free(g2b_model *m);
int g2b_model_info(const g2b_model *m, g2b_model_cfg *cfg, int32_t *arch, int32_t *flags,
                   int32_t *ctx);
/* The attention context the model runs on (stream, tuning, errors). */
g2b_ctx *g2b_model_ctx(g2b_model *m);
/* The model's K and V caches (device, [n_layers][ctx_cap][row] each, in the
 * model's KV mode) and their capacity: what the reference's Model exposes as
 * kcache/vcache or kcq/vcq and ctx (include/g2b.h:82-85), e.g. to fill or
 * read a context with g2b_synth_fill_kv / g2b_kv_read. */
int g2b_model_kv(g2b_model *m, void **kcache, void **vcache, int32_t *ctx_cap);

/* model_forward (l5_model.c:461-606) on the device for `token` at `pos`:
 * embedding row, then per layer rmsnorm, Q/K/V GEMVs, the decode-attention
 * path (QK-RMSNorm, RoPE, KV append, attention: g2b_attn_forward), Wo and the
 * residual, rmsnorm, gate/up GEMVs, SiLU(gate)*up, down and the residual;
 * final rmsnorm and the logits (R_OUTPUT, else the tied R_TOK_EMBD).
 * logits: host array of vocab floats.  As in the reference: pos outside
 * [0, ctx) or token outside [0, vocab) zero the logits and fail (G2B_EPOS /
 * G2B_EINVAL); a missing slot fails with G2B_EINVAL and leaves them. */
int g2b_model_forward(g2b_model *m, int32_t token, int32_t pos, float *logits);

/* on = 1: steps are replayed from HIP graphs, one per position bucket (64,
 * 128, 256, ... positions, the last one the whole context): the first
 * forward in a bucket runs its launches one by one and then captures them
 * (token and pos are read from device memory; the attention is scheduled for
 * the bucket's last position), later forwards in the bucket replay it - one
 * graph launch per step instead of five or six launches per layer.  on = 0
 * (the default): every step is launched eagerly, with the attention
 * scheduled for the step's own position (at short contexts one split and no
 * combine launch: five launches per layer).  Where both schedules cut the
 * context into the same splits (on MI355X, contexts up to 32768) the logits
 * agree bit for bit, else to fp32 summation order.  Changing the fused mode
 * drops the captured steps. */
int g2b_model_use_graph(g2b_model *m, int32_t on);

/* on = 1 (the default): where the weight types allow it (Q8_0 / Q4_0, rows of
 * at most 512 blocks; Q, K and V of one type; gate and up of one type), each
 * layer runs as six launches: rmsnorm + Q/K/V, the attention path (two), Wo
 * + the residual, rmsnorm + gate/up, SiLU(gate) * up + down + the residual;
 * the final rmsnorm goes into the logits GEMV.  on = 0: rmsnorm, SiLU * up
 * and the residual adds as launches of their own, one GEMV per matrix (the
 * path F32 weights always take).  The same arithmetic either way, apart
 * from the order of rmsnorm's fp32 sum of squares.  Changing it drops a
 * captured step; the next forward captures again. */
int g2b_model_set_fused(g2b_model *m, int32_t on);

#ifdef __cplusplus
}
#endif
#endif
