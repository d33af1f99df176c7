/*
 * orc.h - CPU oracle for the gguf2bin2 decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (gguf2bin_amd/, include/)
 * may include, link or call this.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, and only as the checker or as the timed
 * CPU baseline.
 *
 * It restates, operation by operation, the reference arithmetic of
 *   /root/reference/src/l5_model.c:47-67   (Q8_0 KV row codec)
 *   /root/reference/src/l5_model.c:232-265 (KV layout, append, fetch)
 *   /root/reference/src/l5_model.c:448-452 (RoPE dispatch by arch)
 *   /root/reference/src/l5_model.c:513-578 (scores, softmax, V-accumulate)
 *   /root/reference/src/l3_math.c:6-16,52-56,64-102 (fp16, softmax, RoPE)
 *   /root/reference/src/l3_math.c:107-114  (QK-RMSNorm, l5_model.c:505-511)
 *   /root/reference/src/l2_codec.c:35-54   (fp16 -> fp32)
 * Built with the reference's own flags (-O3 -mavx2 -mfma -std=c99, no
 * -ffast-math) so that the AVX2 branch is reproduced bit for bit.
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   orc_f32_to_half / orc_half_to_float : exhaustive over every fp16 and a
 *       dense fp32 sweep against a spec restatement, and against oracle/_ref.
 *   orc_q8_quant_row / orc_q8_dequant_row : golden vectors from the compiled
 *       reference (tests/golden), enumerated special blocks (zero, tiny amax,
 *       exact .5 ties, +-127 clamp, NaN/Inf, partial block).
 *   orc_rope_table / orc_rope : goldens; pos 0 identity; per-pair norm;
 *       NEOX vs LLaMA pairing with one-hot inputs.
 *   orc_qk_rmsnorm : goldens from the compiled reference (random heads and
 *       special inputs); numpy float32 left-to-right accumulation; float64
 *       closed form; forward goldens of model_forward with F_QK_NORM.
 *   orc_softmax / orc_attn_layer : goldens from the reference model_forward;
 *       float64 brute force on small cases; invariants (weights sum to 1,
 *       q = 0 gives uniform weights, constant V gives V).
 */
#ifndef G2B_ORC_H
#define G2B_ORC_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same numeric values as the reference enums (include/g2b.h:17-18). */
enum { ORC_ARCH_LLAMA = 0, ORC_ARCH_QWEN2 = 1, ORC_ARCH_QWEN3 = 2 };

typedef struct {
  int32_t n_layers, n_heads, n_kv_heads, head_dim;
  float rope_theta;
  int32_t arch;   /* ORC_ARCH_LLAMA selects interleaved pairs, else NEOX */
  int32_t kv_q8;  /* 1 = Q8_0 cache (F_KV_Q8), 0 = F32 cache            */
} orc_shape;

/* ---- seeded synthetic inputs (SplitMix64 -> Box-Muller in double -> f32) ---- */
uint64_t orc_splitmix64(uint64_t *state);
double orc_uniform01(uint64_t *state);            /* (0,1], 53-bit */
void orc_normal_f32(uint64_t *state, float *out, size_t n);

/* ---- fp16 (l3_math.c:6-16, l2_codec.c:35-54) ---- */
uint16_t orc_f32_to_half(float f);
float orc_half_to_float(uint16_t h);
void orc_f32_to_half_n(const float *x, uint16_t *out, size_t n);
void orc_half_to_float_n(const uint16_t *h, float *out, size_t n);

/* ---- Q8_0 KV rows (l5_model.c:47-67) ---- */
size_t orc_q8_rowsize(int32_t nkv);
void orc_q8_quant_row(const float *src, uint8_t *dst, int32_t n);
void orc_q8_dequant_row(const uint8_t *src, float *out, int32_t n);

/* ---- RoPE (l3_math.c:64-102, l5_model.c:448-452) ---- */
/* cs[2j] = cos, cs[2j+1] = sin of pos*freq_j, freq_j built by the serial
 * product freq *= powf(theta, -2/hd).  Returns 0, or -1 when hd/2 > 512
 * (the reference prints a message and leaves x untouched). */
int orc_rope_table(int32_t pos, int32_t head_dim, float theta, float *cs);
void orc_rope(int32_t arch, float *x, int32_t len, int32_t pos, int32_t head_dim,
              float theta);

/* ---- QK-RMSNorm (l3_math.c:107-114), applied before RoPE (l5_model.c:505-511) ---- */
/* Per head h: ss = sum_j x_j*x_j (serial, each product rounded), inv =
 * 1/sqrtf(ss/hd + eps), x_j := (w_j*x_j)*inv.  In place. */
void orc_qk_rmsnorm(float *x, const float *w, int32_t n_heads, int32_t head_dim, float eps);

/* ---- softmax (l3_math.c:52-56) ---- */
void orc_softmax(float *x, int32_t n);

/* ---- KV layout (l5_model.c:232-247) ---- */
size_t orc_kv_row_bytes(const orc_shape *s);
/* byte offset of (layer, pos) inside one K (or V) buffer of capacity ctx_cap */
size_t orc_kv_offset(const orc_shape *s, int32_t ctx_cap, int32_t layer, int32_t pos);
/* RoPE k at pos then store k and v rows into the caches (kv_store). */
void orc_kv_append(const orc_shape *s, int32_t ctx_cap, int32_t layer, int32_t pos,
                   uint8_t *kcache, uint8_t *vcache, const float *k_in, const float *v_in);

/* orc_kv_append over rows [pos0, pos0+n_rows); k_rows/v_rows [n_rows][nkv]. */
void orc_kv_prefill(const orc_shape *s, int32_t ctx_cap, int32_t layer, int32_t pos0,
                    int32_t n_rows, uint8_t *kcache, uint8_t *vcache,
                    const float *k_rows, const float *v_rows);

/*
 * One layer of the decode-attention path for one sequence, exactly as
 * model_forward runs it (l5_model.c:513-578):
 *   RoPE(q), RoPE(k) -> kv_store(layer,pos) -> scores over t<=pos ->
 *   softmax per head -> q := sum_t att*v_t.
 * q_inout: [n_heads*hd] in, attention output out (it overwrites q like the
 * reference).  k_in, v_in: [n_kv_heads*hd], pre-RoPE.  att: scratch
 * [n_heads][ctx_cap]; on return it holds the softmax weights of t<=pos.
 * avx2_order: 1 reproduces the __AVX2__ branch (:519-557), 0 the scalar
 * branch (:558-577).  Returns 0, or -1 when pos is outside [0, ctx_cap)
 * (l5_model.c:469-474; nothing is written then).
 */
int orc_attn_layer(const orc_shape *s, int32_t ctx_cap, int32_t layer, int32_t pos,
                   uint8_t *kcache, uint8_t *vcache, float *q_inout,
                   const float *k_in, const float *v_in, float *att, int avx2_order);

/*
 * CPU baseline: the same layer for n_seq independent sequences (each its own
 * KV buffers, pos and ctx_cap), for layers [layer0, layer0+n_layers).
 * q/k/v are [n_layers][n_seq][...].  n_threads <= 1 runs sequences in turn
 * (the reference attention has no OpenMP); > 1 uses an OpenMP parallel for
 * over sequences.  Returns the number of failed calls.
 */
int orc_attn_batch(const orc_shape *s, int32_t layer0, int32_t n_layers, int32_t n_seq,
                   const int32_t *pos, const int32_t *ctx_cap,
                   uint8_t *const *kcache, uint8_t *const *vcache,
                   float *q_inout, const float *k_in, const float *v_in,
                   int n_threads);

/* Seconds from CLOCK_MONOTONIC (the reference bench clock, src/main.c:456-467). */
double orc_now_sec(void);
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
