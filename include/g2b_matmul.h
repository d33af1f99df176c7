/*
 * g2b_matmul.h - device weight GEMVs of gguf2bin2 (C ABI, implemented in HIP
 * by gguf2bin_amd/libg2b_attn.so next to g2b_attn.h).
 *
 * model_forward multiplies every layer's activations by Q/K/V/Wo and the FFN
 * weights through matmul_q (src/l2_codec.c:342-360), which runs the fused
 * kernels matmul_q8_0 (:203-247 AVX2, :306-320 scalar), matmul_q4_0
 * (:249-304, :321-340) and the F32 matmul (src/l3_math.c:17-20) on the CPU,
 * and every other type through a dequantising fallback (:350-366: each row
 * through gguf_dequant, :186-199, then an fp32 dot).  These entry points run
 * the same products on the context's device with the weights resident in
 * HBM, for F32, Q8_0, Q4_0 and the fallback's F16 and Q4_1.  Type ids are
 * GGML's (include/g2b.h:13-14).
 *
 * Results: fp32 arithmetic like the reference (per-block fp32 sums times the
 * fp16 scale, then a sum over blocks); not the reference's summation order, so
 * outputs agree to fp32 rounding (|out - exact| <= 64 * 2^-24 * sum_j
 * |w_ij x_j|), not bit for bit.
 *
 * Not supported (G2B_EUNSUP): the K-quants.  The reference's gguf_dequant
 * writes only part of each 256-element block for Q3_K, Q4_K, Q5_K and Q6_K
 * (the rest of the fallback's row buffer keeps what an earlier row left),
 * reads past each block for Q2_K, and has no case for Q8_K - there is no
 * defined result to reproduce.
 */
#ifndef G2B_MATMUL_H
#define G2B_MATMUL_H
#include <stddef.h>
#include <stdint.h>

#include "g2b_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { G2B_T_F32 = 0, G2B_T_F16 = 1, G2B_T_Q4_0 = 2, G2B_T_Q4_1 = 3, G2B_T_Q8_0 = 8 };

/* Bytes of one weight row of n elements (row_stride, l2_codec.c:340): n*4
 * (F32), n*2 (F16), (n/32)*34 (Q8_0), (n/32)*18 (Q4_0), (n/32)*20 (Q4_1); 0
 * for any other type or n < 0. */
size_t g2b_matmul_row_bytes(int32_t type, int32_t n);

/* matmul_q (l2_codec.c:342-349) on the device: out[i] = sum_j W[i][j] x[j]
 * for i < d, with W = w's d rows of g2b_matmul_row_bytes(type, n) bytes.
 * Q8_0 / Q4_0 use the n/32 whole blocks of a row, as the reference does;
 * Q4_1 needs n a multiple of 32 (G2B_EINVAL otherwise: the reference's
 * fallback would dequantise past its n-element row buffer).
 * out, x, w: device pointers (w 2-byte aligned: blocks are read as dwords
 * from the 4-byte boundary at or before each block).  As in the reference,
 * a null x or w or n <= 0 or d <= 0 writes zeros to out (when out and d > 0)
 * and succeeds.  Other types: G2B_EUNSUP (above).
 * Asynchronous on the context's stream. */
int g2b_matmul(g2b_ctx *ctx, float *out, const float *x, const void *w, int32_t type, int32_t n,
               int32_t d);

/* Same with out and x in host memory (the reference keeps them in m->buf);
 * w stays a device pointer.  Returns when out holds the result. */
int g2b_matmul_host(g2b_ctx *ctx, float *out, const float *x, const void *w, int32_t type,
                    int32_t n, int32_t d);

/* Weight residency: allocate `bytes` of HBM on the context's device, copy
 * `host` into it when non-null (synchronously), and return the pointer. */
int g2b_weights_upload(g2b_ctx *ctx, const void *host, uint64_t bytes, void **dev);
int g2b_weights_free(g2b_ctx *ctx, void *dev);

#ifdef __cplusplus
}
#endif
#endif
