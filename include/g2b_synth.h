/*
 * g2b_synth.h - seeded synthetic inputs generated on the device.
 *
 * These entry points have NO counterpart in the reference: they exist for
 * benchmarks and full-size tests, which need tens of gigabytes of KV that
 * cannot be produced on the host.  They write into caches allocated with
 * g2b_kv_alloc and go through the same RoPE + append arithmetic as
 * g2b_kv_append_rows.
 *
 * Streams: the stream (seq, layer, tensor) has seed
 * g2b_stream_seed(base, seq, layer, tensor); element i of a stream is the
 * i-th float of SplitMix64 -> Box-Muller (double) -> float, pair (2j, 2j+1)
 * taken from generator outputs 2j+1 and 2j+2 as (r*cos, r*sin).  Tensors:
 * 0 = K prefill rows, 1 = V prefill rows, 5 = K row-scale selector.
 * K/V row t uses elements [t*nkv, (t+1)*nkv) of its stream, pre-RoPE.
 */
#ifndef G2B_SYNTH_H
#define G2B_SYNTH_H
#include <stdint.h>

#include "g2b_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { G2B_STREAM_K = 0, G2B_STREAM_V = 1, G2B_STREAM_SEL = 5 };

uint64_t g2b_stream_seed(uint64_t base, int32_t seq, int32_t layer, int32_t tensor);

/* n floats of stream `seed` into device memory `out`. */
int g2b_synth_normal(g2b_ctx *ctx, float *out, uint64_t n, uint64_t seed);

/* Fill rows [pos0, pos0+n_pos) of layers [layer0, layer0+n_layers) of one
 * sequence (`seq` picks its streams): draw k and v, scale a K row by 8 when
 * its selector draw exceeds sel_threshold (pass +INFINITY for none), RoPE k
 * at its position, store (F32) or quantise (Q8_0) both rows.  Asynchronous. */
int g2b_synth_fill_kv(g2b_ctx *ctx, void *kcache, void *vcache, int32_t ctx_cap,
                      int32_t layer0, int32_t n_layers, int32_t pos0, int32_t n_pos,
                      uint64_t base_seed, int32_t seq, float sel_threshold);

/* Plain device copy of nbytes (multiple of 16, 16-byte aligned pointers):
 * the known-size reference kernel used to scale HBM byte counters. */
int g2b_synth_copy(g2b_ctx *ctx, void *dst, const void *src, uint64_t nbytes);

/* Tuning of the decode kernel; 0 keeps the automatic choice for each:
 * split_len = positions per split of the static schedule (automatic: one
 * round of workgroups per launch), chunk = Q8_0 elements per lane (32 = a
 * block, 16 = half a block), stage = how KV rows reach the lanes (-1
 * per-lane loads straight from HBM, 1 chunks of rows pulled into LDS by
 * global_load_lds, 2 chunks loaded into registers one chunk ahead and written
 * to LDS; automatic: 2 wherever the row is a whole number of 16-byte pieces,
 * else -1), piece = the work-queue schedule (-1 static splits only, > 0
 * positions per claimed piece; automatic: work queue when every (sequence,
 * layer) of the call can have a resident workgroup).  Contexts below 128
 * positions without the weights output run the short-context kernel (one
 * workgroup per KV head) unless split_len > 0 or piece != 0 is set. */
int g2b_ctx_tune(g2b_ctx *ctx, int32_t split_len, int32_t chunk, int32_t stage, int32_t piece);

/* Decode kernel choice.  0 automatic: one layer of a single sequence longer
 * than 128 positions whose spans of 128 positions times the KV heads fit one
 * workgroup per CU runs k_short over those spans, which merge their partials
 * in the kernel; k_tiles (K scores on the int8 matrix cores) for
 * Q8_0 KV with head_dim 128, 8 KV heads and 3-4 q heads per KV head when
 * neither the weights output, a chunk nor a stage other than 2 is asked
 * for; else k_layer.  1: k_layer (no k_tiles, no spans).  2: k_tiles where it
 * applies, no spans.  3: spans wherever they apply (any batch), else as 0.
 * Contexts below 128 positions take the single-span k_short in every mode
 * unless g2b_ctx_tune sets a split length or piece. */
int g2b_ctx_tune_kernel(g2b_ctx *ctx, int32_t kernel);

/* The schedule of the last decode call that launched (g2b_attn_layers,
 * g2b_attn_forward and their variants), into out[G2B_SCHED_FIELDS]:
 *   [0] kernel: G2B_KERNEL_LAYER, _TILES, _SHORT or _GENERIC,
 *   [1] positions per split (k_short: per span; 0 under the work queue),
 *   [2] work-queue piece length (0: static splits or spans),
 *   [3] partial slots per (sequence, layer) (splits, spans or queue slots),
 *   [4] workgroups launched,
 *   [5] 1 when the decode kernel wrote the output itself (no combine launch,
 *       or spans merged in the kernel),
 *   [6] how KV rows reach the lanes: 0 per-lane loads straight from HBM,
 *       1 chunks (k_tiles: tiles) pulled into LDS by LDS DMA, 2 chunks
 *       loaded into registers one chunk ahead and written to LDS,
 *   [7] k_layer: row elements per lane (32 = a Q8_0 block, 16); else 0,
 *   [8] 1 when the call wrote the softmax weights.
 * With the shape, [0], [2], [6], [7] and [8] name the kernel instance
 * launched: k_layer<kv_q8, head_dim, [7], group, 2, [8], [6], [2] > 0>, or
 * k_tiles<group, [2] > 0>.  All zero before the first call. */
#define G2B_SCHED_FIELDS 9
#define G2B_KERNEL_LAYER 1
#define G2B_KERNEL_TILES 2
#define G2B_KERNEL_SHORT 3
#define G2B_KERNEL_GENERIC 4
int g2b_ctx_last_schedule(const g2b_ctx *ctx, int32_t *out);

/* Kernel timing with HIP events on the context's stream: while enabled,
 * every decode-kernel launch is bracketed by two events.  _read waits for
 * them, returns the summed milliseconds and the number of launches since
 * the last read, and starts a new window. */
int g2b_ctx_profile(g2b_ctx *ctx, int32_t enable);
int g2b_ctx_profile_read(g2b_ctx *ctx, double *decode_ms, int64_t *launches);

#ifdef __cplusplus
}
#endif
#endif
