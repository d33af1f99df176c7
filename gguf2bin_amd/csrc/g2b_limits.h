/*
 * g2b_limits.h - sizes shared by the device runtime (g2b_api.hip) and the
 * HBM budget (host/g2b_budget.c, C99), so that the budget bounds what the
 * runtime allocates.  Plain C.
 */
#ifndef G2B_LIMITS_H
#define G2B_LIMITS_H
#include <stdint.h>

/* Readable slack after each KV cache: the specialised loaders fetch whole
 * dwords around 34-byte blocks. */
#define G2B_KV_SLACK 256u
/* Floats of one split partial per q head ahead of the accumulator: running
 * max, sum and two pad floats. */
#define G2B_PART_HEAD 4u
/* Work-queue counters: one 128-byte line per (sequence, layer) unit plus one,
 * two sets, at least 256 lines per set. */
#define G2B_WQ_LINE_BYTES 128u
#define G2B_WQ_MIN_LINES 256u
/* Batch descriptor bytes per sequence (SeqDev), at least 64 descriptors. */
#define G2B_SEQ_DESC_BYTES 32u
#define G2B_SEQ_DESC_MIN 64u
/* k_short's span counters: one int32 per (layer of a call, sequence, KV
 * head), at least this many. */
#define G2B_SPAN_CTR_MIN 1024u
/* Work-queue home units: one int32 per workgroup of a launch, at most this
 * many (the resident workgroups of a device: 256 CUs x 8 workgroups, twice). */
#define G2B_HOME_ENTRIES 4096u
/* What one device allocation may take beyond its size (hipMalloc rounds
 * allocations up to pages; 2 MiB covers every size class). */
#define G2B_ALLOC_GRAIN (2u << 20)

/* Split partials per layer of a call: every call keeps n_seq * max_splits at
 * or below this (the schedule lengthens its splits, or caps the work-queue
 * visits per unit, to stay under it). */
static inline uint64_t g2b_splits_per_layer_cap(int32_t n_seq) {
  const uint64_t s = 64u * (uint64_t)(n_seq > 0 ? n_seq : 1);
  return s < 2048u ? 2048u : s;
}

#endif
