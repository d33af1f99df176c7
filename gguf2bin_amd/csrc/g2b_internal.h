// g2b_internal.h - parameter blocks and launchers shared between the C ABI
// (g2b_api.hip) and the kernel translation units.  Not installed.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "g2b_device.h"

namespace g2b {

// Partial state of one split for one q head:
// [m, l, 0, 0, acc[head_dim]] in the log2 domain (m = running max of the
// scaled scores, l = sum of exp2(score - m), acc = sum of exp2(score - m)*v).
constexpr int kPartHead = 4;
constexpr int kWavesPerSplit = 4;      // waves of a 256-thread split workgroup
constexpr int kThreads = 256;
constexpr int kGenericMaxSplit = 1024;  // positions per split in the generic kernel


struct AppendParams {
  ShapeDev sh;
  const SeqDev *seqs;  // nullptr: use `one`
  SeqDev one;
  int32_t n_seq, layer0;
  const float *q_in;   // [L][n_seq][nq] (nullptr in row-prefill mode)
  float *q_rot;        // [L][n_seq][nq]
  const float *k_in;   // [L][n_seq][nkv]  or [n_rows][nkv] in row-prefill mode
  const float *v_in;
  const float *rope;   // [rope_len][head_dim] cos/sin pairs, or nullptr
  NormDev norm;        // QK-RMSNorm weights (norm.w == nullptr: none)
  int32_t pos0;        // row-prefill mode: first position
};

struct DecodeParams {
  ShapeDev sh;
  const SeqDev *seqs;
  SeqDev one;
  int32_t n_seq, layer0;
  int32_t split_len, max_splits;
  const float *q_rot;  // [L][n_seq][nq] rotated q (generic path)
  float *q_out;        // [L][n_seq][nq]: the output overwrites q
  const float *q_in;   // [L][n_seq][nq] pre-RoPE q (single-launch path; == q_out)
  const float *k_in;   // [L][n_seq][nkv] pre-RoPE new k (single-launch path)
  const float *v_in;   // [L][n_seq][nkv] new v (single-launch path)
  const float *rope;   // [rope_len][head_dim] cos/sin pairs, or nullptr
  NormDev norm;        // QK-RMSNorm weights (norm.w == nullptr: none)
  float *part;         // [L][n_seq][n_heads][max_splits][kPartHead+hd]
  float *att;          // nullable: [L][n_seq][n_heads][att_stride]
  int32_t att_stride;
  float qscale;        // (1/sqrtf(hd)) * log2(e)
  int32_t tune_unroll; // 0 = default, else wave-steps per loop trip (2 or 4)
  int32_t tune_chunk;  // 0 = default, else elements per lane for Q8 (16 or 32)
};

// Launchers: return hipSuccess or the launch error.
hipError_t launch_append_batch(const AppendParams &p, int n_layers, hipStream_t s);
hipError_t launch_append_rows(const AppendParams &p, int layer, int n_rows, hipStream_t s);
// Specialised shapes: one launch does RoPE, append and attention (k_layer).
// Generic shapes: launch_append_batch, then this (k_decode_generic).  Both
// are followed by launch_combine.  *used_fast tells which ran.
// Returns hipErrorInvalidValue when split_len is too large for the generic kernel.
hipError_t launch_decode(const DecodeParams &p, int n_layers, hipStream_t s, int *used_fast);
hipError_t launch_combine(const DecodeParams &p, int n_layers, hipStream_t s);
// Whether a specialised decode kernel exists for this shape.
bool decode_fast_available(const ShapeDev &sh);
// Resident 256-thread decode workgroups per CU for this shape (occupancy).
int decode_blocks_per_cu(const ShapeDev &sh);

// Synthetic fill (bench / full-size tests): see g2b_synth.h.
struct SynthParams {
  ShapeDev sh;
  uint8_t *k, *v;
  int32_t ctx_cap, layer0, pos0, n_pos;
  uint64_t base_seed;
  int32_t seq;
  float sel_threshold;  // scale a K row x8 when its selector draw exceeds this
  const float *rope;
};
hipError_t launch_synth_fill(const SynthParams &p, int n_layers, hipStream_t s);
hipError_t launch_synth_normal(float *out, uint64_t n, uint64_t seed, hipStream_t s);
hipError_t launch_copy16(void *dst, const void *src, uint64_t n16, hipStream_t s);

}  // namespace g2b
