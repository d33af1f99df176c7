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

// Staged streaming in k_layer: each wave moves chunks of stage_rows
// contiguous K and V rows into its own LDS region with coalesced 16-byte
// non-temporal loads, and its lanes read their blocks from there.  Needs
// rows that are whole 16-byte pieces.  Mode 1 (global_load_lds straight into
// LDS) and mode 2 (registers one chunk ahead, then LDS) use chunks of about
// 4352 bytes of K (and as much of V); mode 2 at most kStageLoads pieces per
// lane and tensor.  A chunk is a whole number of wave-steps
// (positions_per_wave_step positions each).  0 = not staged.
constexpr int kStageLoads = 5;
__host__ __device__ inline int32_t stage_rows_of(uint32_t row_bytes,
                                                 int32_t positions_per_wave_step, int32_t mode) {
  if (row_bytes == 0 || (row_bytes & 15u) || positions_per_wave_step < 1) return 0;
  if (mode != 1 && mode != 2) return 0;
  const uint32_t target = 4352u;
  const uint32_t per_step = row_bytes * (uint32_t)positions_per_wave_step;
  const uint32_t steps = per_step >= target ? 1u : target / per_step;
  if (mode == 2 && steps * per_step > 1024u * (uint32_t)kStageLoads) return 0;
  return (int32_t)steps * positions_per_wave_step;
}

// k_layer's dynamic LDS: [0, rows) holds the rotated q and the new k and v
// (floats) and a transposed copy of q and k (head_dim x (n_heads +
// n_kv_heads + 1) floats, for the QK-RMSNorm sums) before the stream starts
// and the waves' staging regions (stage_rows > 0) during it;
// then the new K and V rows (row_pad bytes each), n_heads + n_kv_heads
// floats (rounded up to 4) of QK-RMSNorm factors and 3 * head_dim floats of
// setup inputs (the q and k norm weights, the cos/sin row of pos).  After the stream, the wave
// merge of the partials ([wave][head][kPartHead + head_dim] floats) reuses
// everything from 0 (merge_states states per wave).
// Rows the staging regions of layer_lds_layout hold per wave and tensor:
// mode 2 one chunk (the next one waits in registers), mode 1 two (the next
// one is loaded straight into LDS), mode 0 none.
__host__ __device__ inline int32_t layer_stage_rows(int32_t mode, int32_t stage_rows) {
  return mode == 1 ? 2 * stage_rows : mode ? stage_rows : 0;
}
struct LdsLayout {
  uint32_t pre, rows, row_pad, total;  // pre: the setup's bytes at 0
};
// k_layer's position slots per wave that go to the LDS merge as they are
// (1: folded inside the wave first), for lpp lanes per position.  Slots of 32
// or 16 lanes fold through lane swaps; other widths of up to kLdsFoldMax
// slots per wave skip the in-wave fold (a chain of LDS shuffles) and merge
// with the other waves' states in LDS.
constexpr int kLdsFoldMax = 8;
__host__ __device__ inline int layer_merge_states(int lpp) {
  const int ppw = lpp >= 1 && lpp <= 64 ? 64 / lpp : 1;
  return (lpp == 32 || lpp == 16 || ppw <= 1 || ppw > kLdsFoldMax) ? 1 : ppw;
}
// merge_states: layer_merge_states of the variant (the merge area holds that
// many states per wave).
__host__ __device__ inline LdsLayout layer_lds_layout(const ShapeDev &sh, int32_t stage_rows,
                                                      int32_t merge_states = 1) {
  const uint32_t nq = (uint32_t)(sh.n_heads * sh.head_dim);
  const uint32_t nkv = (uint32_t)(sh.n_kv_heads * sh.head_dim);
  const uint32_t pre = nq * 4u + 2u * ((nkv * 4u + 15u) & ~15u) +
                       (uint32_t)(sh.head_dim * (sh.n_heads + sh.n_kv_heads + 1)) * 4u;
  const uint32_t stage = (uint32_t)kWavesPerSplit * 2u * (uint32_t)stage_rows * sh.row_bytes;
  const uint32_t merge = (uint32_t)kWavesPerSplit * (uint32_t)merge_states *
                         (uint32_t)sh.n_heads * (uint32_t)(kPartHead + sh.head_dim) * 4u;
  LdsLayout l;
  l.pre = pre;
  l.row_pad = (sh.row_bytes + 15u) & ~15u;
  l.rows = pre > stage ? pre : stage;
  const uint32_t need =
      l.rows + 2u * l.row_pad +
      (uint32_t)(((sh.n_heads + sh.n_kv_heads + 3) & ~3) + 3 * sh.head_dim) * 4u;
  l.total = need > merge ? need : merge;
  return l;
}


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
  int32_t tune_chunk;  // 0 = default, else elements per lane for Q8 (16 or 32)
  int32_t stage_mode;  // k_layer: 0 direct loads, 1 / 2 staged (stage_rows_of)
  int32_t stage_rows;  // rows per staged chunk (0 with stage_mode 0)
  // Work-queue mode of k_layer (wq != nullptr; stage_mode 2 only): units are
  // (seq, layer) pairs, u = li*n_seq + seq.  wq holds two counter sets of
  // wq_cap units x kWqStride int32 each: [0] = pieces claimed, [1] = partial
  // slots reserved; line n_units holds the next never-assigned unit (used
  // when the grid has fewer workgroups than units).  The launch uses set
  // wq_set; k_combine reads it and zeroes lines [0, wq_zero_units) of the
  // other set.
  int32_t *wq;
  int32_t wq_set, wq_cap, wq_zero_units;
  int32_t wq_grid;      // workgroups of the launch
  // wq_grid entries: the first unit of each workgroup (null: workgroup g
  // starts at unit g % n_units).  Every unit is some workgroup's first.
  const int32_t *home;
  int32_t piece_len;    // positions per small claimed piece (a multiple of stage_rows)
  int32_t piece_big;    // positions per big piece (a multiple of piece_len)
  int32_t n_layers_call;
  // Static schedule with one split per unit (max_splits == 1, no weights
  // output): k_layer writes the normalised output over q itself and no
  // k_combine runs - the value k_combine would give for one partial,
  // (float)((double)acc / (double)l).
  int32_t direct_out;
  int32_t *span_ctr;  // k_short with several spans: [L][n_seq][n_kv_heads] tickets
  // Phase stamps (the library built with G2B_STAMPS only; nullptr in the
  // product build, whose kernels have no stamp code): kStampWords words per
  // workgroup of a static k_layer launch at [g], of its k_combine at
  // [stamp_cap + g], g the linear workgroup id (launches of more than
  // stamp_cap workgroups leave them unwritten).
  uint64_t *stamps;
  int32_t stamp_cap;
};
// Phase stamp words (wall_clock64, 100 MHz): k_layer 0 entry, 1 setup done,
// 2 stream done, 3 fold done, 4 partials stored, 5 exit, 6 split index (work
// queue: visits, phases 1-4 the last visit's), 7 XCD; k_combine 0 entry,
// 5 exit, 7 XCD.
constexpr int kStampWords = 8;
// Grid of a static schedule: x = the splits of a (sequence, layer), the
// fastest index of the linear workgroup order, which the device deals to its
// eight XCDs in turn.  With an even x, sequence q's first split lands on XCD
// (x*q) mod 8 - a few XCDs only - and in a ragged batch its short sequences'
// splits crowd those (c3, 12 splits: 1.28x the average work on the busiest
// XCD).  An odd x (one empty split per sequence more: t0 >= pos+1 for every
// sequence, so it returns at once) starts the sequences on every XCD.
inline dim3 static_grid(const DecodeParams &p, int n_layers) {
  const int x = p.n_seq > 1 ? (p.max_splits | 1) : p.max_splits;
  return dim3((unsigned)x, (unsigned)p.n_seq, (unsigned)n_layers);
}
// The sequence of static-schedule workgroup (y, z) = (blockIdx.y, layer):
// rotated by the layer.  With n_seq a multiple of 8, workgroup (s, y, z)
// lands on XCD (s + x*y) mod 8 in every layer, so without the rotation each
// sequence would run on the same XCD in all layers of a call (c3 over 30
// layers, one split each: the busiest XCD held 1.18x the average work).
__device__ __forceinline__ int static_seq(int y, int z, int n_seq) {
  const int s = y + z;
  return s < n_seq ? s : s % n_seq;
}

constexpr int kWqStride = 32;    // int32 per unit counter pair: one 128-byte line each
constexpr int kWqStealMin = 2;   // unclaimed pieces a unit needs to be worth a visit
constexpr int kWqMinParts = 16;  // partial slots per unit at least
constexpr int kWqClaimsPerWave = 64;   // automatic small piece: about this many per wave
constexpr int kWqUnitPieces = 1024;    // automatic small piece: at most 1/this of a unit
constexpr int kWqMaxWavesPerUnit = 64; // more waves per unit than this: static splits instead
constexpr int kWqBigFactor = 8;        // big piece = this many small pieces
constexpr int kWqTailDiv = 8;          // the last 1/kWqTailDiv of a unit goes in small pieces

// Work-queue pieces of a unit that streams positions [0, n) (guided
// self-scheduling in two sizes): whole big pieces up to n - n/kWqTailDiv,
// then small pieces to the end.  Piece c < nbig covers [c*big, (c+1)*big),
// piece nbig + j covers [small0 + j*small, min(small0 + (j+1)*small, n)).
struct PieceMap {
  int32_t big, small, nbig, small0, npieces;
};
__host__ __device__ inline PieceMap piece_map(int32_t n, int32_t big, int32_t small) {
  PieceMap m;
  m.big = big;
  m.small = small;
  const int32_t head = n - n / kWqTailDiv;
  m.nbig = head > 0 ? head / big : 0;
  m.small0 = m.nbig * big;
  m.npieces = m.nbig + (n - m.small0 + small - 1) / small;
  return m;
}
__host__ __device__ inline void piece_range(const PieceMap &m, int32_t c, int32_t n, int32_t &lo,
                                            int32_t &hi) {
  if (c < m.nbig) {
    lo = c * m.big;
    hi = lo + m.big;
  } else {
    lo = m.small0 + (c - m.nbig) * m.small;
    hi = lo + m.small < n ? lo + m.small : n;
  }
}

// Launchers: return hipSuccess or the launch error.
hipError_t launch_append_batch(const AppendParams &p, int n_layers, hipStream_t s);
hipError_t launch_append_rows(const AppendParams &p, int layer, int n_rows, hipStream_t s);
// Specialised shapes (decode_fast_available, and fast set by the caller):
// one launch does RoPE, append and attention (k_layer).  Otherwise:
// launch_append_batch, then this (k_decode_generic).  Both are followed by
// launch_combine.  *used_fast tells which ran.
// Returns hipErrorInvalidValue when split_len is too large for the generic kernel.
hipError_t launch_decode(const DecodeParams &p, int n_layers, hipStream_t s, bool fast,
                         int *used_fast);
hipError_t launch_combine(const DecodeParams &p, int n_layers, hipStream_t s);
// Whether a specialised decode kernel exists for this shape.
bool decode_fast_available(const ShapeDev &sh);
// k_short (no weights output): RoPE, append and attention with one
// workgroup per (KV head, span of kShortMaxPos positions, sequence, layer);
// DecodeParams.max_splits = the call's spans, ceil((max pos + 1) /
// kShortMaxPos), at most kShortMaxSpans.  A single span writes the output
// over q itself; with several, the spans of a (sequence, layer, KV head)
// write partials and the last to finish merges them (span_ctr: one zeroed
// int32 per (layer of the call, sequence, KV head), left zero again).
constexpr int kShortMaxPos = 128;
constexpr int kShortMaxSpans = 512;
bool short_available(const ShapeDev &sh);
hipError_t launch_short(const DecodeParams &p, int n_layers, hipStream_t s);
// Q8_0 KV with head_dim 128, 8 KV heads and 3 or 4 q heads per KV head, no
// weights output: k_tiles (g2b_tiles.h) does RoPE, append and attention with
// the K scores on the int8 matrix cores, in tiles of kTilesRows positions
// staged per workgroup; schedules (static splits, work queue) and partials
// as k_layer's.
constexpr int kTilesRows = 16;
bool tiles_available(const ShapeDev &sh);
hipError_t launch_tiles(const DecodeParams &p, int n_layers, hipStream_t s);
int tiles_blocks_per_cu(const ShapeDev &sh, bool wq);
// Resident 256-thread decode workgroups per CU for this shape and the
// k_layer variant DecodeParams' tune_chunk / stage_mode / stage_rows / wq
// select (occupancy).
int decode_blocks_per_cu(const ShapeDev &sh, int32_t tune_chunk, int32_t stage_mode,
                         int32_t stage_rows, bool wq);
// DecodeParams.stage_rows for this shape and staging mode (tune_chunk as in
// DecodeParams): 0 when k_layer must load straight from HBM (no specialised
// kernel, or rows that are not whole 16-byte pieces).
int32_t decode_stage_rows(const ShapeDev &sh, int32_t tune_chunk, int32_t mode);
// Positions per wave-step of the specialised kernel (1 for other shapes).
int32_t decode_ppw(const ShapeDev &sh, int32_t tune_chunk);
// Row elements per lane of the k_layer variant launch_layer picks (its CD:
// 32 = a Q8_0 block for groups up to 2, else 16), 0 for other shapes.
int32_t decode_chunk(const ShapeDev &sh, int32_t tune_chunk);
// Staging mode k_layer uses unless tuned otherwise.
constexpr int32_t kDefaultStageMode = 2;
// k_layer for one (KV format 0 = F32 / 1 = Q8_0, head_dim, GQA group),
// defined in g2b_layer.h and instantiated by g2b_layer_inst.hip: the launch,
// and the resident workgroups per CU of the variant a launch would use.
template <int FMT, int HD, int G>
hipError_t launch_layer(const DecodeParams &p, int n_layers, hipStream_t s);
template <int FMT, int HD, int G>
int layer_occupancy(const ShapeDev &sh, int32_t tune_chunk, int32_t stage_mode,
                    int32_t stage_rows, bool wq);

// Device GEMVs (g2b_matmul.hip) for matmul_q's fused types (GGML type ids,
// /root/reference/include/g2b.h:13-14).
constexpr int32_t kTypeF32 = 0, kTypeF16 = 1, kTypeQ4_0 = 2, kTypeQ4_1 = 3, kTypeQ8_0 = 8;
struct GemvParams {
  float *out;          // [d]
  const float *x;      // [n]
  const uint8_t *w;    // d rows of row_bytes
  int32_t n, d;
  int32_t nb;          // blocks per row (Q8_0 / Q4_0: n/32)
  uint32_t row_bytes;
  int32_t steps;       // wave-steps over the rows
  int32_t n_waves;     // waves of the launch
  int32_t vec4;        // F32: 16-byte loads allowed
  int32_t x_vec4;      // Q8_0 / Q4_0: x 16-byte aligned (x kept in registers)
  // Fused forms (Q8_0 / Q4_0 with x in registers only: gemv_fusable).
  // Segments: rows [0, d0) use w / out, [d0, d01) w1 / out1, [d01, d) w2 /
  // out2 - matrices of one type and one n sharing x (Q/K/V, gate/up).  A
  // plain launch has d0 = d01 = d.
  const uint8_t *w1, *w2;
  float *out1, *out2;
  int32_t d0, d01;
  // x as the rows read it: kProNone x; kProRmsnorm (x * nw) * (1 / sqrtf(
  // sum(x^2) / n + eps)); kProSiluMul silu(x) * x2.
  int32_t pro;
  const float *nw, *x2;
  float eps;
  const float *res;    // segment 0: out = res + W x (res may be out itself)
};
constexpr int32_t kProNone = 0, kProRmsnorm = 1, kProSiluMul = 2;
// Whether launch_gemv takes the fused forms for this type and row length.
inline bool gemv_fusable(int32_t type, int32_t n) {
  return (type == kTypeQ8_0 || type == kTypeQ4_0) && n > 0 && n % 32 == 0 && n / 32 <= 512;
}
// Whether launch_gemv runs a plain product of this type and shape on the
// int8 matrix cores (k_gemv_mma: Q8_0 / Q4_0 / Q4_1 rows of 1024 elements,
// at least kGemvMmaMinRows rows - the lm head).
constexpr int32_t kGemvMmaMinRows = 32768;
inline bool gemv_mma_plain(int32_t type, int32_t n, int32_t d) {
  return (type == kTypeQ8_0 || type == kTypeQ4_0 || type == kTypeQ4_1) && n == 1024 &&
         d >= kGemvMmaMinRows;
}
// The prologues keep x * w or SiLU x up of all of x in LDS: n floats within
// 60 KiB.
constexpr int32_t kGemvProMaxN = 15360;
inline bool gemv_fusable_pro(int32_t type, int32_t n) {
  return gemv_fusable(type, n) && n <= kGemvProMaxN;
}
hipError_t launch_gemv(GemvParams p, int32_t type, int n_cu, hipStream_t s);
hipError_t launch_fill_zero(float *out, int32_t n, hipStream_t s);

}  // namespace g2b
struct g2b_ctx;
namespace g2b {
// Decode attention (RoPE, append, attention, combine) of one sequence whose
// descriptor lives in device memory - the kernels read pos from it - with
// the schedule sized for any pos <= max_pos, so the same launches serve
// every step (a captured step graph); the output overwrites q.
int attn_forward_device_seq(g2b_ctx *c, int32_t layer, const SeqDev *d_seq, int32_t max_pos,
                            float *q, const float *k, const float *v);
// The buffers (RoPE table, split partials, counters) of that schedule, with
// nothing launched - before a stream capture, which must not allocate.
int attn_reserve_device_seq(g2b_ctx *c, int32_t max_pos, float *q, const float *k,
                            const float *v);

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
