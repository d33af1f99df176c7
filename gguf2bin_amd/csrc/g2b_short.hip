// g2b_short.hip - k_short: decode attention split by KV head and by spans
// of 128 positions, one workgroup per (KV head, span, sequence, layer).
//
// Same work as k_layer for one (sequence, layer) - l5_model.c:505-516
// (QK-RMSNorm, RoPE, kv_store of the new row) and :518-577 (scores over
// positions 0..pos, softmax with 1/sqrt(hd), V-accumulate, output over q) -
// but split by KV head instead of by positions: at a few hundred positions
// the work is the setup's chain of dependent steps, not the KV bytes (a
// 48-position Qwen3-0.6B layer reads 100 KB), and one KV head's share of
// it - its G query heads, its k and v slice, its slice of every row - is
// independent of the other heads'.  Q8_0 blocks never straddle heads
// (head_dim is a multiple of 32), so each workgroup quantises and stores its
// own slice of the new row bit-exactly with the shared block quantiser.
//
// Per workgroup (256 threads, four waves):
//   1. q of the group's G heads and the new k and v into LDS (one float4
//      each); then every KV load of the call is issued at once (K pieces of
//      positions < pos, and each wave's V elements), to land during 2-4.
//   2. QK-RMSNorm factors: one thread per head, squares summed left to right
//      (qk_rmsnorm_block's order); inv = 1/sqrtf(ss/hd + eps).
//   3. (w * x) * inv, then the RoPE rotation of pos, per pair (ia, ib).
//   4. The new k and v slice: F32 copy or Q8_0 quantisation (four lanes per
//      block) into LDS, then to the caches.
//   5. Scores of positions 0..pos: NB = hd/32 consecutive lanes per
//      position, a 32-element piece each, fp32 dot products with the G
//      heads' q, summed over the NB lanes; position pos from the LDS copy.
//   6. Softmax statistics: wave g for head g (max, exp2, sum).
//   7. V-accumulate: wave w takes positions w, w+4, ..., each lane hd/64
//      elements; the four waves' sums merge in LDS, divided by the sum of
//      weights and written over q.
// Scores are in the log2 domain (q . k * log2(e)/sqrt(hd)), so the weights
// are exp2(s - max): the reference's softmax within fp32 rounding.
//
// Contexts longer than one span (up to 512 spans): workgroup (KV head, span)
// takes positions [128*span, min(pos+1, 128*span+128)), and only the span
// that holds pos appends the new row.  Instead of the output it writes its
// G heads' partials (max m, sum l, unnormalised sums of the weighted V) to
// the partial buffer with device-coherent stores, then takes a ticket from
// the (sequence, layer, KV head)'s counter with an agent-scope atomic: the
// span that draws the last ticket resets the counter to zero (so it is zero
// before every launch without a clearing pass), merges the spans' partials of its
// heads (weights exp2(m_s - M) with M the largest m, float64 sums, folded in
// chunks of 16 spans with a running maximum) and writes the output over q.  The merges of different KV heads run on
// different workgroups at once, and no second launch is needed.  The other
// spans read q before they take their ticket, so the output may overwrite it.
#include "g2b_internal.h"

namespace g2b {
namespace {

constexpr int kSThreads = 256;
constexpr int kSMaxG = 4;  // query heads per KV head (decode_fast_available)

template <int FMT, int HD>
struct ShortGeom {
  static constexpr int NB = HD / 32;                 // 32-element pieces per head slice
  static constexpr int HB = FMT ? NB * 34 : HD * 4;  // bytes of a head's slice of a row
  static constexpr int HBP = (HB + 15) & ~15;        // LDS copy, 16-byte padded
  static constexpr int XS = HD + 4;                  // LDS row of a head (bank offset)
  static constexpr int EPL = HD / 64;                // V elements per lane
};

// Raw bytes of piece b (elements 32b..32b+31) of a head slice (4-byte
// aligned; global or LDS).  Q8_0: block b starts at byte 34b; the nine
// dwords from (34b) & ~3 cover it (two bytes early for odd b, two bytes into
// block b+1 for even b, which exists: NB is even), so the window never
// leaves the slice.  F32: eight float4s.
template <int FMT>
struct PieceRaw {
  uint32_t d[9];
};
template <>
struct PieceRaw<0> {
  float4 f[8];
};

// A load from device (global) memory through a global-address-space
// pointer: the compiler then counts it with the other vector loads (a flat
// load returns out of order with them, so a wait for any load behind it
// becomes a wait for all).
template <typename T>
__device__ __forceinline__ T gload(const void *p) {
  return *(const __attribute__((address_space(1))) T *)p;
}
typedef float gload_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t gload_u32x2 __attribute__((ext_vector_type(2)));
template <>
__device__ __forceinline__ float4 gload<float4>(const void *p) {
  const gload_f32x4 v = *(const __attribute__((address_space(1))) gload_f32x4 *)p;
  return make_float4(v.x, v.y, v.z, v.w);
}
template <>
__device__ __forceinline__ uint2 gload<uint2>(const void *p) {
  const gload_u32x2 v = *(const __attribute__((address_space(1))) gload_u32x2 *)p;
  return make_uint2(v.x, v.y);
}

// Piece b of a head slice in the cache (global memory), as fetch_piece.
template <int FMT>
__device__ __forceinline__ void fetch_piece_g(const uint8_t *slice, int b, PieceRaw<FMT> &r) {
  if constexpr (FMT == 1) {
    const uint8_t *w = slice + ((34 * b) & ~3);
#pragma unroll
    for (int i = 0; i < 9; i++) r.d[i] = gload<uint32_t>(w + 4 * i);
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) r.f[i] = gload<float4>(slice + 128 * b + 16 * i);
  }
}

template <int FMT>
__device__ __forceinline__ void fetch_piece(const uint8_t *slice, int b, PieceRaw<FMT> &r) {
  if constexpr (FMT == 1) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(slice + ((34 * b) & ~3));
#pragma unroll
    for (int i = 0; i < 9; i++) r.d[i] = w[i];
  } else {
    const float4 *p = reinterpret_cast<const float4 *>(slice + 128 * b);
#pragma unroll
    for (int i = 0; i < 8; i++) r.f[i] = p[i];
  }
}

// The piece as 32 floats before the Q8_0 scale; returns the scale (1 for F32).
template <int FMT>
__device__ __forceinline__ float decode_piece(const PieceRaw<FMT> &r, int b, float (&x)[32]) {
  if constexpr (FMT == 1) {
    const bool odd = (b & 1) != 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t q = odd ? r.d[i + 1] : __builtin_amdgcn_alignbit(r.d[i + 1], r.d[i], 16);
      x[4 * i + 0] = (float)(int8_t)(q & 0xFFu);
      x[4 * i + 1] = (float)(int8_t)((q >> 8) & 0xFFu);
      x[4 * i + 2] = (float)(int8_t)((q >> 16) & 0xFFu);
      x[4 * i + 3] = (float)(int8_t)(q >> 24);
    }
    return half_bits_to_f32_hw(odd ? (r.d[0] >> 16) : (r.d[0] & 0xFFFFu));
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      x[4 * i + 0] = r.f[i].x;
      x[4 * i + 1] = r.f[i].y;
      x[4 * i + 2] = r.f[i].z;
      x[4 * i + 3] = r.f[i].w;
    }
    return 1.f;
  }
}

// Raw bytes of V elements e0 .. e0 + EPL - 1 (e0 a multiple of EPL) of a
// head slice: Q8_0 the quants (q) and the block's scale bits (s); F32 the
// values' bits (q, and s for the second).
template <int FMT, int EPL>
__device__ __forceinline__ void fetch_v(const uint8_t *slice, int e0, uint32_t &q, uint32_t &s) {
  if constexpr (FMT == 1) {
    const uint8_t *blk = slice + 34 * (e0 >> 5);
    s = *reinterpret_cast<const uint16_t *>(blk);
    if constexpr (EPL == 2)
      q = *reinterpret_cast<const uint16_t *>(blk + 2 + (e0 & 31));
    else
      q = blk[2 + (e0 & 31)];
  } else {
    const uint32_t *f = reinterpret_cast<const uint32_t *>(slice) + e0;
    if constexpr (EPL == 2) {
      const uint2 t = *reinterpret_cast<const uint2 *>(f);
      q = t.x;
      s = t.y;
    } else {
      q = f[0];
      s = 0u;
    }
  }
}

// The same from the cache (global memory).
template <int FMT, int EPL>
__device__ __forceinline__ void fetch_v_g(const uint8_t *slice, int e0, uint32_t &q, uint32_t &s) {
  if constexpr (FMT == 1) {
    const uint8_t *blk = slice + 34 * (e0 >> 5);
    s = gload<uint16_t>(blk);
    if constexpr (EPL == 2)
      q = gload<uint16_t>(blk + 2 + (e0 & 31));
    else
      q = gload<uint8_t>(blk + 2 + (e0 & 31));
  } else {
    const uint8_t *f = slice + 4 * e0;
    if constexpr (EPL == 2) {
      const uint2 t = gload<uint2>(f);
      q = t.x;
      s = t.y;
    } else {
      q = gload<uint32_t>(f);
      s = 0u;
    }
  }
}

// Dequantised as kv_val_row does (d * q).
template <int FMT, int EPL>
__device__ __forceinline__ void decode_v(uint32_t q, uint32_t s, float (&v)[EPL]) {
  if constexpr (FMT == 1) {
    const float d = half_bits_to_f32_hw(s);
    v[0] = d * (float)(int8_t)(q & 0xFFu);
    if constexpr (EPL == 2) v[1] = d * (float)(int8_t)((q >> 8) & 0xFFu);
  } else {
    v[0] = __uint_as_float(q);
    if constexpr (EPL == 2) v[1] = __uint_as_float(s);
  }
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// A workgroup barrier that orders LDS only: the phases up to the output
// share nothing else, so the KV loads issued with the inputs stay in flight
// through the norm, RoPE and append phases (a full __syncthreads waits for
// every outstanding global load first); the compiler waits for each KV
// register where the scores and V use it.
__device__ __forceinline__ void barrier_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

#ifdef G2B_STAMPS
// Phase stamps of a k_short workgroup (thread 0; one-span calls): 0 entry,
// 1 inputs and the norm factors in, 2 RoPE done, 3 append done, 4 scores
// done, 6 softmax done, 5 exit (after V and the output), 7 XCD.
#define G2B_SSTAMP(i) (sst_[i] = wall_clock64())
#else
#define G2B_SSTAMP(i) ((void)0)
#endif

template <int FMT, int HD>
__global__ __launch_bounds__(kSThreads) void k_short(DecodeParams P) {
#ifdef G2B_STAMPS
  uint64_t sst_[kStampWords] = {};
  G2B_SSTAMP(0);
#endif
  using Geo = ShortGeom<FMT, HD>;
  constexpr int NB = Geo::NB, HB = Geo::HB, XS = Geo::XS, EPL = Geo::EPL;
  constexpr int half = HD / 2;
  constexpr int PPR = kSThreads / NB;                      // score positions per round
  constexpr int RK = (kShortMaxPos + PPR - 1) / PPR;       // score rounds
  constexpr int VI = kShortMaxPos / 4;                     // V positions per wave
  // q heads 0..G-1, the new k (row G) and the new v (row G + 1)
  __shared__ __align__(16) float xs[(kSMaxG + 2) * XS];
  __shared__ __align__(16) uint8_t rowk[Geo::HBP], rowv[Geo::HBP];
  __shared__ float sc[kSMaxG * kShortMaxPos];  // scores, then weights
  // the four waves' V sums
  __shared__ __align__(16) float accs[4 * kSMaxG * HD];
  __shared__ float inv[kSMaxG + 1], lsum[kSMaxG], msh[kSMaxG];
  __shared__ int32_t s_last;

  const ShapeDev &sh = P.sh;
  const int nkvh = sh.n_kv_heads;
  const int kvh = (int)(blockIdx.x % (unsigned)nkvh), span = (int)(blockIdx.x / (unsigned)nkvh);
  const int seq = blockIdx.y, li = blockIdx.z;
  const int layer = P.layer0 + li;
  const int G = sh.n_heads / nkvh;
  const SeqDev sd = P.seqs ? P.seqs[seq] : P.one;
  const int pos = sd.pos;
  // positions [t0, t0 + n_here) of this span; the span of pos appends
  const int t0 = span * kShortMaxPos;
  if (pos < 0 || t0 > pos) return;  // (a shorter sequence of a ragged batch)
  const int n_here = min(pos + 1 - t0, kShortMaxPos);
  const bool owner = t0 + n_here == pos + 1;
  const int nspans = pos / kShortMaxPos + 1;
  // (the host sizes the partials and counters for max_splits spans; a
  // descriptor beyond that leaves its output untouched rather than index
  // past them)
  if (nspans > 1 && (nspans > P.max_splits || !P.span_ctr)) return;
  const size_t sidx = (size_t)li * (size_t)P.n_seq + (size_t)seq;
  const size_t nq = (size_t)sh.n_heads * HD, nkv = (size_t)sh.n_kv_heads * HD;
  float *qo = P.q_out + sidx * nq + (size_t)kvh * G * HD;  // q in; the output goes here
  const float *ki = P.k_in + sidx * nkv + (size_t)kvh * HD;
  const float *vi = P.v_in + sidx * nkv + (size_t)kvh * HD;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t row = sh.row_bytes;
  const size_t lay = (size_t)layer * (size_t)sd.ctx_cap;
  uint8_t *const kb = sd.k + lay * row + (size_t)kvh * HB;
  uint8_t *const vb = sd.v + lay * row + (size_t)kvh * HB;

  // 1. q (G heads), k and v: one float4 per thread, into registers first
  constexpr int P4 = HD / 4;
  const bool has_x = t < (G + 2) * P4;
  const int xh = t / P4, xj = t - xh * P4;
  // (every load of step 1 unconditional, threads without a piece reading
  // one that exists: a load in a per-thread branch is waited for, with all
  // loads before it, where the branches join)
  const int xhc = xh < G + 2 ? xh : G + 1;
  const float *src = xhc < G ? qo + xhc * HD : (xhc == G ? ki : vi);
  const float4 x4 = gload<float4>(src + 4 * xj);
  // Step 3's inputs for this thread's first pair (pair t: head t / half):
  // the norm weights of its two elements and the cos/sin of pos, loaded
  // with the inputs, before the KV loads, so that step 3 waits for neither.
  const float *wq = norm_weights(P.norm, layer, 0, HD);
  const float *wk = norm_weights(P.norm, layer, 1, HD);
  const float *cs = (sh.rope_on && P.rope) ? P.rope + (size_t)pos * HD : nullptr;
  // (unconditional too: a missing table reads q instead, and the values of
  // a thread without a pair or a table are not used)
  float wa0, wb0, c0, s0;
  {
    const int pt = t < (G + 1) * half ? t : 0;
    const int h = pt / half, j = pt - h * half;
    int ia, ib;
    rope_pair_index(sh.arch_llama, j, half, ia, ib);
    const float *w = h < G ? wq : wk;
    const float *ws = w ? w : qo, *cz = cs ? cs : qo;
    wa0 = gload<float>(ws + ia);
    wb0 = gload<float>(ws + ib);
    c0 = gload<float>(cz + 2 * j);
    s0 = gload<float>(cz + 2 * j + 1);
  }
  // Every KV load of the span is issued now, so that it is in flight during
  // the setup: the K pieces of its positions below pos (each thread one
  // piece per round) and, per wave, the V elements of its positions
  // t0 + wave, t0 + wave + 4, ... below pos.  Other slots read row 0 instead
  // (in bounds, never used), which keeps the loads unconditional.  The
  // inputs go to LDS between the K and the V loads: the wait for them counts
  // the K loads issued after them, not the V loads' 2 * VI (more than the
  // wait counter holds), and the barriers up to the scores order LDS only,
  // so the KV bytes land during steps 2-4.
  const int b = t % NB;
  PieceRaw<FMT> kraw[RK];
#pragma unroll
  for (int r = 0; r < RK; r++) {
    const int tp = t0 + r * PPR + t / NB;
    fetch_piece_g<FMT>(kb + (size_t)(tp < pos ? tp : 0) * row, b, kraw[r]);
  }
  if (has_x) *reinterpret_cast<float4 *>(xs + xh * XS + 4 * xj) = x4;
  const int e0 = lane * EPL;
  uint32_t vq[VI], vsb[VI];
#pragma unroll
  for (int i = 0; i < VI; i++) {
    const int tp = t0 + wave + 4 * i;
    fetch_v_g<FMT, EPL>(vb + (size_t)(tp < pos ? tp : 0) * row, e0, vq[i], vsb[i]);
  }
  barrier_lds();

  G2B_SSTAMP(1);
  // 2. QK-RMSNorm factors
  if (t <= G) {
    const float *w = t < G ? wq : wk;
    if (w) {
      const float *x = xs + t * XS;
      float ss = 0.f;
#pragma unroll 8
      for (int j = 0; j < HD; j += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(x + j);
        float sq = v.x * v.x;
        ss = ss + sq;
        sq = v.y * v.y;
        ss = ss + sq;
        sq = v.z * v.z;
        ss = ss + sq;
        sq = v.w * v.w;
        ss = ss + sq;
      }
      inv[t] = __fdiv_rn(1.f, sqrtf(__fdiv_rn(ss, (float)HD) + P.norm.eps));
    }
  }
  barrier_lds();

  // 3. (w * x) * inv, then RoPE(pos), per pair: the thread's first pair
  // from the inputs in registers (no global load here, whose wait would
  // include the V loads still in flight), further ones (more than
  // kSThreads pairs: groups of 4) from the tables
  auto rotate = [&](int i, float wa, float wb, float co, float si) {
    const int h = i / half, j = i - h * half;
    int ia, ib;
    rope_pair_index(sh.arch_llama, j, half, ia, ib);
    float *x = xs + h * XS;
    float a = x[ia], c = x[ib];
    if (h < G ? wq : wk) {
      const float f = inv[h];
      a = (wa * a) * f;
      c = (wb * c) * f;
    }
    if (cs) rope_pair(a, c, co, si);
    x[ia] = a;
    x[ib] = c;
  };
  if (t < (G + 1) * half) rotate(t, wa0, wb0, c0, s0);
  for (int i = t + kSThreads; i < (G + 1) * half; i += kSThreads) {
    const int h = i / half, j = i - h * half;
    int ia, ib;
    rope_pair_index(sh.arch_llama, j, half, ia, ib);
    const float *w = h < G ? wq : wk;
    rotate(i, w ? w[ia] : 1.f, w ? w[ib] : 1.f, cs ? cs[2 * j] : 1.f, cs ? cs[2 * j + 1] : 0.f);
  }
  barrier_lds();

  G2B_SSTAMP(2);
  // 4. the new row's slice (the span of pos only): LDS copy, then the caches
  const float *kr = xs + G * XS, *vr = xs + (G + 1) * XS;
  if (!owner) {
    // nothing to append
  } else if constexpr (FMT == 1) {
    if (t < 8 * NB) {  // blocks 0..NB-1 of k, then of v; four lanes each
      const int bq = t >> 2, part = t & 3;
      const bool is_k = bq < NB;
      const int bb = is_k ? bq : bq - NB;
      q8_quant_block_x4((is_k ? kr : vr) + 32 * bb, 32, (is_k ? rowk : rowv) + 34 * bb, part);
    }
  } else {
    for (int i = t; i < 2 * P4; i += kSThreads) {
      const bool is_k = i < P4;
      const int j = is_k ? i : i - P4;
      const float4 v = *reinterpret_cast<const float4 *>((is_k ? kr : vr) + 4 * j);
      *reinterpret_cast<float4 *>((is_k ? rowk : rowv) + 16 * j) = v;
    }
  }
  barrier_lds();
  if (owner) {
    constexpr int W = HB / 4;  // dwords of a slice (HB is a multiple of 4)
    const size_t off = (size_t)pos * row;
    for (int i = t; i < 2 * W; i += kSThreads) {
      const bool is_k = i < W;
      const int j = is_k ? i : i - W;
      reinterpret_cast<uint32_t *>((is_k ? kb : vb) + off)[j] =
          reinterpret_cast<const uint32_t *>(is_k ? rowk : rowv)[j];
    }
  }

  G2B_SSTAMP(3);
  // 5. scores: position tp's NB pieces on NB consecutive lanes
  const float qscale = P.qscale;
#pragma unroll
  for (int r = 0; r < RK; r++) {
    const int lp = r * PPR + t / NB, tp = t0 + lp;
    if (lp < n_here) {  // (uniform over a position's NB lanes)
      PieceRaw<FMT> pr = kraw[r];
      if (tp == pos) fetch_piece<FMT>(rowk, b, pr);
      float k[32];
      const float d = decode_piece<FMT>(pr, b, k);
#pragma unroll
      for (int g = 0; g < kSMaxG; g++) {
        if (g < G) {
          const float *q = xs + g * XS + 32 * b;
          float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
          for (int j = 0; j < 32; j += 4) {
            const float4 q4 = *reinterpret_cast<const float4 *>(q + j);
            a0 = fmaf(q4.x, k[j + 0], a0);
            a1 = fmaf(q4.y, k[j + 1], a1);
            a2 = fmaf(q4.z, k[j + 2], a2);
            a3 = fmaf(q4.w, k[j + 3], a3);
          }
          float s = ((a0 + a1) + (a2 + a3)) * d;
#pragma unroll
          for (int o = 1; o < NB; o <<= 1) s += __shfl_xor(s, o);
          if (b == 0) sc[g * kShortMaxPos + lp] = s * qscale;
        }
      }
    }
  }
  barrier_lds();

  G2B_SSTAMP(4);
  // 6. softmax statistics: wave g for head g
  if (wave < G) {
    float *s = sc + wave * kShortMaxPos;
    float m = kNegBig;
    for (int i = lane; i < n_here; i += 64) m = fmaxf(m, s[i]);
    m = wave_max(m);
    float l = 0.f;
    for (int i = lane; i < n_here; i += 64) {
      const float p = __builtin_amdgcn_exp2f(s[i] - m);
      s[i] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) {
      lsum[wave] = l;
      msh[wave] = m;
    }
  }
  barrier_lds();

  G2B_SSTAMP(6);
  // 7. V-accumulate, wave w over positions w, w + 4, ... (pos itself from LDS)
  float acc[kSMaxG][EPL];
#pragma unroll
  for (int g = 0; g < kSMaxG; g++)
#pragma unroll
    for (int i = 0; i < EPL; i++) acc[g][i] = 0.f;
  // The weights of the wave's positions: lane i holds position wave + 4i's
  // (one LDS read per head), handed to every lane by readlane in the loop -
  // an LDS read per position and head, each waited for, was 2-5 us of the
  // kernel's 9-12 at 40-100 positions.
  static_assert(VI <= 64, "one lane per position of the wave");
  float pw[kSMaxG];
#pragma unroll
  for (int g = 0; g < kSMaxG; g++)
    pw[g] = (g < G && lane < VI && wave + 4 * lane < n_here)
                ? sc[g * kShortMaxPos + wave + 4 * lane]
                : 0.f;
#pragma unroll
  for (int i = 0; i < VI; i++) {
    const int lp = wave + 4 * i, tp = t0 + lp;
    if (lp < n_here) {
      uint32_t q = vq[i], sb = vsb[i];
      if (tp == pos) fetch_v<FMT, EPL>(rowv, e0, q, sb);
      float v[EPL];
      decode_v<FMT, EPL>(q, sb, v);
#pragma unroll
      for (int g = 0; g < kSMaxG; g++) {
        if (g < G) {
          const float p = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pw[g]), i));
#pragma unroll
          for (int e = 0; e < EPL; e++) acc[g][e] = fmaf(p, v[e], acc[g][e]);
        }
      }
    }
  }
#pragma unroll
  for (int g = 0; g < kSMaxG; g++)
#pragma unroll
    for (int i = 0; i < EPL; i++) accs[(wave * kSMaxG + g) * HD + e0 + i] = acc[g][i];
  barrier_lds();
  if (nspans == 1) {
    for (int i = t; i < G * HD; i += kSThreads) {
      const int g = i / HD, e = i - g * HD;
      const float s = (accs[(0 * kSMaxG + g) * HD + e] + accs[(1 * kSMaxG + g) * HD + e]) +
                      (accs[(2 * kSMaxG + g) * HD + e] + accs[(3 * kSMaxG + g) * HD + e]);
      qo[g * HD + e] = s / lsum[g];
    }
#ifdef G2B_STAMPS
    const uint64_t gw = blockIdx.x + (uint64_t)gridDim.x * (blockIdx.y + (uint64_t)gridDim.y * blockIdx.z);
    if (threadIdx.x == 0 && P.stamps && gw < (uint64_t)P.stamp_cap) {
      G2B_SSTAMP(5);
      sst_[7] = (uint64_t)(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15);
      for (int i = 0; i < kStampWords; i++) P.stamps[gw * kStampWords + i] = sst_[i];
    }
#endif
    return;
  }

  // 8. several spans: this span's partials, a ticket, and the merge by the
  // span that draws the last one
  constexpr int PS = kPartHead + HD;
  const size_t nh = (size_t)sh.n_heads, ms = (size_t)P.max_splits;
  // partial (head kvh*G + g, slot s) of this (sequence, layer)
  auto part_of = [&](int g, int sl) {
    return P.part + ((sidx * nh + (size_t)(kvh * G + g)) * ms + (size_t)sl) * PS;
  };
  // The partials travel through device-coherent accesses: agent-scope
  // atomic stores (write-through to the device's coherence point) that each
  // thread waits for before the barrier, and agent-scope atomic loads in the
  // merging span.  The ticket orders them: after the barrier (workgroup
  // scope: every thread's stores happen before it), thread 0 takes the
  // ticket with an acq_rel agent-scope fetch_add, which releases this
  // span's partials and, in the span that draws the last ticket, acquires
  // every other span's before the barrier that precedes the merge.  One
  // release per workgroup, not per wave (a release fence in every wave cost
  // more than the whole stream here).
  for (int i = t; i < G * HD; i += kSThreads) {
    const int g = i / HD, e = i - g * HD;
    float *pp = part_of(g, span);
    const float a = (accs[(0 * kSMaxG + g) * HD + e] + accs[(1 * kSMaxG + g) * HD + e]) +
                    (accs[(2 * kSMaxG + g) * HD + e] + accs[(3 * kSMaxG + g) * HD + e]);
    __hip_atomic_store(pp + kPartHead + e, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (e == 0) {
      __hip_atomic_store(pp, msh[g], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(pp + 1, lsum[g], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are done
  __syncthreads();
  if (t == 0) {
    int32_t *ctr = P.span_ctr + sidx * (size_t)nkvh + (size_t)kvh;
    const int32_t ticket =
        __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = ticket == nspans - 1;
    if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  // An online merge over chunks of MC spans: each thread folds in, per
  // chunk, the (m, l) pairs and its elements' sums of MC spans, all loaded
  // together (one round trip per chunk rather than a pass for the maxima
  // and another for the sums): M' = max(M, m_s), weights exp2(m_s - M'),
  // the running float64 sums scaled by exp2(M - M').
  constexpr int MC = 16;
  constexpr int EPT = (kSMaxG * HD + kSThreads - 1) / kSThreads;  // elements per thread
  float M[EPT];
  double Lw[EPT], O[EPT];
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    M[j] = kNegBig;
    Lw[j] = 0.0;
    O[j] = 0.0;
  }
  for (int c0 = 0; c0 < nspans; c0 += MC) {
    const int nc = min(MC, nspans - c0);
#pragma unroll
    for (int j = 0; j < EPT; j++) {
      const int i = t + j * kSThreads;
      if (i >= G * HD) break;
      const int g = i / HD, e = i - g * HD;
      uint64_t ml[MC];
      float a[MC];
#pragma unroll
      for (int u = 0; u < MC; u++) {
        if (u < nc) {
          const float *pp = part_of(g, c0 + u);
          ml[u] = __hip_atomic_load(reinterpret_cast<const uint64_t *>(pp), __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
          a[u] = __hip_atomic_load(pp + kPartHead + e, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      float mx = M[j];
#pragma unroll
      for (int u = 0; u < MC; u++)
        if (u < nc) mx = fmaxf(mx, __uint_as_float((uint32_t)ml[u]));
      const double sc = (double)exp2f(M[j] - mx);
      double lw = Lw[j] * sc, o = O[j] * sc;
#pragma unroll
      for (int u = 0; u < MC; u++) {
        if (u < nc) {
          const double w = (double)exp2f(__uint_as_float((uint32_t)ml[u]) - mx);
          lw = fma((double)__uint_as_float((uint32_t)(ml[u] >> 32)), w, lw);
          o = fma((double)a[u], w, o);
        }
      }
      M[j] = mx;
      Lw[j] = lw;
      O[j] = o;
    }
  }
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int i = t + j * kSThreads;
    if (i < G * HD) qo[i] = (float)(O[j] / Lw[j]);
  }
}

}  // namespace

bool short_available(const ShapeDev &sh) {
  return decode_fast_available(sh) && sh.n_heads / sh.n_kv_heads <= kSMaxG;
}

hipError_t launch_short(const DecodeParams &p, int n_layers, hipStream_t s) {
  if (!short_available(p.sh) || n_layers < 1 || p.n_seq < 1 || p.max_splits < 1 ||
      p.max_splits > kShortMaxSpans || (p.max_splits > 1 && (!p.span_ctr || !p.part)))
    return hipErrorInvalidValue;
  dim3 grid(p.sh.n_kv_heads * p.max_splits, p.n_seq, n_layers);
  if (p.sh.kv_q8) {
    if (p.sh.head_dim == 128)
      hipLaunchKernelGGL((k_short<1, 128>), grid, dim3(kSThreads), 0, s, p);
    else
      hipLaunchKernelGGL((k_short<1, 64>), grid, dim3(kSThreads), 0, s, p);
  } else {
    if (p.sh.head_dim == 128)
      hipLaunchKernelGGL((k_short<0, 128>), grid, dim3(kSThreads), 0, s, p);
    else
      hipLaunchKernelGGL((k_short<0, 64>), grid, dim3(kSThreads), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace g2b
