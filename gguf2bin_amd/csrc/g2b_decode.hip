// g2b_decode.hip - the generic decode kernel, the split combine and the
// dispatch of a decode call, gfx950.
//
// Specialised shapes run k_layer (g2b_layer.h, instantiated per KV format,
// head_dim and GQA group by g2b_layer_inst.hip); every other shape runs the
// generic three-pass kernel below after the append kernels.  Both leave one
// partial (m, l, acc[hd]) per split and q head; k_combine merges them.
#include <algorithm>

#include "g2b_internal.h"

namespace g2b {

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- generic
// Any shape (blocks spanning heads, partial blocks, any head_dim): a
// three-pass split per q head with scores staged in LDS.  Correctness path
// for shapes without a specialised kernel.

__device__ __forceinline__ float kv_elem(const uint8_t *rowp, int e, int q8) {
  if (!q8) return reinterpret_cast<const float *>(rowp)[e];
  const uint8_t *blk = rowp + 34 * (e >> 5);
  const float s = half_bits_to_f32(*reinterpret_cast<const uint16_t *>(blk));
  return s * (float)(int8_t)blk[2 + (e & 31)];
}

__device__ float block_reduce(float x, bool is_max, float *scratch) {
  for (int o = 32; o > 0; o >>= 1) {
    const float y = __shfl_xor(x, o);
    x = is_max ? fmaxf(x, y) : x + y;
  }
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[wave] = x;
  __syncthreads();
  float r = scratch[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); w++) r = is_max ? fmaxf(r, scratch[w]) : r + scratch[w];
  return r;
}

__global__ __launch_bounds__(kThreads) void k_decode_generic(DecodeParams P) {
  __shared__ float sc[kGenericMaxSplit];
  __shared__ float red[kThreads / 64];
  const int split = blockIdx.x, li = blockIdx.z;
  const int seq = static_seq((int)blockIdx.y, li, P.n_seq);
  const SeqDev sd = P.seqs ? P.seqs[seq] : P.one;
  const int npos = sd.pos + 1;
  const int t0 = split * P.split_len;
  if (t0 >= npos) return;
  const int t1 = min(npos, t0 + P.split_len);
  const int n = t1 - t0;
  const int HD = P.sh.head_dim, nh = P.sh.n_heads, group = nh / P.sh.n_kv_heads;
  const int layer = P.layer0 + li;
  const size_t sidx = (size_t)li * (size_t)P.n_seq + (size_t)seq;
  const size_t row = P.sh.row_bytes;
  const uint8_t *kb = sd.k + (size_t)layer * (size_t)sd.ctx_cap * row;
  const uint8_t *vb = sd.v + (size_t)layer * (size_t)sd.ctx_cap * row;
  for (int h = 0; h < nh; h++) {
    const int e0 = (h / group) * HD;
    const float *qh = P.q_rot + sidx * (size_t)(nh * HD) + (size_t)h * HD;
    for (int t = threadIdx.x; t < n; t += blockDim.x) {
      const uint8_t *rp = kb + (size_t)(t0 + t) * row;
      float s = 0.f;
      for (int d = 0; d < HD; d++) s = fmaf(qh[d], kv_elem(rp, e0 + d, P.sh.kv_q8), s);
      s *= P.qscale;
      sc[t] = s;
      if (P.att) P.att[(sidx * nh + h) * (size_t)P.att_stride + t0 + t] = s;
    }
    __syncthreads();
    float mx = kNegBig;
    for (int t = threadIdx.x; t < n; t += blockDim.x) mx = fmaxf(mx, sc[t]);
    const float M = block_reduce(mx, true, red);
    float sum = 0.f;
    for (int t = threadIdx.x; t < n; t += blockDim.x) {
      const float p = exp2f(sc[t] - M);
      sc[t] = p;
      sum += p;
    }
    const float L = block_reduce(sum, false, red);
    __syncthreads();
    float *pp = P.part + ((sidx * nh + h) * (size_t)P.max_splits + (size_t)split) *
                             (size_t)(kPartHead + HD);
    for (int d = threadIdx.x; d < HD; d += blockDim.x) {
      float a = 0.f;
      for (int t = 0; t < n; t++) a = fmaf(sc[t], kv_elem(vb + (size_t)(t0 + t) * row, e0 + d, P.sh.kv_q8), a);
      pp[kPartHead + d] = a;
    }
    if (threadIdx.x == 0) {
      pp[0] = M;
      pp[1] = L;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- combine
// One workgroup per (head, seq, layer) merges that head's split partials:
// M = max m_p, w_p = exp2(m_p - M), L = sum l_p w_p, out = sum acc_p w_p / L,
// written over q.  Up to 2048 partials (one per split) per head: the
// max and the sum are block reductions, and the weighted sum of the
// accumulators splits the partials over 256/HD thread groups with four
// independent chains per thread, so the merge is bandwidth- and not
// latency-bound.  The sums are float64: a serial fp32 sum of that many terms
// drifts by ~1e-5 relative once one partial dominates.
constexpr int kCombineThreads = 256;
constexpr int kCombineMaxParts = 2048;
constexpr int kCombineFewParts = 32;  // up to this many partials: one wave per head
constexpr int kCombineRowLoads = 32;  // rows held per thread on the one-round path

__device__ inline float block_max_f(float x, float *red) {
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = x;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); w++) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}

__device__ inline double block_sum_d(double x, double *red) {
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = x;
  __syncthreads();
  double r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); w++) r += red[w];
  __syncthreads();
  return r;
}

#ifdef G2B_STAMPS
// Phase stamps of a combine workgroup (thread 0): entry and exit.
__device__ inline void combine_stamp(const DecodeParams &P, uint64_t in) {
  const uint64_t g = blockIdx.x + (uint64_t)gridDim.x * (blockIdx.y + (uint64_t)gridDim.y * blockIdx.z);
  if (threadIdx.x == 0 && P.stamps && g < (uint64_t)P.stamp_cap) {
    uint64_t *o = P.stamps + ((uint64_t)P.stamp_cap + g) * kStampWords;
    o[0] = in;
    o[5] = (uint64_t)wall_clock64();
    o[7] = (uint64_t)(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15);  // XCD
  }
}
#define G2B_COMBINE_IN const uint64_t stamp_in = (uint64_t)wall_clock64()
#define G2B_COMBINE_OUT combine_stamp(P, stamp_in)
#else
#define G2B_COMBINE_IN ((void)0)
#define G2B_COMBINE_OUT ((void)0)
#endif

__global__ __launch_bounds__(kCombineThreads) void k_combine(DecodeParams P, float *q_out) {
  G2B_COMBINE_IN;
  __shared__ float w[kCombineMaxParts];
  __shared__ double part_sum[4 * kCombineThreads];
  __shared__ double red[kCombineThreads / 64];
  const int h = blockIdx.x, seq = blockIdx.y, li = blockIdx.z;
  const SeqDev sd = P.seqs ? P.seqs[seq] : P.one;
  const int npos = sd.pos + 1;
  const size_t unit = (size_t)li * (size_t)P.n_seq + (size_t)seq;
  int np;
  if (P.wq) {  // work queue: the partial slots the visits reserved
    const int32_t *ctr = P.wq + ((size_t)P.wq_set * P.wq_cap + unit) * kWqStride;
    np = min(ctr[1], P.max_splits);
    // zero the next launch's counter set (its used extent, from the host)
    int32_t *nxt = P.wq + (size_t)(P.wq_set ^ 1) * P.wq_cap * kWqStride;
    const size_t nblk = (size_t)gridDim.x * gridDim.y * gridDim.z;
    const size_t bid = blockIdx.x + (size_t)gridDim.x * (blockIdx.y + (size_t)gridDim.y * blockIdx.z);
    for (size_t uu = bid; uu < (size_t)P.wq_zero_units; uu += nblk)
      if (threadIdx.x < 2) nxt[uu * kWqStride + threadIdx.x] = 0;
  } else {
    np = (npos + P.split_len - 1) / P.split_len;
  }
  const int HD = P.sh.head_dim, nh = P.sh.n_heads;
  const size_t pstr = (size_t)(kPartHead + HD);
  const size_t sidx = (size_t)li * (size_t)P.n_seq + (size_t)seq;
  const float *base =
      P.part + (sidx * nh + h) * (size_t)P.max_splits * pstr;
  const int tid = threadIdx.x;

  // One round of loads where the rows fit the registers (up to
  // kCombineRowLoads float4s of partial rows per thread): every (m, l) pair
  // and every accumulator row is requested before any of them is used, so
  // the merge waits for memory once (a few hundred partials, e.g. a single
  // long sequence's splits, were ~6 us of dependent rounds).
  const int tpr = HD / 4, GRP = (HD & 3) == 0 && tpr <= kCombineThreads ? kCombineThreads / tpr : 0;
  if (GRP > 0 && np >= 1 && np <= GRP * kCombineRowLoads && np <= kCombineThreads) {
    const int grp = tid / tpr, q = tid - grp * tpr;
    // (every load is unconditional - a partial past np reads the last one
    // and gets no weight - so that they are all in flight together: a
    // conditional load waits for itself before the branches join)
    float2 ml = *reinterpret_cast<const float2 *>(base + (size_t)min(tid, np - 1) * pstr);
    if (tid >= np) ml = make_float2(kNegBig, 0.f);
    float4 v[kCombineRowLoads];
    const float *a = base + kPartHead + 4 * (grp < GRP ? q : 0);
#pragma unroll
    for (int u = 0; u < kCombineRowLoads; u++) {
      const int p = min(grp + GRP * u, np - 1);
      v[u] = *reinterpret_cast<const float4 *>(a + (size_t)p * pstr);
    }
    const float M = block_max_f(ml.x, reinterpret_cast<float *>(red));
    double lsum = 0.0;
    if (tid < np) {
      const float wp = exp2f(ml.x - M);
      w[tid] = wp;
      lsum = (double)ml.y * (double)wp;
    }
    const double L = block_sum_d(lsum, red);  // (its barriers also publish w)
    double o[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int u = 0; u < kCombineRowLoads; u++) {
      const int p = grp + GRP * u;
      if (grp < GRP && p < np) {
        const double wp = (double)w[p];
        o[0] = fma((double)v[u].x, wp, o[0]);
        o[1] = fma((double)v[u].y, wp, o[1]);
        o[2] = fma((double)v[u].z, wp, o[2]);
        o[3] = fma((double)v[u].w, wp, o[3]);
      }
    }
    double *gs = part_sum;  // [group][HD], GRP * HD <= 4 * kCombineThreads
    __syncthreads();
    if (grp < GRP)
      for (int j = 0; j < 4; j++) gs[grp * HD + 4 * q + j] = o[j];
    __syncthreads();
    float *out = q_out + sidx * (size_t)(nh * HD) + (size_t)h * HD;
    for (int d = tid; d < HD; d += kCombineThreads) {
      double sum = 0.0;
      for (int g = 0; g < GRP; g++) sum += gs[g * HD + d];
      out[d] = (float)(sum / L);
    }
    if (P.att) {
      float *at = P.att + (sidx * nh + h) * (size_t)P.att_stride;
      for (int t = tid; t < npos; t += blockDim.x)
        at[t] = (float)(exp2((double)at[t] - (double)M) / L);
    }
    G2B_COMBINE_OUT;
    return;
  }

  float mx = kNegBig;
  for (int p = tid; p < np; p += blockDim.x) mx = fmaxf(mx, base[p * pstr]);
  const float M = block_max_f(mx, reinterpret_cast<float *>(red));
  double lsum = 0.0;
  for (int p = tid; p < np; p += blockDim.x) {
    const float wp = exp2f(base[p * pstr] - M);
    w[p] = wp;
    lsum = fma((double)base[p * pstr + 1], (double)wp, lsum);
  }
  const double L = block_sum_d(lsum, red);  // (its barriers also publish w)

  float *out = q_out + sidx * (size_t)(nh * HD) + (size_t)h * HD;
  const int ngrp = HD <= (int)blockDim.x ? (int)blockDim.x / HD : 1;
  const int grp = tid / HD;
  for (int d = tid % HD; d < HD; d += blockDim.x) {
    double o0 = 0.0, o1 = 0.0, o2 = 0.0, o3 = 0.0;
    if (grp < ngrp) {
      const float *a = base + kPartHead + d;
      int p = grp;
      for (; p + 3 * ngrp < np; p += 4 * ngrp) {
        o0 = fma((double)a[(size_t)p * pstr], (double)w[p], o0);
        o1 = fma((double)a[(size_t)(p + ngrp) * pstr], (double)w[p + ngrp], o1);
        o2 = fma((double)a[(size_t)(p + 2 * ngrp) * pstr], (double)w[p + 2 * ngrp], o2);
        o3 = fma((double)a[(size_t)(p + 3 * ngrp) * pstr], (double)w[p + 3 * ngrp], o3);
      }
      for (; p < np; p += ngrp) o0 = fma((double)a[(size_t)p * pstr], (double)w[p], o0);
    }
    const double o = (o0 + o1) + (o2 + o3);
    if (ngrp == 1) {
      out[d] = (float)(o / L);
    } else if (grp < ngrp) {
      part_sum[grp * HD + d] = o;
    }
  }
  if (ngrp > 1) {
    __syncthreads();
    for (int d = tid; d < HD; d += blockDim.x) {
      double o = 0.0;
      for (int g = 0; g < ngrp; g++) o += part_sum[g * HD + d];
      out[d] = (float)(o / L);
    }
  }
  if (P.att) {
    // weights of the scores this kernel used, normalised without an fp32
    // rounding of (score - max)
    float *a = P.att + (sidx * nh + h) * (size_t)P.att_stride;
    for (int t = tid; t < npos; t += blockDim.x)
      a[t] = (float)(exp2((double)a[t] - (double)M) / L);
  }
  G2B_COMBINE_OUT;
}

// k_combine for one unit's many partials (static splits, more than
// kCombineFewParts of them, at most kCombineThreads): each head's dims in
// kCombineParts parts, one workgroup per (head, part), so that a workgroup
// requests R rows of a quarter of the dims instead of a whole head's rows
// (c1 / c2, 129 partials of 16 heads: 16 workgroups of 17 row loads per
// thread became 64 of 5).  The same float64 merge as k_combine - weights
// exp2(m_p - M), sums over the partials in GRP groups, then over the groups
// in order, divided by the sum of the weighted l - with the partials dealt
// to more groups, so the order of the float64 additions differs.
constexpr int kCombineParts = 4;
template <int R>
__global__ __launch_bounds__(kCombineThreads) void k_combine_part(DecodeParams P, float *q_out) {
  G2B_COMBINE_IN;
  __shared__ float w[kCombineThreads];
  __shared__ double gs[4 * kCombineThreads];  // [group][dims of the part]
  __shared__ double red[kCombineThreads / 64];
  const int h = (int)blockIdx.x / kCombineParts, part = (int)blockIdx.x - h * kCombineParts;
  const int seq = blockIdx.y, li = blockIdx.z, tid = threadIdx.x;
  const SeqDev sd = P.seqs ? P.seqs[seq] : P.one;
  const int npos = sd.pos + 1;
  const int np = (npos + P.split_len - 1) / P.split_len;
  const int HD = P.sh.head_dim, nh = P.sh.n_heads, PD = HD / kCombineParts;
  const size_t pstr = (size_t)(kPartHead + HD);
  const size_t sidx = (size_t)li * (size_t)P.n_seq + (size_t)seq;
  const float *base = P.part + (sidx * nh + h) * (size_t)P.max_splits * pstr;
  const int tpr = PD / 4, GRP = kCombineThreads / tpr;  // (the host checks np <= GRP * R)
  const int grp = tid / tpr, q = tid - grp * tpr;
  // every load unconditional, as in k_combine's one-round path
  float2 ml = *reinterpret_cast<const float2 *>(base + (size_t)min(tid, np - 1) * pstr);
  if (tid >= np) ml = make_float2(kNegBig, 0.f);
  float4 v[R];
  const float *a = base + kPartHead + part * PD + 4 * q;
#pragma unroll
  for (int u = 0; u < R; u++) {
    const int p = min(grp + GRP * u, np - 1);
    v[u] = *reinterpret_cast<const float4 *>(a + (size_t)p * pstr);
  }
  const float M = block_max_f(ml.x, reinterpret_cast<float *>(red));
  double lsum = 0.0;
  if (tid < np) {
    const float wp = exp2f(ml.x - M);
    w[tid] = wp;
    lsum = (double)ml.y * (double)wp;
  }
  const double L = block_sum_d(lsum, red);  // (its barriers also publish w)
  double o[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int u = 0; u < R; u++) {
    const int p = grp + GRP * u;
    if (p < np) {
      const double wp = (double)w[p];
      o[0] = fma((double)v[u].x, wp, o[0]);
      o[1] = fma((double)v[u].y, wp, o[1]);
      o[2] = fma((double)v[u].z, wp, o[2]);
      o[3] = fma((double)v[u].w, wp, o[3]);
    }
  }
  for (int j = 0; j < 4; j++) gs[grp * PD + 4 * q + j] = o[j];
  __syncthreads();
  float *out = q_out + sidx * (size_t)(nh * HD) + (size_t)h * HD + (size_t)part * PD;
  for (int d = tid; d < PD; d += kCombineThreads) {
    double sum = 0.0;
    for (int g = 0; g < GRP; g++) sum += gs[g * PD + d];
    out[d] = (float)(sum / L);
  }
  if (P.att && part == 0) {
    float *at = P.att + (sidx * nh + h) * (size_t)P.att_stride;
    for (int t = tid; t < npos; t += blockDim.x)
      at[t] = (float)(exp2((double)at[t] - (double)M) / L);
  }
  G2B_COMBINE_OUT;
}

// k_combine with few partials (max_splits <= kCombineFewParts): one wave per
// head, four heads per workgroup, so the grid has a quarter of the
// workgroups (the launch is bound by dispatching them).  Per head the same
// arithmetic as k_combine with a 64-thread workgroup (its block reductions
// are this wave's), so the two give the same output bit for bit.
__global__ __launch_bounds__(kCombineThreads) void k_combine_waves(DecodeParams P, float *q_out) {
  G2B_COMBINE_IN;
  __shared__ float wsh[kCombineThreads / 64][kCombineFewParts];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = blockIdx.x * (kCombineThreads / 64) + wave;
  const int seq = blockIdx.y, li = blockIdx.z;
  const int HD = P.sh.head_dim, nh = P.sh.n_heads;
  const size_t unit = (size_t)li * (size_t)P.n_seq + (size_t)seq;
  const SeqDev sd = P.seqs ? P.seqs[seq] : P.one;
  const int npos = sd.pos + 1;
  int np;
  if (P.wq) {
    const int32_t *ctr = P.wq + ((size_t)P.wq_set * P.wq_cap + unit) * kWqStride;
    np = min(ctr[1], P.max_splits);
    int32_t *nxt = P.wq + (size_t)(P.wq_set ^ 1) * P.wq_cap * kWqStride;
    const size_t nblk = (size_t)gridDim.x * gridDim.y * gridDim.z;
    const size_t bid = blockIdx.x + (size_t)gridDim.x * (blockIdx.y + (size_t)gridDim.y * blockIdx.z);
    for (size_t uu = bid; uu < (size_t)P.wq_zero_units; uu += nblk)
      if (threadIdx.x < 2) nxt[uu * kWqStride + threadIdx.x] = 0;
  } else {
    np = (npos + P.split_len - 1) / P.split_len;
  }
  if (h >= nh) return;  // (no barrier below)
  const size_t pstr = (size_t)(kPartHead + HD);
  const float *base = P.part + (unit * nh + h) * (size_t)P.max_splits * pstr;
  float *w = wsh[wave];
  float mx = kNegBig;
  for (int p = lane; p < np; p += 64) mx = fmaxf(mx, base[p * pstr]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  const float M = mx;
  double lsum = 0.0;
  for (int p = lane; p < np; p += 64) {
    const float wp = exp2f(base[p * pstr] - M);
    w[p] = wp;
    lsum = fma((double)base[p * pstr + 1], (double)wp, lsum);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o);
  const double L = lsum;
  // (w: written and read by this wave only; LDS keeps its order)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float *out = q_out + unit * (size_t)(nh * HD) + (size_t)h * HD;
  for (int d = lane; d < HD; d += 64) {
    const float *a = base + kPartHead + d;
    double o0 = 0.0, o1 = 0.0, o2 = 0.0, o3 = 0.0;
    int p = 0;
    for (; p + 3 < np; p += 4) {
      o0 = fma((double)a[(size_t)p * pstr], (double)w[p], o0);
      o1 = fma((double)a[(size_t)(p + 1) * pstr], (double)w[p + 1], o1);
      o2 = fma((double)a[(size_t)(p + 2) * pstr], (double)w[p + 2], o2);
      o3 = fma((double)a[(size_t)(p + 3) * pstr], (double)w[p + 3], o3);
    }
    for (; p < np; p++) o0 = fma((double)a[(size_t)p * pstr], (double)w[p], o0);
    out[d] = (float)(((o0 + o1) + (o2 + o3)) / L);
  }
  if (P.att) {
    float *at = P.att + (unit * nh + h) * (size_t)P.att_stride;
    for (int t = lane; t < npos; t += 64) at[t] = (float)(exp2((double)at[t] - (double)M) / L);
  }
  G2B_COMBINE_OUT;
}

// ---------------------------------------------------------------- dispatch

static int fast_chunk(const ShapeDev &sh) {
  const int group = sh.n_heads / sh.n_kv_heads;
  if (sh.kv_q8) return group <= 2 ? 32 : 16;
  return 16;
}

int32_t decode_ppw(const ShapeDev &sh, int32_t tune_chunk) {
  if (!decode_fast_available(sh)) return 1;
  const int cd = tune_chunk == 16 ? 16 : fast_chunk(sh);
  const int lpp = sh.n_kv_heads * (sh.head_dim / cd);
  return lpp >= 1 && lpp <= 64 ? 64 / lpp : 1;
}

int32_t decode_chunk(const ShapeDev &sh, int32_t tune_chunk) {
  if (!decode_fast_available(sh)) return 0;
  return tune_chunk == 16 ? 16 : fast_chunk(sh);
}

int32_t decode_stage_rows(const ShapeDev &sh, int32_t tune_chunk, int32_t mode) {
  if (!decode_fast_available(sh)) return 0;
  return stage_rows_of(sh.row_bytes, decode_ppw(sh, tune_chunk), mode);
}

template <int FMT, int HD>
static int occupancy_hd(const ShapeDev &sh, int group, int32_t chunk, int32_t mode, int32_t sr,
                        bool wq) {
  switch (group) {
    case 1: return layer_occupancy<FMT, HD, 1>(sh, chunk, mode, sr, wq);
    case 2: return layer_occupancy<FMT, HD, 2>(sh, chunk, mode, sr, wq);
    case 3: return layer_occupancy<FMT, HD, 3>(sh, chunk, mode, sr, wq);
    default: return layer_occupancy<FMT, HD, 4>(sh, chunk, mode, sr, wq);
  }
}

int decode_blocks_per_cu(const ShapeDev &sh, int32_t tune_chunk, int32_t stage_mode,
                         int32_t stage_rows, bool wq) {
  if (!decode_fast_available(sh)) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_decode_generic, kThreads, 0) !=
        hipSuccess) {
      (void)hipGetLastError();
      return 1;
    }
    return n > 0 ? n : 1;
  }
  const int group = sh.n_heads / sh.n_kv_heads;
  if (sh.kv_q8)
    return sh.head_dim == 128 ? occupancy_hd<1, 128>(sh, group, tune_chunk, stage_mode, stage_rows, wq)
                              : occupancy_hd<1, 64>(sh, group, tune_chunk, stage_mode, stage_rows, wq);
  return sh.head_dim == 128 ? occupancy_hd<0, 128>(sh, group, tune_chunk, stage_mode, stage_rows, wq)
                            : occupancy_hd<0, 64>(sh, group, tune_chunk, stage_mode, stage_rows, wq);
}

bool decode_fast_available(const ShapeDev &sh) {
  if (sh.head_dim != 64 && sh.head_dim != 128) return false;
  if (sh.n_kv_heads <= 0 || sh.n_heads % sh.n_kv_heads) return false;
  const int group = sh.n_heads / sh.n_kv_heads;
  if (group < 1 || group > 4) return false;
  const int lanes = sh.n_kv_heads * (sh.head_dim / fast_chunk(sh));
  // (k_layer's setup loads at most 8192 q and 2048 k floats per thread set)
  return lanes <= 64 && sh.n_heads * sh.head_dim <= 8192 && sh.n_kv_heads * sh.head_dim <= 2048;
}

template <int FMT, int HD>
static hipError_t launch_hd(const DecodeParams &p, int group, int n_layers, hipStream_t s) {
  switch (group) {
    case 1: return launch_layer<FMT, HD, 1>(p, n_layers, s);
    case 2: return launch_layer<FMT, HD, 2>(p, n_layers, s);
    case 3: return launch_layer<FMT, HD, 3>(p, n_layers, s);
    case 4: return launch_layer<FMT, HD, 4>(p, n_layers, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_decode(const DecodeParams &p, int n_layers, hipStream_t s, bool fast,
                         int *used_fast) {
  if (fast && decode_fast_available(p.sh)) {
    if (used_fast) *used_fast = 1;
    const int group = p.sh.n_heads / p.sh.n_kv_heads;
    if (p.sh.kv_q8)
      return p.sh.head_dim == 128 ? launch_hd<1, 128>(p, group, n_layers, s)
                                  : launch_hd<1, 64>(p, group, n_layers, s);
    return p.sh.head_dim == 128 ? launch_hd<0, 128>(p, group, n_layers, s)
                                : launch_hd<0, 64>(p, group, n_layers, s);
  }
  if (used_fast) *used_fast = 0;
  if (p.split_len > kGenericMaxSplit) return hipErrorInvalidValue;
  const dim3 grid = static_grid(p, n_layers);
  hipLaunchKernelGGL(k_decode_generic, grid, dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_combine(const DecodeParams &p, int n_layers, hipStream_t s) {
  if (p.max_splits > kCombineMaxParts) return hipErrorInvalidValue;
  dim3 grid(p.sh.n_heads, p.n_seq, n_layers);
  // Few partials per head: one wave per head, four heads per workgroup.
  // With thousands of heads in the grid (c4: 4096) the launch is bound by
  // dispatching workgroups (~7 us to start 4096 of four waves), not by the
  // merge; many partials (a single long sequence) need a workgroup's four
  // waves on one head.
  if (p.max_splits <= kCombineFewParts) {
    const int hpw = kCombineThreads / 64;  // heads per workgroup
    dim3 g4((p.sh.n_heads + hpw - 1) / hpw, p.n_seq, n_layers);
    hipLaunchKernelGGL(k_combine_waves, g4, dim3(kCombineThreads), 0, s, p, p.q_out);
    return hipGetLastError();
  }
  // Static splits of few units with many partials: a workgroup per (head,
  // quarter of its dims).
  const int hd = p.sh.head_dim, grp = kCombineThreads / (hd / kCombineParts / 4);
  if (!p.wq && hd % (4 * kCombineParts) == 0 && p.max_splits <= kCombineThreads &&
      p.max_splits <= 8 * grp) {
    dim3 gp(p.sh.n_heads * kCombineParts, p.n_seq, n_layers);
    if (p.max_splits <= 4 * grp)
      hipLaunchKernelGGL(k_combine_part<4>, gp, dim3(kCombineThreads), 0, s, p, p.q_out);
    else
      hipLaunchKernelGGL(k_combine_part<8>, gp, dim3(kCombineThreads), 0, s, p, p.q_out);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_combine, grid, dim3(kCombineThreads), 0, s, p, p.q_out);
  return hipGetLastError();
}

}  // namespace g2b
