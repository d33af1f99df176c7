// g2b_device.h - device-side pieces shared by the gfx950 kernels.
//
// Everything here that produces KV bytes must be bit-exact with the
// reference, so this code is compiled with -ffp-contract=off, IEEE division
// (__fdiv_rn) and fp32 denormals preserved; explicit fmaf() is used only in
// the attention arithmetic, where a tolerance applies.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace g2b {

constexpr float kNegBig = -1.0e30f;  // "no score yet": finite, so m - m == 0

// Per-sequence descriptor as the kernels read it (32 bytes).
struct SeqDev {
  int32_t pos;      // new token position; positions 0..pos are attended
  int32_t ctx_cap;  // layer stride in rows
  int32_t pad0, pad1;
  uint8_t *k;       // [n_layers][ctx_cap][row]
  uint8_t *v;
};

// Shape as the kernels read it.
struct ShapeDev {
  int32_t n_layers, n_heads, n_kv_heads, head_dim;
  int32_t arch_llama;  // 1: interleaved pairs, 0: NEOX halves
  int32_t kv_q8;
  int32_t rope_on;     // 0 when head_dim/2 > 512 (reference leaves x unrotated)
  uint32_t row_bytes;
};

// Per-layer QK-RMSNorm weights as the kernels read them (w == nullptr: no
// layer has any).
struct NormDev {
  const float *w;      // [n_layers][2][head_dim]: q weights, then k weights
  const int32_t *on;   // [n_layers]: bit 0 q, bit 1 k
  float eps;
};

__device__ __forceinline__ const float *norm_weights(const NormDev &n, int layer, int which,
                                                     int hd) {
  if (!n.w || !((n.on[layer] >> which) & 1)) return nullptr;
  return n.w + ((size_t)layer * 2 + (size_t)which) * (size_t)hd;
}

// QK-RMSNorm of /root/reference/src/l3_math.c:107-114 on n_heads heads of x,
// in place.  One thread per head sums the squares left to right with each
// product rounded (no contraction, as the reference's -std=c99 build), then
// inv = 1/sqrtf(ss/hd + eps) with IEEE division and square root, then
// x = (w*x)*inv elementwise.  The square root is sqrtf(), which
// -fhip-fp32-correctly-rounded-divide-sqrt makes correctly rounded on gfx950
// (v_sqrt_f32 plus a residual check of both neighbours); __fsqrt_rn compiles
// to the bare 1-ulp v_sqrt_f32 and would differ from the host's sqrtss.  x is LDS, or global memory that only this block
// touches; inv is LDS scratch of n_heads floats.  Every thread calls it.
__device__ inline void qk_rmsnorm_block(float *x, int n_heads, int hd, const float *w,
                                        float eps, float *inv) {
  for (int h = threadIdx.x; h < n_heads; h += blockDim.x) {
    const float *xh = x + (size_t)h * hd;
    float ss = 0.f;
    for (int j = 0; j < hd; j++) {
      const float sq = xh[j] * xh[j];
      ss = ss + sq;
    }
    inv[h] = __fdiv_rn(1.f, sqrtf(__fdiv_rn(ss, (float)hd) + eps));
  }
  __syncthreads();
  for (int e = threadIdx.x; e < n_heads * hd; e += blockDim.x) {
    const int h = e / hd, j = e - h * hd;
    const float wx = w[j] * x[e];
    x[e] = wx * inv[h];
  }
  __syncthreads();
}

// Truncating fp32 -> fp16 of /root/reference/src/l3_math.c:6-16.
__device__ __forceinline__ uint32_t f32_to_half_trunc(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const int32_t e8 = (int32_t)((u >> 23) & 0xffu);
  if (e8 == 0xff) return sign | 0x7c00u;
  const int32_t e5 = e8 - 112;
  if (e5 <= 0) return sign;
  if (e5 >= 31) return sign | 0x7c00u;
  return sign | ((uint32_t)e5 << 10) | ((u & 0x7fffffu) >> 13);
}

// Exact fp16 -> fp32 of /root/reference/src/l2_codec.c:35-54, built from bits
// (subnormals: m * 2^-24 is exact in fp32).
__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t e5 = (h >> 10) & 0x1fu;
  const uint32_t m10 = h & 0x3ffu;
  if (e5 == 0) {
    const float f = (float)m10 * 5.9604644775390625e-8f;  // 2^-24
    return __uint_as_float(__float_as_uint(f) | sign);
  }
  const uint32_t e8 = (e5 == 31) ? 0xffu : (e5 + 112u);
  return __uint_as_float(sign | (e8 << 23) | (m10 << 13));
}

// fp16 bits (low 16 bits of h) -> fp32 by the hardware conversion
// (v_cvt_f32_f16).  Exact for every finite or infinite half, subnormals
// included: the kernels run with fp16 denormals preserved
// (float_denorm_mode_16_64 = 3).  It differs from half_bits_to_f32 only in
// the payload of a NaN, which no attention output can show (a NaN block
// scale makes the output NaN either way).  The attention loops use it for
// block scales; everything that writes KV bytes uses half_bits_to_f32.
__device__ __forceinline__ float half_bits_to_f32_hw(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// sum(x[i]^2), i < n, over a workgroup of 256 threads (x 16-byte aligned;
// red: 4 floats of LDS), returned to every thread: thread t accumulates the
// float4 pieces t, t + 256, ... in element order (eight loads in flight),
// then, if t < n % 4, element 4 * (n / 4) + t; a tree per wave;
// (w0 + w1) + (w2 + w3).  rmsnorm's sum (l3_math.c:21-37) in another fp32
// order; one order for every kernel that normalises, so they agree bitwise.
// STAGE: also xw[i] = x[i] * w[i] for i < 4 * (n / 4) (xw: LDS).
template <bool STAGE>
__device__ inline float wg256_sumsq_t(const float *x, int n, float *red, const float *w,
                                      float *xw) {
  const int t = threadIdx.x, n4 = n >> 2;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  float s = 0.f;
  for (int i0 = t; i0 < n4; i0 += 8 * 256) {
    float4 v[8];
    [[maybe_unused]] float4 g[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const bool in = i0 + 256 * k < n4;
      v[k] = in ? x4[i0 + 256 * k] : make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (STAGE) {
        const int e = 4 * (i0 + 256 * k);
        g[k] = in ? make_float4(w[e], w[e + 1], w[e + 2], w[e + 3]) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      s = fmaf(v[k].x, v[k].x, s);
      s = fmaf(v[k].y, v[k].y, s);
      s = fmaf(v[k].z, v[k].z, s);
      s = fmaf(v[k].w, v[k].w, s);
      if constexpr (STAGE) {
        if (i0 + 256 * k < n4)
          reinterpret_cast<float4 *>(xw)[i0 + 256 * k] =
              make_float4(v[k].x * g[k].x, v[k].y * g[k].y, v[k].z * g[k].z, v[k].w * g[k].w);
      }
    }
  }
  if (t < (n & 3)) s = fmaf(x[4 * n4 + t], x[4 * n4 + t], s);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if ((t & 63) == 0) red[t >> 6] = s;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ inline float wg256_sumsq(const float *x, int n, float *red) {
  return wg256_sumsq_t<false>(x, n, red, nullptr, nullptr);
}

// (int32)lroundf(r) as glibc on x86-64 gives it: round half away from zero,
// out-of-range and NaN produce LONG_MIN, whose low 32 bits are 0.
__device__ __forceinline__ int32_t lround_i32_like_host(float r) {
  if (!(fabsf(r) < 9.2233720368547758e18f)) return 0;
  return (int32_t)(int64_t)roundf(r);
}

// One Q8_0 block (/root/reference/src/l5_model.c:49-59) of cnt <= 32 floats
// to 34 bytes at dst (2-byte aligned), little-endian fp16 scale first.
__device__ __forceinline__ void q8_quant_block(const float *x, int cnt, uint8_t *dst) {
  float amax = 0.f;
  for (int j = 0; j < cnt; j++) {
    const float a = fabsf(x[j]);
    if (a > amax) amax = a;
  }
  float d = __fdiv_rn(amax, 127.f);
  if (!(d > 0.f)) d = 1e-10f;
  uint16_t *out16 = reinterpret_cast<uint16_t *>(dst);
  out16[0] = (uint16_t)f32_to_half_trunc(d);
#pragma unroll
  for (int j = 0; j < 32; j += 2) {
    int32_t qa = 0, qb = 0;
    if (j < cnt) {
      qa = lround_i32_like_host(__fdiv_rn(x[j], d));
      qa = qa > 127 ? 127 : (qa < -127 ? -127 : qa);
    }
    if (j + 1 < cnt) {
      qb = lround_i32_like_host(__fdiv_rn(x[j + 1], d));
      qb = qb > 127 ? 127 : (qb < -127 ? -127 : qb);
    }
    out16[1 + j / 2] = (uint16_t)((uint32_t)(qa & 0xff) | ((uint32_t)(qb & 0xff) << 8));
  }
}

// The same block quantised by four consecutive lanes of a wave, eight
// elements each (part = 0..3, all four lanes call together): each lane's
// maximum of |x| over its elements (NaN skipped by '>', as in the serial
// loop), combined across the four with the same '>' - an exact maximum, so
// amax, d, the scale bits and every byte equal q8_quant_block's.  x may be
// LDS or global memory; elements at or past cnt are padding (byte 0).
__device__ __forceinline__ void q8_quant_block_x4(const float *x, int cnt, uint8_t *dst,
                                                  int part) {
  float v[8];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int e = 8 * part + j;
    v[j] = e < cnt ? x[e] : 0.f;
    const float a = fabsf(v[j]);
    if (a > amax) amax = a;
  }
  float o = __shfl_xor(amax, 1);
  if (o > amax) amax = o;
  o = __shfl_xor(amax, 2);
  if (o > amax) amax = o;
  float d = __fdiv_rn(amax, 127.f);
  if (!(d > 0.f)) d = 1e-10f;
  uint16_t *out16 = reinterpret_cast<uint16_t *>(dst);
  if (part == 0) out16[0] = (uint16_t)f32_to_half_trunc(d);
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    int32_t qa = 0, qb = 0;
    if (8 * part + j < cnt) {
      qa = lround_i32_like_host(__fdiv_rn(v[j], d));
      qa = qa > 127 ? 127 : (qa < -127 ? -127 : qa);
    }
    if (8 * part + j + 1 < cnt) {
      qb = lround_i32_like_host(__fdiv_rn(v[j + 1], d));
      qb = qb > 127 ? 127 : (qb < -127 ? -127 : qb);
    }
    out16[1 + 4 * part + j / 2] = (uint16_t)((uint32_t)(qa & 0xff) | ((uint32_t)(qb & 0xff) << 8));
  }
}

// RoPE pair rotation of /root/reference/src/l3_math.c:79 and :98-99:
// a' = a*c - b*s, b' = a*s + b*c, each product rounded (no contraction).
__device__ __forceinline__ void rope_pair(float &a, float &b, float c, float s) {
  const float a0 = a, b0 = b;
  a = a0 * c - b0 * s;
  b = a0 * s + b0 * c;
}

// Indices of RoPE pair j inside a head: LLaMA (2j, 2j+1), NEOX (j, j+hd/2).
__device__ __forceinline__ void rope_pair_index(int arch_llama, int j, int half, int &ia,
                                                int &ib) {
  ia = arch_llama ? 2 * j : j;
  ib = arch_llama ? 2 * j + 1 : j + half;
}

// [QK-RMSNorm, then] RoPE(k) [and the same for q into qr when q != nullptr]
// at `pos`, then store the k and v rows at (layer, pos): l5_model.c:505-516
// for one sequence.  Called by every thread of the block; kr is LDS scratch
// of nkv floats, inv of n_heads floats.
__device__ inline void append_row(const ShapeDev &sh, const SeqDev &sd, int layer, int pos,
                                  const float *k, const float *v, const float *q, float *qr,
                                  const float *rope, const NormDev &norm, float *kr,
                                  float *inv) {
  const int hd = sh.head_dim, half = hd / 2;
  const int nkv = sh.n_kv_heads * hd;
  const float *cs = (sh.rope_on && rope) ? rope + (size_t)pos * hd : nullptr;
  const float *wq = q ? norm_weights(norm, layer, 0, hd) : nullptr;
  const float *wk = norm_weights(norm, layer, 1, hd);

  for (int e = threadIdx.x; e < nkv; e += blockDim.x) kr[e] = k[e];
  if (wq)
    for (int e = threadIdx.x; e < sh.n_heads * hd; e += blockDim.x) qr[e] = q[e];
  __syncthreads();
  if (wk) qk_rmsnorm_block(kr, sh.n_kv_heads, hd, wk, norm.eps, inv);
  if (wq) {
    qk_rmsnorm_block(qr, sh.n_heads, hd, wq, norm.eps, inv);
    q = qr;  // rotate the normalised copy in place
  }
  if (cs) {
    for (int p = threadIdx.x; p < sh.n_kv_heads * half; p += blockDim.x) {
      const int h = p / half, j = p - h * half;
      int ia, ib;
      rope_pair_index(sh.arch_llama, j, half, ia, ib);
      rope_pair(kr[h * hd + ia], kr[h * hd + ib], cs[2 * j], cs[2 * j + 1]);
    }
  }
  if (q) {
    for (int p = threadIdx.x; p < sh.n_heads * half; p += blockDim.x) {
      const int h = p / half, j = p - h * half;
      int ia, ib;
      rope_pair_index(sh.arch_llama, j, half, ia, ib);
      float a = q[h * hd + ia], b = q[h * hd + ib];
      if (cs) rope_pair(a, b, cs[2 * j], cs[2 * j + 1]);
      qr[h * hd + ia] = a;
      qr[h * hd + ib] = b;
    }
  }
  __syncthreads();

  const size_t off = ((size_t)layer * (size_t)sd.ctx_cap + (size_t)pos) * sh.row_bytes;
  if (!sh.kv_q8) {
    float *kd = reinterpret_cast<float *>(sd.k + off);
    float *vd = reinterpret_cast<float *>(sd.v + off);
    for (int e = threadIdx.x; e < nkv; e += blockDim.x) {
      kd[e] = kr[e];
      vd[e] = v[e];
    }
    return;
  }
  const int nb = (nkv + 31) / 32;
  for (int b = threadIdx.x; b < 2 * nb; b += blockDim.x) {
    const bool is_k = b < nb;
    const int bb = is_k ? b : b - nb;
    const int cnt = min(32, nkv - 32 * bb);
    const float *src = is_k ? kr + 32 * bb : v + 32 * bb;
    uint8_t *dst = (is_k ? sd.k : sd.v) + off + 34 * (size_t)bb;
    q8_quant_block(src, cnt, dst);
  }
}

}  // namespace g2b
