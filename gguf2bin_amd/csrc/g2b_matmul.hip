// g2b_matmul.hip - device GEMVs of gguf2bin2's weight types: the fused
// matmul_q8_0 / matmul_q4_0 (/root/reference/src/l2_codec.c:203-340) and the
// F32 matmul (src/l3_math.c:17-20), dispatched as matmul_q does
// (l2_codec.c:342-349), and the types matmul_q runs through its dequantising
// fallback (:350-366; gguf_dequant :186-199) whose dequantisation is
// defined: F16 and Q4_1.  out[i] = sum_j W[i][j] * x[j], i < d.
//
// Weight rows are streamed once per call (HBM-bound: 1.0625 B per weight for
// Q8_0, 0.5625 B for Q4_0, 4 B for F32).  Q8_0 / Q4_0: a row of nb = n/32
// blocks is spread over LPR lanes (LPR = nb rounded up to a power of two, at
// most 64), lane c taking blocks c, c + LPR, ...; a wave covers 64/LPR rows
// per step, so one step reads a contiguous run of whole rows.  Each lane
// keeps the x values of its blocks in registers (up to two blocks; more are
// read through the cache) and loads its blocks as dwords from the dword
// boundary at or before the block (blocks are 2-byte aligned), extracting
// the bytes with v_perm.  Arithmetic is fp32 like the reference: per block
// sum_j q_j x_j by FMA, times the fp16 scale, summed over the lane's blocks
// and then across the row's lanes.  Q8_0 over many rows (the lm head) takes
// x as int8 digit planes instead (wg_x_digits): integer dot products per
// block, then the same fp16 scale and sums.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "g2b_internal.h"
#include "g2b_layer.h"  // LDS DMA (dma16, raw_rsrc, lds_addr, wait_vm0)

namespace g2b {

namespace {

typedef float gemv_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t gemv_u32x4 __attribute__((ext_vector_type(4)));
// four dwords at any 4-byte boundary (global memory takes multi-dword loads
// at dword alignment)
typedef uint32_t gemv_u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kGemvThreads = 256;
constexpr int kGemvUnroll = 4;  // steps whose loads are in flight together
constexpr int kGemvGroup = 8;   // blocks per lane in flight (x in LDS or the cache)
constexpr int kGemvMinSteps = 8;            // wave-steps per wave, where there are enough
constexpr int kGemvMaxXLds = 64 * 1024;     // x staged in LDS up to this many bytes
constexpr int kGemvXdMinRows = 32768;       // Q8_0 with x as digit planes (XD) from this many rows

template <typename T>
__device__ __forceinline__ T nt_load(const void *p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) T *)p);
}

// Dwords [B, B + 4N) where B is the dword boundary at or before p, and the
// byte offset of p inside the first one (0 or 2 for 2-byte aligned blocks).
// Default cache policy: neighbouring lanes' windows share their edge dwords,
// which non-temporal loads would fetch twice.
template <int N>
__device__ __forceinline__ void load_dwords(const uint8_t *p, uint32_t (&d)[N], uint32_t &sh) {
  const uintptr_t a = (uintptr_t)p;
  const __attribute__((address_space(1))) uint32_t *base =
      (const __attribute__((address_space(1))) uint32_t *)(a & ~(uintptr_t)3);
  sh = (uint32_t)(a & 3u);
#pragma unroll
  for (int i = 0; i < N; i++) d[i] = base[i];
}

// Quant words j of a block whose payload starts 2 bytes after its first
// byte: bytes 2..5 (sh 0) or 4..7 (sh 2) of the dword pair (d[j], d[j+1]).
__device__ __forceinline__ uint32_t payload_word(const uint32_t *d, int j, uint32_t sh) {
  return __builtin_amdgcn_perm(d[j + 1], d[j], sh ? 0x07060504u : 0x05040302u);
}

__device__ __forceinline__ float scale_of(uint32_t d0, uint32_t sh) {
  return half_bits_to_f32_hw((d0 >> (8u * sh)) & 0xFFFFu);
}

// Block formats of k_gemv_q: FMT 1 = Q8_0 (34 bytes), 2 = Q4_0 (18), 3 =
// Q4_1 (20: fp16 d, fp16 m, 16 bytes of nibbles).
template <int FMT>
constexpr int block_bytes() {
  return FMT == 1 ? 34 : FMT == 2 ? 18 : 20;
}
// Raw block bytes: the dwords covering a 2-byte aligned block (Q8_0 9, Q4_0
// 5, Q4_1 6).
template <int FMT>
struct BlockRaw {
  static constexpr int N = FMT == 1 ? 9 : FMT == 2 ? 5 : 6;
  uint32_t d[N];
  uint32_t sh;
};

template <int FMT>
__device__ __forceinline__ void load_block(BlockRaw<FMT> &r, const uint8_t *p) {
  load_dwords<BlockRaw<FMT>::N>(p, r.d, r.sh);
}

template <int FMT>
__device__ __forceinline__ void zero_block(BlockRaw<FMT> &r) {
#pragma unroll
  for (int i = 0; i < BlockRaw<FMT>::N; i++) r.d[i] = 0u;
  r.sh = 0u;
}

// v_cvt_off_f32_i4 of the low nibble of byte B of t (SDWA byte select, so
// no shift is needed to bring the nibble down).
template <int B>
__device__ __forceinline__ float nib_f(uint32_t t) {
  float r;
  if constexpr (B == 0)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0"
        : "=v"(r) : "v"(t));
  else if constexpr (B == 1)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1"
        : "=v"(r) : "v"(t));
  else if constexpr (B == 2)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2"
        : "=v"(r) : "v"(t));
  else
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3"
        : "=v"(r) : "v"(t));
  return r;
}

// sum_j w_j x_j of one block in fp32 (x: the block's 32 values).
template <int FMT>
__device__ __forceinline__ float block_dot(const BlockRaw<FMT> &r, const float *x) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  if constexpr (FMT == 1) {
    // Q8_0 (l2_codec.c:306-320): d * (int8) q_j, element j = byte j
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t w = payload_word(r.d, j, r.sh);
      a0 = fmaf((float)(int8_t)(w & 0xFFu), x[4 * j + 0], a0);
      a1 = fmaf((float)(int8_t)((w >> 8) & 0xFFu), x[4 * j + 1], a1);
      a2 = fmaf((float)(int8_t)((w >> 16) & 0xFFu), x[4 * j + 2], a2);
      a3 = fmaf((float)(int8_t)(w >> 24), x[4 * j + 3], a3);
    }
    return ((a0 + a1) + (a2 + a3)) * scale_of(r.d[0], r.sh);
  } else if constexpr (FMT == 2) {
    // Q4_0 (l2_codec.c:321-337): byte j holds element j (low nibble) and
    // element j + 16 (high nibble), each (nibble - 8) * d.  v_cvt_off_f32_i4
    // turns a signed nibble s into s / 16; nibble ^ 8 read as signed is
    // nibble - 8, so the block's value is 16 * d * sum(...).
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t t = payload_word(r.d, j, r.sh) ^ 0x88888888u;
      const uint32_t h = t >> 4;
      a0 = fmaf(nib_f<0>(t), x[4 * j + 0], a0);
      a1 = fmaf(nib_f<1>(t), x[4 * j + 1], a1);
      a0 = fmaf(nib_f<2>(t), x[4 * j + 2], a0);
      a1 = fmaf(nib_f<3>(t), x[4 * j + 3], a1);
      a2 = fmaf(nib_f<0>(h), x[16 + 4 * j + 0], a2);
      a3 = fmaf(nib_f<1>(h), x[16 + 4 * j + 1], a3);
      a2 = fmaf(nib_f<2>(h), x[16 + 4 * j + 2], a2);
      a3 = fmaf(nib_f<3>(h), x[16 + 4 * j + 3], a3);
    }
    return ((a0 + a1) + (a2 + a3)) * (16.f * scale_of(r.d[0], r.sh));
  } else {
    // Q4_1 (gguf_dequant's deq_q4_1, l2_codec.c:65-75): byte j holds
    // elements j (low nibble) and j + 16 (high), each d * q + m.  With the
    // same signed-nibble converts as Q4_0 (S = sum (q - 8)/16 * x), the
    // block is 16 d S + (8 d + m) sum x.  (The reference rounds each weight
    // d*q + m to fp32 before its products; the difference is within one
    // fp32 rounding of each product, inside the GEMV bound.)
    float x0 = 0.f, x1 = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t w =
          r.sh ? __builtin_amdgcn_perm(r.d[j + 2], r.d[j + 1], 0x05040302u) : r.d[j + 1];
      const uint32_t t = w ^ 0x88888888u;
      const uint32_t h = t >> 4;
      a0 = fmaf(nib_f<0>(t), x[4 * j + 0], a0);
      a1 = fmaf(nib_f<1>(t), x[4 * j + 1], a1);
      a0 = fmaf(nib_f<2>(t), x[4 * j + 2], a0);
      a1 = fmaf(nib_f<3>(t), x[4 * j + 3], a1);
      a2 = fmaf(nib_f<0>(h), x[16 + 4 * j + 0], a2);
      a3 = fmaf(nib_f<1>(h), x[16 + 4 * j + 1], a3);
      a2 = fmaf(nib_f<2>(h), x[16 + 4 * j + 2], a2);
      a3 = fmaf(nib_f<3>(h), x[16 + 4 * j + 3], a3);
      x0 += (x[4 * j + 0] + x[4 * j + 1]) + (x[4 * j + 2] + x[4 * j + 3]);
      x1 += (x[16 + 4 * j + 0] + x[16 + 4 * j + 1]) + (x[16 + 4 * j + 2] + x[16 + 4 * j + 3]);
    }
    const float d = scale_of(r.d[0], r.sh);
    const float m = half_bits_to_f32_hw(r.sh ? (r.d[1] & 0xFFFFu) : (r.d[0] >> 16));
    return fmaf((a0 + a1) + (a2 + a3), 16.f * d, (x0 + x1) * fmaf(8.f, d, m));
  }
}

// Fused forms (GemvParams): rmsnorm (l3_math.c:21-50) as (x * w) * inv with
// inv = 1 / sqrtf(sum(x^2) / n + eps), computed by every workgroup from the
// whole of x in wg256_sumsq's order (the model's own rmsnorm kernel's);
// x * w goes to LDS (xs: n floats, n a multiple of 32) in the same pass.
__device__ __forceinline__ float wg_rms_stage(const GemvParams &P, float *xs) {
  static_assert(kGemvThreads == 256, "wg256_sumsq");
  __shared__ float red[kGemvThreads / 64];
  const float sum = wg256_sumsq_t<true>(P.x, P.n, red, P.nw, xs);
  return 1.f / sqrtf(sum / (float)P.n + P.eps);
}

// silu(x) * x2 (silu, l3_math.c:57-62, then the product of l5_model.c:595)
// for the whole of x, once per workgroup, into LDS (xs: n floats; n is a
// multiple of 32, x and x2 16-byte aligned): eight float4 pieces of each in
// flight per thread.
__device__ __forceinline__ void wg_silu_mul(const GemvParams &P, float *xs) {
  const int n4 = P.n >> 2;
  const float4 *g4 = reinterpret_cast<const float4 *>(P.x);
  const float4 *u4 = reinterpret_cast<const float4 *>(P.x2);
  for (int i0 = threadIdx.x; i0 < n4; i0 += 8 * kGemvThreads) {
    float4 g[8], u[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      if (i0 + kGemvThreads * k < n4) {
        g[k] = g4[i0 + kGemvThreads * k];
        u[k] = u4[i0 + kGemvThreads * k];
      }
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      if (i0 + kGemvThreads * k < n4) {
        float4 r;
        r.x = (g[k].x / (1.f + expf(-g[k].x))) * u[k].x;
        r.y = (g[k].y / (1.f + expf(-g[k].y))) * u[k].y;
        r.z = (g[k].z / (1.f + expf(-g[k].z))) * u[k].z;
        r.w = (g[k].w / (1.f + expf(-g[k].w))) * u[k].w;
        reinterpret_cast<float4 *>(xs)[i0 + kGemvThreads * k] = r;
      }
    }
  }
  __syncthreads();
}

// x[i..i+4) as the rows read it: plain, rmsnorm'd (x * w from LDS, times
// inv, as rmsnorm's AVX2 loop) or SiLU x up from LDS.  i is a multiple of 4,
// x 16-byte aligned.
__device__ __forceinline__ float4 pro_x4(const GemvParams &P, const float *xs, int i, float inv) {
  if (P.pro == kProNone) return *reinterpret_cast<const float4 *>(P.x + i);
  float4 v = *reinterpret_cast<const float4 *>(xs + i);
  if (P.pro == kProRmsnorm) {
    v.x *= inv;
    v.y *= inv;
    v.z *= inv;
    v.w *= inv;
  }
  return v;
}

// A lane's x blocks (KB of them, blocks b0 + LPR * k below b_hi) in
// registers, through the prologue.
template <int LPR, int KB>
__device__ __forceinline__ void lane_x(const GemvParams &P, const float *xs, int b0, int b_hi,
                                       float inv, float (&xr)[KB][32]) {
#pragma unroll
  for (int k = 0; k < KB; k++) {
    const int b = b0 + LPR * k;
#pragma unroll
    for (int j = 0; j < 32; j += 4) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (b < b_hi) v = pro_x4(P, xs, 32 * b + j, inv);
      xr[k][j] = v.x;
      xr[k][j + 1] = v.y;
      xr[k][j + 2] = v.z;
      xr[k][j + 3] = v.w;
    }
  }
}

// x as four signed int8 digit planes of a 31-bit fixed point per 32-element
// block (the Q8_0 XD form): m = rint(x * 2^(30-e)), 2^(e-1) <= max|x| < 2^e,
// m = d0 + 256 d1 + 65536 d2 + 2^24 d3.  The workgroup makes every block's
// planes once into LDS - dig[b][plane][chunk] (a dword = one plane of four
// elements), then exps[b] and units[b] (1, or NaN for a block with a
// non-finite x: its rows' sums are then NaN) - from x as the rows read it
// (pro_x4), and each lane loads its blocks' planes into registers.  A
// block's sum_j q_j x_j is then four chains of v_dot4_i32_i8 (exact in
// int32), combined in fp32 and scaled by the fp16 scale and 2^(e-30): about
// half the VALU operations of the convert-and-FMA form per weight.  x's
// rounding (2^-31 of its block maximum) is far below fp32's.
__device__ __forceinline__ void wg_x_digits(const GemvParams &P, const float *xs, float inv,
                                            uint32_t *dig) {
  const int nb = P.nb;
  int32_t *exps = reinterpret_cast<int32_t *>(dig + nb * 32);
  float *units = reinterpret_cast<float *>(exps + nb);
  for (int it = threadIdx.x; it < nb * 8; it += kGemvThreads) {
    const int b = it >> 3, j = it & 7;  // chunk j: elements 4j .. 4j+3 of block b
    const float4 v = pro_x4(P, xs, 32 * b + 4 * j, inv);
    float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    mx = fmaxf(mx, __shfl_xor(mx, 1));
    mx = fmaxf(mx, __shfl_xor(mx, 2));
    mx = fmaxf(mx, __shfl_xor(mx, 4));
    int e = 0;
    (void)frexpf(mx, &e);
    const float xv[4] = {v.x, v.y, v.z, v.w};
    uint32_t pl[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      int m = (int)rintf(ldexpf(xv[k], 30 - e));  // |m| <= 2^30, exact scaling
      int d[4];
#pragma unroll
      for (int q = 0; q < 3; q++) {
        d[q] = ((m + 128) & 255) - 128;
        m = (m - d[q]) >> 8;
      }
      d[3] = m;
#pragma unroll
      for (int q = 0; q < 4; q++) pl[q] |= ((uint32_t)d[q] & 0xFFu) << (8 * k);
    }
#pragma unroll
    for (int q = 0; q < 4; q++) dig[(b * 4 + q) * 8 + j] = pl[q];
    if (j == 0) {
      exps[b] = e;
      units[b] = (mx <= 3.402823466e38f) ? 1.f : __int_as_float(0x7fc00000);
    }
  }
  __syncthreads();
}

// A lane's x blocks (KB of them, blocks b0 + LPR * k below nb) as digit
// planes, their exponents and units (zero past nb).
template <int LPR, int KB>
__device__ __forceinline__ void lane_xd(const GemvParams &P, const uint32_t *dig, int b0,
                                        uint32_t (&xd)[KB][4][8], int (&xe)[KB],
                                        float (&xu)[KB]) {
  const int nb = P.nb;
  const int32_t *exps = reinterpret_cast<const int32_t *>(dig + nb * 32);
  const float *units = reinterpret_cast<const float *>(exps + nb);
#pragma unroll
  for (int k = 0; k < KB; k++) {
    const int b = b0 + LPR * k;
    const bool on = b < nb;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint4 a = make_uint4(0u, 0u, 0u, 0u), c = make_uint4(0u, 0u, 0u, 0u);
      if (on) {
        a = *reinterpret_cast<const uint4 *>(dig + (b * 4 + q) * 8);
        c = *reinterpret_cast<const uint4 *>(dig + (b * 4 + q) * 8 + 4);
      }
      xd[k][q][0] = a.x;
      xd[k][q][1] = a.y;
      xd[k][q][2] = a.z;
      xd[k][q][3] = a.w;
      xd[k][q][4] = c.x;
      xd[k][q][5] = c.y;
      xd[k][q][6] = c.z;
      xd[k][q][7] = c.w;
    }
    xe[k] = on ? exps[b] : 0;
    xu[k] = on ? units[b] : 0.f;
  }
}

// sum_j q_j x_j of one Q8_0 block against x's digit planes.
__device__ __forceinline__ float block_dot_xd(const BlockRaw<1> &r, const uint32_t (&d)[4][8],
                                              int e, float u) {
  int s[4];
#pragma unroll
  for (int q = 0; q < 4; q++) s[q] = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t w = payload_word(r.d, j, r.sh);
#pragma unroll
    for (int q = 0; q < 4; q++) s[q] = __builtin_amdgcn_sdot4((int)w, (int)d[q][j], s[q], false);
  }
  // |s3| <= 32*128*64, so s3*256 + s2 fits in int32
  const float t = (float)(s[3] * 256 + s[2]);
  const float sum = fmaf(fmaf(t, 256.f, (float)s[1]), 256.f, (float)s[0]);
  // times the scale, then 2^(e-30) (ldexp: no overflow or early underflow
  // for blocks of very large or very small x)
  return ldexpf(sum * scale_of(r.d[0], r.sh), e - 30) * u;
}

// Row `row` of the launch's concatenated segments: its weights, and the
// store of its result (segment 0 adds the residual res when given:
// x[i] += xb[i], l5_model.c:583, :597).
__device__ __forceinline__ const uint8_t *seg_row(const GemvParams &P, int row) {
  if (row < P.d0) return P.w + (size_t)row * P.row_bytes;
  if (row < P.d01) return P.w1 + (size_t)(row - P.d0) * P.row_bytes;
  return P.w2 + (size_t)(row - P.d01) * P.row_bytes;
}
__device__ __forceinline__ void seg_store(const GemvParams &P, int row, float acc) {
  if (row < P.d0)
    P.out[row] = P.res ? P.res[row] + acc : acc;
  else if (row < P.d01)
    P.out1[row - P.d0] = acc;
  else
    P.out2[row - P.d01] = acc;
}

template <int LPR>
__device__ __forceinline__ float lanes_sum(float v) {
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Q8_0 / Q4_0.  KB > 0: the lane's x blocks (KB of them) live in registers,
// prepared while the first weights are in flight (the fused forms: LDS of n
// floats for SiLU x up); with XD (Q8_0) as digit planes (wg_x_digits, after
// those n floats in LDS); KB == -1: any nb, x staged once per workgroup in
// LDS; KB == 0: any nb, x read per block through the cache.
template <int FMT, int LPR, int KB, bool XD = false>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_q(GemvParams P) {
  static_assert(!XD || (FMT == 1 && KB > 0), "digit planes: Q8_0 with x in registers");
  extern __shared__ float xs[];
  constexpr int RPS = 64 / LPR;  // rows per wave-step
  constexpr int BB = block_bytes<FMT>();
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6);
  const int rr = lane / LPR, c = lane % LPR;
  const int nb = P.nb;
  [[maybe_unused]] float xr[(KB > 0 && !XD) ? KB : 1][32];
  [[maybe_unused]] uint32_t xd[XD ? KB : 1][4][8];
  [[maybe_unused]] int xe[XD ? KB : 1];
  [[maybe_unused]] float xu[XD ? KB : 1];
  if constexpr (KB < 0) {
    const int n4 = nb * 8;
    for (int i0 = threadIdx.x; i0 < n4; i0 += 8 * kGemvThreads) {
      float4 v[8];
#pragma unroll
      for (int k = 0; k < 8; k++)
        if (i0 + k * kGemvThreads < n4)
          v[k] = reinterpret_cast<const float4 *>(P.x)[i0 + k * kGemvThreads];
#pragma unroll
      for (int k = 0; k < 8; k++)
        if (i0 + k * kGemvThreads < n4) reinterpret_cast<float4 *>(xs)[i0 + k * kGemvThreads] = v[k];
    }
    __syncthreads();
  }
  const int stride = P.n_waves;
  if constexpr (KB > 0) {
    // Every wave runs the first trip (rows or not): its weights are issued,
    // then the workgroup prepares x (barriers) while they are in flight.
    // (Twice the steps in flight for Q4_0 measured slower.)
    constexpr int UN = kGemvUnroll;
    for (int s0 = gw, trip = 0;; s0 += stride * UN, trip++) {
      BlockRaw<FMT> raw[UN][KB];
      int row[UN];
      bool ok[UN];
#pragma unroll
      for (int u = 0; u < UN; u++) {
        const int s = s0 + u * stride;
        row[u] = s * RPS + rr;
        ok[u] = s < P.steps && row[u] < P.d;
#pragma unroll
        for (int k = 0; k < KB; k++) {
          const int b = c + LPR * k;
          if (ok[u] && b < nb)
            load_block<FMT>(raw[u][k], seg_row(P, row[u]) + (size_t)b * BB);
          else
            zero_block<FMT>(raw[u][k]);
        }
      }
      if (trip == 0) {
        float inv = 1.f;
        if (P.pro == kProSiluMul) wg_silu_mul(P, xs);
        if (P.pro == kProRmsnorm) inv = wg_rms_stage(P, xs);
        if constexpr (XD) {
          uint32_t *dig = reinterpret_cast<uint32_t *>(xs + (P.pro != kProNone ? P.n : 0));
          wg_x_digits(P, xs, inv, dig);
          lane_xd<LPR, KB>(P, dig, c, xd, xe, xu);
        } else {
          lane_x<LPR, KB>(P, xs, c, nb, inv, xr);
        }
      }
#pragma unroll
      for (int u = 0; u < UN; u++) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < KB; k++) {
          if constexpr (XD)
            acc += block_dot_xd(raw[u][k], xd[k], xe[k], xu[k]);
          else
            acc += block_dot<FMT>(raw[u][k], xr[k]);
        }
        acc = lanes_sum<LPR>(acc);
        if (ok[u] && c == 0) seg_store(P, row[u], acc);
      }
      if (s0 + stride * UN >= P.steps) break;
    }
  } else {
    for (int s0 = gw; s0 < P.steps; s0 += stride * kGemvUnroll) {
      // any number of blocks: kGemvGroup of the lane's blocks in flight at a time
#pragma unroll 1
      for (int u = 0; u < kGemvUnroll; u++) {
        const int s = s0 + u * stride;
        const int row = s * RPS + rr;
        const bool ok = s < P.steps && row < P.d;  // (uniform per row group)
        const uint8_t *wr = P.w + (size_t)row * P.row_bytes;
        float acc = 0.f;
        for (int b0 = c; ok && b0 < nb; b0 += kGemvGroup * LPR) {
          BlockRaw<FMT> r[kGemvGroup];
#pragma unroll
          for (int g = 0; g < kGemvGroup; g++) {
            const int b = b0 + g * LPR;
            if (b < nb)
              load_block<FMT>(r[g], wr + (size_t)b * BB);
            else
              zero_block<FMT>(r[g]);
          }
#pragma unroll
          for (int g = 0; g < kGemvGroup; g++) {
            const int b = b0 + g * LPR;
            if (b < nb) acc += block_dot<FMT>(r[g], (KB < 0 ? xs : P.x) + 32 * b);
          }
        }
        acc = lanes_sum<LPR>(acc);
        if (ok && c == 0) P.out[row] = acc;
      }
    }
  }
}

// Q8_0 / Q4_0 rows of nb = 16 * BPL blocks (BPL even) on the int8 matrix
// cores, for the plain product (no prologue, one segment); dispatched for
// Q4_0 with 1024-element rows (launch_gemv).  v_mfma_i32_4x4x4_16b_i8 computes,
// in each of its 16 groups of four lanes, D[l][i] += dot4(A[4*(l/4) + i],
// B[l]) (the lane layout checked on the device): lane l = 4*g + r takes row
// r of the wave-step's four rows and blocks g*BPL .. g*BPL + BPL - 1 of it,
// so the four lanes of a group read the same block of four rows; B lane l =
// four of its row's quants, A lane 4*g + i = digit plane i of the same four
// elements of x.  x is held as four signed int8 digit planes of a 31-bit
// fixed point relative to each block's largest |x| (m = rint(x * 2^(30-e)),
// 2^(e-1) <= max|x| < 2^e; m = d0 + 256 d1 + 65536 d2 + 2^24 d3), so the
// eight MFMAs of a block give exact int32 plane sums; the block's sum is
// ((D3*256 + D2)*256 + D1)*256 + D0 in fp32, times the block's fp16 scale
// and 2^(e-30), and the lane's blocks and then the row's 16 lanes are summed
// in fp32.  x's rounding (2^-31 of its block maximum) is far below fp32's, so
// outlier channels cost nothing.  Q4_0 quants go in as their nibbles (0..15)
// with the -8 folded in as 8 x the block's digit sums.  Against the VALU path
// (a convert and an FMA per weight) this is ~0.5 VALU operations per weight.
// k_gemv_mma's LDS: x's digit planes, exponents, units and digit sums of nb
// blocks (152 bytes a block), then with DMA two regions per wave of a pair of
// wave-steps' rows (row_bytes x 8, in whole KiB).
__host__ __device__ constexpr size_t mma_dma_lds_offset(int nb) {
  return ((size_t)nb * 152u + 15u) & ~(size_t)15u;
}
__host__ __device__ constexpr size_t mma_dma_region(int block_bytes) {
  return ((size_t)8 * 32 * block_bytes + 1023u) & ~(size_t)1023u;
}
template <int FMT, int BPL, bool DMA = false>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_mma(GemvParams P) {
  extern __shared__ float xs[];  // the digit planes of x
  constexpr int BB = FMT == 1 ? 34 : FMT == 2 ? 18 : 20;
  constexpr int NB = 16 * BPL;
  constexpr int NW = BPL * BB / 4;  // dwords of a lane's span (BPL even)
  // wave-steps in flight: about 72 registers of weights
  constexpr int UN = 72 / NW >= kGemvUnroll ? kGemvUnroll : (72 / NW >= 1 ? 72 / NW : 1);
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6);
  const int r = lane & 3, g = lane >> 2;
  // LDS: digit planes [block][plane][chunk] (a dword = one plane of four
  // elements), per block 1 (or NaN) and its exponent e, and the blocks'
  // per-plane digit sums
  uint32_t *dig = reinterpret_cast<uint32_t *>(xs);
  float *units = reinterpret_cast<float *>(dig + NB * 32);
  int32_t *exps = reinterpret_cast<int32_t *>(units + NB);
  int32_t *dsum = exps + NB;
  // x into digit planes, while the first trip's weights load
  auto x_digits = [&]() {
    for (int it = threadIdx.x; it < NB * 8; it += kGemvThreads) {
      const int b = it >> 3, j = it & 7;  // chunk j: elements 4j .. 4j+3
      const float4 v = *reinterpret_cast<const float4 *>(P.x + 32 * b + 4 * j);
      float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
      mx = fmaxf(mx, __shfl_xor(mx, 1));
      mx = fmaxf(mx, __shfl_xor(mx, 2));
      mx = fmaxf(mx, __shfl_xor(mx, 4));
      int e = 0;
      (void)frexpf(mx, &e);
      const float xv[4] = {v.x, v.y, v.z, v.w};
      uint32_t pl[4] = {0u, 0u, 0u, 0u};
      int ps[4] = {0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        int m = (int)rintf(ldexpf(xv[k], 30 - e));  // |m| <= 2^30, exact scaling
        int d[4];
#pragma unroll
        for (int q = 0; q < 3; q++) {
          d[q] = ((m + 128) & 255) - 128;
          m = (m - d[q]) >> 8;
        }
        d[3] = m;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          pl[q] |= ((uint32_t)d[q] & 0xFFu) << (8 * k);
          ps[q] += d[q];
        }
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        dig[(b * 4 + q) * 8 + j] = pl[q];
        int t = ps[q];
        t += __shfl_xor(t, 1);
        t += __shfl_xor(t, 2);
        t += __shfl_xor(t, 4);
        ps[q] = t;
      }
      if (j == 0) {
        // the block's exponent, and 1 (NaN for a non-finite x: the rows'
        // sums then are NaN)
        exps[b] = e;
        units[b] = (mx <= 3.402823466e38f) ? 1.f : __int_as_float(0x7fc00000);
#pragma unroll
        for (int q = 0; q < 4; q++) dsum[b * 4 + q] = ps[q];
      }
    }
    __syncthreads();
  };
  const int stride = P.n_waves;
  // one wave-step of four rows: the lane's span wv of row rw (stored if real)
  auto step = [&](const uint32_t *wv, int rw, bool real) {
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < BPL; k++) {
      const int b = g * BPL + k;
      // the block's first byte in the span (quants from o + 2; Q4_1: d, m,
      // then the nibbles from o + 4)
      const int o = k * BB;
      typedef int v4i __attribute__((ext_vector_type(4)));
      v4i dd = {0, 0, 0, 0};
      // quant word j of the block: bytes o + 2 + 4j .. (o is even), Q4_1
      // o + 4 + 4j (o a multiple of 4)
      auto qword = [&](int jw) -> uint32_t {
        const int byte = o + (FMT == 3 ? 4 : 2) + 4 * jw;
        const int wi = byte >> 2;
        return (byte & 2) ? __builtin_amdgcn_perm(wv[wi + 1], wv[wi], 0x05040302u) : wv[wi];
      };
      // A: plane r of the block's eight chunks
      const uint4 a03 = *reinterpret_cast<const uint4 *>(dig + (b * 4 + r) * 8);
      const uint4 a47 = *reinterpret_cast<const uint4 *>(dig + (b * 4 + r) * 8 + 4);
      const uint32_t av[8] = {a03.x, a03.y, a03.z, a03.w, a47.x, a47.y, a47.z, a47.w};
      if constexpr (FMT == 1) {
#pragma unroll
        for (int jw = 0; jw < 8; jw++)
          dd = __builtin_amdgcn_mfma_i32_4x4x4i8((int)av[jw], (int)qword(jw), dd, 0, 0, 0);
      } else {
#pragma unroll
        for (int jw = 0; jw < 4; jw++) {
          const uint32_t w = qword(jw);
          dd = __builtin_amdgcn_mfma_i32_4x4x4i8((int)av[jw], (int)(w & 0x0F0F0F0Fu), dd, 0, 0,
                                                 0);
          dd = __builtin_amdgcn_mfma_i32_4x4x4i8((int)av[4 + jw], (int)((w >> 4) & 0x0F0F0F0Fu),
                                                 dd, 0, 0, 0);
        }
        if constexpr (FMT == 2) {
#pragma unroll
          for (int q = 0; q < 4; q++) dd[q] -= 8 * dsum[b * 4 + q];
        }
      }
      const uint32_t sw = wv[o >> 2];
      if constexpr (FMT == 3) {
        // Q4_1 (d q + m: gguf_dequant's deq_q4_1, l2_codec.c:65-75): d *
        // sum q_j m_j + m * sum m_j, both sums exact integers (below 2^39
        // and 2^35) and both products exact in float64, so the block
        // rounds once - taken apart in fp32 the two terms could cancel
        // (a weight d q + m near 0 against an outlier x) and leave their
        // roundings larger than the product
        const double sq = fma((double)(dd[3] * 256 + dd[2]), 65536.0, (double)(dd[1] * 256 + dd[0]));
        const int32_t *ds = dsum + b * 4;
        const double sm = fma((double)(ds[3] * 256 + ds[2]), 65536.0, (double)(ds[1] * 256 + ds[0]));
        const double v = fma((double)half_bits_to_f32_hw(sw & 0xFFFFu), sq,
                             (double)half_bits_to_f32_hw(sw >> 16) * sm);
        acc += (float)ldexp(v, exps[b] - 30) * units[b];
      } else {
        // |D3| <= 32*128*64, so D3*256 + D2 fits in int32
        const float t = (float)(dd[3] * 256 + dd[2]);
        const float sum = fmaf(fmaf(t, 256.f, (float)dd[1]), 256.f, (float)dd[0]);
        const float scl = half_bits_to_f32_hw((o & 2) ? (sw >> 16) : (sw & 0xFFFFu));
        // times the scale, then 2^(e-30) (ldexp: no overflow or early
        // underflow for blocks of very large or very small x)
        acc += ldexpf(sum * scl, exps[b] - 30) * units[b];
      }
    }
    // the row's 16 lanes (lanes r, r + 4, ..., r + 60)
    acc += __shfl_xor(acc, 4);
    acc += __shfl_xor(acc, 8);
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (real && g == 0) P.out[rw] = acc;
  };
  if constexpr (!DMA) {
  for (int s0 = gw, trip = 0;; s0 += stride * UN, trip++) {
    // this trip's spans: UN wave-steps of four rows, each lane its row's
    // BPL blocks (dword loads; a row's 16 lanes cover it, so its lines are
    // fetched once and shared through the cache)
    uint32_t wvs[UN][NW];
    int row[UN];
    bool ok[UN];
#pragma unroll
    for (int u = 0; u < UN; u++) {
      const int st = s0 + u * stride;
      row[u] = st * 4 + r;
      ok[u] = st < P.steps && row[u] < P.d;
      // (global-space 16-byte loads of the 4-byte aligned span, dwords for
      // the rest: as generic-pointer dwords the compiler issued them one by
      // one)
      const __attribute__((address_space(1))) uint32_t *src =
          (const __attribute__((address_space(1))) uint32_t *)(P.w +
                                                              (size_t)(ok[u] ? row[u] : 0) *
                                                                  P.row_bytes +
                                                              g * (BPL * BB));
#pragma unroll
      for (int i = 0; i + 4 <= NW; i += 4) {
        const gemv_u32x4_a4 v = *(const __attribute__((address_space(1))) gemv_u32x4_a4 *)(src + i);
        wvs[u][i] = ok[u] ? v.x : 0u;
        wvs[u][i + 1] = ok[u] ? v.y : 0u;
        wvs[u][i + 2] = ok[u] ? v.z : 0u;
        wvs[u][i + 3] = ok[u] ? v.w : 0u;
      }
#pragma unroll
      for (int i = NW & ~3; i < NW; i++) wvs[u][i] = ok[u] ? src[i] : 0u;
    }
    if (trip == 0) x_digits();
#pragma unroll
    for (int u = 0; u < UN; u++) step(wvs[u], row[u], ok[u]);
    if (s0 + stride * UN >= P.steps) break;
  }
  } else {
    // The weights through LDS: each wave streams pairs of adjacent
    // wave-steps (eight contiguous rows) with LDS DMA into two regions of its
    // own, 1 KiB per load and lane l taking bytes 16 l of each KiB, so every
    // load is one contiguous run (the direct loads above, each lane a span
    // of its row, touch every line of four rows per instruction).  The pair
    // in one region is consumed while the next one lands in the other.
    constexpr int RB = 32 * BB;                 // row bytes (1024-element rows)
    constexpr int PB = 8 * RB;                  // a pair's bytes
    constexpr int NI = (PB + 1023) / 1024;      // loads per pair
    const int wave = threadIdx.x >> 6;
    const uint32_t region0 =
        lds_addr(xs) + (uint32_t)mma_dma_lds_offset(NB) + (uint32_t)wave * 2u * (uint32_t)(NI * 1024);
    const int npairs = (P.steps + 1) / 2;
    const i32x4 rsrc = raw_rsrc(P.w, (uint32_t)((size_t)P.d * RB));
    auto issue = [&](int pr, int k) {
      const uint32_t dst = __builtin_amdgcn_readfirstlane(region0 + (uint32_t)k * (uint32_t)(NI * 1024));
      const uint32_t b0 = (uint32_t)pr * (uint32_t)PB;
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const uint32_t off = 1024u * (uint32_t)i + 16u * (uint32_t)lane;
        if (off < (uint32_t)PB) dma16(rsrc, dst + 1024u * (uint32_t)i, b0 + off);
      }
    };
    const uint8_t *lds_w = reinterpret_cast<const uint8_t *>(xs) + mma_dma_lds_offset(NB) +
                           (size_t)wave * 2 * (NI * 1024);
    int pr = gw;
    issue(pr, 0);
    x_digits();  // (every wave: it holds a workgroup barrier)
    for (int k = 0;; k ^= 1) {
      wait_vm0();  // this pair has landed (nothing else of the wave is in flight)
      __asm__ volatile("" ::: "memory");
      const int pn = pr + stride;
      const bool more = pn < npairs;
      if (more) issue(pn, k ^ 1);
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int st = 2 * pr + u;
        const int rw = st * 4 + r;
        const uint32_t *sp = reinterpret_cast<const uint32_t *>(
            lds_w + (size_t)k * (NI * 1024) + (size_t)(u * 4 + r) * RB + (size_t)g * (BPL * BB));
        uint32_t wv[NW];
#pragma unroll
        for (int i = 0; i < NW; i++) wv[i] = sp[i];
        step(wv, rw, st < P.steps && rw < P.d);
      }
      if (!more) break;
      pr = pn;
    }
  }
}

// Q8_0 / Q4_0 rows of more than 128 blocks: the workgroup's four waves
// split each row's blocks in quarters (a quarter of at most 128 blocks, so
// every lane keeps the x of its KB <= 2 blocks in registers) and add their
// partial sums in LDS.  Workgroups stride over steps of RPS rows.
template <int FMT, int LPR, int KB>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_q_split(GemvParams P) {
  extern __shared__ float xs[];  // the fused SiLU x up: n floats
  constexpr int RPS = 64 / LPR;
  constexpr int BB = block_bytes<FMT>();
  constexpr int NW = kGemvThreads / 64;
  __shared__ float part[kGemvUnroll][NW][RPS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rr = lane / LPR, c = lane % LPR;
  const int nb = P.nb, nbw = (nb + NW - 1) / NW;
  const int b_lo = wave * nbw, b_hi = min(nb, b_lo + nbw);
  const int stride = gridDim.x;
  float xr[KB][32];
  // Every workgroup runs the first trip: its weights are issued, then x is
  // prepared (barriers) while they are in flight.
  for (int s0 = blockIdx.x, trip = 0;; s0 += stride * kGemvUnroll, trip++) {
    BlockRaw<FMT> raw[kGemvUnroll][KB];
#pragma unroll
    for (int u = 0; u < kGemvUnroll; u++) {
      const int s = s0 + u * stride;
      const int row = s * RPS + rr;
      const bool ok = s < P.steps && row < P.d;
#pragma unroll
      for (int k = 0; k < KB; k++) {
        const int b = b_lo + c + LPR * k;
        if (ok && b < b_hi)
          load_block<FMT>(raw[u][k], seg_row(P, row) + (size_t)b * BB);
        else
          zero_block<FMT>(raw[u][k]);
      }
    }
    if (trip == 0) {
      float inv = 1.f;
      if (P.pro == kProSiluMul) wg_silu_mul(P, xs);
      if (P.pro == kProRmsnorm) inv = wg_rms_stage(P, xs);
      lane_x<LPR, KB>(P, xs, b_lo + c, b_hi, inv, xr);
    }
#pragma unroll
    for (int u = 0; u < kGemvUnroll; u++) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < KB; k++) acc += block_dot<FMT>(raw[u][k], xr[k]);
      acc = lanes_sum<LPR>(acc);
      if (c == 0) part[u][wave][rr] = acc;
    }
    __syncthreads();
    if (threadIdx.x < kGemvUnroll * RPS) {
      const int u = threadIdx.x / RPS, r = threadIdx.x % RPS;
      const int s = s0 + u * stride;
      const int row = s * RPS + r;
      if (s < P.steps && row < P.d)
        seg_store(P, row, (part[u][0][r] + part[u][1][r]) + (part[u][2][r] + part[u][3][r]));
    }
    __syncthreads();
    if (s0 + stride * kGemvUnroll >= P.steps) break;
  }
}

// F32 (l3_math.c:17-20): a wave per row, lanes over float4 pieces.  (Four
// rows per wave with their loads issued together, which took F16 from 71% to
// 84% of the HBM peak, ran F32 at 79% against 87%.)
__global__ __launch_bounds__(kGemvThreads) void k_gemv_f32(GemvParams P) {
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6);
  const int n = P.n, n4 = n / 4;
  for (int row = gw; row < P.d; row += P.n_waves) {
    const float *wr = reinterpret_cast<const float *>(P.w + (size_t)row * P.row_bytes);
    float a0 = 0.f, a1 = 0.f;
    if (P.vec4) {
      for (int j = lane; j < n4; j += 64) {
        const gemv_f32x4 w4 = nt_load<gemv_f32x4>(wr + 4 * j);
        const float4 x4 = *reinterpret_cast<const float4 *>(P.x + 4 * j);
        a0 = fmaf(w4.x, x4.x, a0);
        a1 = fmaf(w4.y, x4.y, a1);
        a0 = fmaf(w4.z, x4.z, a0);
        a1 = fmaf(w4.w, x4.w, a1);
      }
      for (int j = 4 * n4 + lane; j < n; j += 64) a0 = fmaf(wr[j], P.x[j], a0);
    } else {
      for (int j = lane; j < n; j += 64) a0 = fmaf(wr[j], P.x[j], a0);
    }
    const float acc = lanes_sum<64>(a0 + a1);
    if (lane == 0) P.out[row] = acc;
  }
}

// F16 (matmul_q's fallback: gguf_dequant's exact half_to_float, then the
// products, l2_codec.c:350-366): a wave per row, lanes over 16-byte pieces
// of eight halves (rows 16-byte aligned), else over single halves.  With
// 16-byte pieces a wave takes kF16Rows rows at a time, their loads issued
// together (one row at a time, each row waited out a memory round trip).
constexpr int kF16Rows = 4;
__global__ __launch_bounds__(kGemvThreads) void k_gemv_f16(GemvParams P) {
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6);
  const int n = P.n, n8 = n / 8;
  if (P.vec4) {
    for (int row0 = gw * kF16Rows; row0 < P.d; row0 += P.n_waves * kF16Rows) {
      float a0[kF16Rows], a1[kF16Rows];
      const uint16_t *wr[kF16Rows];
#pragma unroll
      for (int k = 0; k < kF16Rows; k++) {
        a0[k] = 0.f;
        a1[k] = 0.f;
        // (rows past d read row0's, and are not stored)
        const int row = row0 + k < P.d ? row0 + k : row0;
        wr[k] = reinterpret_cast<const uint16_t *>(P.w + (size_t)row * P.row_bytes);
      }
      for (int j = lane; j < n8; j += 64) {
        gemv_u32x4 w8[kF16Rows];
#pragma unroll
        for (int k = 0; k < kF16Rows; k++) w8[k] = nt_load<gemv_u32x4>(wr[k] + 8 * j);
        const float4 xa = *reinterpret_cast<const float4 *>(P.x + 8 * j);
        const float4 xb = *reinterpret_cast<const float4 *>(P.x + 8 * j + 4);
#pragma unroll
        for (int k = 0; k < kF16Rows; k++) {
          a0[k] = fmaf(half_bits_to_f32_hw(w8[k].x & 0xFFFFu), xa.x, a0[k]);
          a1[k] = fmaf(half_bits_to_f32_hw(w8[k].x >> 16), xa.y, a1[k]);
          a0[k] = fmaf(half_bits_to_f32_hw(w8[k].y & 0xFFFFu), xa.z, a0[k]);
          a1[k] = fmaf(half_bits_to_f32_hw(w8[k].y >> 16), xa.w, a1[k]);
          a0[k] = fmaf(half_bits_to_f32_hw(w8[k].z & 0xFFFFu), xb.x, a0[k]);
          a1[k] = fmaf(half_bits_to_f32_hw(w8[k].z >> 16), xb.y, a1[k]);
          a0[k] = fmaf(half_bits_to_f32_hw(w8[k].w & 0xFFFFu), xb.z, a0[k]);
          a1[k] = fmaf(half_bits_to_f32_hw(w8[k].w >> 16), xb.w, a1[k]);
        }
      }
#pragma unroll
      for (int k = 0; k < kF16Rows; k++) {
        for (int j = 8 * n8 + lane; j < n; j += 64)
          a0[k] = fmaf(half_bits_to_f32_hw(wr[k][j]), P.x[j], a0[k]);
        const float acc = lanes_sum<64>(a0[k] + a1[k]);
        if (lane == 0 && row0 + k < P.d) P.out[row0 + k] = acc;
      }
    }
    return;
  }
  for (int row = gw; row < P.d; row += P.n_waves) {
    const uint16_t *wr = reinterpret_cast<const uint16_t *>(P.w + (size_t)row * P.row_bytes);
    float a0 = 0.f;
    for (int j = lane; j < n; j += 64) a0 = fmaf(half_bits_to_f32_hw(wr[j]), P.x[j], a0);
    const float acc = lanes_sum<64>(a0);
    if (lane == 0) P.out[row] = acc;
  }
}

__global__ void k_fill_zero(float *out, int32_t n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = 0.f;
}

// LDS of the register-x forms: x * w or SiLU x up of the whole of x
inline size_t pro_lds(const GemvParams &p) {
  return p.pro != kProNone ? (size_t)p.n * sizeof(float) : 0;
}

// Resident workgroups per CU of a k_gemv_q instance (with or without the
// prologue's dynamic LDS), queried once.
template <int FMT, int LPR, int KB, bool XD = false>
int occ_q(size_t lds) {
  static int cached[2] = {0, 0};
  int &o = cached[lds ? 1 : 0];
  if (o == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_gemv_q<FMT, LPR, KB, XD>, kGemvThreads,
                                                     lds) != hipSuccess || n < 1) {
      (void)hipGetLastError();
      n = 1;
    }
    o = n;
  }
  return o;
}

// kb: 1, 2 x in registers, -1 x in LDS, 0 x through the cache; Q8_0 only:
// 11, 12 x as digit planes in registers (XD, one or two blocks per lane)
template <int FMT, int LPR>
int occ_q_lpr(int kb, size_t lds) {
  if constexpr (FMT == 1 && LPR >= 16) {
    if (kb == 11) return occ_q<FMT, LPR, 1, true>(lds);
    if (kb == 12) return occ_q<FMT, LPR, 2, true>(lds);
  }
  switch (kb) {
    case 1: return occ_q<FMT, LPR, 1>(lds);
    case 2: return occ_q<FMT, LPR, 2>(lds);
    case -1: return occ_q<FMT, LPR, -1>(lds);
    default: return occ_q<FMT, LPR, 0>(lds);
  }
}

template <int FMT>
int occ_q_fmt(int lpr, int kb, size_t lds) {
  switch (lpr) {
    case 1: return occ_q_lpr<FMT, 1>(kb, lds);
    case 2: return occ_q_lpr<FMT, 2>(kb, lds);
    case 4: return occ_q_lpr<FMT, 4>(kb, lds);
    case 8: return occ_q_lpr<FMT, 8>(kb, lds);
    case 16: return occ_q_lpr<FMT, 16>(kb, lds);
    case 32: return occ_q_lpr<FMT, 32>(kb, lds);
    default: return occ_q_lpr<FMT, 64>(kb, lds);
  }
}

template <int FMT, int LPR>
hipError_t launch_q_lpr(const GemvParams &p, int kb, dim3 grid, hipStream_t s) {
  const dim3 blk(kGemvThreads);
  if constexpr (FMT == 1 && LPR >= 16) {
    if (kb == 11 || kb == 12) {
      const size_t lds = pro_lds(p) + (size_t)p.nb * 34u * 4u;  // + digit planes, exps, units
      if (kb == 11)
        hipLaunchKernelGGL((k_gemv_q<FMT, LPR, 1, true>), grid, blk, lds, s, p);
      else
        hipLaunchKernelGGL((k_gemv_q<FMT, LPR, 2, true>), grid, blk, lds, s, p);
      return hipGetLastError();
    }
  }
  switch (kb) {
    case 1: hipLaunchKernelGGL((k_gemv_q<FMT, LPR, 1>), grid, blk, pro_lds(p), s, p); break;
    case 2: hipLaunchKernelGGL((k_gemv_q<FMT, LPR, 2>), grid, blk, pro_lds(p), s, p); break;
    case -1:
      hipLaunchKernelGGL((k_gemv_q<FMT, LPR, -1>), grid, blk, (size_t)p.nb * 128u, s, p);
      break;
    default: hipLaunchKernelGGL((k_gemv_q<FMT, LPR, 0>), grid, blk, 0, s, p); break;
  }
  return hipGetLastError();
}

template <int FMT, int LPR>
hipError_t launch_split_lpr(const GemvParams &p, int kb, dim3 grid, hipStream_t s) {
  if (kb == 1)
    hipLaunchKernelGGL((k_gemv_q_split<FMT, LPR, 1>), grid, dim3(kGemvThreads), pro_lds(p), s, p);
  else
    hipLaunchKernelGGL((k_gemv_q_split<FMT, LPR, 2>), grid, dim3(kGemvThreads), pro_lds(p), s, p);
  return hipGetLastError();
}

// k_gemv_mma<FMT, 2> (Q8_0 / Q4_0, 1024-element rows): resident workgroups
// per CU, queried once per form.
template <int FMT, bool DMA = false>
int occ_mma(size_t lds) {
  static int cached = 0;
  int &o = cached;
  if (o <= 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_gemv_mma<FMT, 2, DMA>, kGemvThreads, lds) !=
        hipSuccess) {
      (void)hipGetLastError();
      n = 1;
    }
    o = std::max(1, n);
  }
  return o;
}

template <int FMT>
hipError_t launch_split(const GemvParams &p, int lpr, int kb, dim3 grid, hipStream_t s) {
  // a quarter of more than 128 blocks is more than 32: LPR is 64
  (void)lpr;
  return launch_split_lpr<FMT, 64>(p, kb, grid, s);
}

template <int FMT>
hipError_t launch_q(const GemvParams &p, int lpr, int kb, dim3 grid, hipStream_t s) {
  switch (lpr) {
    case 1: return launch_q_lpr<FMT, 1>(p, kb, grid, s);
    case 2: return launch_q_lpr<FMT, 2>(p, kb, grid, s);
    case 4: return launch_q_lpr<FMT, 4>(p, kb, grid, s);
    case 8: return launch_q_lpr<FMT, 8>(p, kb, grid, s);
    case 16: return launch_q_lpr<FMT, 16>(p, kb, grid, s);
    case 32: return launch_q_lpr<FMT, 32>(p, kb, grid, s);
    default: return launch_q_lpr<FMT, 64>(p, kb, grid, s);
  }
}

}  // namespace

hipError_t launch_fill_zero(float *out, int32_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_zero, dim3((n + 255) / 256), dim3(256), 0, s, out, n);
  return hipGetLastError();
}

hipError_t launch_gemv(GemvParams p, int32_t type, int n_cu, hipStream_t s) {
  const int waves_per_wg = kGemvThreads / 64;
  if (p.d0 == 0 && p.d01 == 0) p.d0 = p.d01 = p.d;  // one segment
  const bool fused = p.pro != kProNone || p.res || p.d0 != p.d || p.d01 != p.d;
  // the fused forms exist where x lives in registers (gemv_fusable, x aligned)
  if (fused && (!gemv_fusable(type, p.n) || ((uintptr_t)p.x & 15u) || p.d0 > p.d01 ||
                p.d01 > p.d || (p.pro == kProRmsnorm && !p.nw) ||
                (p.pro != kProNone && p.n > kGemvProMaxN) ||
                (p.pro == kProSiluMul && (!p.x2 || ((uintptr_t)p.x2 & 15u)))))
    return hipErrorInvalidValue;
  if (fused) p.x_vec4 = 1;
  if (type == kTypeF32) {
    p.row_bytes = (uint32_t)p.n * 4u;
    p.vec4 = ((uintptr_t)p.w % 16 == 0 && (uintptr_t)p.x % 16 == 0 && p.n % 4 == 0) ? 1 : 0;
    const int wgs = std::max(1, std::min((p.d + waves_per_wg - 1) / waves_per_wg, n_cu * 8));
    p.n_waves = wgs * waves_per_wg;
    hipLaunchKernelGGL(k_gemv_f32, dim3(wgs), dim3(kGemvThreads), 0, s, p);
    return hipGetLastError();
  }
  if (type == kTypeF16) {
    p.row_bytes = (uint32_t)p.n * 2u;
    p.vec4 = ((uintptr_t)p.w % 16 == 0 && (uintptr_t)p.x % 16 == 0 && p.n % 8 == 0) ? 1 : 0;
    const int rows_per_wave = p.vec4 ? kF16Rows : 1;
    const int wgs = std::max(
        1, std::min((p.d + rows_per_wave * waves_per_wg - 1) / (rows_per_wave * waves_per_wg),
                    n_cu * 8));
    p.n_waves = wgs * waves_per_wg;
    hipLaunchKernelGGL(k_gemv_f16, dim3(wgs), dim3(kGemvThreads), 0, s, p);
    return hipGetLastError();
  }
  const int fmt = type == kTypeQ8_0 ? 1 : type == kTypeQ4_0 ? 2 : 3;
  p.nb = p.n / 32;
  p.row_bytes = (uint32_t)p.nb * (fmt == 1 ? 34u : fmt == 2 ? 18u : 20u);
  if (p.nb > 128 && p.nb <= 4 * 128 && p.x_vec4) {
    // rows split over the workgroup's four waves (x in registers)
    const int nbw = (p.nb + 3) / 4;  // > 32, so 64 lanes per row
    const int kb = (nbw + 63) / 64;
    p.steps = p.d;
    const int wgs = std::min(std::max((p.steps + kGemvMinSteps - 1) / kGemvMinSteps,
                                      std::min(p.steps, n_cu)),
                             n_cu * 4);
    p.n_waves = wgs * waves_per_wg;
    return fmt == 1   ? launch_split<1>(p, 64, kb, dim3(wgs), s)
           : fmt == 2 ? launch_split<2>(p, 64, kb, dim3(wgs), s)
                      : launch_split<3>(p, 64, kb, dim3(wgs), s);
  }
  // The int8 matrix cores (k_gemv_mma) where they pay: plain (unfused) Q8_0
  // and Q4_0 products of 1024-element rows, at least kGemvMmaMinRows of them
  // (gemv_mma_plain; the lm head: Q8_0 26.0 against 30.6 us for x's digit
  // planes on the VALU, Q4_0 16.7 against 26.2 us for the VALU form), x
  // 16-byte and the weights 4-byte aligned.  Each lane loads its row span
  // with 16-byte loads (as single dwords: 34.4 and 19.0 us).  The rmsnorm
  // prologue inside it measured 34.8 us (every workgroup normalising and
  // digitising x before its loads): the model runs its logits as rmsnorm
  // and this plain product instead.  Measured slower elsewhere: Q4_0 4096 x
  // 14336 29.6 against 13.8 us, 4096-row matrices 4.7-5.0 against 4.4 us
  // (the digit prologue of every workgroup).
  if (!fused && p.x_vec4 && gemv_mma_plain(type, p.n, p.d) && ((uintptr_t)p.w & 15u) == 0 &&
      (size_t)p.d * p.row_bytes < ((size_t)1 << 31)) {
    // the LDS-DMA form: pairs of wave-steps per wave
    p.steps = (p.d + 3) / 4;
    const int bb = fmt == 1 ? 34 : fmt == 2 ? 18 : 20;
    const size_t lds = mma_dma_lds_offset(p.nb) + (size_t)waves_per_wg * 2 * mma_dma_region(bb);
    const int occ = fmt == 1   ? occ_mma<1, true>(lds)
                    : fmt == 2 ? occ_mma<2, true>(lds)
                               : occ_mma<3, true>(lds);
    const int npairs = (p.steps + 1) / 2;
    const int waves = std::min(npairs, n_cu * std::max(1, occ) * waves_per_wg);
    const int wgs = std::max(1, (waves + waves_per_wg - 1) / waves_per_wg);
    p.n_waves = wgs * waves_per_wg;
    if (fmt == 1)
      hipLaunchKernelGGL((k_gemv_mma<1, 2, true>), dim3(wgs), dim3(kGemvThreads), lds, s, p);
    else if (fmt == 2)
      hipLaunchKernelGGL((k_gemv_mma<2, 2, true>), dim3(wgs), dim3(kGemvThreads), lds, s, p);
    else
      hipLaunchKernelGGL((k_gemv_mma<3, 2, true>), dim3(wgs), dim3(kGemvThreads), lds, s, p);
    return hipGetLastError();
  }
  if (!fused && p.x_vec4 && gemv_mma_plain(type, p.n, p.d) && ((uintptr_t)p.w & 3u) == 0) {
    p.steps = (p.d + 3) / 4;
    const size_t lds = (size_t)p.nb * (32u * 4u + 4u + 4u + 16u);
    const int occ = fmt == 1 ? occ_mma<1>(lds) : fmt == 2 ? occ_mma<2>(lds) : occ_mma<3>(lds);
    const int waves = std::min(std::max((p.steps + kGemvMinSteps - 1) / kGemvMinSteps,
                                        std::min(p.steps, n_cu * 4)),
                               n_cu * std::max(1, occ) * waves_per_wg);
    const int wgs = std::max(1, (waves + waves_per_wg - 1) / waves_per_wg);
    p.n_waves = wgs * waves_per_wg;
    if (fmt == 1)
      hipLaunchKernelGGL((k_gemv_mma<1, 2>), dim3(wgs), dim3(kGemvThreads), lds, s, p);
    else if (fmt == 2)
      hipLaunchKernelGGL((k_gemv_mma<2, 2>), dim3(wgs), dim3(kGemvThreads), lds, s, p);
    else
      hipLaunchKernelGGL((k_gemv_mma<3, 2>), dim3(wgs), dim3(kGemvThreads), lds, s, p);
    return hipGetLastError();
  }
  int lpr = 1;
  while (lpr < p.nb && lpr < 64) lpr *= 2;
  const int kb = (p.nb + lpr - 1) / lpr;
  const int rps = 64 / lpr;
  p.steps = (p.d + rps - 1) / rps;
  int kbv = !p.x_vec4                     ? 0
            : kb <= 2                     ? kb
            : p.nb * 128 <= kGemvMaxXLds ? -1
                                          : 0;
  // Q8_0 with x in registers over many rows: x as digit planes (the
  // workgroup's digit prologue pays where every wave has many rows; LPR >=
  // 16 keeps the instances few)
  if (fmt == 1 && kbv > 0 && lpr >= 16 && p.d >= kGemvXdMinRows) kbv += 10;
  // every wave loads the x of its blocks once: at least kGemvMinSteps steps
  // per wave where there are enough, at least 4 waves per CU, at most one
  // resident round of workgroups (a partial second round would leave most
  // of the chip idle at the end)
  const size_t lds = kbv < 0    ? (size_t)p.nb * 128u
                     : kbv > 10 ? pro_lds(p) + (size_t)p.nb * 34u * 4u
                                : pro_lds(p);
  const int occ = fmt == 1   ? occ_q_fmt<1>(lpr, kbv, lds)
                  : fmt == 2 ? occ_q_fmt<2>(lpr, kbv, lds)
                             : occ_q_fmt<3>(lpr, kbv, lds);
  const int waves = std::min(std::max((p.steps + kGemvMinSteps - 1) / kGemvMinSteps,
                                      std::min(p.steps, n_cu * 4)),
                             n_cu * std::max(1, occ) * waves_per_wg);
  const int wgs = std::max(1, (waves + waves_per_wg - 1) / waves_per_wg);
  p.n_waves = wgs * waves_per_wg;
  return fmt == 1   ? launch_q<1>(p, lpr, kbv, dim3(wgs), s)
         : fmt == 2 ? launch_q<2>(p, lpr, kbv, dim3(wgs), s)
                    : launch_q<3>(p, lpr, kbv, dim3(wgs), s);
}

}  // namespace g2b
