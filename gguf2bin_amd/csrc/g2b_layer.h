// g2b_layer.h - k_layer, the specialised decode kernel, and its launchers.
// Included only by g2b_layer_inst.hip, which the build compiles once per
// (KV format, head_dim, GQA group) so that the variants build in parallel;
// g2b_decode.hip dispatches to those instantiations.
//
// Replaces the score / softmax / V-accumulate loops of
// /root/reference/src/l5_model.c:518-557 (AVX2) and :558-577 (scalar):
//   att[h][t] = dot(q_h, k_t[h/group]) / sqrt(hd), softmax over t <= pos,
//   out_h = sum_t att[h][t] * v_t[h/group].
// The reference dequantises a whole row per position into a scratch buffer
// (kv_key_row / kv_val_row, l5_model.c:248-265) and walks every q head.  Here
// the row is never materialised: each lane owns one chunk of the row (one
// 32-element Q8_0 block, half a block, or 16 F32 values), keeps the q values
// of the GQA group for that chunk in registers, dequantises in registers,
// and keeps its own online-softmax state.  A position's partial dot products
// are summed over the lanes of a head with DPP.  Nothing goes through LDS in
// the main loop and there is no barrier: each wave streams rows
// independently with wide loads.  Scores are kept in the log2 domain
// (q pre-scaled by log2(e)/sqrt(hd)) so that softmax uses v_exp_f32.
//
// Splits: workgroup (split, seq, layer) covers positions
// [split*split_len, min(pos+1, (split+1)*split_len)); its four waves take
// interleaved groups of PPW positions and each writes one partial
// (m, l, acc[hd]) per q head.  k_combine merges the partials of a
// (seq, layer, head), writes the output over q (as l5_model.c:541-557 does)
// and, when asked, turns the stored scores into the reference's
// att[h*ctx+t] weights.
#pragma once
#include <algorithm>
#include <type_traits>

#include "g2b_internal.h"

namespace g2b {

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of N consecutive lanes; every lane of a group ends
// with the same value (each step adds two equal-order operands).
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
  if constexpr (N >= 2) x += dpp_f<0xB1>(x);   // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (N >= 4) x += dpp_f<0x4E>(x);   // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (N >= 8) x += dpp_f<0x141>(x);  // row_half_mirror: other quad of 8
  if constexpr (N >= 16) x += dpp_f<0x140>(x); // row_mirror: other half of 16
  return x;
}

// x of lane ^ S (S = 32 or 16) through gfx950's lane swaps, on the VALU (no
// LDS traffic).  With both operands x, v_permlane32_swap leaves lanes 0-31 of
// its second result holding lanes 32-63 of x and lanes 32-63 of its first
// result holding lanes 0-31; v_permlane16_swap does the same for each pair of
// 16-lane rows.
template <int S>
__device__ __forceinline__ float lanes_xor(float x) {
  static_assert(S == 32 || S == 16, "swap distance");
  const uint32_t u = __float_as_uint(x);
  if constexpr (S == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
  }
}

__device__ __forceinline__ float i8f(uint32_t w, int byte) {
  return (float)(int8_t)(uint8_t)(w >> (8 * byte));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Loads through the global address space (the cache pointers arrive through a
// descriptor table, so the compiler would otherwise emit flat loads).
template <typename T>
__device__ __forceinline__ T gload(const uint8_t *p) {
  return *(const __attribute__((address_space(1))) T *)(p);
}

// Cache-policy operand of global_load_lds for a non-temporal (streaming)
// load: the nt bit.  Two contiguous streams per workgroup read ~12% faster
// non-temporal than with the default policy on MI355X (7.0 vs 6.2 TB/s), but
// only when each line is requested once, which the staged path guarantees.
constexpr int kAuxNT = 2;
// s_waitcnt operand (gfx9 encoding): vmcnt = 0, expcnt and lgkmcnt not waited.
constexpr int kWaitVmcnt0 = 0x0F70;
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Word 3 of a raw (stride 0) buffer resource on gfx9-family devices: data
// format 32 bits, the rest zero (untyped loads move the bytes as they are;
// the range check is offset < the resource's byte count).
constexpr int32_t kBufferRsrcWord3 = 0x00020000;

// Streamed chunks go straight into LDS through inline assembly, so that the
// compiler's wait-count bookkeeping does not see them: it waits for every
// LDS DMA before any LDS read (which would serialise each chunk's loads with
// the consumption of the one before).  The kernels wait for them themselves,
// with s_waitcnt vmcnt(0) (wait_vm0) before each chunk is read.  Loads the
// compiler cannot see only make its own waits stricter than they need be
// (vmcnt counts in issue order), never too weak.
//
// 16 bytes per lane from buffer resource rsrc at byte voff into LDS at
// lds_addr + 16 * lane, non-temporal (M0 holds the LDS address).  M0 is on
// the clobber list: the statement becomes a definition of M0, so the compiler
// re-initialises M0 before any later instruction of its own that reads it
// (clang warns about clobbering a reserved register; that is the intent).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds_addr, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}
#pragma clang diagnostic pop
// A work-queue claim: lane 0 adds 1 to *ctr (a relaxed agent-scope
// fetch_add, global_atomic_add ... sc0) and holds the old value in its lane
// of the result; the other lanes hold 0.  The atomic is visible to the
// compiler, which therefore waits for its result before any read or copy of
// that register.  The kernels read it (readlane 0) only after a wait_vm0(),
// so no such wait of the compiler's falls inside a chunk's consumption.
__device__ __forceinline__ int32_t claim_lane0(int32_t *ctr, int lane) {
  int32_t r = 0;
  if (lane == 0) r = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return r;
}
// The raw buffer resource of `bytes` bytes at p (p the same in every lane).
__device__ __forceinline__ i32x4 raw_rsrc(const uint8_t *p, uint32_t bytes) {
  const uint64_t u = (uint64_t)(uintptr_t)p;
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)u);
  r.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32)) & 0xFFFF;
  r.z = __builtin_amdgcn_readfirstlane((int)bytes);
  r.w = kBufferRsrcWord3;
  return r;
}
// The LDS address of p (a pointer into __shared__ memory).
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// Every vector memory operation of this wave has completed (the builtin, so
// the compiler knows it and adds no wait of its own for claims read after it).
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(kWaitVmcnt0); }

// Online softmax: how far (log2 units) a score may exceed the reference
// before the accumulators are rescaled.
constexpr float kRescaleSlack = 8.f;

// Per-lane addressing of its chunk inside a row.
struct LaneOff {
  uint32_t o0, o1, o2;  // byte offsets inside the row
  uint32_t sel;         // v_perm_b32 selector that realigns quant dwords
  uint32_t sshift;      // 0 or 16: where the fp16 scale sits in its dword
};

template <int FMT, int CD>
struct Codec;

// F32 rows staged in LDS lie transposed within each row: the 16-byte quarter
// q of lane r (row bytes 64r + 16q) at piece q * lpp + r, lpp = lanes per
// position = row bytes / 64.  A position's lanes then read consecutive pieces
// (reading their own 64-byte runs, every fourth lane would hit the same LDS
// banks).  Piece indices count from the start of a chunk of whole rows.
__device__ __forceinline__ uint32_t f32_lds_piece(uint32_t g, uint32_t lpp) {
  const uint32_t P = 4u * lpp, rw = g / P, rem = g - rw * P;
  return rw * P + (rem & 3u) * lpp + (rem >> 2);  // global piece g -> LDS piece
}
__device__ __forceinline__ uint32_t f32_global_piece(uint32_t p, uint32_t lpp) {
  const uint32_t P = 4u * lpp, rw = p / P, rem = p - rw * P, q = rem / lpp;
  return rw * P + 4u * (rem - q * lpp) + q;  // LDS piece p -> global piece
}

// ---- F32 rows: 16 contiguous floats, four 16-byte loads ----
template <>
struct Codec<0, 16> {
  struct Raw {
    f32x4 x[4];
  };
  // o0: the lane's bytes in a row; in a staged (transposed) row its first
  // quarter at o2 = 16r, the next ones o1 = 16 * lpp apart.
  static __device__ __forceinline__ LaneOff offsets(int elem0, int lpp) {
    LaneOff o;
    o.o0 = (uint32_t)elem0 * 4u;
    o.o1 = 16u * (uint32_t)lpp;
    o.o2 = (uint32_t)elem0;
    o.sel = o.sshift = 0;
    return o;
  }
  // Default cache policy: each of the four loads touches every cache line of
  // the lanes' 64-byte runs, and the later ones hit the lines the first one
  // brought into the vector cache (non-temporal loads would fetch them again).
  static __device__ __forceinline__ void load(Raw &r, const uint8_t *row, const LaneOff &o) {
#pragma unroll
    for (int i = 0; i < 4; i++) r.x[i] = gload<f32x4>(row + o.o0 + 16 * i);
  }
  // a staged row (transposed)
  static __device__ __forceinline__ void load_lds(Raw &r, const uint8_t *row, const LaneOff &o) {
#pragma unroll
    for (int i = 0; i < 4; i++)
      r.x[i] = *reinterpret_cast<const f32x4 *>(row + o.o2 + (uint32_t)i * o.o1);
  }
  // a row as the cache holds it, in LDS (the new row)
  static __device__ __forceinline__ void load_row(Raw &r, const uint8_t *row, const LaneOff &o) {
    const float *p = reinterpret_cast<const float *>(row + o.o0);
#pragma unroll
    for (int i = 0; i < 4; i++) r.x[i] = f32x4{p[4 * i], p[4 * i + 1], p[4 * i + 2], p[4 * i + 3]};
  }
  static __device__ __forceinline__ void values(const Raw &r, float (&f)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      f[4 * i + 0] = r.x[i].x;
      f[4 * i + 1] = r.x[i].y;
      f[4 * i + 2] = r.x[i].z;
      f[4 * i + 3] = r.x[i].w;
    }
  }
};

// ---- Q8_0, one full 34-byte block per lane ----
// Block b starts at byte 34b: for even b the dword window starts at the
// block (scale = low half of dword 0, quants at window bytes 2..33); for odd
// b it starts two bytes earlier (scale = high half, quants at bytes 4..35).
// Nine dwords cover the block either way and, because the last block of a
// row is odd whenever head_dim is a multiple of 64, never leave the row.
template <>
struct Codec<1, 32> {
  struct Raw {
    u32x4 a, b;
    uint32_t c;
  };
  static __device__ __forceinline__ LaneOff offsets(int elem0, int) {
    const uint32_t b = (uint32_t)elem0 >> 5, odd = b & 1u;
    LaneOff o;
    o.o0 = (34u * b) & ~3u;
    o.o1 = o.o2 = 0;
    o.sel = odd ? 0x07060504u : 0x05040302u;
    o.sshift = odd ? 16u : 0u;
    return o;
  }
  static __device__ __forceinline__ void load(Raw &r, const uint8_t *row, const LaneOff &o) {
    const uint8_t *p = row + o.o0;
    r.a = gload<u32x4>(p);
    r.b = gload<u32x4>(p + 16);
    r.c = gload<uint32_t>(p + 32);
  }
  static __device__ __forceinline__ void load_lds(Raw &r, const uint8_t *row, const LaneOff &o) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row + o.o0);
    r.a = u32x4{p[0], p[1], p[2], p[3]};
    r.b = u32x4{p[4], p[5], p[6], p[7]};
    r.c = p[8];
  }
  static __device__ __forceinline__ void load_row(Raw &r, const uint8_t *row, const LaneOff &o) {
    load_lds(r, row, o);
  }
  // the 32 int8 quants as 8 aligned dwords, and the block scale
  static __device__ __forceinline__ void quants(const Raw &r, uint32_t (&w)[8], float &scale,
                                                const LaneOff &o) {
    const uint32_t d[9] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c};
    scale = half_bits_to_f32_hw(d[0] >> o.sshift);
#pragma unroll
    for (int j = 0; j < 8; j++) w[j] = __builtin_amdgcn_perm(d[j + 1], d[j], o.sel);
  }
};

// ---- Q8_0, half a block (16 quants) per lane ----
// Scale dword at (34b)&~3; quant window at (34b+2+16h)&~3 (two bytes early
// for even b).  For odd b the window is aligned and only four dwords are
// used; the fifth load is pointed inside the block so it never leaves it.
template <>
struct Codec<1, 16> {
  struct Raw {
    uint32_t s;
    u32x4 a;
    uint32_t c;
  };
  static __device__ __forceinline__ LaneOff offsets(int elem0, int) {
    const uint32_t b = (uint32_t)elem0 >> 5, odd = b & 1u, h = ((uint32_t)elem0 >> 4) & 1u;
    const uint32_t qstart = 34u * b + 2u + 16u * h;
    LaneOff o;
    o.o0 = (34u * b) & ~3u;
    o.o1 = qstart & ~3u;
    o.o2 = odd ? o.o1 + 12u : o.o1 + 16u;
    o.sel = odd ? 0x03020100u : 0x05040302u;
    o.sshift = odd ? 16u : 0u;
    return o;
  }
  static __device__ __forceinline__ void load(Raw &r, const uint8_t *row, const LaneOff &o) {
    r.s = gload<uint32_t>(row + o.o0);
    r.a = gload<u32x4>(row + o.o1);
    r.c = gload<uint32_t>(row + o.o2);
  }
  static __device__ __forceinline__ void load_lds(Raw &r, const uint8_t *row, const LaneOff &o) {
    r.s = *reinterpret_cast<const uint32_t *>(row + o.o0);
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row + o.o1);
    r.a = u32x4{p[0], p[1], p[2], p[3]};
    r.c = *reinterpret_cast<const uint32_t *>(row + o.o2);
  }
  static __device__ __forceinline__ void load_row(Raw &r, const uint8_t *row, const LaneOff &o) {
    load_lds(r, row, o);
  }
  static __device__ __forceinline__ void quants(const Raw &r, uint32_t (&w)[4], float &scale,
                                                const LaneOff &o) {
    const uint32_t d[5] = {r.a.x, r.a.y, r.a.z, r.a.w, r.c};
    scale = half_bits_to_f32_hw(r.s >> o.sshift);
#pragma unroll
    for (int j = 0; j < 4; j++) w[j] = __builtin_amdgcn_perm(d[j + 1], d[j], o.sel);
  }
};

// q for the integer K dot products: each q value of a (head, chunk) becomes
// m = rint(q * 2^(kQBits-e)) with 2^e > max|q| (so |m| <= 2^30: 31 bits of
// the chunk maximum), split into kQPlanes signed base-256 digits packed four
// per dword.  sum_j m_j k_j is then kQPlanes chains of v_dot4_i32_i8 (exact
// in int32) and one fp32 combination; the quantisation of q costs at most
// 2^-31 * max|q| per element, well below what an fp32 FMA chain over the
// same int8 values loses, also where one element of a chunk is 10^3 times
// the others (three planes, 23 bits, were not: such a chunk left its other
// elements ~2^-13 relative precision).
constexpr int kQPlanes = 4;
constexpr int kQBits = 8 * kQPlanes - 2;  // 30
template <int CD>
struct QDigits {
  uint32_t d[kQPlanes][CD / 4];
  float unit;  // 2^(e-30): value of one m step
};

// The digits of m (|m| <= 2^30): planes 0..2 in [-128, 127], plane 3 the
// rest (|d3| <= 64).
__device__ __forceinline__ void split_digits(int m, int (&d)[kQPlanes]) {
#pragma unroll
  for (int p = 0; p < kQPlanes - 1; p++) {
    d[p] = ((m + 128) & 255) - 128;
    m = (m - d[p]) >> 8;
  }
  d[kQPlanes - 1] = m;
}

template <int CD>
__device__ __forceinline__ QDigits<CD> make_digits(const float (&q)[CD]) {
  QDigits<CD> r;
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < CD; j++) mx = fmaxf(mx, fabsf(q[j]));
  int e = 0;
  (void)frexpf(mx, &e);
  const float up = ldexpf(1.f, kQBits - e);
  r.unit = ldexpf(1.f, e - kQBits);
#pragma unroll
  for (int k = 0; k < kQPlanes; k++)
#pragma unroll
    for (int j = 0; j < CD / 4; j++) r.d[k][j] = 0u;
#pragma unroll
  for (int j = 0; j < CD; j++) {
    int d[kQPlanes];
    split_digits((int)rintf(q[j] * up), d);
    const int sh = 8 * (j & 3);
#pragma unroll
    for (int k = 0; k < kQPlanes; k++) r.d[k][j >> 2] |= ((uint32_t)d[k] & 0xffu) << sh;
  }
  return r;
}

// A chunk's value from its plane sums c[p] = sum_j d_pj k_j (at most 32
// elements: |c[0..2]| <= 32*128*127, |c[3]| <= 32*64*127), in units of m:
// c3*2^24 + c2*2^16 + c1*2^8 + c0 = (c3*256 + c2) * 65536 + (c1*256 + c0),
// both parts exact in int32.
//
// k_layer takes it times the chunk's scale su (fp16 block scale x 2^(e-30),
// exact) in one fp32 rounding: fma(hi, su * 65536, lo * su), where (float)hi
// is exact below 2^24 (it rounds only for chunks near the int8 limits in
// every element) and lo * su is 2^-16 of the value's scale.  A head's score
// then adds its chunks in fp32 - a few roundings of the score's size, as
// many as the reference's fp32 dot (l5_model.c:520-536) has.
__device__ __forceinline__ float chunk_value(int c0, int c1, int c2, int c3, float su) {
  const int hi = c3 * 256 + c2, lo = c1 * 256 + c0;
  return fmaf((float)hi, su * 65536.f, (float)lo * su);
}
// k_tiles takes the value exactly in float64 (below 2^43) and sums a head's
// blocks in float64 before one fp32 rounding: free there, where the VALU
// does little else per block.
__device__ __forceinline__ double chunk_value_exact(int c0, int c1, int c2, int c3) {
  const int hi = c3 * 256 + c2, lo = c1 * 256 + c0;
  return fma((double)hi, 65536.0, (double)lo);
}

// The first product of a dot chain, a.b with a zero accumulator: the
// VOP3P form takes the 0 as an inline constant, where the compiler's
// v_dot4c (accumulate into the destination) first needs a v_mov of 0 - one
// VALU instruction per chain, 4% of k_layer's loop.
__device__ __forceinline__ int sdot4_first(uint32_t a, uint32_t b) {
  int r;
  asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// sum_j q_j * k_j for the chunk: the integer dot product of the digit planes
// with the chunk's quants w, times su (chunk_value).
template <int NW>
__device__ __forceinline__ float qk_int(const uint32_t (&w)[NW],
                                        const uint32_t (&d)[kQPlanes][NW], float su) {
  int s[kQPlanes];
#pragma unroll
  for (int p = 0; p < kQPlanes; p++) s[p] = sdot4_first(w[0], d[p][0]);
#pragma unroll
  for (int j = 1; j < NW; j++)
#pragma unroll
    for (int p = 0; p < kQPlanes; p++)
      s[p] = __builtin_amdgcn_sdot4((int)w[j], (int)d[p][j], s[p], false);
  static_assert(kQPlanes == 4, "chunk_value takes four planes");
  return chunk_value(s[0], s[1], s[2], s[3], su);
}

__device__ __forceinline__ float fast_exp2(float x) {
  // v_exp_f32; results below 2^-126 (weights under 1e-38 of the maximum)
  // may flush to zero, which no output can see.
  return __builtin_amdgcn_exp2f(x);
}

// Work-queue visits: the new row of the workgroup that owns position pos:
// [QK-RMSNorm,] RoPE(k), then F32 copy
// or Q8_0 quantisation of k and v into LDS (rowk, rowv), then a copy of both
// rows to the caches.  The workgroup later reads pos from LDS, so no other
// workgroup and no cache level is involved.  Every thread calls it.
__device__ inline void append_new_row(const ShapeDev &sh, const SeqDev &sd, int layer, int pos,
                                      const float *k, const float *v, const float *rope,
                                      const NormDev &norm, float *kr, float *vr, uint8_t *rowk,
                                      uint8_t *rowv, float *inv) {
  const int hd = sh.head_dim, half = hd / 2;
  const int nkv = sh.n_kv_heads * hd;
  const float *cs = (sh.rope_on && rope) ? rope + (size_t)pos * hd : nullptr;
  for (int e = threadIdx.x; e < nkv; e += blockDim.x) {
    kr[e] = k[e];
    vr[e] = v[e];
  }
  __syncthreads();
  if (const float *wk = norm_weights(norm, layer, 1, hd))
    qk_rmsnorm_block(kr, sh.n_kv_heads, hd, wk, norm.eps, inv);
  if (cs) {
    for (int p = threadIdx.x; p < sh.n_kv_heads * half; p += blockDim.x) {
      const int h = p / half, j = p - h * half;
      int ia, ib;
      rope_pair_index(sh.arch_llama, j, half, ia, ib);
      rope_pair(kr[h * hd + ia], kr[h * hd + ib], cs[2 * j], cs[2 * j + 1]);
    }
  }
  __syncthreads();
  if (sh.kv_q8) {
    // four lanes per block (a multiple of 4 items, so a block's four lanes
    // are active together)
    const int nb = (nkv + 31) / 32;
    for (int it = threadIdx.x; it < 8 * nb; it += blockDim.x) {
      const int b = it >> 2, part = it & 3;
      const bool is_k = b < nb;
      const int bb = is_k ? b : b - nb;
      const int cnt = min(32, nkv - 32 * bb);
      q8_quant_block_x4((is_k ? kr : vr) + 32 * bb, cnt, (is_k ? rowk : rowv) + 34 * bb, part);
    }
  } else {
    float *fk = reinterpret_cast<float *>(rowk), *fv = reinterpret_cast<float *>(rowv);
    for (int e = threadIdx.x; e < nkv; e += blockDim.x) {
      fk[e] = kr[e];
      fv[e] = vr[e];
    }
  }
  __syncthreads();
  const size_t off = ((size_t)layer * (size_t)sd.ctx_cap + (size_t)pos) * sh.row_bytes;
  uint32_t *gk = reinterpret_cast<uint32_t *>(sd.k + off);
  uint32_t *gv = reinterpret_cast<uint32_t *>(sd.v + off);
  const uint32_t *lk = reinterpret_cast<const uint32_t *>(rowk);
  const uint32_t *lv = reinterpret_cast<const uint32_t *>(rowv);
  for (uint32_t i = threadIdx.x; i < sh.row_bytes / 4; i += blockDim.x) {
    gk[i] = lk[i];
    gv[i] = lv[i];
  }
}

// The setup of a static-schedule visit (every thread calls it; owns_new is
// uniform), shaped for latency: the visit is one workgroup's whole job.
// Threads own rope groups - four pairs (j, j + hd/2) for NEOX, (2j, 2j + 1)
// for LLaMA, j = 4i..4i+3, of one q head or (owner) new k head - and bring
// their two float4s of x, of the norm weights and of the cos/sin row of pos
// (l3_math.c:65-102) into registers in one round of global loads, with the
// owner's v.  QK-RMSNorm (l3_math.c:107-114) needs each head's sum of
// squares first: one thread per head, left to right with every product
// rounded, inv = 1/sqrtf(ss/hd + eps) with IEEE division and square root,
// over a transposed LDS copy.  Then (w * x) * inv and the rotation in
// registers, into qrot (rotated q) and kr (rotated new k).  With DIG (Q8_0
// KV), the q digit planes of every (head, CD-element chunk) - make_digits of
// qrot * qscale - are computed once here, four threads per chunk, into dig.
// Then, for the owner, F32 copy or Q8_0 quantisation of k and v into LDS
// (rowk, rowv) and a copy of both rows to the caches (kv_store,
// l5_model.c:235-247).  The owner later reads pos from LDS, so no other
// workgroup and no cache level is involved.
// scr: norm factors (n_heads + n_kv_heads floats).  tr: hd x (n_heads +
// n_kv_heads + 1) floats holding q and k transposed in float4 groups -
// elements 4i..4i+3 of head H at float4 [i][H] - so each head's sum reads
// 16-byte pieces without bank conflicts; dig (DIG) reuses tr once the sums
// are done, or is digp where the caller gives it (outside qrot, kr and vr):
// dig_dwords<CD>(n_heads * hd / CD) dwords, chunk h * (hd / CD) + c.  In tr
// they fit for every shape the specialised kernels take: n_heads * (hd/CD)
// * (4 * CD/4 + 1) <= hd * (n_heads + n_kv_heads + 1) for CD 16 or 32 and
// n_heads <= 4 * n_kv_heads.
// The digit planes of a chunk: dig_stride<CD>() dwords (kQPlanes planes of
// CD/4 dwords, 16-byte rows); the chunks' units 2^(e-30) follow all the
// chunks' planes, one float each (dig_unit).
template <int CD>
__host__ __device__ constexpr int dig_stride() {
  return kQPlanes * (CD / 4);
}
// Where chunk ch's unit lies, and the dwords of n_chunks chunks' digits.
template <int CD>
__host__ __device__ constexpr int dig_unit_at(int n_chunks, int ch) {
  return n_chunks * dig_stride<CD>() + ch;
}
template <int CD>
__host__ __device__ constexpr int dig_dwords(int n_chunks) {
  return n_chunks * (dig_stride<CD>() + 1);
}

template <int HD, int CD, bool DIG>
__device__ inline void visit_setup(const ShapeDev &sh, const SeqDev &sd, int layer, bool owns_new,
                                   const float *qi, const float *ki, const float *vi,
                                   const float *rope, const NormDev &norm, float qscale,
                                   float *qrot, float *kr, float *vr, uint8_t *rowk,
                                   uint8_t *rowv, float *scr, float *tr,
                                   uint32_t *digp = nullptr) {
  constexpr int half = HD / 2;
  constexpr int gph = half / 4;  // rope groups per head
  static_assert(half % 4 == 0, "four pairs per group");
  const int nh = sh.n_heads, nkvh = sh.n_kv_heads;
  const int nkv = nkvh * HD;
  const float *wq = norm_weights(norm, layer, 0, HD);
  const float *wk = owns_new ? norm_weights(norm, layer, 1, HD) : nullptr;
  const float *cs = (sh.rope_on && rope) ? rope + (size_t)sd.pos * HD : nullptr;
  const bool llama = sh.arch_llama != 0;
  float *inv = scr;
  const int nt = nh + nkvh + 1;  // float4 row length of tr
  // group gi < ngq: q head gi / gph; else k head (gi - ngq) / gph.  A
  // thread's groups gi = t, t + 256, ... all sit at i4 = t % gph (256 is a
  // multiple of gph), so its weights and cos/sin are one set.
  static_assert(kThreads % gph == 0, "one group position per thread");
  constexpr int kG = 5;  // groups per thread: nq <= 8192 and nkv <= 2048
  const int ngq = nh * gph, ng = ngq + (owns_new ? nkvh * gph : 0);
  const int i4 = (int)threadIdx.x % gph;
  const int oa = llama ? 8 * i4 : 4 * i4, ob = llama ? 8 * i4 + 4 : half + 4 * i4;
  float4 xa[kG], xb[kG], qwa, qwb, kwa, kwb, c0, c1;
#pragma unroll
  for (int u = 0; u < kG; u++) {
    const int gi = (int)threadIdx.x + kThreads * u;
    if (gi < ng) {
      const bool is_q = gi < ngq;
      const float *x = is_q ? qi + (gi / gph) * HD : ki + ((gi - ngq) / gph) * HD;
      xa[u] = *reinterpret_cast<const float4 *>(x + oa);
      xb[u] = *reinterpret_cast<const float4 *>(x + ob);
    }
  }
  if (wq) {
    qwa = *reinterpret_cast<const float4 *>(wq + oa);
    qwb = *reinterpret_cast<const float4 *>(wq + ob);
  }
  if (wk) {
    kwa = *reinterpret_cast<const float4 *>(wk + oa);
    kwb = *reinterpret_cast<const float4 *>(wk + ob);
  }
  if (cs) {
    c0 = *reinterpret_cast<const float4 *>(cs + 8 * i4);
    c1 = *reinterpret_cast<const float4 *>(cs + 8 * i4 + 4);
  }
  // the owner's v, as it is (two pieces per thread: nkv <= 2048)
  const int nv4 = owns_new ? nkv / 4 : 0;
  const int v0 = (int)threadIdx.x, v1 = (int)threadIdx.x + kThreads;
  float4 tv0 = make_float4(0.f, 0.f, 0.f, 0.f), tv1 = tv0;
  if (v0 < nv4) tv0 = reinterpret_cast<const float4 *>(vi)[v0];
  if (v1 < nv4) tv1 = reinterpret_cast<const float4 *>(vi)[v1];
  if (v0 < nv4) reinterpret_cast<float4 *>(vr)[v0] = tv0;
  if (v1 < nv4) reinterpret_cast<float4 *>(vr)[v1] = tv1;
  // QK-RMSNorm factors over the transposed copy: thread h < nh for q head h,
  // nh + g for k head g
  if (wq || wk) {
#pragma unroll
    for (int u = 0; u < kG; u++) {
      const int gi = (int)threadIdx.x + kThreads * u;
      if (gi < ng) {
        const bool is_q = gi < ngq;
        if (is_q ? wq != nullptr : wk != nullptr) {
          const int H = is_q ? gi / gph : nh + (gi - ngq) / gph;
          // the group's elements as float4s of consecutive j: LLaMA's two
          // pieces already are; NEOX's a and b pieces are j = 4i4.. and
          // half + 4i4..
          const int ia = llama ? 2 * i4 : i4, ib = llama ? 2 * i4 + 1 : gph + i4;
          reinterpret_cast<float4 *>(tr)[ia * nt + H] = xa[u];
          reinterpret_cast<float4 *>(tr)[ib * nt + H] = xb[u];
        }
      }
    }
    __syncthreads();
    for (int h = threadIdx.x; h < nh + nkvh; h += kThreads) {
      const bool is_q = h < nh;
      if (is_q ? !wq : !wk) continue;
      float ss = 0.f;
#pragma unroll 8
      for (int i = 0; i < HD / 4; i++) {
        const float4 x = reinterpret_cast<const float4 *>(tr)[i * nt + h];
        float sq = x.x * x.x;
        ss = ss + sq;
        sq = x.y * x.y;
        ss = ss + sq;
        sq = x.z * x.z;
        ss = ss + sq;
        sq = x.w * x.w;
        ss = ss + sq;
      }
      inv[h] = __fdiv_rn(1.f, sqrtf(__fdiv_rn(ss, (float)HD) + norm.eps));
    }
    __syncthreads();
  }
  // (w * x) * inv, then the rotation, in registers; into qrot / kr
#pragma unroll
  for (int u = 0; u < kG; u++) {
    const int gi = (int)threadIdx.x + kThreads * u;
    if (gi < ng) {
      const bool is_q = gi < ngq;
      const int h = is_q ? gi / gph : (gi - ngq) / gph;
      const float4 wa = is_q ? qwa : kwa, wb = is_q ? qwb : kwb;
      float a[4], b[4], fa[4], fb[4];
      if (llama) {
        a[0] = xa[u].x; b[0] = xa[u].y; a[1] = xa[u].z; b[1] = xa[u].w;
        a[2] = xb[u].x; b[2] = xb[u].y; a[3] = xb[u].z; b[3] = xb[u].w;
        fa[0] = wa.x; fb[0] = wa.y; fa[1] = wa.z; fb[1] = wa.w;
        fa[2] = wb.x; fb[2] = wb.y; fa[3] = wb.z; fb[3] = wb.w;
      } else {
        a[0] = xa[u].x; a[1] = xa[u].y; a[2] = xa[u].z; a[3] = xa[u].w;
        b[0] = xb[u].x; b[1] = xb[u].y; b[2] = xb[u].z; b[3] = xb[u].w;
        fa[0] = wa.x; fa[1] = wa.y; fa[2] = wa.z; fa[3] = wa.w;
        fb[0] = wb.x; fb[1] = wb.y; fb[2] = wb.z; fb[3] = wb.w;
      }
      if (is_q ? wq != nullptr : wk != nullptr) {
        const float f = inv[is_q ? h : nh + h];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          a[k] = (fa[k] * a[k]) * f;
          b[k] = (fb[k] * b[k]) * f;
        }
      }
      if (cs) {
        rope_pair(a[0], b[0], c0.x, c0.y);
        rope_pair(a[1], b[1], c0.z, c0.w);
        rope_pair(a[2], b[2], c1.x, c1.y);
        rope_pair(a[3], b[3], c1.z, c1.w);
      }
      float *xh = (is_q ? qrot : kr) + h * HD;
      if (llama) {
        *reinterpret_cast<float4 *>(xh + oa) = make_float4(a[0], b[0], a[1], b[1]);
        *reinterpret_cast<float4 *>(xh + ob) = make_float4(a[2], b[2], a[3], b[3]);
      } else {
        *reinterpret_cast<float4 *>(xh + oa) = make_float4(a[0], a[1], a[2], a[3]);
        *reinterpret_cast<float4 *>(xh + ob) = make_float4(b[0], b[1], b[2], b[3]);
      }
    }
  }
  __syncthreads();
  if constexpr (DIG) {
    // make_digits per (head, chunk): thread quarter k of a chunk takes its
    // elements k*CD/4 .. (k+1)*CD/4 - 1; the chunk maximum over the quarter's
    // four lanes (consecutive threads)
    constexpr int QE = CD / 4;
    uint32_t *dig = digp ? digp : reinterpret_cast<uint32_t *>(tr);
    const int nch = nh * (HD / CD);
    for (int it = threadIdx.x; it < 4 * nch; it += kThreads) {
      const int ch = it >> 2, k = it & 3;
      const float *src = qrot + ch * CD + k * QE;
      float q[QE];
#pragma unroll
      for (int j = 0; j < QE; j += 4) {
        const float4 v4 = *reinterpret_cast<const float4 *>(src + j);
        q[j] = v4.x * qscale;
        q[j + 1] = v4.y * qscale;
        q[j + 2] = v4.z * qscale;
        q[j + 3] = v4.w * qscale;
      }
      float mx = 0.f;
#pragma unroll
      for (int j = 0; j < QE; j++) mx = fmaxf(mx, fabsf(q[j]));
      mx = fmaxf(mx, __shfl_xor(mx, 1));
      mx = fmaxf(mx, __shfl_xor(mx, 2));
      int e = 0;
      (void)frexpf(mx, &e);
      const float up = ldexpf(1.f, kQBits - e);
      uint32_t d[kQPlanes][QE / 4];
#pragma unroll
      for (int pl = 0; pl < kQPlanes; pl++)
#pragma unroll
        for (int j = 0; j < QE / 4; j++) d[pl][j] = 0u;
#pragma unroll
      for (int j = 0; j < QE; j++) {
        int dj[kQPlanes];
        split_digits((int)rintf(q[j] * up), dj);
        const int sh8 = 8 * (j & 3);
#pragma unroll
        for (int pl = 0; pl < kQPlanes; pl++) d[pl][j >> 2] |= ((uint32_t)dj[pl] & 0xffu) << sh8;
      }
      uint32_t *o = dig + ch * dig_stride<CD>();
#pragma unroll
      for (int pl = 0; pl < kQPlanes; pl++)
#pragma unroll
        for (int j = 0; j < QE / 4; j++) o[pl * (CD / 4) + k * (QE / 4) + j] = d[pl][j];
      if (k == 0) dig[dig_unit_at<CD>(nch, ch)] = __float_as_uint(ldexpf(1.f, e - kQBits));
    }
  }
  if (owns_new) {
    if (sh.kv_q8) {
      // four lanes per block (a multiple of 4 items, so a block's four
      // lanes are active together)
      const int nb = (nkv + 31) / 32;
      for (int it = threadIdx.x; it < 8 * nb; it += kThreads) {
        const int b = it >> 2, part = it & 3;
        const bool is_k = b < nb;
        const int bb = is_k ? b : b - nb;
        const int cnt = min(32, nkv - 32 * bb);
        q8_quant_block_x4((is_k ? kr : vr) + 32 * bb, cnt, (is_k ? rowk : rowv) + 34 * bb, part);
      }
    } else {
      float *fk = reinterpret_cast<float *>(rowk), *fv = reinterpret_cast<float *>(rowv);
      for (int e = threadIdx.x; e < nkv; e += kThreads) {
        fk[e] = kr[e];
        fv[e] = vr[e];
      }
    }
  }
  if (!DIG && !owns_new) return;  // qrot was published by the barrier above
  __syncthreads();
  if (!owns_new) return;
  const size_t off = ((size_t)layer * (size_t)sd.ctx_cap + (size_t)sd.pos) * sh.row_bytes;
  uint32_t *gk = reinterpret_cast<uint32_t *>(sd.k + off);
  uint32_t *gv = reinterpret_cast<uint32_t *>(sd.v + off);
  const uint32_t *lk = reinterpret_cast<const uint32_t *>(rowk);
  const uint32_t *lv = reinterpret_cast<const uint32_t *>(rowv);
  for (uint32_t i = threadIdx.x; i < sh.row_bytes / 4; i += kThreads) {
    gk[i] = lk[i];
    gv[i] = lv[i];
  }
}

// Specialised shapes.  A workgroup "visit" handles one unit (sequence,
// layer) over a set of positions: it [QK-RMSNorms and] rotates the unit's q
// into LDS, appends the new row if it owns pos (and reads that row back from
// LDS, not HBM), streams its positions, merges its four waves' softmax
// states and writes one partial per head into its partial slot; k_combine
// merges the partials and writes the output over q (l5_model.c:513-578).
//
// Static mode (WQ = false): workgroup (split, seq, layer) visits positions
// [split*split_len, min(pos+1, (split+1)*split_len)) of its unit once, and
// the split that holds pos appends.  Work-queue mode (WQ = true, STG = 2): a
// grid of resident workgroups, each starting at home unit blockIdx.x %
// n_units; positions [0, pos) of a unit are cut into pieces of
// P.piece_len positions that the waves of every workgroup visiting the unit
// claim one by one from the unit's counter (relaxed device-scope atomics,
// one claim ahead), so workgroups on busier parts of the memory system take
// fewer pieces.  With more units than workgroups, a workgroup done with its
// unit first takes the next never-assigned unit from a counter; after that,
// a workgroup whose unit has no pieces left moves to another unit with
// pieces left.  Each visit first reserves a partial slot from the
// unit's slot counter; the visit that gets slot 0 appends and consumes pos.
// At most P.max_splits visits per unit are admitted, and all counters only
// grow, so every workgroup finishes.  k_combine reads the slot count and
// zeroes the counter set of the next launch.
// A merge of the partials inside this kernel (last workgroup of a unit by
// an atomic counter) measured slower than the separate k_combine launch:
// its agent-scope fences cost more than one more launch.
// FMT: 0 = F32 KV, 1 = Q8_0 KV.  HD: head_dim.  CD: elements per lane.
// G: q heads per KV head.  U: wave-steps per loop trip of the per-lane (STG = 0) path.
// ATT: also write the raw scores for the reference-layout softmax weights.
// STG: how KV rows reach the lanes.  0: per-lane loads straight from HBM.
// 1: chunks of P.stage_rows rows pulled into the wave's LDS region by
// global_load_lds, then read from there.  2: the same chunks loaded into
// registers with coalesced non-temporal loads one chunk ahead (in flight
// while the current chunk is consumed) and written to LDS.
#ifdef G2B_STAMPS
#define G2B_STAMP(i) (stamp_[i] = wall_clock64())
#else
#define G2B_STAMP(i) ((void)0)
#endif

template <int FMT, int HD, int CD, int G, int U, bool ATT, int STG, bool WQ>
__global__ __launch_bounds__(kThreads) void k_layer(DecodeParams P) {
#ifdef G2B_STAMPS
  uint64_t stamp_[kStampWords] = {};
  G2B_STAMP(0);
#endif
  static_assert(!WQ || STG != 0, "the work queue streams through LDS");
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ int32_t s_bcast;
  constexpr int LPH = HD / CD;  // lanes per head
  using C = Codec<FMT, CD>;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int LPP = P.sh.n_kv_heads * LPH;  // lanes per position (<= 64, checked on host)
  const int PPW = 64 / LPP;               // positions per wave-step
  const int slot = lane / LPP;
  const bool lane_on = slot < PPW;
  const int slot_ld = lane_on ? slot : 0;  // idle lanes shadow slot 0's rows
  const int r = lane_on ? lane - slot * LPP : 0;
  const int g = r / LPH, c = r - g * LPH;
  const int n_heads = P.sh.n_heads;
  const int nkv = P.sh.n_kv_heads * HD;
  const size_t nq = (size_t)n_heads * HD;
  const size_t row = P.sh.row_bytes;
  const LaneOff lo = C::offsets(g * HD + c * CD, LPP);
  const int stride = kWavesPerSplit * PPW;    // positions between a wave's steps
  const size_t ustep = (size_t)stride * row;  // bytes between them

  // LDS: rotated q (nq floats), rotated new k and new v (nkv floats each) at 0 - with
  // STG, the waves' staging regions overlap them once q is in registers -
  // then the new K and V rows and the QK-RMSNorm scratch (n_heads floats).
  const LdsLayout ll = layer_lds_layout(P.sh, layer_stage_rows(STG, P.stage_rows));
  float *qrot = reinterpret_cast<float *>(lds);
  float *kr = reinterpret_cast<float *>(lds + nq * 4);
  float *vr = reinterpret_cast<float *>(lds + nq * 4 + ((nkv * 4 + 15) & ~15u));
  uint8_t *rowk = lds + ll.rows;
  uint8_t *rowv = rowk + ll.row_pad;
  float *scr = reinterpret_cast<float *>(rowv + ll.row_pad);  // norm factors, setup inputs
  float *trq = reinterpret_cast<float *>(lds + nq * 4 + 2 * ((nkv * 4 + 15) & ~15u));

  // One visit of unit (seq, li): positions [t0, tend) from HBM (static
  // mode) or the unit's claimed pieces (work queue), plus pos itself when
  // owns_new; the merged state goes to partial slot `pslot`.
  // (sd must be wave-uniform - loaded with a uniform index - or every KV
  // address derived from it lives in VGPRs.)
  auto visit = [&](const SeqDev &sd, int seq, int li, int t0, int tend, bool owns_new,
                   int pslot, int32_t *ctr) {
    const int layer = P.layer0 + li;
    const size_t sidx = (size_t)li * (size_t)P.n_seq + (size_t)seq;
    const uint8_t *kb = sd.k + ((size_t)layer * (size_t)sd.ctx_cap) * row;
    const uint8_t *vb = sd.v + ((size_t)layer * (size_t)sd.ctx_cap) * row;
    // Register staging (STG 2): the next chunk's 16-byte pieces, lane l
    // taking pieces l, l + 64, ... of the chunk's K and V bytes (at most
    // kStageLoads per lane and tensor).
    [[maybe_unused]] u32x4 rk[kStageLoads], rv[kStageLoads];
    [[maybe_unused]] auto issue = [&](int cs0) {
      const uint32_t np = (uint32_t)min(P.stage_rows, tend - cs0) * (uint32_t)row / 16u;
      const uint8_t *gk = kb + (size_t)cs0 * row + 16u * (uint32_t)lane;
      const uint8_t *gv = vb + (size_t)cs0 * row + 16u * (uint32_t)lane;
#pragma unroll
      for (int i = 0; i < kStageLoads; i++) {
        if (64u * (uint32_t)i + (uint32_t)lane < np) {
          rk[i] = __builtin_nontemporal_load(
              (const __attribute__((address_space(1))) u32x4 *)(gk + 1024u * i));
          rv[i] = __builtin_nontemporal_load(
              (const __attribute__((address_space(1))) u32x4 *)(gv + 1024u * i));
        }
      }
    };
    // Per-lane loads (STG 0): trip tb is UP wave-steps at positions
    // tb + u*stride + slot; positions past tend (and idle lanes) load row t0
    // and are masked out of the softmax.  Two register sets: the next trip
    // loads while the current one is consumed.  (F32 rows with 3 or 4 heads
    // per group: one wave-step per trip, to stay within 256 VGPRs.)
    constexpr int UP = (FMT == 0 && G >= 3) ? 1 : U;
    [[maybe_unused]] typename C::Raw ka[UP], va[UP], kn[UP], vn[UP];
    [[maybe_unused]] auto fetch = [&](int tb, typename C::Raw(&kk)[UP],
                                      typename C::Raw(&vv)[UP]) {
      const size_t base = (size_t)(tb + slot_ld) * row;
#pragma unroll
      for (int u = 0; u < UP; u++) {
        size_t off = base + (size_t)u * ustep;
        if (!(lane_on && tb + u * stride + slot < tend)) off = (size_t)t0 * row;
        C::load(kk[u], kb + off, lo);
        C::load(vv[u], vb + off, lo);
      }
    };
    // LDS DMA staging (STG 1): two regions per wave and tensor, region 0 of
    // every wave in the upper half of the staging area and region 1 in the
    // lower half, where the setup's scratch lies (so that a static
    // schedule's first chunk can land in region 0 during the setup when the
    // scratch fits the lower half).  Chunk cs0 of nrows rows goes straight
    // into region k (buffer_load_dwordx4 ... lds, non-temporal) once the
    // wave's reads of that region are done.
    [[maybe_unused]] const uint32_t cbytes = (uint32_t)P.stage_rows * (uint32_t)row;
    [[maybe_unused]] auto region = [&](int k) {
      return lds + (size_t)((k ? 0 : kWavesPerSplit) + wave) * 2 * cbytes;
    };
    [[maybe_unused]] auto dma_chunk = [&](int k, int cs0, int nrows) {
      const uint32_t np = (uint32_t)nrows * (uint32_t)row / 16u;  // 16-byte pieces
      const size_t base = (size_t)cs0 * row;
      const i32x4 rk = raw_rsrc(kb + base, np * 16u), rv = raw_rsrc(vb + base, np * 16u);
      const uint32_t la = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_addr(region(k)));
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the region's reads are done
      for (uint32_t i = 0; 64u * i < np; i++) {
        if (64u * i + (uint32_t)lane < np) {
          // (F32: LDS piece p holds the row piece that lies transposed there)
          const uint32_t p = 64u * i + (uint32_t)lane;
          const uint32_t voff = 16u * (FMT == 0 ? f32_global_piece(p, (uint32_t)LPP) : p);
          dma16(rk, la + 1024u * i, voff);
          dma16(rv, la + cbytes + 1024u * i, voff);
        }
      }
    };
    [[maybe_unused]] const bool early = ll.pre <= (uint32_t)kWavesPerSplit * 2u * cbytes;
    // Static schedule: the wave's first chunk or trip is in flight during
    // the setup.
    if constexpr (STG == 2 && !WQ) {
      if (t0 + wave * P.stage_rows < tend) issue(t0 + wave * P.stage_rows);
    }
    if constexpr (STG == 1 && !WQ) {
      if (early && t0 + wave * P.stage_rows < tend)
        dma_chunk(0, t0 + wave * P.stage_rows, min(P.stage_rows, tend - t0 - wave * P.stage_rows));
    }
    if constexpr (STG == 0) {
      if (t0 + wave * PPW < tend) fetch(t0 + wave * PPW, ka, va);
    }
    if constexpr (WQ) {
      {
        // [QK-RMSNorm (l3_math.c:107-114),] RoPE(q) for every head, pair by
        // pair as the append does (l3_math.c:74-101)
        const float *cs = (P.sh.rope_on && P.rope) ? P.rope + (size_t)sd.pos * HD : nullptr;
        const float *qi = P.q_in + sidx * nq;
        if (const float *wq = norm_weights(P.norm, layer, 0, HD)) {
          for (int e = threadIdx.x; e < (int)nq; e += blockDim.x) qrot[e] = qi[e];
          __syncthreads();
          qk_rmsnorm_block(qrot, n_heads, HD, wq, P.norm.eps, scr);
          qi = qrot;  // rotate in place: each pair is read and written by one thread
        }
        constexpr int half = HD / 2;
        for (int pr = threadIdx.x; pr < n_heads * half; pr += blockDim.x) {
          const int h = pr / half, j = pr - h * half;
          int ia, ib;
          rope_pair_index(P.sh.arch_llama, j, half, ia, ib);
          float a = qi[h * HD + ia], b = qi[h * HD + ib];
          if (cs) rope_pair(a, b, cs[2 * j], cs[2 * j + 1]);
          qrot[h * HD + ia] = a;
          qrot[h * HD + ib] = b;
        }
      }
      if (owns_new)  // (its barriers also publish qrot)
        append_new_row(P.sh, sd, layer, sd.pos, P.k_in + sidx * nkv, P.v_in + sidx * nkv,
                       P.rope, P.norm, kr, vr, rowk, rowv, scr);
      else
        __syncthreads();
    } else {
      // one round of loads, QK-RMSNorm, RoPE, the digit planes (Q8_0 KV)
      // and the owner's append
      visit_setup<HD, CD, FMT == 1>(P.sh, sd, layer, owns_new, P.q_in + sidx * nq,
                                    P.k_in + sidx * nkv, P.v_in + sidx * nkv, P.rope, P.norm,
                                    P.qscale, qrot, kr, vr, rowk, rowv, scr, trq);
    }
    G2B_STAMP(1);
    constexpr bool kDig = FMT == 1 && !WQ;  // the digit planes come from the setup

    // q in registers: F32 rows take the values, Q8_0 rows the digit planes
    // (from the setup's LDS copy, or made here from the values)
    [[maybe_unused]] float q[G][CD];
    [[maybe_unused]] QDigits<CD> qd[G];
    if constexpr (kDig) {
      const uint32_t *dig = reinterpret_cast<const uint32_t *>(trq);
#pragma unroll
      for (int i = 0; i < G; i++) {
        const int ch = (g * G + i) * (HD / CD) + c;
        const uint32_t *o = dig + ch * dig_stride<CD>();
#pragma unroll
        for (int pl = 0; pl < kQPlanes; pl++)
#pragma unroll
          for (int j = 0; j < CD / 4; j += 4) {
            const uint4 v4 = *reinterpret_cast<const uint4 *>(o + pl * (CD / 4) + j);
            qd[i].d[pl][j] = v4.x;
            qd[i].d[pl][j + 1] = v4.y;
            qd[i].d[pl][j + 2] = v4.z;
            qd[i].d[pl][j + 3] = v4.w;
          }
        qd[i].unit = __uint_as_float(dig[dig_unit_at<CD>(n_heads * (HD / CD), ch)]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < G; i++)
#pragma unroll
        for (int j = 0; j < CD; j += 4) {
          const float4 v4 =
              *reinterpret_cast<const float4 *>(qrot + (size_t)(g * G + i) * HD + c * CD + j);
          q[i][j + 0] = v4.x * P.qscale;
          q[i][j + 1] = v4.y * P.qscale;
          q[i][j + 2] = v4.z * P.qscale;
          q[i][j + 3] = v4.w * P.qscale;
        }
      if constexpr (FMT == 1) {
#pragma unroll
        for (int i = 0; i < G; i++) qd[i] = make_digits<CD>(q[i]);
      }
    }
    if constexpr (STG != 0) __syncthreads();  // every wave has its q: staging may overwrite qrot

    float m[G], l[G], acc[G][CD];
#pragma unroll
    for (int i = 0; i < G; i++) {
      m[i] = kNegBig;
      l[i] = 0.f;
#pragma unroll
      for (int j = 0; j < CD; j++) acc[i][j] = 0.f;
    }
    [[maybe_unused]] float *att_h = nullptr;
    if constexpr (ATT)
      att_h = P.att + (sidx * (size_t)n_heads + (size_t)g * G) * (size_t)P.att_stride;

    // Scores, online softmax and V for UU positions already loaded.
    auto consume = [&](const typename C::Raw *kr_, const typename C::Raw *vr_,
                       const bool *valid, const int *tpos, auto nu, auto check) {
      constexpr int UU = decltype(nu)::value;
      constexpr bool CHECK = decltype(check)::value;
      float sc[UU][G];
#pragma unroll
      for (int u = 0; u < UU; u++) {
        if constexpr (FMT == 1) {
          uint32_t w[CD / 4];
          float ks;
          C::quants(kr_[u], w, ks, lo);
#pragma unroll
          for (int i = 0; i < G; i++) {
            const float s = group_sum<LPH>(qk_int<CD / 4>(w, qd[i].d, ks * qd[i].unit));
            sc[u][i] = (!CHECK || valid[u]) ? s : -INFINITY;
          }
        } else {
          float kf[CD];
          C::values(kr_[u], kf);
#pragma unroll
          for (int i = 0; i < G; i++) {
            float s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (int j = 0; j < CD; j += 2) {
              s0 = fmaf(q[i][j], kf[j], s0);
              s1 = fmaf(q[i][j + 1], kf[j + 1], s1);
            }
            const float s = group_sum<LPH>(s0 + s1);
            sc[u][i] = (!CHECK || valid[u]) ? s : -INFINITY;
          }
        }
      }
      // m is a reference, not necessarily the running maximum: it is raised
      // (rescaling l and acc) only when a score exceeds it by more than
      // kRescaleSlack, so p = exp2(s - m) <= 2^kRescaleSlack and l, acc stay
      // far from overflow; any reference gives the same softmax, and the
      // merges scale each partial by its own m.  Rescales, which touch every
      // accumulator of the wave, become rare.
      bool need = false;
      float mn[G];
#pragma unroll
      for (int i = 0; i < G; i++) {
        float mx = m[i];
#pragma unroll
        for (int u = 0; u < UU; u++) mx = fmaxf(mx, sc[u][i]);
        mn[i] = mx;
        need |= mx > m[i] + kRescaleSlack;
      }
      if (__any(need)) {
#pragma unroll
        for (int i = 0; i < G; i++) {
          const float a = fast_exp2(m[i] - mn[i]);
          l[i] *= a;
#pragma unroll
          for (int j = 0; j < CD; j++) acc[i][j] *= a;
          m[i] = mn[i];
        }
      }
#pragma unroll
      for (int u = 0; u < UU; u++) {
        float p[G];
#pragma unroll
        for (int i = 0; i < G; i++) {
          p[i] = fast_exp2(sc[u][i] - m[i]);
          l[i] += p[i];
        }
        if constexpr (FMT == 1) {
          uint32_t w[CD / 4];
          float vs;
          C::quants(vr_[u], w, vs, lo);
          float pv[G];
#pragma unroll
          for (int i = 0; i < G; i++) pv[i] = p[i] * vs;
#pragma unroll
          for (int j = 0; j < CD / 4; j++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
              const float x = i8f(w[j], b);
#pragma unroll
              for (int i = 0; i < G; i++) acc[i][4 * j + b] = fmaf(pv[i], x, acc[i][4 * j + b]);
            }
        } else {
          float vf[CD];
          C::values(vr_[u], vf);
#pragma unroll
          for (int j = 0; j < CD; j++)
#pragma unroll
            for (int i = 0; i < G; i++) acc[i][j] = fmaf(p[i], vf[j], acc[i][j]);
        }
        if constexpr (ATT) {
          if (c == 0 && valid[u]) {
#pragma unroll
            for (int i = 0; i < G; i++) att_h[(size_t)i * P.att_stride + tpos[u]] = sc[u][i];
          }
        }
      }
    };

    if constexpr (STG != 0) {
      // Chunks of R contiguous positions.  A chunk's K and V bytes are
      // contiguous (rows of a layer are), so they move as 16-byte pieces,
      // lane l taking pieces l, l + 64, ..., into the wave's LDS region (each
      // HBM byte fetched once, by one lane, non-temporal); then every lane
      // reads its blocks from there.
      const int R = P.stage_rows;
      uint8_t *sk = lds + (size_t)wave * 2 * cbytes, *sv = sk + cbytes;
      const int steps = R / PPW;
      // U wave-steps of the chunk from LDS; rows past nrows (and idle lanes)
      // read row 0 of the chunk and are masked out of the softmax.
      auto lds_trip = [&](int cs0, int s, int nrows, auto nu, auto check) {
        constexpr int UU = decltype(nu)::value;
        constexpr bool CHECK = decltype(check)::value;
        typename C::Raw krr[UU], vrr[UU];
        bool valid[UU];
        int tpos[UU];
#pragma unroll
        for (int u = 0; u < UU; u++) {
          const int rr = (s + u) * PPW + slot;
          valid[u] = CHECK ? (lane_on && rr < nrows) : lane_on;
          const size_t ro = valid[u] ? (size_t)rr * row : 0;
          tpos[u] = cs0 + rr;
          C::load_lds(krr[u], sk + ro, lo);
          C::load_lds(vrr[u], sv + ro, lo);
        }
        consume(krr, vrr, valid, tpos, nu, check);
      };
      // Every lane's blocks of a chunk of nrows rows, read from LDS.
      auto consume_chunk = [&](int cs0, int nrows) {
        if (nrows == R) {
          for (int s = 0; s < steps; s++)
            lds_trip(cs0, s, nrows, std::integral_constant<int, 1>{}, std::false_type{});
        } else {
          for (int s = 0; s * PPW < nrows; s++)
            lds_trip(cs0, s, nrows, std::integral_constant<int, 1>{}, std::true_type{});
        }
      };
      const int cstride = kWavesPerSplit * R;  // positions between a wave's chunks (static)
      // Work queue: pieces of [0, tend) (piece_map: big ones, then small
      // ones for the last part; multiples of R) claimed from ctr[0], two
      // claims in flight while a piece is streamed.  Chunks never cross a
      // piece boundary.
      [[maybe_unused]] const PieceMap pm = piece_map(WQ ? tend : 0, P.piece_big, P.piece_len);
      [[maybe_unused]] const int npieces = WQ ? pm.npieces : 0;
      // A claim returns lane 0's fetched value in a VGPR without waiting for
      // it; the value is read (readfirstlane, which waits) only at the next
      // piece switch, so the atomic's latency overlaps a whole piece.
      [[maybe_unused]] auto claim_async = [&]() {
        int32_t v = 0;
        if (lane == 0)
          v = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return v;
      };
      if constexpr (STG == 1) {
        // Chunk c+1 goes into the wave's other region while chunk c is
        // consumed; each wave waits for its own loads only (s_waitcnt
        // vmcnt(0) opens every chunk: nothing else of the wave is then in
        // flight).
        auto consume_region = [&](int k, int cs0, int nrows) {
          sk = region(k);
          sv = sk + cbytes;
          consume_chunk(cs0, nrows);
        };
        if constexpr (!WQ) {
          int cs0 = t0 + wave * R;
          if (!early && cs0 < tend) dma_chunk(0, cs0, min(R, tend - cs0));
          for (int k = 0; cs0 < tend; k ^= 1, cs0 += cstride) {
            wait_vm0();
            const int ns = cs0 + cstride;
            if (ns < tend) dma_chunk(k ^ 1, ns, min(R, tend - ns));
            consume_region(k, cs0, min(R, tend - cs0));
          }
        } else {
          // this wave's pieces: a claim (lane 0) is issued when
          // a piece starts and read when it runs out - at a later chunk, so
          // after a wait for all of the wave's loads
          int32_t c0 = claim_lane0(ctr, lane);
          int32_t pend = claim_lane0(ctr, lane);
          wait_vm0();
          int pc = __builtin_amdgcn_readlane(c0, 0);
          int cs0 = 0, ce = 0;
          bool live = pc >= 0 && pc < npieces;
          if (live) {
            piece_range(pm, pc, tend, cs0, ce);
            cs0 = __builtin_amdgcn_readfirstlane(cs0);
            ce = __builtin_amdgcn_readfirstlane(ce);
            dma_chunk(0, cs0, min(R, ce - cs0));
          }
          for (int k = 0; live; k ^= 1) {
            wait_vm0();
            int ns = cs0 + R, nce = ce;
            bool nlive = true;
            if (ns >= ce) {  // next piece
              const int nc = __builtin_amdgcn_readlane(pend, 0);
              nlive = nc >= 0 && nc < npieces;
              if (nlive) {
                piece_range(pm, nc, tend, ns, nce);
                ns = __builtin_amdgcn_readfirstlane(ns);
                nce = __builtin_amdgcn_readfirstlane(nce);
                pend = claim_lane0(ctr, lane);
              }
            }
            if (nlive) dma_chunk(k ^ 1, ns, min(R, nce - ns));
            consume_region(k, cs0, min(R, ce - cs0));
            live = nlive;
            cs0 = ns;
            ce = nce;
          }
        }
      } else {
        // Registers hold the next chunk while the current one is consumed.
        auto stash = [&](int cs0) {
          const uint32_t np = (uint32_t)min(R, tend - cs0) * (uint32_t)row / 16u;
#pragma unroll
          for (int i = 0; i < kStageLoads; i++) {
            const uint32_t pc = 64u * (uint32_t)i + (uint32_t)lane;
            if (pc < np) {
              const uint32_t lp = FMT == 0 ? f32_lds_piece(pc, (uint32_t)LPP) : pc;
              *reinterpret_cast<u32x4 *>(sk + 16u * lp) = rk[i];
              *reinterpret_cast<u32x4 *>(sv + 16u * lp) = rv[i];
            }
          }
        };
        if constexpr (!WQ) {
          int cs0 = t0 + wave * R;  // (its loads were issued before the setup)
          for (; cs0 < tend; cs0 += cstride) {
            // (the previous chunk's LDS reads were all used before this point)
            stash(cs0);
            if (cs0 + cstride < tend) issue(cs0 + cstride);
            consume_chunk(cs0, min(R, tend - cs0));
          }
        } else {
          int pc = __builtin_amdgcn_readfirstlane(claim_async());
          int32_t pn1 = claim_async(), pn2 = claim_async();
          int cs0 = 0, ce = 0;
          if (pc < npieces) {
            piece_range(pm, pc, tend, cs0, ce);
            issue(cs0);
          }
          while (pc < npieces) {
            stash(cs0);
            int ns = cs0 + R, nce = ce, nc = pc;
            if (ns >= ce) {  // next piece
              nc = __builtin_amdgcn_readfirstlane(pn1);
              pn1 = pn2;
              if (nc < npieces) {
                piece_range(pm, nc, tend, ns, nce);
                pn2 = claim_async();
              }
            }
            if (nc < npieces) issue(ns);
            consume_chunk(cs0, min(R, ce - cs0));
            pc = nc;
            cs0 = ns;
            ce = nce;
          }
        }
      }
    } else {
      // Per-lane loads, one trip ahead (the first was issued before the setup).
      auto pipe_step = [&](int tb, typename C::Raw(&kc)[UP], typename C::Raw(&vc)[UP],
                           typename C::Raw(&kx)[UP], typename C::Raw(&vx)[UP]) {
        if (tb + stride * UP < tend) fetch(tb + stride * UP, kx, vx);
        bool valid[UP];
        int tpos[UP];
#pragma unroll
        for (int u = 0; u < UP; u++) {
          tpos[u] = tb + u * stride + slot;
          valid[u] = lane_on && tpos[u] < tend;
        }
        consume(kc, vc, valid, tpos, std::integral_constant<int, UP>{}, std::true_type{});
      };
      // (two steps per loop trip, so the register sets swap roles without copies)
      for (int tb = t0 + wave * PPW; tb < tend; tb += 2 * stride * UP) {
        pipe_step(tb, ka, va, kn, vn);
        if (tb + stride * UP >= tend) break;
        pipe_step(tb + stride * UP, kn, vn, ka, va);
      }
    }
    G2B_STAMP(2);
    if (owns_new) {
      typename C::Raw krr[1], vrr[1];
      C::load_row(krr[0], rowk, lo);
      C::load_row(vrr[0], rowv, lo);
      const bool valid[1] = {wave == 0 && slot == 0};
      const int tpos[1] = {sd.pos};
      consume(krr, vrr, valid, tpos, std::integral_constant<int, 1>{}, std::true_type{});
    }

    // Fold the PPW position slots of the wave into slot 0.  Slots of 32 or
    // 16 lanes: a butterfly through the lane swaps, every lane merging its
    // state with lane ^ 32's (then lane ^ 16's), so all lanes end with the
    // wave's state.  Otherwise every lane takes part in LDS shuffles, but only
    // slot-0 lanes update their state, so the state read from slot k is always
    // slot k's own.
    auto fold_xor = [&](auto dist) {
      constexpr int S = decltype(dist)::value;
#pragma unroll
      for (int i = 0; i < G; i++) {
        const float m2 = lanes_xor<S>(m[i]);
        const float l2 = lanes_xor<S>(l[i]);
        const float M = fmaxf(m[i], m2);
        const float f1 = exp2f(m[i] - M), f2 = exp2f(m2 - M);
        l[i] = l[i] * f1 + l2 * f2;
#pragma unroll
        for (int j = 0; j < CD; j++) acc[i][j] = acc[i][j] * f1 + lanes_xor<S>(acc[i][j]) * f2;
        m[i] = M;
      }
    };
    const int S = layer_merge_states(LPP);  // slots kept apart for the LDS merge
    if (LPP == 32 || LPP == 16) {
      fold_xor(std::integral_constant<int, 32>{});
      if (LPP == 16) fold_xor(std::integral_constant<int, 16>{});
    } else if (S == 1) {
      const bool gather = slot == 0;
      for (int k = 1; k < PPW; k++) {
        const int src = (lane + k * LPP) & 63;
#pragma unroll
        for (int i = 0; i < G; i++) {
          const float m2 = __shfl(m[i], src);
          const float l2 = __shfl(l[i], src);
          const float M = fmaxf(m[i], m2);
          const float f1 = exp2f(m[i] - M), f2 = exp2f(m2 - M);
          l[i] = gather ? l[i] * f1 + l2 * f2 : l[i];
#pragma unroll
          for (int j = 0; j < CD; j++) {
            const float a2 = __shfl(acc[i][j], src);
            acc[i][j] = gather ? acc[i][j] * f1 + a2 * f2 : acc[i][j];
          }
          m[i] = gather ? M : m[i];
        }
      }
    }
    // Merge the four waves' states in LDS (the rows and q there are no
    // longer read once every wave is past this barrier) and write one
    // partial per head.  LDS: [wave][slot][head][kPartHead + HD] floats, S
    // slots per wave (1 when the wave folded them).
    constexpr int pstr = kPartHead + HD;
    G2B_STAMP(3);
    __syncthreads();
    float *ws = reinterpret_cast<float *>(lds);
    if (S > 1 ? lane_on : slot == 0) {
      const int st = wave * S + (S > 1 ? slot : 0);
#pragma unroll
      for (int i = 0; i < G; i++) {
        float *pw = ws + ((size_t)st * n_heads + (size_t)(g * G + i)) * pstr;
        if (c == 0) {
          pw[0] = m[i];
          pw[1] = l[i];
        }
#pragma unroll
        for (int j = 0; j < CD; j += 4)
          *reinterpret_cast<float4 *>(pw + kPartHead + c * CD + j) =
              make_float4(acc[i][j], acc[i][j + 1], acc[i][j + 2], acc[i][j + 3]);
      }
    }
    __syncthreads();
    // (four elements of one head per thread and step)
    const size_t wstr = (size_t)n_heads * pstr;
    const int NW = kWavesPerSplit * S;
    for (int e4 = threadIdx.x; e4 < n_heads * (HD / 4); e4 += blockDim.x) {
      const int h = e4 / (HD / 4), d = 4 * (e4 - h * (HD / 4));
      const float *pw = ws + (size_t)h * pstr;
      float M = pw[0];
      for (int w = 1; w < NW; w++) M = fmaxf(M, pw[w * wstr]);
      float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
      float lsum = 0.f;
      for (int w = 0; w < NW; w++) {
        const float f = exp2f(pw[w * wstr] - M);
        const float4 a = *reinterpret_cast<const float4 *>(pw + w * wstr + kPartHead + d);
        o.x = fmaf(a.x, f, o.x);
        o.y = fmaf(a.y, f, o.y);
        o.z = fmaf(a.z, f, o.z);
        o.w = fmaf(a.w, f, o.w);
        lsum = fmaf(pw[w * wstr + 1], f, lsum);
      }
      if (!WQ && P.direct_out) {
        // the only partial of the unit: the output itself, over q
        float *out = P.q_out + sidx * nq + (size_t)h * HD + d;
        const double L = (double)lsum;
        *reinterpret_cast<float4 *>(out) =
            make_float4((float)((double)o.x / L), (float)((double)o.y / L),
                        (float)((double)o.z / L), (float)((double)o.w / L));
        continue;
      }
      float *pp = P.part + ((sidx * (size_t)n_heads + (size_t)h) * (size_t)P.max_splits +
                            (size_t)pslot) * pstr;
      *reinterpret_cast<float4 *>(pp + kPartHead + d) = o;
      if (d == 0) {
        pp[0] = M;
        pp[1] = lsum;
      }
    }
    G2B_STAMP(4);
    __syncthreads();  // LDS is free for the next visit
  };

  if constexpr (!WQ) {
    const int split = blockIdx.x, li = blockIdx.z;
    const int seq = static_seq((int)blockIdx.y, li, P.n_seq);
    const SeqDev sd = P.seqs ? P.seqs[seq] : P.one;
    const int npos = sd.pos + 1;
    const int t0 = split * P.split_len;
    if (t0 >= npos) return;  // a shorter sequence of a ragged batch: no split here
    const int t1 = min(npos, t0 + P.split_len);
    const bool owns_new = t1 == npos;  // this split holds position pos
    // Positions [t0, tend) stream from HBM; pos itself, when owned, from LDS.
    visit(sd, seq, li, t0, owns_new ? t1 - 1 : t1, owns_new, split, nullptr);
#ifdef G2B_STAMPS
    const uint64_t g = blockIdx.x + (uint64_t)gridDim.x * (blockIdx.y + (uint64_t)gridDim.y * blockIdx.z);
    if (threadIdx.x == 0 && P.stamps && g < (uint64_t)P.stamp_cap) {
      G2B_STAMP(5);
      stamp_[6] = (uint64_t)split;
      // HW_REG_XCC_ID (hwreg 20), bits 3:0: the XCD the workgroup ran on
      stamp_[7] = (uint64_t)(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15);
      for (int i = 0; i < kStampWords; i++) P.stamps[g * kStampWords + i] = stamp_[i];
    }
#endif
  } else {
    const int n_units = P.n_seq * P.n_layers_call;
    int32_t *const wq = P.wq + (size_t)P.wq_set * (size_t)P.wq_cap * kWqStride;
    int unit = __builtin_amdgcn_readfirstlane(
        P.home ? P.home[blockIdx.x] : (int)(blockIdx.x % (unsigned)n_units));
    uint32_t probe = blockIdx.x * 2654435761u;  // where the next search starts
    // More units than workgroups: units [gridDim.x, n_units) are handed out
    // in order from the counter in line n_units before any search.
    int32_t *const fresh = wq + (size_t)n_units * kWqStride;
    bool fresh_left = (int)gridDim.x < n_units;
    for (;;) {
      int32_t *ctr = wq + (size_t)unit * kWqStride;
      if (threadIdx.x == 0)
        s_bcast = __hip_atomic_fetch_add(ctr + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      const int pslot = __builtin_amdgcn_readfirstlane(s_bcast);
      __syncthreads();
      if (pslot < P.max_splits) {
        const int seq = unit % P.n_seq, li = unit / P.n_seq;
        const SeqDev sd = P.seqs ? P.seqs[seq] : P.one;
        visit(sd, seq, li, 0, sd.pos, pslot == 0, pslot, ctr);
#ifdef G2B_STAMPS
        stamp_[6]++;  // visits (phases 1-4 are the last visit's)
#endif
      }
      if (fresh_left) {
        if (threadIdx.x == 0)
          s_bcast = (int)gridDim.x +
                    __hip_atomic_fetch_add(fresh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const int nu = __builtin_amdgcn_readfirstlane(s_bcast);
        __syncthreads();
        if (nu < n_units) {
          unit = nu;
          continue;
        }
        fresh_left = false;
      }
      // Next unit: one with at least kWqStealMin unclaimed pieces and a free
      // partial slot, searched by wave 0 from a per-workgroup offset.
      if (wave == 0) {
        int found = -1;
        probe = probe * 1664525u + 1013904223u;
        const int start = (int)(probe % (uint32_t)n_units);
        for (int b = 0; b < n_units && found < 0; b += 64) {
          const int v = b + lane;
          bool ok = false;
          if (v < n_units) {
            const int uu = (start + v) % n_units;
            const int32_t *cu = wq + (size_t)uu * kWqStride;
            const int pos2 = P.seqs ? P.seqs[uu % P.n_seq].pos : P.one.pos;
            const int np2 = piece_map(pos2, P.piece_big, P.piece_len).npieces;
            const int32_t nx = __hip_atomic_load(cu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int32_t ns = __hip_atomic_load(cu + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = nx + kWqStealMin <= np2 && ns < P.max_splits;
          }
          const uint64_t mask = __ballot(ok);
          if (mask) found = (start + b + (int)__builtin_ctzll(mask)) % n_units;
        }
        if (lane == 0) s_bcast = found;
      }
      __syncthreads();
      unit = __builtin_amdgcn_readfirstlane(s_bcast);
      __syncthreads();
      if (unit < 0) break;
    }
#ifdef G2B_STAMPS
    const uint64_t g = blockIdx.x;
    if (threadIdx.x == 0 && P.stamps && g < (uint64_t)P.stamp_cap) {
      G2B_STAMP(5);
      stamp_[7] = (uint64_t)(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15);
      for (int i = 0; i < kStampWords; i++) P.stamps[g * kStampWords + i] = stamp_[i];
    }
#endif
  }
}

// ---------------------------------------------------------------- launchers

// (CD elements per lane: the variant's merge states)
template <int HD, int CD>
static inline size_t layer_lds_bytes(const ShapeDev &sh, int32_t stage_rows) {
  return layer_lds_layout(sh, stage_rows, layer_merge_states(sh.n_kv_heads * (HD / CD))).total;
}

template <int FMT, int HD, int CD, int G, int U, int STG, bool WQ>
static hipError_t launch_fast_s(const DecodeParams &p, int n_layers, hipStream_t s) {
  const dim3 grid = WQ ? dim3(p.wq_grid) : static_grid(p, n_layers);
  const size_t lds = layer_lds_bytes<HD, CD>(p.sh, layer_stage_rows(STG, p.stage_rows));
  if (p.att)
    hipLaunchKernelGGL((k_layer<FMT, HD, CD, G, U, true, STG, WQ>), grid, dim3(kThreads), lds, s, p);
  else
    hipLaunchKernelGGL((k_layer<FMT, HD, CD, G, U, false, STG, WQ>), grid, dim3(kThreads), lds, s,
                       p);
  return hipGetLastError();
}

template <int FMT, int HD, int CD, int G, int U>
static hipError_t launch_fast_u(const DecodeParams &p, int n_layers, hipStream_t s) {
  if (p.stage_rows > 0 && p.stage_mode == 2) {
    if (p.wq) return launch_fast_s<FMT, HD, CD, G, U, 2, true>(p, n_layers, s);
    return launch_fast_s<FMT, HD, CD, G, U, 2, false>(p, n_layers, s);
  }
  if (p.stage_rows > 0 && p.stage_mode == 1) {
    if (p.wq) return launch_fast_s<FMT, HD, CD, G, U, 1, true>(p, n_layers, s);
    return launch_fast_s<FMT, HD, CD, G, U, 1, false>(p, n_layers, s);
  }
  return launch_fast_s<FMT, HD, CD, G, U, 0, false>(p, n_layers, s);
}

template <int FMT, int HD, int CD, int G>
static hipError_t launch_fast(const DecodeParams &p, int n_layers, hipStream_t s) {
  return launch_fast_u<FMT, HD, CD, G, 2>(p, n_layers, s);
}

// Q8_0 with group <= 2 defaults to a whole block per lane (half a block when
// tuned so); every other shape uses 16 elements per lane.
template <int FMT, int HD, int G>
hipError_t launch_layer(const DecodeParams &p, int n_layers, hipStream_t s) {
  if constexpr (FMT == 1 && G <= 2) {
    if (p.tune_chunk == 16) return launch_fast<1, HD, 16, G>(p, n_layers, s);
    return launch_fast<1, HD, 32, G>(p, n_layers, s);
  } else {
    return launch_fast<FMT, HD, 16, G>(p, n_layers, s);
  }
}

template <int FMT, int HD, int CD, int G, int STG, bool WQ>
static int occupancy_of(const ShapeDev &sh, int32_t stage_rows) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_layer<FMT, HD, CD, G, 2, false, STG, WQ>,
                                                   kThreads,
                                                   layer_lds_bytes<HD, CD>(sh, layer_stage_rows(STG, stage_rows))) !=
      hipSuccess) {
    (void)hipGetLastError();
    return 1;
  }
  return n > 0 ? n : 1;
}

template <int FMT, int HD, int CD, int G>
static int occupancy_cd(const ShapeDev &sh, int32_t stage_mode, int32_t stage_rows, bool wq) {
  if (stage_rows > 0 && stage_mode == 2)
    return wq ? occupancy_of<FMT, HD, CD, G, 2, true>(sh, stage_rows)
              : occupancy_of<FMT, HD, CD, G, 2, false>(sh, stage_rows);
  if (stage_rows > 0 && stage_mode == 1)
    return wq ? occupancy_of<FMT, HD, CD, G, 1, true>(sh, stage_rows)
              : occupancy_of<FMT, HD, CD, G, 1, false>(sh, stage_rows);
  return occupancy_of<FMT, HD, CD, G, 0, false>(sh, 0);
}

template <int FMT, int HD, int G>
int layer_occupancy(const ShapeDev &sh, int32_t tune_chunk, int32_t stage_mode,
                    int32_t stage_rows, bool wq) {
  if constexpr (FMT == 1 && G <= 2) {
    if (tune_chunk == 16) return occupancy_cd<1, HD, 16, G>(sh, stage_mode, stage_rows, wq);
    return occupancy_cd<1, HD, 32, G>(sh, stage_mode, stage_rows, wq);
  } else {
    return occupancy_cd<FMT, HD, 16, G>(sh, stage_mode, stage_rows, wq);
  }
}

}  // namespace g2b
