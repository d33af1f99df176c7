// g2b_tiles.h - k_tiles, the decode kernel for Q8_0 KV with wide GQA groups,
// whose K scores run on the int8 matrix cores.
//
// Replaces the score / softmax / V-accumulate loops of
// /root/reference/src/l5_model.c:518-557 for Q8_0 KV caches with head_dim
// 128, 8 KV heads and 3 or 4 q heads per KV head (Llama-3-8B's shape).  With
// that many q heads per KV head, k_layer's per-lane integer dot products
// (four v_dot4 chains per head and 4 bytes) make the loop bound by VALU
// issue; here one v_mfma_i32_16x16x32_i8 computes, for one 32-element block
// of one KV head and 16 positions, all G x 4 digit-plane dot products:
//   A (16 x 32 int8): row 4h + p = digit plane p of q head h of the group
//                     (heads >= G are zero rows),
//   B (32 x 16 int8): the block's 32 quants of 16 positions (the cache bytes
//                     as they are),
//   C (16 x 16 int32): exact sums; lane (h = lane/16, t = lane%16) holds the
//                     four planes of head h at position t.
// q is held as four signed int8 digits of a 31-bit fixed point relative to
// each (head, block)'s largest |q| (the digit planes k_layer uses), so the
// block's score is (d3*2^24 + d2*2^16 + d1*2^8 + d0)-weighted sums, exact in
// int32 per plane and combined exactly in float64 (chunk_value_exact), times
// the block's fp16 scale; blocks are summed in float64 and the score is
// rounded to fp32 once.  Softmax stays in that layout (each lane one (head, position); the
// running maximum of a head is shared by its 16 lanes through DPP), and V is
// accumulated in fp32 on the matrix cores as well: lane (KV head of the
// wave's pair, four dims) takes p * v_scale for its block from a per-wave LDS
// exchange, and four v_mfma_f32_4x4x1_16b_f32 per position add p * v_scale *
// v for every head of the group to the lane's four dims.
//
// Streaming: a workgroup streams tiles of 16 positions - the K and V rows of
// 16 consecutive positions are two contiguous runs of 16 x 1088 bytes - from
// HBM straight into one of two LDS tile buffers (buffer_load_dwordx4 ... lds,
// non-temporal, 36 loads of 1 KiB per tile, nine per wave): tile i+1 is
// issued into the other buffer right after the workgroup barrier that opens
// tile i and lands while tile i is consumed.  In LDS each 1088-byte row is
// padded to 1104 bytes (a 16-byte slot no load writes): at the plain stride
// the 16 positions' operand reads all fell on 2 of 32 banks (an 8-way
// conflict that made LDS the bound).
// Each wave owns two KV heads of every tile, so the waves of a workgroup
// never merge states: each writes the partials (or, with one split, the
// output) of its own heads.
//
// Schedules are k_layer's: static splits (workgroup = split x sequence x
// layer) or the work queue (pieces of a unit claimed per workgroup by wave 0,
// which hands each tile's first row and row count to the waves through LDS
// one tile ahead).  The
// setup (QK-RMSNorm, RoPE, digit planes, the owner's append) is k_layer's
// visit_setup; the owner consumes its new row from LDS.
#pragma once
#include "g2b_layer.h"

namespace g2b {

constexpr int kTileRows = kTilesRows;  // positions per tile (the MFMA's 16 columns)
constexpr int kTilesKvPerWave = 2;
constexpr int kTilesHd = 128;
// A tile tensor (16 K or V rows) in LDS: rows of 68 16-byte slots of data
// and one of padding (a pitch of 71 slots measured the same).
constexpr int kTilesRowData = 68;
constexpr int kTilesRowSlots = kTilesRowData + 1;
constexpr uint32_t kTilesLdsRow = 16u * kTilesRowSlots;
constexpr int kTilesSlots = kTileRows * kTilesRowSlots;   // per tensor
constexpr int kTilesLoadsT = (kTilesSlots + 63) / 64;     // 1 KiB loads per tensor
constexpr int kTilesLoads = 2 * kTilesLoadsT;             // per tile
constexpr int kTilesWaveLoads = kTilesLoads / kWavesPerSplit;  // wave w: loads w, w + 4, ...
static_assert(kTilesLoads % kWavesPerSplit == 0, "the same loads per wave");
constexpr uint32_t kTilesTensorBytes = (uint32_t)kTilesSlots * 16u;
constexpr uint32_t kTilesTileBytes = 2u * kTilesTensorBytes;

// Shapes k_tiles serves.
__host__ __device__ inline bool tiles_shape_ok(const ShapeDev &sh) {
  if (!sh.kv_q8 || sh.head_dim != kTilesHd) return false;
  if (sh.n_kv_heads != kWavesPerSplit * kTilesKvPerWave) return false;
  if (sh.row_bytes != 16u * kTilesRowData) return false;
  if (sh.n_heads % sh.n_kv_heads) return false;
  const int g = sh.n_heads / sh.n_kv_heads;
  return g >= 3 && g <= 4;
}

// k_tiles' dynamic LDS: tile buffer 0, each wave's exchange of p * v_scale
// ([kv][block][head][position]) and rescale factors ([kv][head]), tile
// buffer 1.  The setup's scratch starts at the exchange and lies over it and
// buffer 1 (never over buffer 0, whose loads the static schedule issues
// before the setup): rotated q at 0, the new k after it, the digit planes
// after that and the new v, then the new K and V rows and the norm factors;
// the transposed copy for the QK-RMSNorm sums lies over q, k and the digit
// planes, which are written only after the sums (the v copy is written before
// them, so it stays clear).  The exchange overlaps only q and k, dead by the
// time the owner consumes its new row; buffer 1 is loaded after a barrier
// that follows that.  ~78 KiB for Llama-3-8B's heads: two workgroups per CU.
struct TilesLds {
  uint32_t scr0;                              // the setup scratch (absolute)
  uint32_t kr, dig, vr, rows, row_pad, scr;  // (relative to scr0)
  uint32_t px, buf1, total;                   // (absolute)
};
// The exchange holds one group of 4 heads x kTileRows floats per (KV head,
// block), kTilesPxGroup floats apart: the V loop's lanes read the eight
// groups together (four positions of one head each), and at 64 floats (256
// bytes) apart such reads all fell on the same four banks.
constexpr int kTilesPxGroup = kTileRows * 4 + 4;
__host__ __device__ inline uint32_t tiles_px_floats() {
  return (uint32_t)(kTilesKvPerWave * (kTilesHd / 32) * kTilesPxGroup + kTilesKvPerWave * 4);
}
__host__ __device__ inline TilesLds tiles_lds_layout(const ShapeDev &sh) {
  const uint32_t nq = (uint32_t)(sh.n_heads * sh.head_dim);
  const uint32_t nkv4 = ((uint32_t)(sh.n_kv_heads * sh.head_dim) * 4u + 15u) & ~15u;
  const uint32_t digb = (uint32_t)dig_dwords<32>(sh.n_heads * (sh.head_dim / 32)) * 4u;
  const uint32_t trb = (uint32_t)(sh.head_dim * (sh.n_heads + sh.n_kv_heads + 1)) * 4u;
  TilesLds l;
  l.kr = nq * 4u;
  l.dig = l.kr + nkv4;
  const uint32_t dig_end = l.dig + digb;
  l.vr = ((dig_end > trb ? dig_end : trb) + 15u) & ~15u;
  l.row_pad = (sh.row_bytes + 15u) & ~15u;
  l.rows = l.vr + nkv4;
  l.scr = l.rows + 2u * l.row_pad;
  const uint32_t scr_floats =
      (uint32_t)(((sh.n_heads + sh.n_kv_heads + 3) & ~3) + 3 * sh.head_dim);
  const uint32_t scr_end = l.scr + scr_floats * 4u;
  l.px = kTilesTileBytes;
  l.scr0 = l.px;
  l.buf1 = l.px + (uint32_t)kWavesPerSplit * tiles_px_floats() * 4u;
  const uint32_t end = l.buf1 + kTilesTileBytes;
  l.total = end > l.scr0 + scr_end ? end : ((l.scr0 + scr_end + 15u) & ~15u);
  return l;
}

template <int N>
__device__ __forceinline__ float group_max(float x) {
  static_assert(N == 16, "rows of 16 lanes");
  x = fmaxf(x, dpp_f<0xB1>(x));   // lane ^ 1
  x = fmaxf(x, dpp_f<0x4E>(x));   // lane ^ 2
  x = fmaxf(x, dpp_f<0x141>(x));  // other quad of 8
  x = fmaxf(x, dpp_f<0x140>(x));  // other half of 16
  return x;
}

// G: q heads per KV head (3 or 4).  WQ: work-queue schedule.
template <int G, bool WQ>
__global__ __launch_bounds__(kThreads) void k_tiles(DecodeParams P) {
  constexpr int HD = kTilesHd, NB = HD / 32, KPW = kTilesKvPerWave, TP = kTileRows;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ int32_t s_bcast;
  __shared__ int32_t s_desc[2][2];  // work queue: tile t's (first row, rows) at [t & 1]
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n_heads = P.sh.n_heads;
  const int nkv = P.sh.n_kv_heads * HD;
  const size_t nq = (size_t)n_heads * HD;
  const uint32_t row = P.sh.row_bytes;
  const TilesLds ll = tiles_lds_layout(P.sh);
  uint8_t *const sb = lds + ll.scr0;
  float *qrot = reinterpret_cast<float *>(sb);
  float *kr = reinterpret_cast<float *>(sb + ll.kr);
  float *vr = reinterpret_cast<float *>(sb + ll.vr);
  float *trq = reinterpret_cast<float *>(sb);  // the norm sums' transposed copy
  uint32_t *digs = reinterpret_cast<uint32_t *>(sb + ll.dig);
  uint8_t *rowk = sb + ll.rows, *rowv = rowk + ll.row_pad;
  float *scr = reinterpret_cast<float *>(sb + ll.scr);
  float *px = reinterpret_cast<float *>(lds + ll.px) + (size_t)wave * tiles_px_floats();
  float *pfac = px + KPW * NB * kTilesPxGroup;  // [kv][head] rescale factors
  auto buf = [&](int k) { return lds + (k ? ll.buf1 : 0u); };

  // This wave's tile loads u: load j = wave + 4u of the tile, tensor j / 18
  // (K, V), slots 64 (j % 18) + lane of it; slot s is row s / 69, bytes
  // 16 (s % 69) of it, and slot 68 of a row is padding (lane off).
  // Loop-invariant registers: a load's offset register must not be
  // rewritten while the load is in flight.
  uint32_t goff[kTilesWaveLoads];
  uint32_t gon = 0u;  // bit u: this lane takes part in load u
#pragma unroll
  for (int u = 0; u < kTilesWaveLoads; u++) {
    const int j = wave + kWavesPerSplit * u;
    const int sl = 64 * (j % kTilesLoadsT) + lane;
    const int r = sl / kTilesRowSlots, c = sl - r * kTilesRowSlots;
    goff[u] = (uint32_t)r * row + 16u * (uint32_t)c;
    if (sl < kTilesSlots && c < kTilesRowData) gon |= 1u << u;
  }

  // lane roles: MFMA row / column (A row, B and C column = position) and
  // quarter (A/B k-quarter, C row group = q head of the group)
  const int col = lane & 15, quarter = lane >> 4;
  // V: KV head of the wave's pair, four dims 4*vd .. 4*vd+3 (block vd / 8)
  const int vkv = lane >> 5, vd = lane & 31, vblk = vd >> 3;

  auto visit = [&](const SeqDev &sd, int seq, int li, int t0, int tend, bool owns_new,
                   int pslot, int32_t *ctr) {
    // (the workgroup's positions: scalar registers)
    t0 = __builtin_amdgcn_readfirstlane(t0);
    tend = __builtin_amdgcn_readfirstlane(tend);
    const int layer = P.layer0 + li;
    const size_t sidx = (size_t)li * (size_t)P.n_seq + (size_t)seq;
    const uint8_t *kb = sd.k + ((size_t)layer * (size_t)sd.ctx_cap) * row;
    const uint8_t *vb = sd.v + ((size_t)layer * (size_t)sd.ctx_cap) * row;
    // This wave's loads of the tile of n rows at ts into buffer k.  Slots of
    // rows at or past n load the run's first bytes instead (never read), so
    // that every load keeps its lanes.
    auto issue = [&](int k, int ts, int n) {
      const size_t base = (size_t)ts * row;
      const uint32_t span = (uint32_t)TP * row;
      const i32x4 rk = raw_rsrc(kb + base, span), rv = raw_rsrc(vb + base, span);
      const uint32_t la = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_addr(buf(k)));
      const uint32_t lim = (uint32_t)n * row;
#pragma unroll
      for (int u = 0; u < kTilesWaveLoads; u++) {
        const int j = wave + kWavesPerSplit * u;
        const bool is_v = j >= kTilesLoadsT;
        const uint32_t dst = la + (is_v ? kTilesTensorBytes : 0u) +
                             1024u * (uint32_t)(is_v ? j - kTilesLoadsT : j);
        if ((gon >> u) & 1u) dma16(is_v ? rv : rk, dst, goff[u] < lim ? goff[u] : 0u);
      }
    };
    const int ntiles = t0 < tend ? (tend - t0 + TP - 1) / TP : 0;  // static schedule
    auto static_rows = [&](int t) { return t < ntiles ? min(TP, tend - (t0 + TP * t)) : 0; };
    // Static schedule: the first tile is in flight during the setup.
    if (!WQ && ntiles > 0) issue(0, t0, static_rows(0));
    // Work queue: wave 0 claims the visit's first two pieces (first, pend),
    // in flight during the setup.
    int32_t first = 0, pend = 0;
    if (WQ && wave == 0) {
      first = claim_lane0(ctr, lane);
      pend = claim_lane0(ctr, lane);
    }

    // [QK-RMSNorm,] RoPE, the digit planes of q (32-element chunks = the
    // Q8_0 blocks) and the owner's append, all in LDS
    visit_setup<HD, 32, true>(P.sh, sd, layer, owns_new, P.q_in + sidx * nq, P.k_in + sidx * nkv,
                              P.v_in + sidx * nkv, P.rope, P.norm, P.qscale, qrot, kr, vr, rowk,
                              rowv, scr, trq, digs);
    // A operands: digit plane (col & 3) of head (col >> 2), bytes
    // 8*quarter .. of block b; and the C lanes' units 2^(e-30) of
    // (head quarter, block b)
    uint64_t qa[KPW][NB];
    float un[KPW][NB];
    {
      const uint32_t *dig = digs;
      constexpr int DS = dig_stride<32>();
      static_assert(kQPlanes == 4, "A rows 4h + p: four digit planes per head");
      const int ah = col >> 2, ap = col & 3;
      const int nch = P.sh.n_heads * NB;
#pragma unroll
      for (int kk = 0; kk < KPW; kk++) {
        const int kvg = wave * KPW + kk;
#pragma unroll
        for (int b = 0; b < NB; b++) {
          uint64_t a = 0;
          if (ah < G) {
            const uint32_t *o = dig + ((kvg * G + ah) * NB + b) * DS + ap * 8 + 2 * quarter;
            a = (uint64_t)o[0] | ((uint64_t)o[1] << 32);
          }
          qa[kk][b] = a;
          un[kk][b] = quarter < G
                          ? __uint_as_float(dig[dig_unit_at<32>(nch, (kvg * G + quarter) * NB + b)])
                          : 0.f;
        }
      }
    }

    // acc[j][h]: head h of the lane's KV head at dim 4*vd + j (the C/D
    // layout of v_mfma_f32_4x4x1_16b_f32, below)
    float m[KPW], l[KPW];
    f32x4 acc[4];
#pragma unroll
    for (int kk = 0; kk < KPW; kk++) {
      m[kk] = kNegBig;
      l[kk] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // V lane addressing inside a row: dims 4*vd.. of head (wave*KPW + vkv)
    const uint32_t voff = 34u * (uint32_t)((wave * KPW + vkv) * NB + vblk) + 2u + 4u * (vd & 7);
    const uint32_t vsel = (voff & 2u) ? 0x05040302u : 0x03020100u;
    const uint32_t valn = voff & ~3u;

    // One tile: rows [0, nrows) at K / V, `stride` bytes apart (rows past
    // nrows read row 0 and are masked).
    auto consume = [&](const uint8_t *K, const uint8_t *V, int nrows, uint32_t stride) {
      const int rr = col < nrows ? col : 0;
      const uint8_t *krow = K + (size_t)rr * stride;
      const uint8_t *vrow = V + (size_t)rr * stride;
      const bool valid = col < nrows && quarter < G;
      float s[KPW];
#pragma unroll
      for (int kk = 0; kk < KPW; kk++) {
        const int kvg = wave * KPW + kk;
        // the KV head's four blocks: operands first, then the MFMAs in pairs
        // into separate accumulators (so they issue back to back), then the
        // sums in block order
        uint64_t bop[NB];
        float ks[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
          const uint32_t blk = (uint32_t)(kvg * NB + b);
          const uint32_t off = 34u * blk + 2u + 8u * (uint32_t)quarter;
          const uint32_t *w = reinterpret_cast<const uint32_t *>(krow + (off & ~3u));
          const uint32_t sel = (off & 2u) ? 0x05040302u : 0x03020100u;
          const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
          bop[b] = (uint64_t)__builtin_amdgcn_perm(w1, w0, sel) |
                   ((uint64_t)__builtin_amdgcn_perm(w2, w1, sel) << 32);
          const uint32_t sw = *reinterpret_cast<const uint32_t *>(krow + ((34u * blk) & ~3u));
          ks[b] = half_bits_to_f32_hw(sw >> ((blk & 1u) * 16u));
        }
        double sc = 0.0;  // (exact block values, summed in float64: chunk_value_exact)
#pragma unroll
        for (int b0 = 0; b0 < NB; b0 += 2) {
          // two at a time (four accumulators would cost the second wave per SIMD)
          i32x4 c[2];
#pragma unroll
          for (int j = 0; j < 2; j++)
            c[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)qa[kk][b0 + j], (long)bop[b0 + j],
                                                         i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 2; j++) {
            const double part = chunk_value_exact(c[j][0], c[j][1], c[j][2], c[j][3]);
            sc = fma(part, (double)ks[b0 + j] * (double)un[kk][b0 + j], sc);
          }
        }
        s[kk] = valid ? (float)sc : -INFINITY;
      }
      // online softmax per (KV head, q head): the 16 lanes of a head share
      // its reference m (raised lazily, as k_layer does)
      bool need = false;
      float mt[KPW];
#pragma unroll
      for (int kk = 0; kk < KPW; kk++) {
        const float mx = group_max<16>(s[kk]);
        mt[kk] = fmaxf(m[kk], mx);
        need |= mx > m[kk] + kRescaleSlack;
      }
      const bool rescale = __any(need);
      if (rescale) {
#pragma unroll
        for (int kk = 0; kk < KPW; kk++) {
          const float a = fast_exp2(m[kk] - mt[kk]);
          l[kk] *= a;
          m[kk] = mt[kk];
          if (col == 0) pfac[kk * 4 + quarter] = a;
        }
      }
#pragma unroll
      for (int kk = 0; kk < KPW; kk++) {
        const int kvg = wave * KPW + kk;
        const float p = fast_exp2(s[kk] - m[kk]);  // 0 for masked lanes
        l[kk] += p;
        // p * (the V row's block scale) for each block of the KV head
#pragma unroll
        for (int b = 0; b < NB; b++) {
          const uint32_t blk = (uint32_t)(kvg * NB + b);
          const uint32_t sw = *reinterpret_cast<const uint32_t *>(vrow + ((34u * blk) & ~3u));
          const float vs = half_bits_to_f32_hw(sw >> ((blk & 1u) * 16u));
          px[(kk * NB + b) * kTilesPxGroup + quarter * TP + col] = p * vs;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (rescale) {
        const float4 f = *reinterpret_cast<const float4 *>(pfac + vkv * 4);
        const f32x4 fa = {f.x, f.y, f.z, f.w};
#pragma unroll
        for (int j = 0; j < 4; j++) acc[j] *= fa;
      }
      // V on the matrix cores: v_mfma_f32_4x4x1_16b_f32 is 16 blocks of
      // D[i][n] += A[i] B[n] with block g = lanes 4g..4g+3, A[i] from lane
      // 4g+i, B[n] from lane 4g+n and D[i][n] in register i of lane 4g+n.
      // A lane's block shares its KV head and Q8_0 block, so A = p x v_scale
      // of head (lane & 3) and B = the lane's own int8 at dim 4*vd + j put
      // head i's sum over positions for that dim in register i of the lane
      // (fp32 products accumulated in fp32, position by position).
      const float *pv = px + (vkv * NB + vblk) * kTilesPxGroup + (lane & 3) * TP;
      auto vstep = [&](int t, float a) {
        const uint32_t *w = reinterpret_cast<const uint32_t *>(V + (size_t)t * stride + valn);
        const uint32_t x = __builtin_amdgcn_perm(w[1], w[0], vsel);
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[j] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, i8f(x, j), acc[j], 0, 0, 0);
      };
      if (nrows == TP) {
#pragma unroll
        for (int t = 0; t < TP; t += 4) {  // four positions' p x v_scale in one read
          const float4 a4 = *reinterpret_cast<const float4 *>(pv + t);
          vstep(t, a4.x);
          vstep(t + 1, a4.y);
          vstep(t + 2, a4.z);
          vstep(t + 3, a4.w);
        }
      } else {
        for (int t = 0; t < nrows; t++) vstep(t, pv[t]);
      }
      // (px is written again only after these reads: the wave's next K
      // phase)
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // Work queue: wave 0 turns claimed pieces of [0, tend) into tiles, one
    // tile ahead of the issue.  A claim is issued when a piece starts and
    // read when it runs out, at a later tile: after the wait for all of the
    // wave's loads that opens every tile.
    const PieceMap pm = piece_map(WQ ? tend : 0, P.piece_big, P.piece_len);
    int nx = 0, pe = 0;  // the piece being cut: next row, end
    bool live = false;
    auto take_piece = [&](int pc) {
      live = pc >= 0 && pc < pm.npieces;
      if (live) {
        piece_range(pm, pc, tend, nx, pe);
        nx = __builtin_amdgcn_readfirstlane(nx);
        pe = __builtin_amdgcn_readfirstlane(pe);
      }
    };
    auto publish = [&](int t) {  // (wave 0) tile t's descriptor, for all
      if (live && nx >= pe) {
        take_piece(__builtin_amdgcn_readlane(pend, 0));
        if (live) pend = claim_lane0(ctr, lane);
      }
      int ts = 0, n = 0;
      if (live) {
        ts = nx;
        n = __builtin_amdgcn_readfirstlane(min(TP, pe - nx));
        nx += n;
      }
      if (lane == 0) {
        s_desc[t & 1][0] = ts;
        s_desc[t & 1][1] = n;
      }
    };
    auto desc = [&](int t, int &ts, int &n) {
      if constexpr (WQ) {
        ts = __builtin_amdgcn_readfirstlane(s_desc[t & 1][0]);
        n = __builtin_amdgcn_readfirstlane(s_desc[t & 1][1]);
      } else {
        ts = __builtin_amdgcn_readfirstlane(t0 + TP * t);
        n = __builtin_amdgcn_readfirstlane(static_rows(t));
      }
    };
    if constexpr (WQ) {
      if (wave == 0) {
        wait_vm0();  // (nothing else of this wave is in flight)
        take_piece(__builtin_amdgcn_readlane(first, 0));
        publish(0);
        publish(1);
      }
    }

    // The owner's new row first: it sits in the setup's scratch, which
    // buffer 1 overlaps.
    if (owns_new) consume(rowk, rowv, 1, row);
    __syncthreads();  // operands held, new row taken, descriptors published

    int ts = 0, n0 = 0;  // rows of tile i
    desc(0, ts, n0);
    if (WQ && n0 > 0) issue(0, ts, n0);  // (static: issued before the setup)
    for (int i = 0; n0 > 0; i++) {
      // this wave's loads of tile i are done; after the barrier everyone's
      // are, and everyone is done with tile i-1, whose buffer takes tile i+1
      wait_vm0();
      __syncthreads();
      int n1 = 0;
      desc(i + 1, ts, n1);
      if (n1 > 0) issue((i + 1) & 1, ts, n1);
      if (WQ && wave == 0) publish(i + 2);
      uint8_t *cur = buf(i & 1);
      consume(cur, cur + kTilesTensorBytes, n0, kTilesLdsRow);
      n0 = n1;
    }

    // The partials (or the output) of the wave's heads: the sums of each
    // head's 16 lanes; m is already shared by them.
    float lsum[KPW];
#pragma unroll
    for (int kk = 0; kk < KPW; kk++) lsum[kk] = group_sum<16>(l[kk]);
    constexpr int pstr = kPartHead + HD;
#pragma unroll
    for (int h = 0; h < G; h++) {
      // this V lane's head: (wave*KPW + vkv)*G + h; its m and l sit in the
      // lanes of row group h
      // (readlane moves the bits as an int)
      const int m0 = __builtin_amdgcn_readlane(__float_as_int(m[0]), 16 * h);
      const int m1 = __builtin_amdgcn_readlane(__float_as_int(m[1]), 16 * h);
      const int l0 = __builtin_amdgcn_readlane(__float_as_int(lsum[0]), 16 * h);
      const int l1 = __builtin_amdgcn_readlane(__float_as_int(lsum[1]), 16 * h);
      const float mh = __int_as_float(vkv ? m1 : m0);
      const float lh = __int_as_float(vkv ? l1 : l0);
      const int head = (wave * KPW + vkv) * G + h;
      if (!WQ && P.direct_out) {
        float *out = P.q_out + sidx * nq + (size_t)head * HD + 4 * vd;
        const double L = (double)lh;
        *reinterpret_cast<float4 *>(out) =
            make_float4((float)((double)acc[0][h] / L), (float)((double)acc[1][h] / L),
                        (float)((double)acc[2][h] / L), (float)((double)acc[3][h] / L));
      } else {
        float *pp = P.part + ((sidx * (size_t)n_heads + (size_t)head) * (size_t)P.max_splits +
                              (size_t)pslot) * pstr;
        *reinterpret_cast<float4 *>(pp + kPartHead + 4 * vd) =
            make_float4(acc[0][h], acc[1][h], acc[2][h], acc[3][h]);
        if (vd == 0) {
          pp[0] = mh;
          pp[1] = lh;
        }
      }
    }
    __syncthreads();  // LDS is free for the next visit
  };

  if constexpr (!WQ) {
    const int split = blockIdx.x, li = blockIdx.z;
    const int seq = static_seq((int)blockIdx.y, li, P.n_seq);
    const SeqDev sd = P.seqs ? P.seqs[seq] : P.one;
    const int npos = sd.pos + 1;
    const int t0 = split * P.split_len;
    if (t0 >= npos) return;
    const int t1 = min(npos, t0 + P.split_len);
    const bool owns_new = t1 == npos;
    visit(sd, seq, li, t0, owns_new ? t1 - 1 : t1, owns_new, split, nullptr);
  } else {
    const int n_units = P.n_seq * P.n_layers_call;
    int32_t *const wq = P.wq + (size_t)P.wq_set * (size_t)P.wq_cap * kWqStride;
    int unit = __builtin_amdgcn_readfirstlane(
        P.home ? P.home[blockIdx.x] : (int)(blockIdx.x % (unsigned)n_units));
    uint32_t probe = blockIdx.x * 2654435761u;
    int32_t *const fresh = wq + (size_t)n_units * kWqStride;
    bool fresh_left = (int)gridDim.x < n_units;
    for (;;) {
      int32_t *ctr = wq + (size_t)unit * kWqStride;
      if (tid == 0)
        s_bcast = __hip_atomic_fetch_add(ctr + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      const int pslot = __builtin_amdgcn_readfirstlane(s_bcast);
      __syncthreads();
      if (pslot < P.max_splits) {
        const int seq = unit % P.n_seq, li = unit / P.n_seq;
        const SeqDev sd = P.seqs ? P.seqs[seq] : P.one;
        visit(sd, seq, li, 0, sd.pos, pslot == 0, pslot, ctr);
      }
      if (fresh_left) {
        if (tid == 0)
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
  }
}

}  // namespace g2b
