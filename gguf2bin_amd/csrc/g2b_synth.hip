// g2b_synth.hip - device generation of the seeded synthetic KV used by the
// benchmark and the full-size tests (no reference counterpart).  The stream
// definition matches oracle/orc_rng.c so that small cases can be checked
// against the host generator.
#include <algorithm>

#include "g2b_internal.h"

namespace g2b {

constexpr uint64_t kGamma = 0x9e3779b97f4a7c15ull;

__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t stream_seed(uint64_t base, int32_t seq, int32_t layer,
                                                int32_t tensor) {
  uint64_t z = mix64(base ^ ((uint64_t)tensor * 0xD1B54A32D192ED03ull));
  z = mix64(z + (uint64_t)(seq + 1) * kGamma);
  return mix64(z + (uint64_t)(layer + 1) * 0xC2B2AE3D27D4EB4Full);
}

// Elements 2j and 2j+1 of stream `seed`.
__device__ inline void normal_pair(uint64_t seed, uint64_t j, float &even, float &odd) {
  const uint64_t z1 = mix64(seed + (2 * j + 1) * kGamma);
  const uint64_t z2 = mix64(seed + (2 * j + 2) * kGamma);
  const double u1 = (double)((z1 >> 11) + 1ull) * (1.0 / 9007199254740992.0);
  const double u2 = (double)((z2 >> 11) + 1ull) * (1.0 / 9007199254740992.0);
  const double r = sqrt(-2.0 * log(u1));
  const double a = 6.283185307179586476925286766559 * u2;
  even = (float)(r * cos(a));
  odd = (float)(r * sin(a));
}

__device__ inline float normal_elem(uint64_t seed, uint64_t i) {
  float e, o;
  normal_pair(seed, i >> 1, e, o);
  return (i & 1) ? o : e;
}

__global__ __launch_bounds__(kThreads) void k_synth_normal(float *out, uint64_t n,
                                                           uint64_t seed) {
  const uint64_t j = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (2 * j >= n) return;
  float e, o;
  normal_pair(seed, j, e, o);
  out[2 * j] = e;
  if (2 * j + 1 < n) out[2 * j + 1] = o;
}

constexpr int kSynthRowsPerBlock = 8;

// grid (ceil(n_pos / rows), n_layers): each block draws, rotates and stores
// kSynthRowsPerBlock rows of K and V through append_row.
__global__ __launch_bounds__(kThreads) void k_synth_fill(SynthParams p) {
  extern __shared__ float lds[];
  const int nkv = p.sh.n_kv_heads * p.sh.head_dim;
  float *kraw = lds, *vraw = lds + nkv, *kr = lds + 2 * nkv;
  const int li = blockIdx.y, layer = p.layer0 + li;
  const uint64_t sk = stream_seed(p.base_seed, p.seq, layer, 0);
  const uint64_t sv = stream_seed(p.base_seed, p.seq, layer, 1);
  const uint64_t ss = stream_seed(p.base_seed, p.seq, layer, 5);
  SeqDev sd;
  sd.pos = 0;
  sd.ctx_cap = p.ctx_cap;
  sd.pad0 = sd.pad1 = 0;
  sd.k = p.k;
  sd.v = p.v;
  for (int rr = 0; rr < kSynthRowsPerBlock; rr++) {
    const int r = blockIdx.x * kSynthRowsPerBlock + rr;
    if (r >= p.n_pos) break;  // uniform across the block
    const int pos = p.pos0 + r;
    const uint64_t base = (uint64_t)pos * (uint64_t)nkv;
    float scale = 1.f;
    if (p.sel_threshold < INFINITY && normal_elem(ss, (uint64_t)pos) > p.sel_threshold)
      scale = 8.f;
    // nkv is even (head_dim is), so row t starts on a pair boundary
    for (int e2 = threadIdx.x; 2 * e2 < nkv; e2 += blockDim.x) {
      const uint64_t j = (base >> 1) + (uint64_t)e2;
      float a, b;
      normal_pair(sk, j, a, b);
      kraw[2 * e2] = a * scale;
      kraw[2 * e2 + 1] = b * scale;
      normal_pair(sv, j, a, b);
      vraw[2 * e2] = a;
      vraw[2 * e2 + 1] = b;
    }
    __syncthreads();
    append_row(p.sh, sd, layer, pos, kraw, vraw, nullptr, nullptr, p.rope, NormDev{}, kr,
               nullptr);  // synthetic rows stand for post-norm k: no QK-RMSNorm
    __syncthreads();
  }
}

hipError_t launch_synth_normal(float *out, uint64_t n, uint64_t seed, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const uint64_t pairs = (n + 1) / 2;
  const uint64_t blocks = (pairs + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(k_synth_normal, dim3((unsigned)blocks), dim3(kThreads), 0, s, out, n,
                     seed);
  return hipGetLastError();
}

hipError_t launch_synth_fill(const SynthParams &p, int n_layers, hipStream_t s) {
  const int nkv = p.sh.n_kv_heads * p.sh.head_dim;
  const size_t lds = (size_t)3 * nkv * sizeof(float);
  dim3 grid((p.n_pos + kSynthRowsPerBlock - 1) / kSynthRowsPerBlock, n_layers);
  hipLaunchKernelGGL(k_synth_fill, grid, dim3(kThreads), lds, s, p);
  return hipGetLastError();
}

__global__ __launch_bounds__(kThreads) void k_copy16(uint4 *dst, const uint4 *src,
                                                      uint64_t n16) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    dst[i] = src[i];
}

hipError_t launch_copy16(void *dst, const void *src, uint64_t n16, hipStream_t s) {
  if (n16 == 0) return hipSuccess;
  const uint64_t blocks = std::min<uint64_t>((n16 + kThreads - 1) / kThreads, 256u * 64u);
  hipLaunchKernelGGL(k_copy16, dim3((unsigned)blocks), dim3(kThreads), 0, s, (uint4 *)dst,
                     (const uint4 *)src, n16);
  return hipGetLastError();
}

}  // namespace g2b

extern "C" uint64_t g2b_stream_seed(uint64_t base, int32_t seq, int32_t layer, int32_t tensor) {
  return g2b::stream_seed(base, seq, layer, tensor);
}
