// g2b_append.hip - RoPE + KV append for gfx950.
//
// Replaces /root/reference/src/l5_model.c:505-516: QK-RMSNorm when the layer
// has norm weights (l3_math.c:107-114), apply_rope on q and on the new k
// (l5_model.c:448-452, l3_math.c:64-102), then kv_store
// (l5_model.c:235-247) which memcpy's F32 rows or quantises Q8_0 rows
// (l5_model.c:49-59).  The cos/sin table comes from the host C library (the
// same powf/cosf/sinf the reference calls), so rotated values and therefore
// the stored bytes are bit-exact; the quantiser follows the reference
// operation by operation (IEEE division, round half away from zero,
// truncating fp16 scale).  This work is two rows per (sequence, layer), so
// the kernel favours plain code over speed: one workgroup per row pair.
#include "g2b_internal.h"

namespace g2b {

// LDS: kr[nkv], then inv[n_heads]
__global__ __launch_bounds__(kThreads) void k_append_batch(AppendParams p) {
  extern __shared__ float kr[];
  const int seq = blockIdx.x, li = blockIdx.y;
  const SeqDev sd = p.seqs ? p.seqs[seq] : p.one;
  const size_t slot = (size_t)li * (size_t)p.n_seq + (size_t)seq;
  const size_t nq = (size_t)p.sh.n_heads * p.sh.head_dim;
  const size_t nkv = (size_t)p.sh.n_kv_heads * p.sh.head_dim;
  append_row(p.sh, sd, p.layer0 + li, sd.pos, p.k_in + slot * nkv, p.v_in + slot * nkv,
             p.q_in + slot * nq, p.q_rot + slot * nq, p.rope, p.norm, kr, kr + nkv);
}

__global__ __launch_bounds__(kThreads) void k_append_rows(AppendParams p, int layer) {
  extern __shared__ float kr[];
  const int r = blockIdx.x;
  const size_t nkv = (size_t)p.sh.n_kv_heads * p.sh.head_dim;
  append_row(p.sh, p.one, layer, p.pos0 + r, p.k_in + (size_t)r * nkv,
             p.v_in + (size_t)r * nkv, nullptr, nullptr, p.rope, p.norm, kr, kr + nkv);
}

static size_t append_lds_bytes(const ShapeDev &sh) {
  return ((size_t)sh.n_kv_heads * sh.head_dim + (size_t)sh.n_heads) * sizeof(float);
}

hipError_t launch_append_batch(const AppendParams &p, int n_layers, hipStream_t s) {
  const size_t lds = append_lds_bytes(p.sh);
  hipLaunchKernelGGL(k_append_batch, dim3(p.n_seq, n_layers), dim3(kThreads), lds, s, p);
  return hipGetLastError();
}

hipError_t launch_append_rows(const AppendParams &p, int layer, int n_rows, hipStream_t s) {
  const size_t lds = append_lds_bytes(p.sh);
  hipLaunchKernelGGL(k_append_rows, dim3(n_rows), dim3(kThreads), lds, s, p, layer);
  return hipGetLastError();
}

}  // namespace g2b
