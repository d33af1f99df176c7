// g2b_model.hip - model_forward (/root/reference/src/l5_model.c:461-606) on
// the device: the G2BX weight blob resident in HBM, the rest of the layer as
// small kernels (embedding row, rmsnorm, SiLU * up, residual add), the
// weight GEMVs of g2b_matmul.hip and the decode-attention path of k_layer
// (through g2b_attn_forward), all in order on the context's stream.
//
// The element-wise kernels are HBM/latency-trivial next to the GEMVs; they
// follow the reference's arithmetic: rmsnorm (l3_math.c:21-50) as
// o = (x * w) * (1 / sqrtf(sum(x^2) / n + eps)) with the sum in another order
// (tree, fp32), silu (l3_math.c:57-62) as x / (1 + expf(-x)) then * up
// (l5_model.c:594-595), embedding rows dequantised exactly as gguf_dequant
// (l2_codec.c:55-82: scale * (q - 8) for Q4_0, scale * q for Q8_0).
#include <hip/hip_runtime.h>

#include <string.h>

#include <vector>

#include "g2b_attn.h"
#include "g2b_internal.h"
#include "g2b_matmul.h"
#include "g2b_model.h"

namespace g2b {
namespace {

constexpr int kEwThreads = 256;

// gguf_dequant of one embedding row (l2_codec.c:186-199) for the types the
// device supports; the products are exact in fp32.  The token comes from
// device memory (checked against vocab on the host before it is written).
__global__ void k_embed_row(float *out, const uint8_t *emb, const int32_t *tok, uint64_t stride,
                            int32_t type, int32_t n) {
  const uint8_t *row = emb + (size_t)(*tok) * stride;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    float v;
    if (type == kTypeF32) {
      v = reinterpret_cast<const float *>(row)[i];
    } else if (type == 1) {  // F16
      v = half_bits_to_f32(reinterpret_cast<const uint16_t *>(row)[i]);
    } else if (type == kTypeQ8_0) {
      const uint8_t *b = row + (size_t)(i / 32) * 34;
      const float s = half_bits_to_f32((uint32_t)b[0] | (uint32_t)b[1] << 8);
      v = s * (float)(int8_t)b[2 + i % 32];
    } else if (type == kTypeQ4_1) {  // deq_q4_1 (l2_codec.c:65-75): s*q + m
      const uint8_t *b = row + (size_t)(i / 32) * 20;
      const float s = half_bits_to_f32((uint32_t)b[0] | (uint32_t)b[1] << 8);
      const float mn = half_bits_to_f32((uint32_t)b[2] | (uint32_t)b[3] << 8);
      const int j = i % 32;
      const int q = j < 16 ? (b[4 + j] & 0x0f) : (b[4 + j - 16] >> 4);
      v = s * (float)q + mn;
    } else {  // Q4_0
      const uint8_t *b = row + (size_t)(i / 32) * 18;
      const float s = half_bits_to_f32((uint32_t)b[0] | (uint32_t)b[1] << 8);
      const int j = i % 32;
      const int q = j < 16 ? (b[2 + j] & 0x0f) : (b[2 + j - 16] >> 4);
      v = s * (float)(q - 8);
    }
    out[i] = v;
  }
}

// rmsnorm (l3_math.c:21-50) by one workgroup of kEwThreads: o may alias x
// (the final norm runs in place): every read of x happens before the barrier
// that precedes the writes.
__global__ __launch_bounds__(kEwThreads) void k_rmsnorm(float *o, const float *x, const float *w,
                                                        int32_t n, float eps) {
  __shared__ float red[kEwThreads / 64];
  // (the fused GEMVs' order, so both give the same normalised x)
  static_assert(kEwThreads == 256, "wg256_sumsq");
  const float sum = wg256_sumsq(x, n, red);
  const float inv = 1.f / sqrtf(sum / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) o[i] = (x[i] * w[i]) * inv;
}

// silu(gate) * up (l3_math.c:57-62, l5_model.c:594-595), into gate.
__global__ void k_silu_mul(float *gate, const float *up, int32_t n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const float g = gate[i];
    const float sg = g / (1.f + expf(-g));
    gate[i] = sg * up[i];
  }
}

// x += y (l5_model.c:583, :597)
__global__ void k_add(float *x, const float *y, int32_t n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    x[i] += y[i];
}

int ew_blocks(int32_t n) { return (n + kEwThreads - 1) / kEwThreads < 1024 ? (n + kEwThreads - 1) / kEwThreads : 1024; }

// matmul_q's types with a device GEMV (g2b_matmul); embeddings: the same
// (gguf_dequant of a row).  The K-quants are refused (include/g2b_matmul.h).
bool matrix_type_ok(int32_t t) {
  return t == kTypeF32 || t == kTypeF16 || t == kTypeQ8_0 || t == kTypeQ4_0 || t == kTypeQ4_1;
}
bool embed_type_ok(int32_t t) { return matrix_type_ok(t); }

// row_stride (l5_model.c:444-446) for the supported types.
uint64_t row_stride_of(int32_t t, int32_t n) {
  switch (t) {
    case kTypeF32: return (uint64_t)n * 4u;
    case 1: return (uint64_t)n * 2u;
    case kTypeQ8_0: return (uint64_t)(n / 32) * 34u;
    case kTypeQ4_0: return (uint64_t)(n / 32) * 18u;
    case kTypeQ4_1: return (uint64_t)(n / 32) * 20u;
    default: return 0;
  }
}

}  // namespace
}  // namespace g2b

using namespace g2b;

struct g2b_model {
  g2b_ctx *ctx = nullptr;
  int32_t device = 0, n_cu = 1;
  bool fuse = true;  // fused GEMV launches where the weight types allow them
  g2b_model_cfg cfg{};
  int32_t arch = 0, flags = 0;
  std::vector<g2b_slot> slots;  // the table; offsets into dblob
  uint8_t *dblob = nullptr;
  void *kc = nullptr, *vc = nullptr;
  int32_t ctx_cap = 0;
  float *act = nullptr;  // x, xb, hb, hb2, q, k, v, logits (device)
  // step inputs: the sequence descriptor (pos) and the token, in device
  // memory so that a captured step graph reads them; pinned staging
  uint8_t *d_step = nullptr, *h_step = nullptr;
  SeqDev *d_seq = nullptr;
  int32_t *d_tok = nullptr;
  bool use_graph = false;
  // captured steps, one per position bucket: the attention of bucket b is
  // scheduled for positions up to max_pos (64, 128, 256, ... positions, the
  // last one the whole context)
  struct GraphBucket {
    int32_t max_pos;
    hipGraphExec_t exec;
    bool tried;
  };
  std::vector<GraphBucket> graphs;
  void drop_graphs() {
    for (GraphBucket &b : graphs)
      if (b.exec) (void)hipGraphExecDestroy(b.exec);
    graphs.clear();
  }
  int32_t bucket_max_pos(int32_t pos) const {
    int64_t n = 64;
    while (n < (int64_t)pos + 1) n *= 2;
    return (int32_t)(n < ctx_cap ? n : ctx_cap) - 1;
  }
  float *x = nullptr, *xb = nullptr, *hb = nullptr, *hb2 = nullptr, *q = nullptr,
        *k = nullptr, *v = nullptr, *logits = nullptr;
  // slot_get's index (l5_model.c:34-45): per layer and role, and global
  std::vector<const g2b_slot *> ix_layer, ix_global;

  const g2b_slot *get(int role, int layer) const {
    if (layer < 0) return ix_global[role];
    if (layer >= cfg.n_layers) return nullptr;
    return ix_layer[(size_t)layer * G2B_R_COUNT + role];
  }
  const uint8_t *ptr(const g2b_slot *s) const { return s ? dblob + s->off : nullptr; }
};

extern "C" {

int g2b_model_free(g2b_model *m) {
  if (!m) return G2B_EINVAL;
  if (m->ctx) {
    (void)g2b_sync(m->ctx);
    m->drop_graphs();
    if (m->h_step) (void)hipHostFree(m->h_step);
    if (m->d_step) (void)g2b_weights_free(m->ctx, m->d_step);
    if (m->kc || m->vc) (void)g2b_kv_free(m->ctx, m->kc, m->vc);
    if (m->dblob) (void)g2b_weights_free(m->ctx, m->dblob);
    if (m->act) (void)g2b_weights_free(m->ctx, m->act);
    (void)g2b_ctx_destroy(m->ctx);
  }
  delete m;
  return G2B_OK;
}

int g2b_model_load_g2bx(g2b_model **out, int32_t device, const char *path, int32_t kv_q8,
                        int32_t ctx) {
  if (!out) return G2B_EINVAL;
  *out = nullptr;
  g2b_g2bx g;
  if (int rc = g2b_g2bx_open(path, &g)) return rc;
  const g2b_model_cfg &c = g.cfg;
  auto bail = [&](int rc, g2b_model *m) {
    g2b_g2bx_close(&g);
    if (m) g2b_model_free(m);
    return rc;
  };
  if (c.dim <= 0 || c.hidden_dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 ||
      c.n_kv_heads <= 0 || c.head_dim <= 0 || c.vocab <= 0)
    return bail(G2B_EINVAL, nullptr);
  // types the device forward runs
  for (uint32_t i = 0; i < g.n_slots; i++) {
    const g2b_slot &s = g.slots[i];
    if (s.role >= G2B_R_COUNT) continue;
    const bool vec = s.role == G2B_R_OUT_NORM || s.role == G2B_R_ATTN_NORM ||
                     s.role == G2B_R_FFN_NORM || s.role == G2B_R_ATTN_Q_NORM ||
                     s.role == G2B_R_ATTN_K_NORM;
    const bool ok = vec ? s.type == kTypeF32
                        : (s.role == G2B_R_TOK_EMBD ? embed_type_ok(s.type)
                                                    : matrix_type_ok(s.type));
    if (!ok) return bail(G2B_EUNSUP, nullptr);
  }
  g2b_model *m = new g2b_model;
  m->device = device;
  {
    int n_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
      (void)hipGetLastError();
      n_cu = 1;
    }
    m->n_cu = n_cu > 0 ? n_cu : 1;
  }
  m->cfg = c;
  m->arch = g.arch;
  m->flags = g.flags;
  m->slots.assign(g.slots, g.slots + g.n_slots);
  m->ix_global.assign(G2B_R_COUNT, nullptr);
  m->ix_layer.assign((size_t)c.n_layers * G2B_R_COUNT, nullptr);
  for (const g2b_slot &s : m->slots) {
    if (s.role >= G2B_R_COUNT) continue;
    if (s.layer == 0xFFFF)
      m->ix_global[s.role] = &s;
    else if (s.layer < c.n_layers)
      m->ix_layer[(size_t)s.layer * G2B_R_COUNT + s.role] = &s;
  }
  // every slot the forward reads must hold what its role needs: the kernels
  // read rows x row_stride bytes from it (the reference trusts the file)
  {
    const uint64_t nq = (uint64_t)c.n_heads * c.head_dim, nkv = (uint64_t)c.n_kv_heads * c.head_dim;
    auto fits = [&](int role, int layer, uint64_t rows, int32_t n) {
      const g2b_slot *s = m->get(role, layer);
      if (!s) return true;  // missing: the forward reports it, as the reference does
      const bool vec = role == G2B_R_OUT_NORM || role == G2B_R_ATTN_NORM ||
                       role == G2B_R_FFN_NORM || role == G2B_R_ATTN_Q_NORM ||
                       role == G2B_R_ATTN_K_NORM;
      const uint64_t need = vec ? (uint64_t)n * 4u : rows * row_stride_of(s->type, n);
      // (the slot must also lie inside the blob: g2b_g2bx_open refuses
      // offsets that wrap, and sizes the blob to the largest slot end)
      return s->nbytes >= need && s->off <= g.data_size && s->nbytes <= g.data_size - s->off;
    };
    bool ok = fits(G2B_R_TOK_EMBD, -1, (uint64_t)c.vocab, c.dim) &&
              fits(G2B_R_OUTPUT, -1, (uint64_t)c.vocab, c.dim) &&
              fits(G2B_R_OUT_NORM, -1, 1, c.dim);
    for (int32_t L = 0; ok && L < c.n_layers; L++)
      ok = fits(G2B_R_ATTN_NORM, L, 1, c.dim) && fits(G2B_R_ATTN_Q, L, nq, c.dim) &&
           fits(G2B_R_ATTN_K, L, nkv, c.dim) && fits(G2B_R_ATTN_V, L, nkv, c.dim) &&
           fits(G2B_R_ATTN_O, L, (uint64_t)c.dim, (int32_t)nq) &&
           fits(G2B_R_ATTN_Q_NORM, L, 1, c.head_dim) && fits(G2B_R_ATTN_K_NORM, L, 1, c.head_dim) &&
           fits(G2B_R_FFN_NORM, L, 1, c.dim) && fits(G2B_R_FFN_GATE, L, (uint64_t)c.hidden_dim, c.dim) &&
           fits(G2B_R_FFN_UP, L, (uint64_t)c.hidden_dim, c.dim) &&
           fits(G2B_R_FFN_DOWN, L, (uint64_t)c.dim, c.hidden_dim);
    if (!ok) return bail(G2B_EINVAL, m);
  }
  g2b_shape sh{};
  sh.n_layers = c.n_layers;
  sh.n_heads = c.n_heads;
  sh.n_kv_heads = c.n_kv_heads;
  sh.head_dim = c.head_dim;
  sh.rope_theta = c.rope_theta;
  sh.arch = g.arch;
  sh.kv_q8 = kv_q8 ? 1 : 0;
  if (int rc = g2b_ctx_create(&m->ctx, device, &sh)) return bail(rc, m);
  // the blob, once (slot offsets stay valid)
  if (int rc = g2b_weights_upload(m->ctx, g.data, g.data_size ? g.data_size : 64,
                                  (void **)&m->dblob))
    return bail(rc, m);
  // QK-RMSNorm weights (l5_model.c:505-511), host copies from the file
  if (g.flags & G2B_F_QK_NORM) {
    for (int32_t L = 0; L < c.n_layers; L++) {
      const g2b_slot *qn = m->get(G2B_R_ATTN_Q_NORM, L), *kn = m->get(G2B_R_ATTN_K_NORM, L);
      if (!qn && !kn) continue;
      if ((qn && qn->nbytes < (uint32_t)c.head_dim * 4u) ||
          (kn && kn->nbytes < (uint32_t)c.head_dim * 4u))
        return bail(G2B_EINVAL, m);
      if (int rc = g2b_set_qk_norm(m->ctx, L,
                                   qn ? reinterpret_cast<const float *>(g.data + qn->off) : nullptr,
                                   kn ? reinterpret_cast<const float *>(g.data + kn->off) : nullptr,
                                   c.eps))
        return bail(rc, m);
    }
  }
  // model_set_ctx (l5_model.c:166-174): the clamp, then the KV
  m->ctx_cap = g2b_clamp_ctx(ctx > 0 ? ctx : c.seq_len, c.seq_len);
  if (int rc = g2b_kv_alloc(m->ctx, m->ctx_cap, &m->kc, &m->vc)) return bail(rc, m);
  const size_t nq = (size_t)c.n_heads * c.head_dim, nkv = (size_t)c.n_kv_heads * c.head_dim;
  auto up4 = [](size_t n) { return (n + 3) & ~(size_t)3; };  // 16-byte aligned pieces
  const size_t floats = up4(c.dim) * 2 + up4(c.hidden_dim) * 2 + up4(nq) + up4(nkv) * 2 +
                        up4((size_t)c.vocab);
  if (int rc = g2b_weights_upload(m->ctx, nullptr, floats * 4, (void **)&m->act))
    return bail(rc, m);
  float *p = m->act;
  m->x = p; p += up4(c.dim);
  m->xb = p; p += up4(c.dim);
  m->hb = p; p += up4(c.hidden_dim);
  m->hb2 = p; p += up4(c.hidden_dim);
  m->q = p; p += up4(nq);
  m->k = p; p += up4(nkv);
  m->v = p; p += up4(nkv);
  m->logits = p;
  if (int rc = g2b_weights_upload(m->ctx, nullptr, 64, (void **)&m->d_step)) return bail(rc, m);
  if (hipHostMalloc((void **)&m->h_step, 64, hipHostMallocDefault) != hipSuccess) {
    m->h_step = nullptr;
    (void)hipGetLastError();
    return bail(G2B_ENOMEM, m);
  }
  m->d_seq = reinterpret_cast<SeqDev *>(m->d_step);
  m->d_tok = reinterpret_cast<int32_t *>(m->d_step + 32);
  g2b_g2bx_close(&g);
  *out = m;
  return G2B_OK;
}

int g2b_model_info(const g2b_model *m, g2b_model_cfg *cfg, int32_t *arch, int32_t *flags,
                   int32_t *ctx) {
  if (!m) return G2B_EINVAL;
  if (cfg) *cfg = m->cfg;
  if (arch) *arch = m->arch;
  if (flags) *flags = m->flags;
  if (ctx) *ctx = m->ctx_cap;
  return G2B_OK;
}

g2b_ctx *g2b_model_ctx(g2b_model *m) { return m ? m->ctx : nullptr; }

int g2b_model_use_graph(g2b_model *m, int32_t on) {
  if (!m) return G2B_EINVAL;
  m->use_graph = on != 0;
  return G2B_OK;
}

int g2b_model_kv(g2b_model *m, void **kcache, void **vcache, int32_t *ctx_cap) {
  if (!m || !kcache || !vcache || !ctx_cap) return G2B_EINVAL;
  *kcache = m->kc;
  *vcache = m->vc;
  *ctx_cap = m->ctx_cap;
  return G2B_OK;
}

int g2b_model_set_fused(g2b_model *m, int32_t on) {
  if (!m) return G2B_EINVAL;
  if (m->fuse != (on != 0)) {
    m->fuse = on != 0;
    // a captured step holds the other launches: capture again
    m->drop_graphs();
  }
  return G2B_OK;
}

}  // extern "C"

namespace {

// Every launch of one decode step, reading the token and pos from the step
// inputs in device memory: the same sequence runs eagerly and is captured.
// The attention is scheduled for positions up to max_pos: the step's own pos
// when eager (one split, no combine launch at short contexts), the whole
// context when captured.
int enqueue_step(g2b_model *m, int32_t max_pos) {
  const g2b_model_cfg &c = m->cfg;
  const int32_t dim = c.dim, hid = c.hidden_dim;
  const int32_t nq = c.n_heads * c.head_dim, nkv = c.n_kv_heads * c.head_dim;
  g2b_ctx *cx = m->ctx;
  hipStream_t st = (hipStream_t)g2b_ctx_stream(cx);
#define G2B_MODEL_HIP(call)                        \
  do {                                             \
    if ((call) != hipSuccess) return G2B_EDEVICE; \
  } while (0)
#define G2B_MODEL_RC(call)      \
  do {                          \
    const int rc_ = (call);     \
    if (rc_) return rc_;        \
  } while (0)
  const g2b_slot *emb = m->get(G2B_R_TOK_EMBD, -1);
  if (!emb) return G2B_EINVAL;  // require_slot("tok_embd")
  hipLaunchKernelGGL(k_embed_row, dim3(ew_blocks(dim)), dim3(kEwThreads), 0, st, m->x,
                     m->ptr(emb), m->d_tok, row_stride_of(emb->type, dim), (int32_t)emb->type,
                     dim);
  G2B_MODEL_HIP(hipGetLastError());
  // A plain GEMV, or a fused one (launch_gemv: rmsnorm or SiLU x up on x,
  // segments sharing x, a residual added to the output).
  auto gemv = [&](float *out, const float *x, const g2b_slot *w, int32_t n, int32_t d) {
    return g2b_matmul(cx, out, x, m->ptr(w), w->type, n, d);
  };
  auto fused = [&](GemvParams p, int32_t type) {
    return launch_gemv(p, type, m->n_cu, st) == hipSuccess ? G2B_OK : G2B_EDEVICE;
  };
  auto rmsnorm = [&](float *o, const float *x, const g2b_slot *w) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kEwThreads), 0, st, o, x,
                       (const float *)m->ptr(w), dim, c.eps);
    return hipGetLastError() == hipSuccess ? G2B_OK : G2B_EDEVICE;
  };
  auto add = [&](float *x, const float *y, int32_t n) {
    hipLaunchKernelGGL(k_add, dim3(ew_blocks(n)), dim3(kEwThreads), 0, st, x, y, n);
    return hipGetLastError() == hipSuccess ? G2B_OK : G2B_EDEVICE;
  };
  for (int32_t L = 0; L < c.n_layers; L++) {
    const g2b_slot *an = m->get(G2B_R_ATTN_NORM, L);
    const g2b_slot *wq = m->get(G2B_R_ATTN_Q, L), *wk = m->get(G2B_R_ATTN_K, L),
                   *wv = m->get(G2B_R_ATTN_V, L), *wo = m->get(G2B_R_ATTN_O, L);
    const g2b_slot *fn = m->get(G2B_R_FFN_NORM, L);
    const g2b_slot *wg = m->get(G2B_R_FFN_GATE, L), *wu = m->get(G2B_R_FFN_UP, L),
                   *wd = m->get(G2B_R_FFN_DOWN, L);
    if (!an || !wq || !wk || !wv || !wo || !fn || !wg || !wu || !wd) return G2B_EINVAL;
    // rmsnorm, then Q, K, V (l5_model.c:495-503): one launch when the three
    // matrices share a type the fused GEMV takes
    if (m->fuse && wq->type == wk->type && wq->type == wv->type &&
        gemv_fusable_pro(wq->type, dim)) {
      GemvParams p{};
      p.out = m->q;
      p.out1 = m->k;
      p.out2 = m->v;
      p.x = m->x;
      p.w = m->ptr(wq);
      p.w1 = m->ptr(wk);
      p.w2 = m->ptr(wv);
      p.n = dim;
      p.d0 = nq;
      p.d01 = nq + nkv;
      p.d = nq + 2 * nkv;
      p.x_vec4 = 1;
      p.pro = kProRmsnorm;
      p.nw = (const float *)m->ptr(an);
      p.eps = c.eps;
      G2B_MODEL_RC(fused(p, wq->type));
    } else {
      G2B_MODEL_RC(rmsnorm(m->xb, m->x, an));
      G2B_MODEL_RC(gemv(m->q, m->xb, wq, dim, nq));
      G2B_MODEL_RC(gemv(m->k, m->xb, wk, dim, nkv));
      G2B_MODEL_RC(gemv(m->v, m->xb, wv, dim, nkv));
    }
    // QK-RMSNorm, RoPE, KV append, attention over the positions up to pos;
    // the output over q
    G2B_MODEL_RC(attn_forward_device_seq(cx, L, m->d_seq, max_pos, m->q, m->k, m->v));
    // Wo and the residual (l5_model.c:580-583)
    if (m->fuse && gemv_fusable(wo->type, nq)) {
      GemvParams p{};
      p.out = m->x;
      p.res = m->x;
      p.x = m->q;
      p.w = m->ptr(wo);
      p.n = nq;
      p.d = dim;
      p.x_vec4 = 1;
      G2B_MODEL_RC(fused(p, wo->type));
    } else {
      G2B_MODEL_RC(gemv(m->xb, m->q, wo, nq, dim));
      G2B_MODEL_RC(add(m->x, m->xb, dim));
    }
    // rmsnorm, gate and up (l5_model.c:585-593)
    if (m->fuse && wg->type == wu->type && gemv_fusable_pro(wg->type, dim)) {
      GemvParams p{};
      p.out = m->hb;
      p.out1 = m->hb2;
      p.x = m->x;
      p.w = m->ptr(wg);
      p.w1 = m->ptr(wu);
      p.n = dim;
      p.d0 = hid;
      p.d01 = 2 * hid;
      p.d = 2 * hid;
      p.x_vec4 = 1;
      p.pro = kProRmsnorm;
      p.nw = (const float *)m->ptr(fn);
      p.eps = c.eps;
      G2B_MODEL_RC(fused(p, wg->type));
    } else {
      G2B_MODEL_RC(rmsnorm(m->xb, m->x, fn));
      G2B_MODEL_RC(gemv(m->hb, m->xb, wg, dim, hid));
      G2B_MODEL_RC(gemv(m->hb2, m->xb, wu, dim, hid));
    }
    // SiLU(gate) x up, down and the residual (l5_model.c:594-597)
    if (m->fuse && gemv_fusable_pro(wd->type, hid)) {
      GemvParams p{};
      p.out = m->x;
      p.res = m->x;
      p.x = m->hb;
      p.x2 = m->hb2;
      p.pro = kProSiluMul;
      p.w = m->ptr(wd);
      p.n = hid;
      p.d = dim;
      p.x_vec4 = 1;
      G2B_MODEL_RC(fused(p, wd->type));
    } else {
      hipLaunchKernelGGL(k_silu_mul, dim3(ew_blocks(hid)), dim3(kEwThreads), 0, st, m->hb, m->hb2,
                         hid);
      G2B_MODEL_HIP(hipGetLastError());
      G2B_MODEL_RC(gemv(m->xb, m->hb, wd, hid, dim));
      G2B_MODEL_RC(add(m->x, m->xb, dim));
    }
  }
  // final rmsnorm and the logits (l5_model.c:600-605)
  const g2b_slot *on = m->get(G2B_R_OUT_NORM, -1);
  if (!on) return G2B_EINVAL;
  const g2b_slot *out = m->get(G2B_R_OUTPUT, -1);
  if (!out) out = emb;  // tied embeddings (l5_model.c:602)
  // (an output matrix the int8 matrix cores take - 1024-element rows, many
  // of them - gets the rmsnorm as its own launch and the plain product:
  // normalising and digitising x in every workgroup of the product cost more
  // than the launch)
  if (m->fuse && gemv_fusable_pro(out->type, dim) && !gemv_mma_plain(out->type, dim, c.vocab)) {
    GemvParams p{};
    p.out = m->logits;
    p.x = m->x;
    p.w = m->ptr(out);
    p.n = dim;
    p.d = c.vocab;
    p.x_vec4 = 1;
    p.pro = kProRmsnorm;
    p.nw = (const float *)m->ptr(on);
    p.eps = c.eps;
    G2B_MODEL_RC(fused(p, out->type));
  } else {
    G2B_MODEL_RC(rmsnorm(m->x, m->x, on));
    G2B_MODEL_RC(gemv(m->logits, m->x, out, dim, c.vocab));
  }
#undef G2B_MODEL_HIP
#undef G2B_MODEL_RC
  return G2B_OK;
}

}  // namespace

extern "C" {

int g2b_model_forward(g2b_model *m, int32_t token, int32_t pos, float *logits) {
  if (!m || !logits) return G2B_EINVAL;
  const g2b_model_cfg &c = m->cfg;
  // the forward's own checks (l5_model.c:469-483)
  if (pos < 0 || pos >= m->ctx_cap || token < 0 || token >= c.vocab) {
    memset(logits, 0, (size_t)c.vocab * sizeof(float));
    return pos < 0 || pos >= m->ctx_cap ? G2B_EPOS : G2B_EINVAL;
  }
  hipStream_t st = (hipStream_t)g2b_ctx_stream(m->ctx);
  if (hipSetDevice(m->device) != hipSuccess) return G2B_EDEVICE;
  // step inputs (the previous step's copies have completed: every forward
  // ends with a stream synchronisation)
  SeqDev sd{};
  sd.pos = pos;
  sd.ctx_cap = m->ctx_cap;
  sd.k = (uint8_t *)m->kc;
  sd.v = (uint8_t *)m->vc;
  memcpy(m->h_step, &sd, sizeof sd);
  memcpy(m->h_step + 32, &token, sizeof token);
  if (hipMemcpyAsync(m->d_step, m->h_step, 64, hipMemcpyHostToDevice, st) != hipSuccess)
    return G2B_EDEVICE;
  g2b_model::GraphBucket *bucket = nullptr;
  if (m->use_graph) {
    const int32_t bmax = m->bucket_max_pos(pos);
    for (g2b_model::GraphBucket &b : m->graphs)
      if (b.max_pos == bmax) bucket = &b;
    if (!bucket) {
      m->graphs.push_back({bmax, nullptr, false});
      bucket = &m->graphs.back();
    }
  }
  if (bucket && bucket->exec) {
    if (hipGraphLaunch(bucket->exec, st) != hipSuccess) return G2B_EDEVICE;
  } else {
    if (int rc = enqueue_step(m, pos)) return rc;
    if (bucket && !bucket->tried) {
      // capture this bucket's step once (nothing runs while capturing); on
      // any failure the bucket keeps running eagerly
      bucket->tried = true;
      hipGraph_t graph = nullptr;
      // (the bucket's attention buffers first: the capture must not allocate)
      if (attn_reserve_device_seq(m->ctx, bucket->max_pos, m->q, m->k, m->v) == G2B_OK &&
          hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed) == hipSuccess) {
        const int rc = enqueue_step(m, bucket->max_pos);
        const hipError_t e = hipStreamEndCapture(st, &graph);
        if (rc == G2B_OK && e == hipSuccess && graph &&
            hipGraphInstantiate(&bucket->exec, graph, nullptr, nullptr, 0) != hipSuccess)
          bucket->exec = nullptr;
        if (graph) (void)hipGraphDestroy(graph);
      }
      (void)hipGetLastError();
    }
  }
  if (hipMemcpyAsync(logits, m->logits, (size_t)c.vocab * 4, hipMemcpyDeviceToHost, st) !=
      hipSuccess)
    return G2B_EDEVICE;
  if (hipStreamSynchronize(st) != hipSuccess) return G2B_EDEVICE;
  return G2B_OK;
}

}  // extern "C"
