/*
 * ref_driver.c - drives the COMPILED REFERENCE for golden vectors.
 * TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile (target `ref`) into
 * oracle/_ref/ from the reference sources where they lie under
 * /root/reference; nothing of the reference is copied into this repository.
 * The reference's path lives in static helpers and inline in model_forward,
 * so this translation unit includes src/l5_model.c to reach them.
 *
 * ref_forward_case() builds an in-memory one-or-more-layer model whose
 * weights make model_forward run exactly the decode-attention path on chosen
 * inputs:
 *   - dim = nq + 2*nkv, token embeddings are the caller's rows (F32);
 *   - attn_norm = 1, so xb = rmsnorm(x) (returned to the caller: it is the
 *     q|k|v the reference actually uses);
 *   - Wq/Wk/Wv are F32 0/1 selector matrices, so q, k, v are exact slices of
 *     xb (the F32 GEMV of l3_math.c:17-20 adds exact zeros);
 *   - Wo and the FFN are zero, so every layer sees the same xb.
 * Positions [0, n_pre) are prefilled with the reference's own apply_rope and
 * kv_store; positions [n_pre, n_pre+n_fwd) go through model_forward.
 * ref_forward_case_qkn() adds attn_q_norm / attn_k_norm slots and F_QK_NORM
 * (l5_model.c:505-511); its prefill applies the reference's qk_rmsnorm to
 * each k row before apply_rope, as model_forward would.
 */
#define _POSIX_C_SOURCE 200809L
#define _DEFAULT_SOURCE
#include <time.h>

#include "l5_model.c"

void ref_q8_quant_row(const f32 *src, u8 *dst, i32 n) { q8_quant_row(src, dst, n); }
void ref_q8_dequant_row(const u8 *src, f32 *out, i32 n) { q8_dequant_row(src, out, n); }
u16 ref_f32_to_half(f32 f) { return f32_to_half(f); }
f32 ref_half_to_float(u16 h) { return half_to_float(h); }
void ref_f32_to_half_n(const f32 *x, u16 *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = f32_to_half(x[i]);
}
void ref_half_to_float_n(const u16 *h, f32 *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = half_to_float(h[i]);
}
void ref_softmax(f32 *x, i32 n) { softmax(x, n); }
void ref_qk_rmsnorm(f32 *x, const f32 *w, i32 n_heads, i32 hd, f32 eps) {
  qk_rmsnorm(x, w, n_heads, hd, eps);
}
void ref_rope(i32 arch, f32 *x, i32 len, i32 pos, i32 hd, f32 theta) {
  Model m;
  memset(&m, 0, sizeof m);
  m.arch = (u8)arch;
  apply_rope(&m, x, len, pos, hd, theta);
}

static void put_slot(Slot *sl, u32 *ns, u64 *cur, u8 role, u16 layer, u64 nfloats) {
  Slot *s = &sl[*ns];
  s->role = role;
  s->layer = layer;
  s->type = T_F32;
  s->nbytes = (u32)(nfloats * 4u);
  s->off = *cur;
  *cur = ALIGN64(*cur + nfloats * 4u);
  (*ns)++;
}

int ref_forward_case_qkn(i32 n_layers, i32 n_heads, i32 n_kv_heads, i32 head_dim, f32 theta,
                         i32 arch, i32 kv_q8, i32 ctx_cap,
                         i32 n_pre, const f32 *k_pre, const f32 *v_pre,
                         i32 n_fwd, const f32 *x_rows,
                         const f32 *q_norm, const f32 *k_norm, f32 eps,
                         f32 *xb_out, f32 *out_per_step, f32 *att_out,
                         u8 *kc_out, u8 *vc_out) {
  const i32 hd = head_dim, nq = n_heads * hd, nkv = n_kv_heads * hd;
  const i32 dim = nq + 2 * nkv, hid = 32, vocab = n_fwd > 0 ? n_fwd : 1;
  Model m;
  memset(&m, 0, sizeof m);
  m.fd = -1;
  m.swap_fd = -1;
  m.c.dim = dim;
  m.c.hidden_dim = hid;
  m.c.n_layers = n_layers;
  m.c.n_heads = n_heads;
  m.c.n_kv_heads = n_kv_heads;
  m.c.vocab = vocab;
  m.c.seq_len = ctx_cap;
  m.c.head_dim = hd;
  m.c.eps = eps;
  m.c.rope_theta = theta;
  m.arch = (u8)arch;
  m.flags = (kv_q8 ? F_KV_Q8 : 0) | ((q_norm || k_norm) ? F_QK_NORM : 0);

  u32 max_slots = 2 + (u32)n_layers * 11u;
  Slot *sl = calloc(max_slots, sizeof(Slot));
  u32 ns = 0;
  u64 cur = 0;
  put_slot(sl, &ns, &cur, R_TOK_EMBD, 0xFFFF, (u64)vocab * dim);
  put_slot(sl, &ns, &cur, R_OUT_NORM, 0xFFFF, (u64)dim);
  for (i32 L = 0; L < n_layers; L++) {
    put_slot(sl, &ns, &cur, R_ATTN_NORM, (u16)L, (u64)dim);
    put_slot(sl, &ns, &cur, R_ATTN_Q, (u16)L, (u64)nq * dim);
    put_slot(sl, &ns, &cur, R_ATTN_K, (u16)L, (u64)nkv * dim);
    put_slot(sl, &ns, &cur, R_ATTN_V, (u16)L, (u64)nkv * dim);
    put_slot(sl, &ns, &cur, R_ATTN_O, (u16)L, (u64)dim * nq);
    put_slot(sl, &ns, &cur, R_FFN_NORM, (u16)L, (u64)dim);
    put_slot(sl, &ns, &cur, R_FFN_GATE, (u16)L, (u64)hid * dim);
    put_slot(sl, &ns, &cur, R_FFN_UP, (u16)L, (u64)hid * dim);
    put_slot(sl, &ns, &cur, R_FFN_DOWN, (u16)L, (u64)dim * hid);
    if (q_norm) put_slot(sl, &ns, &cur, R_ATTN_Q_NORM, (u16)L, (u64)hd);
    if (k_norm) put_slot(sl, &ns, &cur, R_ATTN_K_NORM, (u16)L, (u64)hd);
  }
  u8 *blob = calloc(1, (size_t)cur + 64);
  if (!sl || !blob) { free(sl); free(blob); return -1; }
  m.slots = sl;
  m.n_slots = ns;
  m.data = blob;
  m.data_size = (size_t)cur;
  m.own_data = 0;

  for (u32 i = 0; i < ns; i++) {
    f32 *w = (f32 *)(blob + sl[i].off);
    u64 nf = sl[i].nbytes / 4u;
    switch (sl[i].role) {
      case R_TOK_EMBD:
        if (n_fwd > 0) memcpy(w, x_rows, (size_t)n_fwd * dim * 4u);
        break;
      case R_OUT_NORM: case R_ATTN_NORM: case R_FFN_NORM:
        for (u64 j = 0; j < nf; j++) w[j] = 1.f;
        break;
      case R_ATTN_Q:
        for (i32 r = 0; r < nq; r++) w[(size_t)r * dim + r] = 1.f;
        break;
      case R_ATTN_K:
        for (i32 r = 0; r < nkv; r++) w[(size_t)r * dim + nq + r] = 1.f;
        break;
      case R_ATTN_V:
        for (i32 r = 0; r < nkv; r++) w[(size_t)r * dim + nq + nkv + r] = 1.f;
        break;
      case R_ATTN_Q_NORM:
        memcpy(w, q_norm + (size_t)sl[i].layer * hd, (size_t)hd * 4u);
        break;
      case R_ATTN_K_NORM:
        memcpy(w, k_norm + (size_t)sl[i].layer * hd, (size_t)hd * 4u);
        break;
      default:
        break; /* Wo and FFN stay zero */
    }
  }
  build_index(&m);
  if (model_set_ctx(&m, ctx_cap)) { free(blob); model_free(&m); return -2; }
  size_t half_bytes = kv_q8 ? (size_t)n_layers * ctx_cap * kv_q8_rowsize(nkv)
                            : (size_t)n_layers * ctx_cap * (size_t)nkv * 4u;
  if (kv_q8) { memset(m.kcq, 0, half_bytes); memset(m.vcq, 0, half_bytes); }
  else { memset(m.kcache, 0, half_bytes); memset(m.vcache, 0, half_bytes); }

  f32 *tmp = malloc((size_t)nkv * 4u);
  for (i32 t = 0; t < n_pre; t++)
    for (i32 L = 0; L < n_layers; L++) {
      memcpy(tmp, k_pre + (size_t)t * nkv, (size_t)nkv * 4u);
      if (k_norm) qk_rmsnorm(tmp, k_norm + (size_t)L * hd, n_kv_heads, hd, eps);
      apply_rope(&m, tmp, nkv, t, hd, theta);
      kv_store(&m, L, t, tmp, v_pre + (size_t)t * nkv);
    }
  free(tmp);

  f32 *ones = malloc((size_t)dim * 4u);
  f32 *logits = malloc((size_t)vocab * 4u);
  for (i32 j = 0; j < dim; j++) ones[j] = 1.f;
  f32 *qbuf = m.buf + 3 * dim + 2 * hid; /* q region, see model_forward :485-486 */
  for (i32 i = 0; i < n_fwd; i++) {
    rmsnorm(xb_out + (size_t)i * dim, (f32 *)(x_rows + (size_t)i * dim), ones, dim, m.c.eps);
    model_forward(&m, i, n_pre + i, logits);
    memcpy(out_per_step + (size_t)i * nq, qbuf, (size_t)nq * 4u);
  }
  if (n_fwd > 0 && att_out)
    memcpy(att_out, qbuf + nq + 2 * nkv, (size_t)n_heads * ctx_cap * 4u);
  if (kc_out) memcpy(kc_out, kv_q8 ? (void *)m.kcq : (void *)m.kcache, half_bytes);
  if (vc_out) memcpy(vc_out, kv_q8 ? (void *)m.vcq : (void *)m.vcache, half_bytes);
  free(ones);
  free(logits);
  model_free(&m);
  free(blob);
  return 0;
}

int ref_forward_case(i32 n_layers, i32 n_heads, i32 n_kv_heads, i32 head_dim, f32 theta,
                     i32 arch, i32 kv_q8, i32 ctx_cap,
                     i32 n_pre, const f32 *k_pre, const f32 *v_pre,
                     i32 n_fwd, const f32 *x_rows,
                     f32 *xb_out, f32 *out_per_step, f32 *att_out,
                     u8 *kc_out, u8 *vc_out) {
  return ref_forward_case_qkn(n_layers, n_heads, n_kv_heads, head_dim, theta, arch, kv_q8,
                              ctx_cap, n_pre, k_pre, v_pre, n_fwd, x_rows, NULL, NULL, 1e-6f,
                              xb_out, out_per_step, att_out, kc_out, vc_out);
}

/* The reference's RAM budgeting on an in-memory Model with the given config
 * (no tokenizer, no weights): est_for (l5_model.c:174-187) and
 * model_auto_budget (:218-230), which allocates the runtime through
 * model_set_ctx; the chosen context and KV mode are read back and the
 * runtime is freed. */
static void budget_model(Model *m, i32 dim, i32 hid, i32 n_layers, i32 n_heads, i32 n_kv_heads,
                         i32 vocab, i32 seq_len, i32 head_dim, int q8) {
  memset(m, 0, sizeof *m);
  m->c.dim = dim;
  m->c.hidden_dim = hid;
  m->c.n_layers = n_layers;
  m->c.n_heads = n_heads;
  m->c.n_kv_heads = n_kv_heads;
  m->c.vocab = vocab;
  m->c.seq_len = seq_len;
  m->c.head_dim = head_dim;
  m->flags = q8 ? F_KV_Q8 : 0;
#if !defined(_WIN32)
  m->fd = -1;
  m->swap_fd = -1;
#endif
}
u64 ref_est_for(i32 dim, i32 hid, i32 n_layers, i32 n_heads, i32 n_kv_heads, i32 vocab,
                i32 seq_len, i32 head_dim, i32 ctx, int q8) {
  Model m;
  budget_model(&m, dim, hid, n_layers, n_heads, n_kv_heads, vocab, seq_len, head_dim, q8);
  return est_for(&m, ctx, q8);
}
int ref_auto_budget(i32 dim, i32 hid, i32 n_layers, i32 n_heads, i32 n_kv_heads, i32 vocab,
                    i32 seq_len, i32 head_dim, int q8, u64 max_ram, i32 *ctx_out, i32 *q8_out) {
  Model m;
  budget_model(&m, dim, hid, n_layers, n_heads, n_kv_heads, vocab, seq_len, head_dim, q8);
  const int rc = model_auto_budget(&m, max_ram);
  *ctx_out = m.ctx;
  *q8_out = (m.flags & F_KV_Q8) ? 1 : 0;
  free_rt(&m);
  return rc;
}

/* The reference's G2BX loader (model_load_g2bx, l5_model.c:393-408) on a file:
 * its parsed ModelCfg (40 packed bytes), arch, flags, slot count and packed
 * 16-byte slots (at most max_slots copied).  0 on success. */
int ref_g2bx_info(const char *path, u8 *cfg40, int *arch, int *flags, u32 *n_slots,
                  u8 *slots16, u32 max_slots) {
  Model m;
  if (model_load_g2bx(path, &m)) return -1;
  memcpy(cfg40, &m.c, sizeof m.c);
  *arch = m.arch;
  *flags = m.flags;
  *n_slots = m.n_slots;
  for (u32 i = 0; i < m.n_slots && i < max_slots; i++) memcpy(slots16 + 16 * i, &m.slots[i], 16);
  model_free(&m);
  return 0;
}

/* model_forward (l5_model.c:461-606) over tokens[0..n) at positions 0..n-1
 * of a G2BX file, KV in Q8_0 when kv_q8, context ctx (<= 0: seq_len):
 * logits of every step into out[n][vocab].  0 on success. */
/* Loads a G2BX file and runs model_forward over tokens at positions 0..n-1.
 * secs (may be NULL) receives the wall time of the token loop alone
 * (CLOCK_MONOTONIC), without the load and the KV allocation. */
int ref_model_forward_g2bx(const char *path, int kv_q8, int ctx, const i32 *tokens, int n,
                           f32 *out, double *secs) {
  Model m;
  if (model_load_g2bx(path, &m)) return -1;
  if (kv_q8) m.flags |= F_KV_Q8;
  if (model_set_ctx(&m, ctx > 0 ? ctx : m.c.seq_len)) {
    model_free(&m);
    return -2;
  }
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  for (int i = 0; i < n; i++) model_forward(&m, tokens[i], i, out + (size_t)i * m.c.vocab);
  clock_gettime(CLOCK_MONOTONIC, &t1);
  if (secs) *secs = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
  model_free(&m);
  return 0;
}

/* model_forward over tokens at positions pos0..pos0+n-1 of a G2BX file whose
 * KV positions [0, pos0) are given as bytes (kbytes, vbytes: the K and V
 * caches [n_layers][ctx][row] in the mode kv_q8 selects, ctx = the model's
 * effective context after model_set_ctx(ctx), which must equal cap): the
 * reference's own decode step at a long context, without a prefill through
 * pos0 forwards.  Logits of every step into out[n][vocab]; secs (may be NULL)
 * receives the wall time of the token loop alone (CLOCK_MONOTONIC). */
int ref_model_forward_g2bx_kv(const char *path, int kv_q8, int ctx, int cap, const u8 *kbytes,
                              const u8 *vbytes, int pos0, const i32 *tokens, int n, f32 *out,
                              double *secs) {
  Model m;
  if (model_load_g2bx(path, &m)) return -1;
  if (kv_q8) m.flags |= F_KV_Q8;
  if (model_set_ctx(&m, ctx > 0 ? ctx : m.c.seq_len) || m.ctx != cap) {
    model_free(&m);
    return -2;
  }
  const i32 nkv = m.c.n_kv_heads * m.c.head_dim;
  const size_t row = kv_q8 ? kv_q8_rowsize(nkv) : (size_t)nkv * sizeof(f32);
  const size_t nbytes = (size_t)m.c.n_layers * (size_t)m.ctx * row;
  memcpy(kv_q8 ? (void *)m.kcq : (void *)m.kcache, kbytes, nbytes);
  memcpy(kv_q8 ? (void *)m.vcq : (void *)m.vcache, vbytes, nbytes);
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  for (int i = 0; i < n; i++) model_forward(&m, tokens[i], pos0 + i, out + (size_t)i * m.c.vocab);
  clock_gettime(CLOCK_MONOTONIC, &t1);
  if (secs) *secs = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
  model_free(&m);
  return 0;
}
