/*
 * g2b_c_caller.c - a plain C99 program that drives the decode-attention ABI
 * the way gguf2bin2's model_forward drives its attention: one context per
 * Model, the KV allocated where alloc_rt allocates it, then for every token
 * and layer one call with q, k, v in host memory, the output written over q
 * (/root/reference/src/l5_model.c:113-149 for the KV, :493-578 for the layer
 * loop and the attention block this call replaces).  Built with
 * `gcc -std=c99 -Wall -Werror` against include/g2b_attn.h only and linked
 * to libg2b_attn.so; tests/test_gpu_c_caller.py runs it and checks it
 * against the CPU oracle.
 *
 *   g2b_c_caller IN OUT
 *
 * IN:  int32 n_layers, n_heads, n_kv_heads, head_dim, arch, kv_q8, ctx_cap,
 *      n_tokens, with_qk_norm; float32 rope_theta, eps;
 *      with_qk_norm: float32 [n_layers][2][head_dim] norm weights (q, k);
 *      then for token t = 0..n_tokens-1 (pos = t) and layer L:
 *      float32 q[nq], k[nkv], v[nkv] (pre-norm, pre-RoPE).
 * OUT: float32 out[n_tokens][n_layers][nq], then the K cache bytes and the V
 *      cache bytes ([n_layers][ctx_cap][row] each).
 * Exit status 0 on success; a G2B_* failure prints its text and exits 1.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "g2b_attn.h"

static int read_all(FILE *f, void *p, size_t n) { return fread(p, 1, n, f) == n; }

static int fail(const char *what, int rc, g2b_ctx *ctx) {
  fprintf(stderr, "g2b_c_caller: %s: %s (%s)\n", what, g2b_strerror(rc),
          ctx ? g2b_ctx_last_error(ctx) : "");
  return 1;
}

int main(int argc, char **argv) {
  if (argc != 3) {
    fprintf(stderr, "usage: g2b_c_caller IN OUT\n");
    return 2;
  }
  FILE *in = fopen(argv[1], "rb");
  if (!in) {
    perror(argv[1]);
    return 2;
  }
  int32_t h[9];
  float hf[2];
  if (!read_all(in, h, sizeof h) || !read_all(in, hf, sizeof hf)) {
    fprintf(stderr, "g2b_c_caller: short header\n");
    fclose(in);
    return 2;
  }
  g2b_shape s;
  s.n_layers = h[0];
  s.n_heads = h[1];
  s.n_kv_heads = h[2];
  s.head_dim = h[3];
  s.arch = h[4];
  s.kv_q8 = h[5];
  s.rope_theta = hf[0];
  const int32_t ctx_cap = h[6], n_tokens = h[7], with_norm = h[8];
  const float eps = hf[1];
  const size_t nq = (size_t)s.n_heads * (size_t)s.head_dim;
  const size_t nkv = (size_t)s.n_kv_heads * (size_t)s.head_dim;

  int status = 1;
  g2b_ctx *ctx = NULL;
  void *kc = NULL, *vc = NULL;
  float *q = malloc(nq * sizeof(float)), *k = malloc(nkv * sizeof(float));
  float *v = malloc(nkv * sizeof(float));
  float *norm = with_norm ? malloc((size_t)2 * (size_t)s.head_dim * sizeof(float)) : NULL;
  uint8_t *cache = NULL;
  FILE *out = NULL;
  int rc;
  if (!q || !k || !v || (with_norm && !norm)) goto done;

  /* model load: the context; with F_QK_NORM the per-layer norm weights */
  if ((rc = g2b_ctx_create(&ctx, 0, &s)) != G2B_OK) {
    status = fail("g2b_ctx_create", rc, NULL);
    goto done;
  }
  for (int32_t L = 0; with_norm && L < s.n_layers; L++) {
    if (!read_all(in, norm, (size_t)2 * (size_t)s.head_dim * sizeof(float))) goto done;
    if ((rc = g2b_set_qk_norm(ctx, L, norm, norm + s.head_dim, eps)) != G2B_OK) {
      status = fail("g2b_set_qk_norm", rc, ctx);
      goto done;
    }
  }
  /* alloc_rt: the KV half in HBM */
  if ((rc = g2b_kv_alloc(ctx, ctx_cap, &kc, &vc)) != G2B_OK) {
    status = fail("g2b_kv_alloc", rc, ctx);
    goto done;
  }
  out = fopen(argv[2], "wb");
  if (!out) {
    perror(argv[2]);
    goto done;
  }
  /* model_forward's layer loop, attention block only */
  for (int32_t t = 0; t < n_tokens; t++) {
    for (int32_t L = 0; L < s.n_layers; L++) {
      if (!read_all(in, q, nq * sizeof(float)) || !read_all(in, k, nkv * sizeof(float)) ||
          !read_all(in, v, nkv * sizeof(float))) {
        fprintf(stderr, "g2b_c_caller: short input at token %d layer %d\n", (int)t, (int)L);
        goto done;
      }
      rc = g2b_attn_forward_host(ctx, L, t, ctx_cap, kc, vc, q, k, v, NULL);
      if (rc != G2B_OK) {
        status = fail("g2b_attn_forward_host", rc, ctx);
        goto done;
      }
      if (fwrite(q, sizeof(float), nq, out) != nq) goto done;
    }
  }
  /* the caches, as a tool reading Model.kcache/kcq would see them */
  {
    const uint64_t nbytes = g2b_kv_bytes(&s, ctx_cap);
    cache = malloc((size_t)nbytes);
    if (!cache) goto done;
    void *caches[2] = {kc, vc};
    for (int i = 0; i < 2; i++) {
      if ((rc = g2b_kv_read(ctx, caches[i], 0, nbytes, cache)) != G2B_OK) {
        status = fail("g2b_kv_read", rc, ctx);
        goto done;
      }
      if (fwrite(cache, 1, (size_t)nbytes, out) != (size_t)nbytes) goto done;
    }
  }
  status = 0;
done:
  if (out && fclose(out) != 0) status = 1;
  if (ctx) {
    if (kc && (rc = g2b_kv_free(ctx, kc, vc)) != G2B_OK) status = fail("g2b_kv_free", rc, ctx);
    g2b_ctx_destroy(ctx);
  }
  free(cache);
  free(norm);
  free(q);
  free(k);
  free(v);
  fclose(in);
  return status;
}
