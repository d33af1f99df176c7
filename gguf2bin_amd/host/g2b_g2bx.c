/*
 * g2b_g2bx.c - the G2BX container on the host, C99.
 *
 * Layout (written by exp_synth_qwen_tiny, /root/reference/src/l5_model.c:
 * 668-676; read by load_header_body, :286-301): "G2BX", u16 version, u8
 * arch, u8 flags, the packed 40-byte ModelCfg, u32 n_slots, n_slots packed
 * 16-byte slots, then the weight blob of ALIGN64(max(off + nbytes)) bytes.
 * Fields are little-endian and read byte by byte, so the parse does not
 * depend on the host's struct packing.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g2b_model.h"

static uint32_t le32(const uint8_t *p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
static uint64_t le64(const uint8_t *p) { return (uint64_t)le32(p) | (uint64_t)le32(p + 4) << 32; }
static float lef32(const uint8_t *p) {
  const uint32_t u = le32(p);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void g2b_g2bx_close(g2b_g2bx *g) {
  if (!g) return;
  free(g->slots);
  free(g->data);
  memset(g, 0, sizeof *g);
}

int g2b_g2bx_open(const char *path, g2b_g2bx *out) {
  if (!out) return G2B_EINVAL;
  memset(out, 0, sizeof *out);
  if (!path) return G2B_EINVAL;
  FILE *f = fopen(path, "rb");
  if (!f) return G2B_EINVAL;
  uint8_t h[4 + 2 + 1 + 1 + 40 + 4];
  if (fread(h, 1, sizeof h, f) != sizeof h || memcmp(h, "G2BX", 4) != 0) {
    fclose(f);
    return G2B_EINVAL;
  }
  out->version = (uint16_t)(h[4] | h[5] << 8);
  out->arch = h[6];
  out->flags = h[7];
  const uint8_t *c = h + 8;
  g2b_model_cfg *cfg = &out->cfg;
  cfg->dim = (int32_t)le32(c);
  cfg->hidden_dim = (int32_t)le32(c + 4);
  cfg->n_layers = (int32_t)le32(c + 8);
  cfg->n_heads = (int32_t)le32(c + 12);
  cfg->n_kv_heads = (int32_t)le32(c + 16);
  cfg->vocab = (int32_t)le32(c + 20);
  cfg->seq_len = (int32_t)le32(c + 24);
  cfg->head_dim = (int32_t)le32(c + 28);
  cfg->eps = lef32(c + 32);
  cfg->rope_theta = lef32(c + 36);
  out->n_slots = le32(h + 48);
  if (out->n_slots > (1u << 24)) {
    fclose(f);
    return G2B_EINVAL;
  }
  out->slots = (g2b_slot *)calloc(out->n_slots ? out->n_slots : 1, sizeof(g2b_slot));
  if (!out->slots) {
    fclose(f);
    return G2B_ENOMEM;
  }
  uint64_t max_end = 0;
  for (uint32_t i = 0; i < out->n_slots; i++) {
    uint8_t s[16];
    if (fread(s, 1, 16, f) != 16) {
      fclose(f);
      g2b_g2bx_close(out);
      return G2B_EINVAL;
    }
    g2b_slot *sl = &out->slots[i];
    sl->role = s[0];
    sl->layer = (uint16_t)(s[1] | s[2] << 8);
    sl->type = s[3];
    sl->nbytes = le32(s + 4);
    sl->off = le64(s + 8);
    /* an offset whose end wraps would pass every later size check */
    if (sl->off > UINT64_MAX - sl->nbytes) {
      fclose(f);
      g2b_g2bx_close(out);
      return G2B_EINVAL;
    }
    const uint64_t e = sl->off + sl->nbytes;
    if (e > max_end) max_end = e;
  }
  out->data_size = (max_end + 63u) & ~(uint64_t)63u;
  out->data = (uint8_t *)malloc(out->data_size ? (size_t)out->data_size : 1);
  if (!out->data) {
    fclose(f);
    g2b_g2bx_close(out);
    return G2B_ENOMEM;
  }
  if (fread(out->data, 1, (size_t)out->data_size, f) != (size_t)out->data_size) {
    fclose(f);
    g2b_g2bx_close(out);
    return G2B_EINVAL;  /* "model: truncado" (l5_model.c:368-370) */
  }
  fclose(f);
  if (cfg->seq_len <= 0) cfg->seq_len = 2048;
  return G2B_OK;
}

const g2b_slot *g2b_g2bx_slot(const g2b_g2bx *g, int32_t role, int32_t layer) {
  if (!g || role < 0 || role >= G2B_R_COUNT) return NULL;
  if (layer >= g->cfg.n_layers) return NULL;
  const g2b_slot *hit = NULL;
  for (uint32_t i = 0; i < g->n_slots; i++) {
    const g2b_slot *s = &g->slots[i];
    if (s->role != (uint8_t)role) continue;
    if (layer < 0 ? s->layer == 0xFFFF : s->layer == (uint16_t)layer) hit = s;
  }
  return hit;
}
