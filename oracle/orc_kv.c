/*
 * orc_kv.c - fp16 conversion, Q8_0 KV rows, RoPE, softmax and KV layout,
 * restated from the reference for the CPU oracle.  TEST INFRASTRUCTURE ONLY
 * (see orc.h).  Compile with -O3 -mavx2 -mfma -std=c99 (reference Makefile:3);
 * -std=c99 keeps GCC from contracting a*b+c into fma, as in the reference.
 */
#include "orc.h"
#include <math.h>
#include <string.h>
#include <stdio.h>
#include <stdlib.h>

/* Truncating fp32 -> fp16.  Follows /root/reference/src/l3_math.c:6-16:
 * exponent rebias by -112, mantissa cut to 10 bits (no rounding), results
 * below the normal range become signed zero, overflow and Inf/NaN become
 * signed Inf. */
uint16_t orc_f32_to_half(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  int32_t e8 = (int32_t)((u >> 23) & 0xffu);
  if (e8 == 0xff) return (uint16_t)(sign | 0x7c00u);
  int32_t e5 = e8 - 112;
  if (e5 <= 0) return sign;
  if (e5 >= 31) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | ((uint32_t)e5 << 10) | ((u & 0x7fffffu) >> 13));
}

/* Exact fp16 -> fp32 including subnormals and Inf/NaN payloads.
 * Follows /root/reference/src/l2_codec.c:35-54. */
float orc_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) & 1u;
  uint32_t e5 = (uint32_t)(h >> 10) & 0x1fu;
  uint32_t m10 = (uint32_t)h & 0x3ffu;
  uint32_t u;
  float f;
  if (e5 == 0) {
    if (m10 == 0) {
      u = sign << 31;
      memcpy(&f, &u, 4);
      return f;
    }
    /* mant/1024 * 2^-14, both steps exact in fp32 */
    f = (float)m10 / 1024.f;
    f *= 1.f / 16384.f;
    return sign ? -f : f;
  }
  if (e5 == 31) u = (sign << 31) | (0xffu << 23) | (m10 << 13);
  else u = (sign << 31) | ((e5 + 112u) << 23) | (m10 << 13);
  memcpy(&f, &u, 4);
  return f;
}

void orc_f32_to_half_n(const float *x, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_half(x[i]);
}

void orc_half_to_float_n(const uint16_t *h, float *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = orc_half_to_float(h[i]);
}

/* Bytes per Q8_0 row of nkv floats: ceil(nkv/32) blocks of 34 bytes.
 * /root/reference/src/l5_model.c:47 */
size_t orc_q8_rowsize(int32_t nkv) { return ((size_t)nkv + 31u) / 32u * 34u; }

/* /root/reference/src/l5_model.c:49-59.  Per 32-element block: amax over
 * |x| (a NaN never wins the '>' test), d = amax/127 in fp32 (1e-10 when d is
 * not > 0), the truncated fp16 of d stored little-endian in bytes 0-1, then
 * q = clamp((int32)lroundf(x/d), -127, 127) using the unrounded fp32 d;
 * a partial last block is zero padded. */
void orc_q8_quant_row(const float *src, uint8_t *dst, int32_t n) {
  for (int32_t base = 0; base < n; base += 32) {
    int32_t cnt = (n - base) < 32 ? (n - base) : 32;
    float amax = 0.f;
    for (int32_t j = 0; j < cnt; j++) {
      float a = fabsf(src[base + j]);
      if (a > amax) amax = a;
    }
    float d = amax / 127.f;
    if (!(d > 0.f)) d = 1e-10f;
    uint16_t hd = orc_f32_to_half(d);
    dst[0] = (uint8_t)(hd & 0xffu);
    dst[1] = (uint8_t)(hd >> 8);
    for (int32_t j = 0; j < 32; j++) {
      int32_t q = 0;
      if (j < cnt) {
        q = (int32_t)lroundf(src[base + j] / d);
        if (q > 127) q = 127;
        else if (q < -127) q = -127;
      }
      dst[2 + j] = (uint8_t)(int8_t)q;
    }
    dst += 34;
  }
}

/* /root/reference/src/l5_model.c:60-67: out = fp16 scale * int8, exact. */
void orc_q8_dequant_row(const uint8_t *src, float *out, int32_t n) {
  for (int32_t base = 0; base < n; base += 32) {
    uint16_t hs = (uint16_t)(src[0] | ((uint16_t)src[1] << 8));
    float sc = orc_half_to_float(hs);
    int32_t cnt = (n - base) < 32 ? (n - base) : 32;
    for (int32_t j = 0; j < cnt; j++) out[base + j] = sc * (float)(int8_t)src[2 + j];
    src += 34;
  }
}

/* Angle table of /root/reference/src/l3_math.c:68-73 (LLaMA) and :87-92 (NEOX),
 * which are the same: freq starts at 1 and is multiplied serially by
 * powf(theta, -2/hd); ang = (float)pos * freq. */
int orc_rope_table(int32_t pos, int32_t head_dim, float theta, float *cs) {
  int32_t half = head_dim / 2;
  if (half > 512) return -1;
  float step = powf(theta, -2.0f / (float)head_dim);
  float freq = 1.0f;
  for (int32_t j = 0; j < half; j++) {
    float ang = (float)pos * freq;
    cs[2 * j] = cosf(ang);
    cs[2 * j + 1] = sinf(ang);
    freq *= step;
  }
  return 0;
}

/* apply_rope (/root/reference/src/l5_model.c:448-452): ARCH_LLAMA rotates
 * adjacent pairs (2i, 2i+1) (l3_math.c:74-81); every other arch rotates the
 * half-split pairs (j, j+hd/2) (l3_math.c:93-101).  a' = a*c - b*s,
 * b' = a*s + b*c, in place, head by head. */
/* l3_math.c:107-114.  ss accumulates left to right with each square rounded
 * (-std=c99 keeps contraction off, and without -ffast-math GCC does not
 * reassociate the sum); ss/head_dim divides by the int converted to float;
 * the output is (w*x)*inv, rounded after each product. */
void orc_qk_rmsnorm(float *x, const float *w, int32_t n_heads, int32_t head_dim, float eps) {
  for (int32_t h = 0; h < n_heads; h++) {
    float *xh = x + (size_t)h * (size_t)head_dim;
    float ss = 0.f;
    for (int32_t j = 0; j < head_dim; j++) {
      const float sq = xh[j] * xh[j];
      ss = ss + sq;
    }
    const float inv = 1.f / sqrtf(ss / (float)head_dim + eps);
    for (int32_t j = 0; j < head_dim; j++) {
      const float wx = w[j] * xh[j];
      xh[j] = wx * inv;
    }
  }
}

void orc_rope(int32_t arch, float *x, int32_t len, int32_t pos, int32_t head_dim,
              float theta) {
  float cs[1024];
  if (orc_rope_table(pos, head_dim, theta, cs)) {
    fprintf(stderr, "rope: head_dim %d > 1024 (no soportado)\n", head_dim);
    return;
  }
  int32_t half = head_dim / 2;
  for (int32_t h = 0; h < len; h += head_dim) {
    float *xh = x + h;
    for (int32_t j = 0; j < half; j++) {
      float c = cs[2 * j], s = cs[2 * j + 1];
      int32_t ia = arch == ORC_ARCH_LLAMA ? 2 * j : j;
      int32_t ib = arch == ORC_ARCH_LLAMA ? 2 * j + 1 : j + half;
      float a = xh[ia], b = xh[ib];
      xh[ia] = a * c - b * s;
      xh[ib] = a * s + b * c;
    }
  }
}

/* /root/reference/src/l3_math.c:52-56: max, expf(x-max) with a serial fp32
 * sum, then a true division by the sum. */
void orc_softmax(float *x, int32_t n) {
  float mx = x[0];
  for (int32_t i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];
  float sum = 0.f;
  for (int32_t i = 0; i < n; i++) {
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  for (int32_t i = 0; i < n; i++) x[i] /= sum;
}

/* Row bytes: kv_q8_rowsize(nkv) for Q8_0, nkv*4 for F32
 * (/root/reference/src/l5_model.c:131-132). */
size_t orc_kv_row_bytes(const orc_shape *s) {
  int32_t nkv = s->n_kv_heads * s->head_dim;
  return s->kv_q8 ? orc_q8_rowsize(nkv) : (size_t)nkv * 4u;
}

/* [layer][ctx_cap][row]: /root/reference/src/l5_model.c:232-234 (F32, in
 * floats) and :239-240 (Q8, in bytes); here always in bytes. */
size_t orc_kv_offset(const orc_shape *s, int32_t ctx_cap, int32_t layer, int32_t pos) {
  return ((size_t)layer * (size_t)ctx_cap + (size_t)pos) * orc_kv_row_bytes(s);
}

/* RoPE on k at pos (l5_model.c:514) then kv_store (l5_model.c:235-247). */
void orc_kv_append(const orc_shape *s, int32_t ctx_cap, int32_t layer, int32_t pos,
                   uint8_t *kcache, uint8_t *vcache, const float *k_in, const float *v_in) {
  int32_t nkv = s->n_kv_heads * s->head_dim;
  float kbuf[8192];
  float *k = kbuf;
  float *heap = NULL;
  if (nkv > 8192) {
    heap = (float *)malloc((size_t)nkv * sizeof(float));
    k = heap;
  }
  memcpy(k, k_in, (size_t)nkv * sizeof(float));
  orc_rope(s->arch, k, nkv, pos, s->head_dim, s->rope_theta);
  size_t off = orc_kv_offset(s, ctx_cap, layer, pos);
  if (s->kv_q8) {
    orc_q8_quant_row(k, kcache + off, nkv);
    orc_q8_quant_row(v_in, vcache + off, nkv);
  } else {
    memcpy(kcache + off, k, (size_t)nkv * 4u);
    memcpy(vcache + off, v_in, (size_t)nkv * 4u);
  }
  free(heap);
}

/* orc_kv_append for rows [pos0, pos0+n_rows) of one layer; k_rows/v_rows are
 * [n_rows][nkv], pre-RoPE. */
void orc_kv_prefill(const orc_shape *s, int32_t ctx_cap, int32_t layer, int32_t pos0,
                    int32_t n_rows, uint8_t *kcache, uint8_t *vcache,
                    const float *k_rows, const float *v_rows) {
  const size_t nkv = (size_t)s->n_kv_heads * (size_t)s->head_dim;
  for (int32_t r = 0; r < n_rows; r++)
    orc_kv_append(s, ctx_cap, layer, pos0 + r, kcache, vcache, k_rows + (size_t)r * nkv,
                  v_rows + (size_t)r * nkv);
}
