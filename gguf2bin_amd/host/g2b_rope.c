/*
 * g2b_rope.c - host side of the RoPE step, C99.
 *
 * The reference computes the rotation angles with the C library on every
 * call (/root/reference/src/l3_math.c:68-73 for LLaMA, :87-92 for NEOX; the
 * two tables are identical): inv_step = powf(theta, -2/hd), freq starts at 1
 * and is multiplied serially, ang = (float)pos * freq, then cosf and sinf.
 * Rotated values feed the Q8_0 quantiser, so the device must see the very
 * same cos/sin bits; the table is therefore built here, on the host, with the
 * same library calls, and uploaded once per context (g2b_kv_alloc,
 * g2b_batch_begin) instead of being recomputed per layer.
 */
#include <math.h>
#include <stddef.h>

#include "g2b_attn.h"

int g2b_rope_table(int32_t pos0, int32_t n_pos, int32_t head_dim, float theta, float *cs) {
  if (!cs || n_pos < 0 || pos0 < 0 || head_dim < 2 || (head_dim & 1)) return G2B_EINVAL;
  const int32_t half = head_dim / 2;
  if (half > 512) return G2B_EUNSUP;
  float freq[512];
  const float step = powf(theta, -2.0f / (float)head_dim);
  float f = 1.0f;
  for (int32_t j = 0; j < half; j++) {
    freq[j] = f;
    f *= step;
  }
  for (int32_t i = 0; i < n_pos; i++) {
    const float p = (float)(pos0 + i);
    float *row = cs + (size_t)i * (size_t)head_dim;
    for (int32_t j = 0; j < half; j++) {
      const float ang = p * freq[j];
      row[2 * j] = cosf(ang);
      row[2 * j + 1] = sinf(ang);
    }
  }
  return G2B_OK;
}
