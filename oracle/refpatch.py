#!/usr/bin/env python3
"""Apply the maintainer's drop-in patch for the reference to a COPY of the
reference sources (test infrastructure: build recipe of oracle/_ref).

    python3 oracle/refpatch.py /root/reference /tmp/g2b_refpatch

copies REF/src and REF/include into OUT (outside this repository; nothing of
the reference is kept) and inserts this repository's integration code at
anchors in include/g2b.h and src/l5_model.c:
  - a `gpu` context field in Model (include/g2b.h:77-105);
  - gpu_attach at model load (after build_index, l5_model.c:382), which
    creates the context when G2B_GPU is set and hands it the QK-RMSNorm
    weights;
  - the KV half of alloc_rt / free_rt in HBM (:113-149);
  - model_forward's attention block (:505-578) as one g2b_attn_forward_host
    call when the context exists;
  - the context's release in model_free (:418-434).
Every snippet below is also shown, verbatim, in the repository's integration
guide for maintainers (checked by tests/test_refpatch.py).  Each anchor must match exactly once; the script
fails otherwise, so a reference that moved under the patch is reported, not
silently mis-patched.
"""
import os
import re
import shutil
import sys

H_INCLUDE = '#include "g2b_attn.h"\n'

H_FIELD = "  g2b_ctx *gpu;          /* non-NULL: KV in HBM, attention on the MI355X */\n"

C_ATTACH = r'''static void load_vec_f32(Model *m, Slot *s, f32 *dst, i32 n);
static void gpu_attach(Model *m){
  g2b_shape s = { m->c.n_layers, m->c.n_heads, m->c.n_kv_heads, m->c.head_dim,
                  m->c.rope_theta, m->arch, (m->flags & F_KV_Q8) ? 1 : 0 };
  if (!getenv("G2B_GPU") || g2b_ctx_create(&m->gpu, 0, &s) != G2B_OK) { m->gpu = NULL; return; }
  if (m->flags & F_QK_NORM) {
    f32 *qw = malloc(m->c.head_dim * sizeof(f32)), *kw = malloc(m->c.head_dim * sizeof(f32));
    for (i32 L = 0; qw && kw && L < m->c.n_layers; L++) {
      Slot *qn = slot_get(m, R_ATTN_Q_NORM, L), *kn = slot_get(m, R_ATTN_K_NORM, L);
      if (qn) load_vec_f32(m, qn, qw, m->c.head_dim);
      if (kn) load_vec_f32(m, kn, kw, m->c.head_dim);
      g2b_set_qk_norm(m->gpu, L, qn ? qw : NULL, kn ? kw : NULL, m->c.eps);
    }
    free(qw); free(kw);
  }
}
'''

C_ATTACH_CALL = "  gpu_attach(m);\n"

C_FREE_RT = r'''  if (m->gpu) {
    if (m->kcq || m->kcache)
      g2b_kv_free(m->gpu, m->kcq ? (void*)m->kcq : (void*)m->kcache,
                          m->vcq ? (void*)m->vcq : (void*)m->vcache);
    m->kcache = m->vcache = NULL; m->kcq = m->vcq = NULL;
    return;
  }
'''

C_ALLOC_RT = r'''  if (m->gpu) {
    if (m->swap_path) return -1;                 /* file-backed KV cannot live in HBM (G2B_ESWAP) */
    g2b_ctx_destroy(m->gpu); m->gpu = NULL;      /* F_KV_Q8 may have changed since the load: */
    gpu_attach(m);                               /* the KV mode is part of the context's shape */
    if (!m->gpu) return -1;
    void *k = NULL, *v = NULL;
    if (g2b_kv_alloc(m->gpu, ctx, &k, &v) != G2B_OK) return -1;
    if (q8) { m->kcq = k; m->vcq = v; } else { m->kcache = k; m->vcache = v; }
    return 0;
  }
'''

C_FWD_OPEN = r'''    if (m->gpu) {
      f32 *att_dbg = NULL;   /* or att, to get the reference [n_heads][ctx] weights */
      int rc = g2b_attn_forward_host(m->gpu, L, pos, ctx,
                                     m->kcq ? (void*)m->kcq : (void*)m->kcache,
                                     m->vcq ? (void*)m->vcq : (void*)m->vcache,
                                     q, k, v, att_dbg);
      if (rc != G2B_OK) {
        fprintf(stderr, "fwd: gpu attention: %s (%s)\n", g2b_strerror(rc),
                g2b_ctx_last_error(m->gpu));
        if (logits) memset(logits, 0, (size_t)c->vocab * sizeof(f32));
        return;
      }
    } else {
'''

C_FWD_CLOSE = "    }  /* m->gpu */\n"

C_MODEL_FREE = "  if (m->gpu) { g2b_ctx_destroy(m->gpu); m->gpu = NULL; }\n"

# (file, anchor regex (one match, MULTILINE), 'before' | 'after' the anchor's
# line, code)
EDITS = [
    ("include/g2b.h", r"^#include <stdio\.h>[ \t]*$", "after", H_INCLUDE),
    ("include/g2b.h", r"^\} Model;[ \t]*$", "before", H_FIELD),
    ("src/l5_model.c", r"^static void free_rt\(Model \*m\)\{[ \t]*$", "before", C_ATTACH),
    ("src/l5_model.c", r"^[ \t]*m->buf=NULL; m->kvrow=NULL;[ \t]*$", "after", C_FREE_RT),
    ("src/l5_model.c", r"^[ \t]*if\(m->swap_path && kv_swap_alloc\(m,usize\)==0\)\{[ \t]*$",
     "before", C_ALLOC_RT),
    ("src/l5_model.c", r"^[ \t]*build_index\(m\);[ \t]*$", "after", C_ATTACH_CALL),
    ("src/l5_model.c", r"^[ \t]*if\(m->flags & F_QK_NORM\)\{[ \t]*$", "before", C_FWD_OPEN),
    ("src/l5_model.c", r"^#endif[ \t]*\n[ \t]*\n[ \t]*Slot \*wo=slot_get\(m,R_ATTN_O,L\);", "after",
     C_FWD_CLOSE),
    ("src/l5_model.c", r"^[ \t]*free_rt\(m\);[ \t]*\n[ \t]*free\(m->swap_path\);", "after",
     C_MODEL_FREE),
]


def apply(text: str, anchor: str, where: str, code: str, name: str) -> str:
    hits = list(re.finditer(anchor, text, re.M))
    if len(hits) != 1:
        raise SystemExit(f"refpatch: anchor {anchor!r} matches {len(hits)} times in {name}")
    m = hits[0]
    if where == "before":
        at = text.rfind("\n", 0, m.start()) + 1
    else:  # after the anchor's first line
        at = text.find("\n", m.start()) + 1
    return text[:at] + code + text[at:]


def main():
    if len(sys.argv) != 3:
        raise SystemExit("usage: refpatch.py REFERENCE_DIR OUT_DIR")
    ref, out = sys.argv[1], sys.argv[2]
    if os.path.abspath(out).startswith(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))):
        raise SystemExit("refpatch: OUT_DIR must lie outside this repository")
    shutil.rmtree(out, ignore_errors=True)
    for sub in ("src", "include"):
        shutil.copytree(os.path.join(ref, sub), os.path.join(out, sub))
    for rel, anchor, where, code in EDITS:
        p = os.path.join(out, rel)
        with open(p) as f:
            text = f.read()
        with open(p, "w") as f:
            f.write(apply(text, anchor, where, code, rel))
    print(f"refpatch: {len(EDITS)} edits applied in {out}")


if __name__ == "__main__":
    main()
