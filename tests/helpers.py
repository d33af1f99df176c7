"""Shared test helpers: golden fixtures, seeded inputs, oracle runs and
device runs of the same case."""
from __future__ import annotations

import hashlib
import os
from statistics import NormalDist

import numpy as np

from oracle import orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def load_golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def fwd_cases():
    return sorted(f for f in os.listdir(GOLDEN) if f.startswith("fwd_") and f.endswith(".npz"))


def golden_shape(d: dict) -> orc.Shape:
    L, nh, nkv, hd, arch, q8 = [int(x) for x in d["shape"]]
    return orc.Shape(L, nh, nkv, hd, float(d["theta"]), arch, bool(q8))


def case_inputs(shape: orc.Shape, n_pre: int, n_fwd: int, seed: int, p_scale: float):
    """Seeded inputs of a forward case: pre-RoPE k/v prefill rows and x rows.

    A prefill K row is scaled x8 when its own N(0,1) selector draw exceeds
    the (1 - p_scale) quantile."""
    nkv = shape.nkv
    dim = shape.nq + 2 * nkv
    kp = orc.normal(seed * 16 + 0, n_pre * nkv).reshape(n_pre, nkv)
    vp = orc.normal(seed * 16 + 1, n_pre * nkv).reshape(n_pre, nkv)
    if p_scale > 0 and n_pre:
        thr = float(NormalDist().inv_cdf(1.0 - p_scale))
        sel = orc.normal(seed * 16 + 3, n_pre)
        kp[sel > thr] *= np.float32(8.0)
    xr = orc.normal(seed * 16 + 2, n_fwd * dim).reshape(n_fwd, dim)
    return kp, vp, xr


def golden_inputs(d: dict):
    shape = golden_shape(d)
    kp, vp, xr = case_inputs(shape, int(d["n_pre"]), int(d["n_fwd"]), int(d["seed"]),
                             float(d["p_scale"]))
    assert d["inputs_sha"].item().decode() == sha(kp) + sha(vp) + sha(xr), "RNG drift"
    return shape, kp, vp


def golden_norms(d: dict):
    """(q_norm [L, hd] or None, k_norm [L, hd] or None, eps) of a golden case."""
    eps = float(d["qkn_eps"]) if "qkn_eps" in d else 1e-6
    return d.get("q_norm"), d.get("k_norm"), eps


def normed(x: np.ndarray, w, n_heads: int, head_dim: int, eps: float) -> np.ndarray:
    """x (any number of rows of n_heads heads) through the oracle's QK-RMSNorm
    with weights w; x itself when w is None."""
    if w is None:
        return np.asarray(x, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    n = x.size // head_dim
    return orc.qk_rmsnorm(x.reshape(-1), w, n, head_dim, eps).reshape(x.shape)


def split_xb(shape: orc.Shape, xb: np.ndarray):
    nq, nkv = shape.nq, shape.nkv
    return xb[:nq], xb[nq:nq + nkv], xb[nq + nkv:nq + 2 * nkv]


def oracle_run_case(d: dict):
    """The oracle on a golden case: prefill, then every forward step on every
    layer (all layers see the same q/k/v, as in the reference selector model;
    with QK-RMSNorm weights, each layer normalises them with its own).
    Returns (outs [n_fwd, nq], att of the last step [n_heads, pos+1], kc, vc)."""
    shape, kp, vp = golden_inputs(d)
    qn, kn, eps = golden_norms(d)
    hd = shape.head_dim
    ctx_cap, n_pre = int(d["ctx_cap"]), int(d["n_pre"])
    avx2 = d["variant"].item().decode() == "avx2"
    kc, vc = orc.alloc_kv(shape, ctx_cap)
    for L in range(shape.n_layers):
        kpl = normed(kp, None if kn is None else kn[L], shape.n_kv_heads, hd, eps)
        orc.kv_prefill(shape, ctx_cap, L, 0, kc, vc, kpl, vp)
    outs, att = [], None
    for i, xb in enumerate(d["xb"]):
        q, k, v = split_xb(shape, xb)
        for L in range(shape.n_layers):
            ql = normed(q, None if qn is None else qn[L], shape.n_heads, hd, eps)
            kl = normed(k, None if kn is None else kn[L], shape.n_kv_heads, hd, eps)
            o, att = orc.attn_layer(shape, ctx_cap, L, n_pre + i, kc, vc, ql, kl, v, avx2)
        outs.append(o)
    return np.array(outs), att, kc, vc


def kv_rows(shape: orc.Shape, buf: np.ndarray, ctx_cap: int, n_rows: int) -> np.ndarray:
    return buf.reshape(shape.n_layers, ctx_cap, shape.row_bytes)[:, :n_rows]


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def q8_special_rows() -> np.ndarray:
    """Rows of 64 floats whose blocks exercise every branch of q8_quant_row."""
    rows = []
    z = np.zeros(64, np.float32)
    rows.append(z.copy())                                  # zero blocks: d -> 1e-10
    r = z.copy(); r[0] = 127.0; r[1:32] = np.arange(31) - 15 + 0.5   # d = 1: exact .5 ties
    r[32] = -127.0; r[33:64] = -(np.arange(31) - 15 + 0.5)
    rows.append(r)
    r = z.copy(); r[:32] = np.linspace(-0.007, 0.007, 32); r[32:] = 1e-6   # amax < 2^-14*127
    rows.append(r)
    r = z.copy(); r[:32] = np.float32(5e-39); r[40] = np.float32(1e-45)    # subnormal inputs
    rows.append(r)
    r = np.linspace(-3, 3, 64).astype(np.float32); r[5] = np.nan             # NaN skipped by '>'
    rows.append(r)
    r = np.linspace(-3, 3, 64).astype(np.float32); r[7] = np.inf; r[40] = -np.inf
    rows.append(r)
    r = np.linspace(-1, 1, 64).astype(np.float32) * np.float32(1e30)        # fp16 scale overflow
    rows.append(r)
    r = np.full(64, -0.0, np.float32); r[63] = 1e-3                          # negative zeros
    rows.append(r)
    r = np.linspace(-65504 * 127, 65504 * 127, 64).astype(np.float32)      # near fp16 max scale
    rows.append(r)
    rng = np.random.default_rng(7)
    for s in (1e-4, 1e-2, 1.0, 8.0, 300.0):
        rows.append((rng.standard_normal(64) * s).astype(np.float32))
    return np.stack(rows).astype(np.float32)


def dequant_rows(shape: orc.Shape, buf: np.ndarray, ctx_cap: int, layer: int,
                 n_rows: int) -> np.ndarray:
    """Rows [0, n_rows) of one layer as float64, decoded with numpy (float16
    scale times int8, exact), independent of the C codec."""
    rb = shape.row_bytes
    raw = buf[layer * ctx_cap * rb:(layer * ctx_cap + n_rows) * rb].reshape(n_rows, rb)
    if not shape.kv_q8:
        return raw.copy().view(np.float32).astype(np.float64)
    nb = rb // 34
    blk = raw.reshape(n_rows, nb, 34)
    scale = blk[:, :, :2].copy().view(np.float16).astype(np.float64)  # [n, nb, 1]
    q = blk[:, :, 2:].copy().view(np.int8).astype(np.float64)
    return (scale * q).reshape(n_rows, nb * 32)[:, :shape.nkv]


def exact_attention(shape: orc.Shape, ctx_cap: int, layer: int, pos: int, kc: np.ndarray,
                    vc: np.ndarray, q: np.ndarray):
    """float64 attention over the given cache bytes.  q is rotated in float32
    by the oracle (bit-exact with the reference and the device), so only the
    score/softmax/V arithmetic is evaluated exactly.
    Returns (out [nq], weights [n_heads, pos+1])."""
    hd, nh = shape.head_dim, shape.n_heads
    group = nh // shape.n_kv_heads
    qr = orc.rope(shape.arch, q, pos, hd, shape.rope_theta).astype(np.float64).reshape(nh, hd)
    K = dequant_rows(shape, kc, ctx_cap, layer, pos + 1)
    V = dequant_rows(shape, vc, ctx_cap, layer, pos + 1)
    out = np.zeros((nh, hd))
    W = np.zeros((nh, pos + 1))
    for h in range(nh):
        g = h // group
        sc = K[:, g * hd:(g + 1) * hd] @ qr[h] / np.sqrt(np.float64(hd))
        w = np.exp(sc - sc.max())
        w /= w.sum()
        W[h] = w
        out[h] = w @ V[:, g * hd:(g + 1) * hd]
    return out.ravel(), W


OUT_ATOL = 1e-4
W_RTOL = 1e-5


def check_out(got, ref, exact, atol: float = OUT_ATOL):
    """Attention outputs.  got must be within atol of the float64 evaluation
    and within atol + (the reference's own float32 error) of the reference.
    Where the reference is accurate (almost always: ~1e-7) this is plain
    max |got - ref| <= atol; where its serial float32 sums drift (32k
    contexts with dominant rows), the reference's measured error is added."""
    got, ref, exact = (np.asarray(a, np.float64) for a in (got, ref, exact))
    own = float(np.max(np.abs(ref - exact)))
    e_ex = float(np.max(np.abs(got - exact)))
    e_ref = float(np.max(np.abs(got - ref)))
    assert e_ex <= atol, f"max |out - float64| = {e_ex:.3g} > {atol}"
    assert e_ref <= atol + own, f"max |out - ref| = {e_ref:.3g} > {atol} + ref's own {own:.3g}"
    return e_ref, e_ex, own


def check_weights(got, ref, exact, rtol: float = W_RTOL, as_accurate_as_ref: bool = False):
    """Softmax weights, relative, with the same rule as check_out; weights
    below 1e-30 are compared absolutely (1e-35).

    as_accurate_as_ref: the float64 bar becomes rtol + twice the reference's
    own relative error - the reference's accuracy class: its score is an
    fp32 dot times an fp32 scale, a couple of roundings of the score's size.
    For scores so large that rounding them to fp32 once moves the weights by
    about rtol (a q channel 10^2-10^3 times the rest: |score| in the tens to
    hundreds, 2^-24 of it ~1e-6-1e-5), where the reference itself misses
    rtol and any fp32 evaluation that rounds once or twice more or less than
    it lands within a small factor of its error."""
    got, ref, exact = (np.asarray(a, np.float64) for a in (got, ref, exact))
    big = exact > 1e-30
    r_ex = 0.0
    if big.any():
        own = float(np.max(np.abs(ref[big] - exact[big]) / exact[big]))
        r_ex = float(np.max(np.abs(got[big] - exact[big]) / exact[big]))
        r_ref = float(np.max(np.abs(got[big] - ref[big]) / ref[big]))
        bar = rtol + 2.0 * own if as_accurate_as_ref else rtol
        assert r_ex <= bar, f"max rel |w - float64| = {r_ex:.3g} > {bar:.3g}"
        # (against the reference: its own error adds to ours, so within bar + own)
        assert r_ref <= bar + own, f"max rel |w - ref| = {r_ref:.3g} > {bar:.3g} + own {own:.3g}"
    # (the relative bar at the 1e-30 level: 1e-35 for the plain rtol)
    small_bar = 1e-30 * (rtol + 2.0 * own if as_accurate_as_ref and big.any() else rtol)
    assert np.all(np.abs(got[~big] - exact[~big]) <= small_bar)
    return r_ex


# ---------------------------------------------------------------- G2BX files
# Roles and flags of the container (include/g2b.h:18-24).
R_TOK_EMBD, R_OUT_NORM, R_OUTPUT = 0, 1, 2
(R_ATTN_NORM, R_ATTN_Q, R_ATTN_K, R_ATTN_V, R_ATTN_O, R_ATTN_Q_NORM, R_ATTN_K_NORM,
 R_FFN_NORM, R_FFN_GATE, R_FFN_UP, R_FFN_DOWN) = range(3, 14)
F_TIE_EMBD, F_QK_NORM = 1, 2
G2BX_CFG = ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab", "seq_len",
            "head_dim", "eps", "rope_theta")


def write_g2bx(path, cfg: dict, arch: int, flags: int, slots, version: int = 1):
    """A G2BX container laid out as the reference's writer lays it out
    (exp_synth_qwen_tiny, /root/reference/src/l5_model.c:666-676): header,
    packed 40-byte ModelCfg, slot table, then each slot's bytes at a 64-byte
    aligned offset, zero padding to the aligned end.  slots: (role, layer,
    type, bytes) with layer 0xFFFF for global slots."""
    import struct
    offs, cur = [], 0
    for s in slots:
        offs.append(cur)
        cur = (cur + len(s[3]) + 63) & ~63
    head = b"G2BX" + struct.pack("<HBB", version, arch, flags)
    head += struct.pack("<8i2f", *[cfg[k] for k in G2BX_CFG])
    head += struct.pack("<I", len(slots))
    for (role, layer, typ, data), off in zip(slots, offs):
        head += struct.pack("<BHBIQ", role, layer, typ, len(data), off)
    blob = bytearray(cur)
    for (_, _, _, data), off in zip(slots, offs):
        blob[off:off + len(data)] = data
    with open(path, "wb") as f:
        f.write(head + bytes(blob))


def random_matrix_bytes(rng, t: int, rows: int, n: int, gain: float = 1.0) -> bytes:
    """rows x n weights of type t with values ~ gain * U(-1, 1) / sqrt(n) (Q8_0,
    Q4_0, Q4_1: random quants with fp16 block scales; F32, F16: normal /
    sqrt(n))."""
    if t == 0:
        return (rng.standard_normal((rows, n)) * gain / np.sqrt(n)).astype(np.float32).tobytes()
    if t == 1:
        return (rng.standard_normal((rows, n)) * gain / np.sqrt(n)).astype(np.float16).tobytes()
    nb = n // 32
    if t == 8:
        blk = np.zeros((rows, nb, 34), np.uint8)
        blk[:, :, 2:] = rng.integers(-127, 128, (rows, nb, 32)).astype(np.int8).view(np.uint8)
        sc = np.full((rows, nb), gain / (127 * np.sqrt(n)) * 1.7, np.float32)
    elif t == 3:  # Q4_1: d, m (about -8 d: nibbles centred), 16 bytes of nibbles
        blk = np.zeros((rows, nb, 20), np.uint8)
        blk[:, :, 4:] = rng.integers(0, 256, (rows, nb, 16), dtype=np.uint8)
        sc = (np.full((rows, nb), gain / (8 * np.sqrt(n)) * 1.7, np.float32)
              * rng.uniform(0.5, 1.5, (rows, nb)).astype(np.float32))
        mn = (-8.0 * sc * rng.uniform(0.8, 1.2, (rows, nb))).astype(np.float16)
        blk[:, :, :2] = sc.astype(np.float16).view(np.uint8).reshape(rows, nb, 2)
        blk[:, :, 2:4] = mn.view(np.uint8).reshape(rows, nb, 2)
        return blk.tobytes()
    else:
        blk = np.zeros((rows, nb, 18), np.uint8)
        blk[:, :, 2:] = rng.integers(0, 256, (rows, nb, 16), dtype=np.uint8)
        sc = np.full((rows, nb), gain / (8 * np.sqrt(n)) * 1.7, np.float32)
    sc *= rng.uniform(0.5, 1.5, (rows, nb)).astype(np.float32)
    blk[:, :, :2] = sc.astype(np.float16).view(np.uint8).reshape(rows, nb, 2)
    return blk.tobytes()


def random_model_slots(rng, cfg: dict, flags: int, mat_type: int, emb_type: int,
                       out_type=None):
    """Every slot model_forward reads, random: norms near 1 (F32), matrices
    of mat_type (a GGML type id, or a dict role -> type with "*" for the
    rest), embeddings of emb_type, an untied output of out_type (None: tied
    to the embeddings, F_TIE_EMBD)."""
    d, h, nl = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"]
    types = mat_type if isinstance(mat_type, dict) else {"*": mat_type}

    def mt(role):
        return types.get(role, types["*"])
    nq, nkv, hd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"], cfg["head_dim"]
    G = 0xFFFF

    def norm(n):
        return (1.0 + 0.2 * rng.standard_normal(n)).astype(np.float32).tobytes()

    slots = [(R_TOK_EMBD, G, emb_type, random_matrix_bytes(rng, emb_type, cfg["vocab"], d,
                                                           gain=np.sqrt(d))),
             (R_OUT_NORM, G, 0, norm(d))]
    if out_type is not None:
        slots.append((R_OUTPUT, G, out_type, random_matrix_bytes(rng, out_type, cfg["vocab"], d)))
    for L in range(nl):
        slots += [(R_ATTN_NORM, L, 0, norm(d))]
        slots += [(r, L, mt(r), random_matrix_bytes(rng, mt(r), rows, n))
                  for r, rows, n in ((R_ATTN_Q, nq, d), (R_ATTN_K, nkv, d), (R_ATTN_V, nkv, d),
                                     (R_ATTN_O, d, nq))]
        if flags & F_QK_NORM:
            slots += [(R_ATTN_Q_NORM, L, 0, norm(hd)), (R_ATTN_K_NORM, L, 0, norm(hd))]
        slots += [(R_FFN_NORM, L, 0, norm(d))]
        slots += [(r, L, mt(r), random_matrix_bytes(rng, mt(r), rows, n))
                  for r, rows, n in ((R_FFN_GATE, h, d), (R_FFN_UP, h, d), (R_FFN_DOWN, d, h))]
    return slots


def require_ref(variant: str = "avx2"):
    """The compiled reference (oracle/_ref, built from /root/reference by
    build() in the build container and shipped with the tree).  Its absence
    fails the test instead of skipping it: the model, budget, loader and
    GEMV parity rest on it, and a run without it must not read as green."""
    import pytest
    from oracle import orc

    L = orc.ref_lib(variant)
    if L is None:
        pytest.fail(f"compiled reference oracle/_ref/libg2bref_{variant}.so is missing: build it "
                    "with `make -C oracle ref` (needs /root/reference) before running the "
                    "parity tests", pytrace=False)
    return L
