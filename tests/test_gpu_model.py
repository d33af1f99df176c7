"""A whole decode step on the device (include/g2b_model.h) against the
compiled reference's own model_load_g2bx + model_forward on the same G2BX
files (random weights written by tests/helpers.write_g2bx, and the
reference's tiny.g2bx).

Bar, F32 KV: the logits of every step within 2e-5 x max(1, max|reference
logits|).  Both sides are fp32 with different summation orders (GEMVs,
rmsnorm sums, attention); measured 2.6e-7 - 8.1e-7 of the largest logit over
24 steps.  Q8_0 KV: within 2e-3 x the same scale.  The appended k and v come
from GEMVs whose fp32 sums differ from the reference's in the last bits, and
an element within that distance of a Q8_0 rounding boundary quantises one
step (its block's amax/127) differently; that moves the position's scores
and weights.  Measured up to 1.2e-4 of the logit scale.  In both modes the
argmax must agree wherever the reference's top-two gap exceeds twice the bar.
"""
import os

import numpy as np
import pytest

from helpers import (F_QK_NORM, F_TIE_EMBD, R_ATTN_K, R_ATTN_O, R_ATTN_Q, R_FFN_DOWN,
                     random_model_slots, require_ref, write_g2bx)
from oracle import orc
from gguf2bin_amd import attn

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
TINY = os.path.join(HERE, "golden", "tiny.g2bx")

CASES = {
    # name: (cfg, arch, flags, matrix type, embedding type, output type or None (tied))
    "qwen3_q8_tied": (dict(dim=128, hidden_dim=256, n_layers=2, n_heads=4, n_kv_heads=2,
                           vocab=300, seq_len=64, head_dim=32, eps=1e-6, rope_theta=1e6),
                      attn.ARCH_QWEN3, F_QK_NORM | F_TIE_EMBD, 8, 8, None),
    "llama_q4_f16emb": (dict(dim=256, hidden_dim=512, n_layers=3, n_heads=8, n_kv_heads=2,
                             vocab=500, seq_len=128, head_dim=32, eps=1e-5, rope_theta=5e5),
                        attn.ARCH_LLAMA, 0, 2, 1, 0),
    "qwen3_hd128_q8": (dict(dim=512, hidden_dim=1024, n_layers=2, n_heads=8, n_kv_heads=4,
                            vocab=1000, seq_len=256, head_dim=128, eps=1e-6, rope_theta=1e6),
                       attn.ARCH_QWEN3, F_QK_NORM, 8, 8, 8),
    "qwen2_f32": (dict(dim=128, hidden_dim=192, n_layers=2, n_heads=4, n_kv_heads=4, vocab=200,
                       seq_len=64, head_dim=32, eps=1e-5, rope_theta=1e4),
                  attn.ARCH_QWEN2, 0, 0, 0, 0),
    # Q/K/V of mixed types and an F32 Wo (their plain launches), gate/up in one
    # launch, down over 144 blocks per row (the split-row GEMV with SiLU x up)
    "mixed_types": (dict(dim=256, hidden_dim=4608, n_layers=2, n_heads=4, n_kv_heads=2,
                         vocab=300, seq_len=64, head_dim=64, eps=1e-6, rope_theta=1e6),
                    attn.ARCH_QWEN3, F_QK_NORM, {"*": 8, R_ATTN_K: 2, R_ATTN_O: 0, R_FFN_DOWN: 2},
                    8, 2),
    # the types matmul_q runs through its dequantising fallback: F16
    # matrices, embeddings and output; Q4_1 matrices and tied Q4_1 embeddings
    "llama_f16": (dict(dim=256, hidden_dim=512, n_layers=2, n_heads=8, n_kv_heads=2,
                       vocab=400, seq_len=64, head_dim=32, eps=1e-5, rope_theta=5e5),
                  attn.ARCH_LLAMA, 0, 1, 1, 1),
    "qwen3_q4_1_tied": (dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2,
                             vocab=300, seq_len=64, head_dim=64, eps=1e-6, rope_theta=1e6),
                        attn.ARCH_QWEN3, F_QK_NORM | F_TIE_EMBD, 3, 3, None),
    # an output matrix of 40000 Q8_0 rows: rmsnorm + logits with x as digit
    # planes (the lm-head form)
    "qwen3_q8_big_vocab": (dict(dim=512, hidden_dim=1024, n_layers=1, n_heads=8, n_kv_heads=4,
                                vocab=40000, seq_len=64, head_dim=64, eps=1e-6, rope_theta=1e6),
                           attn.ARCH_QWEN3, F_QK_NORM, 8, 8, 8),
    # 1024-element rows and 33000 output rows: rmsnorm + logits on the int8
    # matrix cores (tied Q8_0 embeddings; a Q4_0 output matrix)
    "qwen3_q8_mma_lm_head": (dict(dim=1024, hidden_dim=1024, n_layers=1, n_heads=8, n_kv_heads=4,
                                  vocab=33000, seq_len=64, head_dim=128, eps=1e-6,
                                  rope_theta=1e6),
                             attn.ARCH_QWEN3, F_QK_NORM | F_TIE_EMBD, 8, 8, None),
    "llama_q4_mma_lm_head": (dict(dim=1024, hidden_dim=1024, n_layers=1, n_heads=8, n_kv_heads=2,
                                  vocab=33000, seq_len=64, head_dim=128, eps=1e-5,
                                  rope_theta=5e5),
                             attn.ARCH_LLAMA, 0, 2, 2, 2),
    # rows of 132 blocks: rmsnorm + Q/K/V, rmsnorm + gate/up and rmsnorm +
    # logits on the split-row GEMV
    "wide_dim_q4": (dict(dim=4224, hidden_dim=512, n_layers=1, n_heads=4, n_kv_heads=4,
                         vocab=128, seq_len=64, head_dim=64, eps=1e-5, rope_theta=5e5),
                    attn.ARCH_LLAMA, 0, 2, 0, 8),
}


def make(tmp_path, name, seed=0):
    cfg, arch, flags, mt, et, ot = CASES[name]
    rng = np.random.default_rng(seed + sum(map(ord, name)))
    p = str(tmp_path / f"{name}.g2bx")
    write_g2bx(p, cfg, arch, flags, random_model_slots(rng, cfg, flags, mt, et, ot))
    return p, cfg, rng


def check(dev, ref, what, kv_q8=False):
    rel = 2e-3 if kv_q8 else 2e-5
    for i in range(len(ref)):
        scale = max(1.0, float(np.abs(ref[i]).max()))
        err = float(np.abs(dev[i] - ref[i]).max())
        assert err <= rel * scale, f"{what} step {i}: {err:.3e} (scale {scale:.3e})"
        top2 = np.sort(ref[i])[-2:]
        if top2[1] - top2[0] > 2 * rel * scale:
            assert dev[i].argmax() == ref[i].argmax(), f"{what} step {i}: argmax"


@pytest.mark.parametrize("kv_q8", [False, True])
@pytest.mark.parametrize("name", sorted(CASES))
def test_forward_matches_reference(gpu_device, tmp_path, name, kv_q8):
    require_ref()
    p, cfg, rng = make(tmp_path, name)
    toks = rng.integers(0, cfg["vocab"], 24)
    print(f"[model] {name} kv_q8={kv_q8}", flush=True)
    ref = orc.ref_model_forward(p, toks, cfg["vocab"], kv_q8, 0)
    with attn.Model(p, kv_q8=kv_q8) as m:
        assert m.cfg["dim"] == cfg["dim"] and m.ctx_cap == cfg["seq_len"]
        dev = np.stack([m.forward(int(t), i) for i, t in enumerate(toks)])
    check(dev, ref, name, kv_q8)


def test_forward_long_context(gpu_device, tmp_path):
    """300 steps of one model: attention over many splits as pos grows."""
    require_ref()
    cfg = dict(dim=256, hidden_dim=384, n_layers=2, n_heads=4, n_kv_heads=2, vocab=256,
               seq_len=512, head_dim=64, eps=1e-6, rope_theta=1e6)
    rng = np.random.default_rng(77)
    p = str(tmp_path / "long.g2bx")
    write_g2bx(p, cfg, attn.ARCH_QWEN3, F_QK_NORM, random_model_slots(rng, cfg, F_QK_NORM, 8, 8, 2))
    toks = rng.integers(0, cfg["vocab"], 300)
    ref = orc.ref_model_forward(p, toks, cfg["vocab"], True, 0)
    with attn.Model(p, kv_q8=True) as m:
        dev = np.stack([m.forward(int(t), i) for i, t in enumerate(toks)])
    check(dev, ref, "long", True)


@pytest.mark.parametrize("kv_q8", [False, True])
def test_graph_replays_match_eager(gpu_device, tmp_path, kv_q8):
    """With the graph on, the first forward of each position bucket (64,
    128, ... positions) captures its step and later ones replay it; stepped
    in turn with an eager model of the same file (its launches one by one,
    scheduled for the step's own position; the synchronisation that ends
    every forward between the replays), each replay must give the eager
    step's logits bit for bit.  200 positions cover three buckets: 63 and
    127, whose captured attention is k_short (as every eager step below 128
    positions), and 255, whose captured attention is k_layer over two splits
    and k_combine, replayed against eager steps at positions 128-199 (k_layer
    with one or two splits: its own output, or k_combine)."""
    p, cfg, rng = make(tmp_path, "qwen3_hd128_q8", seed=5)
    toks = [int(t) for t in rng.integers(0, cfg["vocab"], 200)]
    with attn.Model(p, kv_q8=kv_q8) as g, attn.Model(p, kv_q8=kv_q8) as e:
        g.use_graph(True)
        e.use_graph(False)
        for i, t in enumerate(toks):
            a, b = g.forward(t, i), e.forward(t, i)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {i}"


@pytest.mark.parametrize("name", ["qwen3_q8_tied", "llama_q4_f16emb", "mixed_types",
                                  "wide_dim_q4", "qwen3_q8_big_vocab", "qwen3_q8_mma_lm_head",
                                  "llama_q4_mma_lm_head"])
def test_fused_launches_match_separate(gpu_device, tmp_path, name):
    """The fused GEMV launches (rmsnorm, SiLU x up and the residual inside
    them, Q/K/V and gate/up as segments of one launch) against the same step
    as separate launches, both eager: the same arithmetic in the same order,
    so the logits agree bit for bit."""
    p, cfg, rng = make(tmp_path, name, seed=9)
    toks = [int(t) for t in rng.integers(0, cfg["vocab"], 12)]
    with attn.Model(p, kv_q8=True) as f, attn.Model(p, kv_q8=True) as u:
        f.use_graph(False)
        u.use_graph(False)
        u.set_fused(False)
        for i, t in enumerate(toks):
            a, b = f.forward(t, i), u.forward(t, i)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {i}"


def test_tiny_g2bx(gpu_device):
    """The reference's own tiny model (all-zero Q4_0 weights: logits 0)."""
    require_ref()
    ref = orc.ref_model_forward(TINY, [1, 5, 9], 128)
    with attn.Model(TINY) as m:
        assert m.arch == attn.ARCH_QWEN3 and m.flags == 3
        dev = np.stack([m.forward(t, i) for i, t in enumerate([1, 5, 9])])
    assert np.array_equal(dev, ref)


def test_forward_errors(gpu_device, tmp_path):
    """model_forward's checks (l5_model.c:469-483: pos and token out of range
    zero the logits) and the loader's rejections."""
    p, cfg, rng = make(tmp_path, "qwen2_f32")
    with attn.Model(p) as m:
        rc, out = m.forward_rc(0, cfg["seq_len"])
        assert rc == attn.G2B_EPOS and not out.any()
        rc, out = m.forward_rc(cfg["vocab"], 0)
        assert rc == attn.G2B_EINVAL and not out.any()
        rc, out = m.forward_rc(-1, 0)
        assert rc == attn.G2B_EINVAL and not out.any()
    cfg0, arch, flags, mt, et, ot = CASES["qwen2_f32"]
    slots = random_model_slots(np.random.default_rng(1), cfg0, flags, mt, et, ot)
    # a layer without ffn_down: the forward fails (require_slot) and leaves the logits
    q = str(tmp_path / "missing.g2bx")
    write_g2bx(q, cfg0, arch, flags, [s for s in slots if not (s[0] == R_FFN_DOWN and s[1] == 1)])
    with attn.Model(q) as m:
        rc, out = m.forward_rc(3, 0)
        assert rc == attn.G2B_EINVAL and np.all(out == 7.0)
    # a K-quant matrix: no device GEMV
    u = str(tmp_path / "q6k.g2bx")
    write_g2bx(u, cfg0, arch, flags, [(s[0], s[1], 14 if s[0] == R_ATTN_Q else s[2], s[3])
                                      for s in slots])
    with pytest.raises(attn.G2BError) as e:
        attn.Model(u)
    assert e.value.code == attn.G2B_EUNSUP
    # a slot too small for its role is refused before anything reads it
    t = str(tmp_path / "short.g2bx")
    write_g2bx(t, cfg0, arch, flags, [(s[0], s[1], s[2], s[3][:-4] if s[0] == R_ATTN_Q else s[3])
                                      for s in slots])
    with pytest.raises(attn.G2BError) as e:
        attn.Model(t)
    assert e.value.code == attn.G2B_EINVAL


@pytest.mark.parametrize("name", ["qwen3_q8_tied", "qwen3_hd128_q8", "llama_q4_f16emb"])
@pytest.mark.parametrize("kv_q8", [False, True])
def test_patched_reference_runs_device_attention(gpu_device, tmp_path, name, kv_q8):
    """The reference's own model_forward with the maintainer's drop-in patch
    applied (oracle/refpatch.py; KV from g2b_kv_alloc in alloc_rt, the attention block
    as g2b_attn_forward_host, QK-RMSNorm weights handed over at load) against
    the unpatched reference on the same file: everything but the attention
    is the reference's own code.  140 tokens reach the split kernel.  F32 KV:
    within 2e-5 of the logit scale; Q8_0 KV: the appended rows are the same
    bytes for the same k/v, but a last-bit difference of the attention output
    reaches the next layer's k/v (the bar of test_forward_matches_reference)."""
    require_ref()
    require_ref("gpu")
    p, cfg, rng = make(tmp_path, name, seed=13)
    n = min(140, cfg["seq_len"])
    toks = [int(t) for t in rng.integers(0, cfg["vocab"], n)]
    ref = orc.ref_model_forward(p, toks, cfg["vocab"], kv_q8, 0)
    dev = orc.ref_model_forward(p, toks, cfg["vocab"], kv_q8, 0, variant="gpu")
    check(dev, ref, f"{name} patched reference", kv_q8)
