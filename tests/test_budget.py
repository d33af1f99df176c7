"""HBM budgeting (include/g2b_attn.h: g2b_model_kv_bytes, g2b_clamp_ctx,
g2b_hbm_bytes, g2b_auto_budget) - host arithmetic, no GPU.

Chain of checks:
  1. the oracle's est_for and model_auto_budget restatements against the
     compiled reference (oracle/_ref, a Model with no tokenizer), on grids of
     shapes, contexts and budgets that cross every branch of the loop;
  2. the product's decision (g2b_auto_budget) against the pinned oracle loop
     driven by the product's own HBM estimate;
  3. the HBM estimate's KV term against g2b_kv_bytes (pinned to the
     reference's alloc_rt sizes in test_abi.py), and its other terms by
     linearity in n_seq and ctx.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import require_ref
from oracle import orc
from gguf2bin_amd import attn

# (dim, hidden, n_layers, n_heads, n_kv_heads, vocab, head_dim)
CFGS = [
    (64, 128, 2, 4, 2, 1000, 32),      # nkv = 64: whole Q8 blocks
    (96, 200, 3, 6, 2, 50, 16),        # nkv = 32
    (48, 64, 1, 3, 3, 70000, 16),      # vocab dominates the buffer; nkv = 48 (partial block)
    (1024, 3072, 28, 16, 8, 151936, 128),
]
SEQ_LENS = [0, 1, 100, 256, 257, 300, 4096, 40000]


@pytest.mark.parametrize("cfg", CFGS)
def test_oracle_est_for_matches_reference(cfg):
    L = require_ref()
    dim, hid, nl, nh, nkvh, vocab, hd = cfg
    for ctx in (1, 255, 256, 2048, 40000):
        for q8 in (0, 1):
            want = L.ref_est_for(dim, hid, nl, nh, nkvh, vocab, 4096, hd, ctx, q8)
            assert orc.est_for_ram(dim, hid, nl, nh, nkvh, vocab, hd, ctx, q8) == want


@pytest.mark.parametrize("cfg", CFGS[:3])
def test_oracle_auto_budget_matches_reference(cfg):
    """Budgets around every threshold of the loop: below the floor, between
    halvings, just under / at / over the F32 and Q8_0 estimates."""
    L = require_ref()
    dim, hid, nl, nh, nkvh, vocab, hd = cfg
    for seq_len in SEQ_LENS:
        for q8 in (0, 1):
            start = seq_len if seq_len > 0 else 2048
            marks = set()
            c = start
            while True:
                for m in (0, 1):
                    e = orc.est_for_ram(dim, hid, nl, nh, nkvh, vocab, hd, c, m)
                    marks.update((e - 1, e, e + 1))
                if c <= 256:
                    break
                c //= 2
            marks.update((1, 10, 1 << 40))
            for budget in sorted(b for b in marks if b > 0):
                ctx, q, rc = C.c_int32(), C.c_int32(), None
                rc = L.ref_auto_budget(dim, hid, nl, nh, nkvh, vocab, seq_len, hd, q8, budget,
                                       C.byref(ctx), C.byref(q))
                est = lambda cc, qq: orc.est_for_ram(dim, hid, nl, nh, nkvh, vocab, hd, cc, qq)
                octx, oq8, _ = orc.auto_budget(est, seq_len, q8, budget)
                assert rc == 0
                assert (octx, oq8) == (ctx.value, q.value), (seq_len, q8, budget)


def shape(nl, nh, nkvh, hd, q8):
    return attn.Shape(nl, nh, nkvh, hd, 1e4, attn.ARCH_LLAMA, q8)


@pytest.mark.parametrize("nl,nh,nkvh,hd", [(2, 4, 2, 32), (3, 6, 2, 16), (28, 16, 8, 128),
                                           (32, 32, 8, 128)])
@pytest.mark.parametrize("q8_in", [False, True])
@pytest.mark.parametrize("n_seq", [1, 7, 256])
def test_auto_budget_follows_reference_loop(nl, nh, nkvh, hd, q8_in, n_seq):
    s = shape(nl, nh, nkvh, hd, q8_in)
    for seq_len in SEQ_LENS:
        est = lambda c, q: attn.hbm_bytes(shape(nl, nh, nkvh, hd, bool(q)), c, bool(q), n_seq)
        start = seq_len if seq_len > 0 else 2048
        marks = {1, 1 << 62}
        c = start
        while True:
            for m in (0, 1):
                e = est(c, m)
                marks.update((e - 1, e, e + 1))
            if c <= 256:
                break
            c //= 2
        for budget in sorted(b for b in marks if b > 0):
            q8, ctx, fits = attn.auto_budget(s, seq_len, n_seq, budget)
            octx, oq8, ofits = orc.auto_budget(est, seq_len, int(q8_in), budget)
            assert (ctx, int(q8), fits) == (octx, oq8, ofits), (seq_len, budget)
            # the decision's own properties, independent of the restatement:
            # ctx is on the halving sequence from start, the one before it
            # did not fit, and it fits unless it is the floor
            seq = [start]
            while seq[-1] > 256:
                seq.append(seq[-1] // 2)
            assert ctx in seq
            k = seq.index(ctx)
            if k > 0:
                assert est(seq[k - 1], int(q8)) > budget
            assert fits == (est(ctx, int(q8)) <= budget)
            if not fits:
                assert k == len(seq) - 1
            if q8 and not q8_in:
                assert est(start, 0) > budget


def _grain(b, g=2 << 20):
    return -(-b // g) * g


def test_hbm_bytes_terms():
    """The estimate's structure: whole allocation grains; two caches per
    sequence (each its cache bytes and 256 bytes of read slack, rounded up);
    the partials of a call over all layers at the per-layer cap of
    max(2048, 64*n_seq) splits; monotone in n_seq and ctx.  That the runtime
    stays within it is measured on the device (test_gpu_budget.py)."""
    G = 2 << 20
    for (nl, nh, nkvh, hd) in [(2, 4, 2, 32), (28, 16, 8, 128), (30, 9, 3, 64)]:
        for q8 in (False, True):
            s = shape(nl, nh, nkvh, hd, q8)
            for ctx in (1, 300, 8193):
                cache = _grain(attn.kv_bytes(s, ctx) + 256)
                prev = 0
                for n_seq in (1, 2, 31, 32, 33, 100, 101):
                    b = attn.hbm_bytes(s, ctx, q8, n_seq)
                    assert b % G == 0
                    assert b > prev
                    prev = b
                    splits = max(2048, 64 * n_seq)
                    parts = nl * splits * nh * (4 + hd) * 4
                    assert b >= 2 * n_seq * cache + _grain(parts) + _grain(ctx * hd * 4)
                    # the sequence-independent part does not depend on n_seq
                    # below the split floor (n_seq <= 32), nor the caches'
                    # share on anything but n_seq
                    if n_seq <= 31:
                        nxt = attn.hbm_bytes(s, ctx, q8, n_seq + 1)
                        assert nxt - b >= 2 * cache
                assert attn.hbm_bytes(s, ctx + 1, q8, 3) >= attn.hbm_bytes(s, ctx, q8, 3)
            assert attn.model_kv_bytes(s, 4096, q8) == 2 * attn.kv_bytes(s, 4096)
            assert attn.model_kv_bytes(s, 0, q8) == 0


def test_clamp_ctx_and_errors():
    assert attn.clamp_ctx(0, 4096) == 256
    assert attn.clamp_ctx(-5, 100) == 100  # 256, then capped at seq_len
    assert attn.clamp_ctx(5000, 4096) == 4096
    assert attn.clamp_ctx(5000, 0) == 5000
    s = shape(2, 4, 2, 32, False)
    for args in ((0, 1, 0), (0, 0, 100)):  # budget 0; n_seq 0
        seq_len, n_seq, budget = 4096, args[1], args[2]
        with pytest.raises(attn.G2BError):
            attn.auto_budget(s, seq_len, n_seq, budget)
    L = attn.lib()
    q8, ctx = C.c_int32(), C.c_int32()
    assert L.g2b_auto_budget(None, 4096, 1, 1 << 30, C.byref(q8), C.byref(ctx)) == attn.G2B_EINVAL
    assert attn.hbm_bytes(s, 0, False, 1) == 0
    # too small for anything: ENOMEM with the floor values written
    q8b, ctxb, fits = attn.auto_budget(s, 4096, 1, 10)
    assert (q8b, ctxb, fits) == (True, 256, False)
