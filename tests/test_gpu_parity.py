"""Device parity through the C ABI (libg2b_attn.so) against the reference
goldens and the CPU oracle on the same seeded inputs.

Bars (from the task's north star):
  * KV bytes (F32 rows and Q8_0 blocks) bit-exact;
  * attention outputs within max-abs 1e-4, softmax weights within relative
    1e-5 (helpers.check_out / check_weights): of a float64 evaluation of the
    same cache bytes, and of the reference up to the reference's own float32
    error measured against that float64 evaluation (about 1e-7 except at 32k
    contexts with dominant rows, where its serial fp32 sums drift by ~4e-4).
"""
import zlib

import numpy as np
import pytest

from helpers import (bits, check_out, check_weights, exact_attention, fwd_cases, golden_inputs,
                     golden_norms, kv_rows, load_golden, normed, q8_special_rows, sha, split_xb)
from oracle import orc

from gguf2bin_amd import attn, hip

pytestmark = pytest.mark.gpu

def ashape(o: orc.Shape) -> attn.Shape:
    return attn.Shape(o.n_layers, o.n_heads, o.n_kv_heads, o.head_dim, o.rope_theta, o.arch,
                      o.kv_q8)


class DevSeq:
    """One sequence's KV on the device, prefilled through g2b_kv_append_rows."""

    def __init__(self, ctx: attn.Context, o: orc.Shape, ctx_cap: int):
        self.ctx, self.o, self.ctx_cap = ctx, o, ctx_cap
        self.k, self.v = ctx.kv_alloc(ctx_cap)
        self.nbytes = attn.kv_bytes(ctx.shape, ctx_cap)

    def prefill(self, layer, kp, vp, pos0=0):
        if len(kp):
            kd, vd = hip.to_device(kp), hip.to_device(vp)
            self.ctx.kv_append_rows(self.k, self.v, self.ctx_cap, layer, pos0, len(kp), kd.ptr,
                                    vd.ptr)
            self.ctx.sync()

    def download(self):
        return (hip.copy_d2h(self.k, np.uint8, self.nbytes),
                hip.copy_d2h(self.v, np.uint8, self.nbytes))

    def free(self):
        self.ctx.kv_free(self.k, self.v)


# ---------------------------------------------------------------- reference goldens

@pytest.mark.parametrize("name", fwd_cases())
def test_golden_forward_case(gpu_device, name):
    d = load_golden(name)
    o, kp, vp = golden_inputs(d)
    ctx_cap, n_pre = int(d["ctx_cap"]), int(d["n_pre"])
    pos = n_pre + int(d["n_fwd"]) - 1
    qn, kn, eps = golden_norms(d)
    print(f"[golden] {name} shape={o} ctx_cap={ctx_cap} pos={pos}", flush=True)
    with attn.Context(ashape(o)) as ctx:
        if qn is not None or kn is not None:
            for L in range(o.n_layers):
                ctx.set_qk_norm(L, None if qn is None else qn[L], None if kn is None else kn[L],
                                eps)
        seq = DevSeq(ctx, o, ctx_cap)
        try:
            for L in range(o.n_layers):
                seq.prefill(L, kp, vp)
            att = hip.DeviceBuffer(o.n_heads * ctx_cap * 4)
            outs = []
            for i, xb in enumerate(d["xb"]):
                q, k, v = split_xb(o, xb)
                kd, vd = hip.to_device(k), hip.to_device(v)
                for L in range(o.n_layers):
                    qd = hip.to_device(q)
                    ctx.attn_forward(L, n_pre + i, ctx_cap, seq.k, seq.v, qd.ptr, kd.ptr, vd.ptr,
                                     att.ptr)
                ctx.sync()
                outs.append(qd.download(np.float32, o.nq))
            w = att.download(np.float32, o.n_heads * ctx_cap).reshape(o.n_heads, ctx_cap)
            w = w[:, :pos + 1]
            kc, vc = seq.download()
        finally:
            seq.free()
    kr, vr = kv_rows(o, kc, ctx_cap, pos + 1), kv_rows(o, vc, ctx_cap, pos + 1)
    assert sha(kr) == d["kc_sha"].item().decode(), "K bytes differ from the reference"
    assert sha(vr) == d["vc_sha"].item().decode(), "V bytes differ from the reference"
    last = o.n_layers - 1
    for i, xb in enumerate(d["xb"]):
        ql = normed(split_xb(o, xb)[0], None if qn is None else qn[last], o.n_heads,
                    o.head_dim, eps)
        ex, wex = exact_attention(o, ctx_cap, last, n_pre + i, kc, vc, ql)
        e_ref, e_ex, own = check_out(outs[i], d["out"][i], ex)
    print(f"[golden] {name}: |out-ref|={e_ref:.2e} |out-f64|={e_ex:.2e} ref own={own:.2e}")
    if "att_heads" in d:
        check_weights(w[d["att_heads"]], d["att"], wex[d["att_heads"]])
    else:
        check_weights(w, d["att"], wex)


def test_codec_special_rows_on_device(gpu_device):
    """Every branch of the quantiser (zero, tiny, subnormal, NaN, Inf, ties,
    fp16 overflow, -0) through the device append, V side (no RoPE) against
    the reference bytes, K side (RoPE at pos 0) against the oracle."""
    codec = load_golden("codec_q8_fp16.npz")
    rows = q8_special_rows()
    assert np.array_equal(bits(rows), bits(codec["rows"]))
    o = orc.Shape(1, 2, 1, 64, 1e4, orc.ARCH_QWEN3, True)
    n = rows.shape[0]
    with attn.Context(ashape(o)) as ctx:
        seq = DevSeq(ctx, o, n)
        try:
            for t in range(n):  # one row per call so that every row is at pos t
                seq.prefill(0, rows[t:t + 1], rows[t:t + 1], pos0=t)
            kc, vc = seq.download()
        finally:
            seq.free()
    vr = kv_rows(o, vc, n, n)[0]
    assert np.array_equal(vr, codec["q"])
    okc, ovc = orc.alloc_kv(o, n)
    for t in range(n):
        orc.kv_prefill(o, n, 0, t, okc, ovc, rows[t:t + 1], rows[t:t + 1])
    assert np.array_equal(kv_rows(o, kc, n, n), kv_rows(o, okc, n, n))


@pytest.mark.parametrize("heads", [(2, 1, 64), (16, 8, 128)])
def test_codec_special_rows_through_decode(gpu_device, heads):
    """The same quantiser branches through the append of a decode step (the
    new row that the attention kernel itself quantises, four lanes per
    block): row t of the special rows, tiled (and rolled) across nkv, is the
    new k and v at pos t.  K and V bytes must equal the oracle's (reference
    quantiser; K after RoPE at t)."""
    rows = q8_special_rows()
    nh, nkvh, hd = heads
    o = orc.Shape(1, nh, nkvh, hd, 1e4, orc.ARCH_QWEN3, True)
    n, nkv = rows.shape[0], o.nkv
    tiled = np.stack([np.roll(np.tile(rows[t], nkv // 64), 7 * t) for t in range(n)])
    tiled = tiled.astype(np.float32)
    rng = np.random.default_rng(11)
    print(f"[codec-decode] shape={o} rows={n}", flush=True)
    with attn.Context(ashape(o)) as ctx:
        seq = DevSeq(ctx, o, n)
        try:
            for t in range(n):
                q = rng.standard_normal(o.nq).astype(np.float32)
                ctx.attn_forward_host(0, t, n, seq.k, seq.v, q, tiled[t], tiled[t])
            kc, vc = seq.download()
        finally:
            seq.free()
    okc, ovc = orc.alloc_kv(o, n)
    for t in range(n):
        orc.kv_prefill(o, n, 0, t, okc, ovc, tiled[t:t + 1], tiled[t:t + 1])
    assert np.array_equal(kv_rows(o, vc, n, n), kv_rows(o, ovc, n, n))
    assert np.array_equal(kv_rows(o, kc, n, n), kv_rows(o, okc, n, n))


# ---------------------------------------------------------------- oracle comparisons

SHAPES = {
    # name: (n_heads, n_kv_heads, head_dim, arch, q8)  -> kernel variant exercised
    "qwen3_q8_g2": (16, 8, 128, orc.ARCH_QWEN3, True),     # Q8, CD=32, G=2
    "qwen3_f32_g2": (16, 8, 128, orc.ARCH_QWEN3, False),   # F32, HD=128, G=2
    "smollm2_f32_g3": (9, 3, 64, orc.ARCH_LLAMA, False),   # F32, HD=64, G=3, 5 pos/wave
    "llama3_q8_g4": (32, 8, 128, orc.ARCH_LLAMA, True),    # Q8, CD=16, G=4
    "mha_q8_g1": (8, 8, 128, orc.ARCH_QWEN3, True),        # Q8, CD=32, G=1
    "hd64_q8_g2": (8, 4, 64, orc.ARCH_LLAMA, True),        # Q8, HD=64
    "hd64_q8_g3": (6, 2, 64, orc.ARCH_QWEN3, True),        # Q8, HD=64, CD=16
    "f32_g4_hd64": (16, 4, 64, orc.ARCH_QWEN3, False),     # F32, G=4
    "f32_g1_hd128": (4, 4, 128, orc.ARCH_LLAMA, False),    # F32, G=1
    "tiny_q8_generic": (4, 2, 16, orc.ARCH_QWEN3, True),   # generic: blocks span heads
    "hd24_q8_generic": (4, 2, 24, orc.ARCH_QWEN3, True),   # generic: partial block
    "hd256_f32_generic": (4, 2, 256, orc.ARCH_LLAMA, False),
    "g8_q8_generic": (16, 2, 128, orc.ARCH_QWEN3, True),   # generic: group 8
}


# Schedules of the decode call: (all layers in one call?, g2b_ctx_tune arguments
# (split_len, chunk, stage, piece)).  "wq" forces the work queue (piece > 0),
# "static" forces static splits, "dma" / "dma_wq" the KV rows loaded straight
# into LDS (static splits, work queue), "direct" per-lane loads.
MODES = {
    "fused": (True, None),
    "layers": (False, None),
    "wq": (False, (0, 0, 2, 1)),
    "wq_fused": (True, (0, 0, 2, 8)),
    "static": (False, (0, 0, 2, -1)),
    "dma": (True, (0, 0, 1, -1)),
    "dma_wq": (False, (0, 0, 1, 1)),
    "direct": (False, (0, 0, -1, -1)),
}


def run_batch_case(o: orc.Shape, caps, poss, seed, fused: bool, want_att=True, norms=None,
                   setup=None, tune=None, misalign=0, kernel=0, sched=None, q_gain=None,
                   w_as_accurate_as_ref=False, errs=None):
    """n_seq ragged sequences, all layers: device (one fused call or layer by
    layer) against the oracle, sequence by sequence.  tune: None or the
    g2b_ctx_tune arguments for the context.  norms: None, or
    (q_norm, k_norm, eps) with q_norm/k_norm None or indexable by layer (an
    entry None: that layer has no such weights); the oracle side normalises
    its inputs with them, and they are set on the context unless setup(ctx)
    is given to do that itself.  misalign: byte offset of q, k and v in their
    device buffers (not a multiple of 16: the generic kernels run).  kernel:
    g2b_ctx_tune_kernel (0 automatic, 1 k_layer only).  sched: None or a
    dict that receives the last call's schedule (g2b_ctx_last_schedule).
    q_gain: None or nq floats that multiply every q (outlier channels).
    w_as_accurate_as_ref: the weights' float64 bar (helpers.check_weights).
    errs: None or a list that receives (max |out - float64|, max relative
    |w - float64| or None, the oracle's own relative weight error or None)
    per (sequence, layer)."""
    n_seq, nL = len(caps), o.n_layers
    rng_seed = seed * 1000
    qn, kn, eps = norms if norms else (None, None, 1e-6)
    hd = o.head_dim

    def nq_(x, L):
        return normed(x, None if qn is None else qn[L], o.n_heads, hd, eps)

    def nk_(x, L):
        return normed(x, None if kn is None else kn[L], o.n_kv_heads, hd, eps)

    with attn.Context(ashape(o)) as ctx:
        if tune:
            ctx.tune(*tune)
        ctx.tune_kernel(kernel)
        if setup:
            setup(ctx)
        elif norms:
            for L in range(nL):
                ctx.set_qk_norm(L, None if qn is None else qn[L], None if kn is None else kn[L],
                                eps)
        seqs = [DevSeq(ctx, o, c) for c in caps]
        hosts = [orc.alloc_kv(o, c) for c in caps]
        try:
            for i, (c, p) in enumerate(zip(caps, poss)):
                for L in range(nL):
                    kp = orc.normal(rng_seed + 10 * i + L, p * o.nkv).reshape(p, o.nkv)
                    vp = orc.normal(rng_seed + 500 + 10 * i + L, p * o.nkv).reshape(p, o.nkv)
                    seqs[i].prefill(L, kp, vp)
                    orc.kv_prefill(o, c, L, 0, hosts[i][0], hosts[i][1], nk_(kp, L), vp)
            q = orc.normal(seed + 1, nL * n_seq * o.nq).reshape(nL, n_seq, o.nq)
            k = orc.normal(seed + 2, nL * n_seq * o.nkv).reshape(nL, n_seq, o.nkv)
            v = orc.normal(seed + 3, nL * n_seq * o.nkv).reshape(nL, n_seq, o.nkv)
            if q_gain is not None:
                q = (q * np.asarray(q_gain, np.float32)).astype(np.float32)
            if misalign:
                qd, kd, vd = (hip.DeviceBuffer(a.nbytes + 64) for a in (q, k, v))
                for buf, a in ((qd, q), (kd, k), (vd, v)):
                    buf.upload(a, misalign)
            else:
                qd, kd, vd = hip.to_device(q), hip.to_device(k), hip.to_device(v)
            base = misalign
            stride = max(poss) + 1
            att = hip.DeviceBuffer(nL * n_seq * o.n_heads * stride * 4) if want_att else None
            ctx.batch_begin([(p, c, s.k, s.v) for p, c, s in zip(poss, caps, seqs)])
            if fused:
                ctx.attn_layers(0, nL, qd.ptr + base, kd.ptr + base, vd.ptr + base,
                                att.ptr if att else None, stride)
            else:
                for L in range(nL):
                    off_q = base + L * n_seq * o.nq * 4
                    off_k = base + L * n_seq * o.nkv * 4
                    off_a = L * n_seq * o.n_heads * stride * 4
                    ctx.attn_layers(L, 1, qd.ptr + off_q, kd.ptr + off_k, vd.ptr + off_k,
                                    (att.ptr + off_a) if att else None, stride)
            ctx.sync()
            if sched is not None:
                sched.update(ctx.last_schedule())
            out = qd.download(np.float32, q.size, base).reshape(q.shape)
            w = (att.download(np.float32, nL * n_seq * o.n_heads * stride)
                 .reshape(nL, n_seq, o.n_heads, stride) if att else None)
            dev_kv = [s.download() for s in seqs]
        finally:
            for s in seqs:
                s.free()
    for i, (c, p) in enumerate(zip(caps, poss)):
        kc, vc = hosts[i]
        for L in range(nL):
            ql, kl = nq_(q[L, i], L), nk_(k[L, i], L)
            ref, ratt = orc.attn_layer(o, c, L, p, kc, vc, ql, kl, v[L, i])
            ex, wex = exact_attention(o, c, L, p, kc, vc, ql)
            e_out = check_out(out[L, i], ref, ex)[1]
            r_w = own_w = None
            if w is not None:
                r_w = check_weights(w[L, i, :, :p + 1], ratt, wex,
                                    as_accurate_as_ref=w_as_accurate_as_ref)
                bw = wex > 1e-30
                own_w = float(np.max(np.abs(ratt[bw] - wex[bw]) / wex[bw]))
            if errs is not None:
                errs.append((e_out, r_w, own_w))
        assert np.array_equal(dev_kv[i][0], kc), f"K bytes of sequence {i}"
        assert np.array_equal(dev_kv[i][1], vc), f"V bytes of sequence {i}"
    return out


@pytest.mark.parametrize("name", sorted(SHAPES))
@pytest.mark.parametrize("mode", sorted(MODES))
def test_batched_ragged_vs_oracle(gpu_device, name, mode):
    nh, nkv, hd, arch, q8 = SHAPES[name]
    o = orc.Shape(2, nh, nkv, hd, 1e5 if arch == orc.ARCH_LLAMA else 1e6, arch, q8)
    caps = [1, 37, 300, 700, 129]
    poss = [0, 36, 211, 650, 64]  # pos 0 (attends to itself only), full, ragged
    fused, tune = MODES[mode]
    print(f"[batch] {name} mode={mode}", flush=True)
    run_batch_case(o, caps, poss, seed=zlib.crc32(name.encode()) % 1000, fused=fused, tune=tune)


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("arch", [orc.ARCH_LLAMA, orc.ARCH_QWEN3])
def test_head_dim_over_1024_leaves_q_and_k_unrotated(gpu_device, arch, q8):
    """head_dim 2048: the reference's RoPE prints a message and leaves q and
    k as they are (/root/reference/src/l3_math.c:67,86; the oracle's branch
    is pinned against the compiled reference in test_oracle_golden.py).  The
    device takes the generic kernels with RoPE off: appended K bytes
    bit-exact with the oracle's (the unrotated k), outputs and weights
    within the bars, which fail if q were rotated."""
    o = orc.Shape(2, 4, 2, 2048, 1e4, arch, q8)
    print(f"[hd2048] arch={arch} q8={q8}", flush=True)
    sched = {}
    run_batch_case(o, [1, 40, 129], [0, 39, 100], seed=2048 + arch, fused=False, sched=sched)
    assert sched["kernel"] == "k_decode_generic", sched


@pytest.mark.parametrize("name", ["qwen3_q8_g2", "qwen3_f32_g2", "smollm2_f32_g3",
                                  "llama3_q8_g4", "hd64_q8_g3", "mha_q8_g1"])
def test_static_splits_without_weights(gpu_device, name):
    """Static splits without the weights output (the decode kernel skips the
    raw-score writes; a single split writes the output itself): against the
    oracle, and, k_layer on both sides, bit for bit against the same call
    with the weights requested.  One sequence in 2..32 splits, then a ragged batch, then a
    batch of short sequences (one split each)."""
    nh, nkv, hd, arch, q8 = SHAPES[name]
    o = orc.Shape(2, nh, nkv, hd, 1e5 if arch == orc.ARCH_LLAMA else 1e6, arch, q8)
    print(f"[noatt] {name}", flush=True)
    tune = (0, 0, 0, -1)  # static splits
    # (k_layer on both sides: without the weights, shapes that k_tiles serves
    # would otherwise take it, whose sums differ in the last bits)
    plain = run_batch_case(o, [900], [899], seed=31, fused=False, want_att=False, tune=tune,
                           kernel=1)
    with_w = run_batch_case(o, [900], [899], seed=31, fused=False, want_att=True, tune=tune,
                            kernel=1)
    assert np.array_equal(plain.view(np.uint32), with_w.view(np.uint32))
    run_batch_case(o, [1, 70, 900, 300], [0, 69, 899, 150], seed=32, fused=False,
                   want_att=False, tune=tune)
    # every sequence within one split: each unit's k_layer workgroup writes the
    # output itself and no k_combine runs
    run_batch_case(o, [1, 20, 33], [0, 19, 32], seed=33, fused=True, want_att=False, tune=tune)


@pytest.mark.parametrize("name", ["qwen3_q8_g2", "qwen3_f32_g2", "smollm2_f32_g3", "hd64_q8_g3"])
@pytest.mark.parametrize("split", [3, 8, 16, 28])
def test_many_partials_merge_bit_exact(gpu_device, name, split):
    """Many partials per head: one sequence of 900 positions in 300 splits
    (more than 256: k_combine's merge in rounds) and 113 / 57 / 33 (33-256:
    k_combine_part, a workgroup per head and quarter of its dims) against the
    oracle, and the same output bits with and without the weights output (the
    weights are a separate pass over the raw scores)."""
    nh, nkv, hd, arch, q8 = SHAPES[name]
    o = orc.Shape(2, nh, nkv, hd, 1e5 if arch == orc.ARCH_LLAMA else 1e6, arch, q8)
    tune = (split, 0, 0, -1)
    print(f"[merge] {name} split={split}", flush=True)
    sched = {}
    plain = run_batch_case(o, [900], [899], seed=61, fused=False, want_att=False, tune=tune,
                           kernel=1, sched=sched)
    assert sched["max_splits"] == -(-900 // split) > 32, sched
    with_w = run_batch_case(o, [900], [899], seed=61, fused=False, want_att=True, tune=tune,
                            kernel=1)
    assert np.array_equal(plain.view(np.uint32), with_w.view(np.uint32))


@pytest.mark.parametrize("name", ["qwen3_q8_g2", "smollm2_f32_g3", "llama3_q8_g4"])
@pytest.mark.parametrize("split,stage", [(64, 0), (100, 0), (100, 2), (128, 2)])
def test_static_grid_odd_splits_and_layer_rotation(gpu_device, name, split, stage):
    """Static schedules launch an odd number of splits per sequence (an even
    count gets one empty split more) and rotate each layer's sequences over
    the grid's y index.  Eight ragged sequences, three layers in one call (so
    the rotation wraps) and layer by layer, splits of 64/128 positions (9 and
    5 per sequence: odd already) and 100 (6: one empty split added), per-lane
    and staged rows: against the oracle, KV bytes bit for bit."""
    nh, nkv, hd, arch, q8 = SHAPES[name]
    o = orc.Shape(3, nh, nkv, hd, 1e5 if arch == orc.ARCH_LLAMA else 1e6, arch, q8)
    caps = [1, 40, 130, 300, 513, 64, 257, 100]
    poss = [c - 1 for c in caps]
    tune = (split, 0, stage, -1)
    print(f"[grid] {name} split={split} stage={stage}", flush=True)
    for fused in (True, False):
        sched = {}
        run_batch_case(o, caps, poss, seed=41 + split, fused=fused, want_att=False, tune=tune,
                       sched=sched)
        assert sched["split_len"] == split and sched["max_splits"] == -(-513 // split), sched


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("norm", [False, True])
def test_stepping_across_splits(gpu_device, q8, norm):
    """A decode loop: one layer stepped one position per call from 120 to 200
    on one context, each call appending its row (k_short below 128, then
    k_layer's splits and the combine as their count grows; the first of
    those calls allocates the context's buffers), every step against the
    oracle; 8 query heads, 4 KV heads, head_dim 128, with and without
    QK-RMSNorm."""
    o = orc.Shape(1, 8, 4, 128, 1e6, orc.ARCH_QWEN3, q8)
    cap, eps = 256, 1e-6
    rng = np.random.default_rng(7 + 2 * int(q8) + int(norm))
    qn = (1 + 0.25 * rng.standard_normal(o.head_dim)).astype(np.float32) if norm else None
    kn = (1 + 0.25 * rng.standard_normal(o.head_dim)).astype(np.float32) if norm else None
    print(f"[stepping] q8={q8} norm={norm}", flush=True)
    with attn.Context(ashape(o)) as ctx:
        if norm:
            ctx.set_qk_norm(0, qn, kn, eps)
        kc, vc = ctx.kv_alloc(cap)
        host = orc.alloc_kv(o, cap)
        try:
            kp = rng.standard_normal((120, o.nkv)).astype(np.float32)
            vp = rng.standard_normal((120, o.nkv)).astype(np.float32)
            kd, vd = hip.to_device(kp), hip.to_device(vp)
            ctx.kv_append_rows(kc, vc, cap, 0, 0, 120, kd.ptr, vd.ptr)
            ctx.sync()
            orc.kv_prefill(o, cap, 0, 0, host[0], host[1],
                           normed(kp, kn, o.n_kv_heads, o.head_dim, eps), vp)
            for pos in range(120, 200):
                q = rng.standard_normal(o.nq).astype(np.float32)
                k = rng.standard_normal(o.nkv).astype(np.float32)
                v = rng.standard_normal(o.nkv).astype(np.float32)
                qd, kk, vv = hip.to_device(q), hip.to_device(k), hip.to_device(v)
                ctx.attn_forward(0, pos, cap, kc, vc, qd.ptr, kk.ptr, vv.ptr)
                ctx.sync()
                out = qd.download(np.float32, q.size)
                ql = normed(q, qn, o.n_heads, o.head_dim, eps)
                kl = normed(k, kn, o.n_kv_heads, o.head_dim, eps)
                ref, _ = orc.attn_layer(o, cap, 0, pos, host[0], host[1], ql, kl, v)
                ex, _ = exact_attention(o, cap, 0, pos, host[0], host[1], ql)
                check_out(out, ref, ex)
        finally:
            ctx.kv_free(kc, vc)



@pytest.mark.parametrize("name", ["qwen3_q8_g2", "smollm2_f32_g3"])
def test_unaligned_qkv_take_generic_kernels(gpu_device, name):
    """q/k/v that are not 16-byte aligned (the fast kernel reads 16-byte
    pieces): the call runs the generic kernels, with the same parity."""
    nh, nkv, hd, arch, q8 = SHAPES[name]
    o = orc.Shape(2, nh, nkv, hd, 1e5 if arch == orc.ARCH_LLAMA else 1e6, arch, q8)
    print(f"[unaligned] {name}", flush=True)
    run_batch_case(o, [1, 37, 300], [0, 36, 211], seed=7, fused=False, misalign=4)


SHORT_SHAPES = sorted(n for n in SHAPES if "generic" not in n)


@pytest.mark.parametrize("name", SHORT_SHAPES)
@pytest.mark.parametrize("norm", ["none", "qk"])
def test_short_contexts_vs_oracle(gpu_device, name, norm):
    """Every pos below 128 and no weights output: the short-context kernel
    (one workgroup per KV head, sequence and layer; output written over q,
    no combine) - outputs within the bars and K/V bytes bit-exact against
    the oracle, all layers in one call and layer by layer, pos 0 and 127
    (the last position it takes) included; then the same inputs through the
    split kernel (an explicit split length of 64 keeps it)."""
    nh, nkv, hd, arch, q8 = SHAPES[name]
    o = orc.Shape(2, nh, nkv, hd, 1e5 if arch == orc.ARCH_LLAMA else 1e6, arch, q8)
    seed = zlib.crc32(name.encode()) % 1000 + (7 if norm == "qk" else 0)
    norms = None
    if norm == "qk":
        qn = (1 + 0.25 * orc.normal(seed + 40, 2 * hd)).reshape(2, hd)
        kn = (1 + 0.25 * orc.normal(seed + 41, 2 * hd)).reshape(2, hd)
        norms = (qn, kn, 1e-6)
    caps, poss = [1, 2, 37, 128, 129], [0, 1, 36, 127, 64]
    print(f"[short] {name} norm={norm}", flush=True)
    a = run_batch_case(o, caps, poss, seed, fused=True, want_att=False, norms=norms)
    b = run_batch_case(o, caps, poss, seed, fused=False, want_att=False, norms=norms)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    run_batch_case(o, caps, poss, seed, fused=True, want_att=False, norms=norms,
                   tune=(64, 0, 0, 0))


QKN_SHAPES = {
    # name: (SHAPES entry, which norms, eps)
    "qwen3_q8_g2": ("qwen3_q8_g2", "qk", 1e-6),
    "qwen3_f32_g2": ("qwen3_f32_g2", "qk", 1e-6),
    "llama3_q8_g4_konly": ("llama3_q8_g4", "k", 1e-5),
    "smollm2_f32_g3_qonly": ("smollm2_f32_g3", "q", 1e-5),
    "hd24_q8_generic": ("hd24_q8_generic", "qk", 1e-6),
    "hd64_q8_g3": ("hd64_q8_g3", "qk", 1e-6),
}


@pytest.mark.parametrize("name", sorted(QKN_SHAPES))
@pytest.mark.parametrize("fused", [True, False])
def test_batched_qk_norm_vs_oracle(gpu_device, name, fused):
    """QK-RMSNorm (l5_model.c:505-511) before RoPE on the device, in the
    prefill append, the single-launch kernel and the generic path: K bytes
    bit-exact with the oracle, outputs and weights within the bars.  Layer 1
    gets different weights from layer 0."""
    base, which, eps = QKN_SHAPES[name]
    nh, nkv, hd, arch, q8 = SHAPES[base]
    o = orc.Shape(2, nh, nkv, hd, 1e5 if arch == orc.ARCH_LLAMA else 1e6, arch, q8)
    seed = zlib.crc32(name.encode()) % 1000
    qn = (1 + 0.25 * orc.normal(seed + 40, 2 * hd)).reshape(2, hd) if "q" in which else None
    kn = (1 + 0.25 * orc.normal(seed + 41, 2 * hd)).reshape(2, hd) if "k" in which else None
    print(f"[qknorm] {name} fused={fused}", flush=True)
    run_batch_case(o, [1, 37, 300, 129], [0, 36, 211, 64], seed=seed, fused=fused,
                   norms=(qn, kn, eps))


def test_qk_norm_off_and_eps_rules(gpu_device):
    """Weights can be cleared per layer (the layer runs without the norm);
    eps is one value per model."""
    o = orc.Shape(2, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True)
    w = 1 + 0.25 * orc.normal(3, o.head_dim)

    def setup(ctx):
        ctx.set_qk_norm(0, w, w, 1e-6)
        with pytest.raises(attn.G2BError) as e:
            ctx.set_qk_norm(1, w, w, 1e-5)
        assert e.value.code == attn.G2B_EINVAL
        with pytest.raises(attn.G2BError):
            ctx.set_qk_norm(2, w, w, 1e-6)  # no layer 2
        ctx.set_qk_norm(1, None, w, 1e-6)
        ctx.set_qk_norm(0, None, None, 1e-6)  # layer 0 off again

    # afterwards: layer 0 without norm, layer 1 with the k norm only
    print("[qknorm] off/eps rules", flush=True)
    run_batch_case(o, [50, 90], [49, 80], seed=11, fused=True,
                   norms=(None, [None, w], 1e-6), setup=setup)


@pytest.mark.parametrize("q8", [True, False])
@pytest.mark.parametrize("mode", ["layers", "wq"])
def test_many_splits_single_sequence(gpu_device, q8, mode):
    """A long single sequence, layer by layer: hundreds of splits (or
    hundreds of work-queue pieces claimed by many workgroups), every boundary
    crossed, partial last split or piece."""
    o = orc.Shape(1, 16, 8, 128, 1e6, orc.ARCH_QWEN3, q8)
    print(f"[splits] q8={q8} mode={mode}", flush=True)
    run_batch_case(o, [6000], [5999], seed=77, fused=False,
                   tune=(0, 0, 2, 12) if mode == "wq" else None)


@pytest.mark.parametrize("piece", [0, 8])
def test_work_queue_more_units_than_workgroups(gpu_device, piece):
    """One call over 24 layers x 32 ragged sequences (768 units, more than
    the resident workgroups of the work-queue grid): workgroups take the
    never-assigned units from the counter in turn, then steal pieces."""
    o = orc.Shape(24, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True)
    rng = np.random.default_rng(41 + piece)
    poss = [int(x) for x in rng.integers(40, 200, 32)]
    caps = [p + 1 + int(x) for p, x in zip(poss, rng.integers(0, 5, 32))]
    print(f"[wq-units] piece={piece} units={o.n_layers * len(poss)}", flush=True)
    run_batch_case(o, caps, poss, 2600 + piece, fused=True, tune=(0, 0, 2, piece))


def test_work_queue_counters_across_calls(gpu_device):
    """One context, work-queue calls with different unit counts in turn (one
    layer, both layers, the other layer, a smaller batch, both layers
    again): the per-launch counters are zeroed between calls over the extent
    any earlier call used, so every call matches the oracle."""
    o = orc.Shape(2, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True)
    caps, poss = [400, 90, 257], [399, 60, 256]
    nL, n_seq = o.n_layers, len(caps)
    with attn.Context(ashape(o)) as ctx:
        ctx.tune(0, 0, 2, 4)
        seqs = [DevSeq(ctx, o, c) for c in caps]
        hosts = [orc.alloc_kv(o, c) for c in caps]
        try:
            for i, (c, p) in enumerate(zip(caps, poss)):
                for L in range(nL):
                    kp = orc.normal(900 + 10 * i + L, p * o.nkv).reshape(p, o.nkv)
                    vp = orc.normal(950 + 10 * i + L, p * o.nkv).reshape(p, o.nkv)
                    seqs[i].prefill(L, kp, vp)
                    orc.kv_prefill(o, c, L, 0, hosts[i][0], hosts[i][1], kp, vp)
            q = orc.normal(31, nL * n_seq * o.nq).reshape(nL, n_seq, o.nq)
            k = orc.normal(32, nL * n_seq * o.nkv).reshape(nL, n_seq, o.nkv)
            v = orc.normal(33, nL * n_seq * o.nkv).reshape(nL, n_seq, o.nkv)
            refs = {}
            for i, (c, p) in enumerate(zip(caps, poss)):
                for L in range(nL):
                    kc, vc = orc.alloc_kv(o, c)
                    kc[:], vc[:] = hosts[i][0], hosts[i][1]
                    ref, _ = orc.attn_layer(o, c, L, p, kc, vc, q[L, i], k[L, i], v[L, i])
                    ex, _ = exact_attention(o, c, L, p, kc, vc, q[L, i])
                    refs[(L, i)] = (ref, ex)
            for step, (batch, layers) in enumerate([([0, 1, 2], [0]), ([0, 1, 2], [0, 1]),
                                                    ([0, 1, 2], [1]), ([1], [0, 1]),
                                                    ([2, 0], [1]), ([0, 1, 2], [0, 1])]):
                ctx.batch_begin([(poss[i], caps[i], seqs[i].k, seqs[i].v) for i in batch])
                L0, nl, nb = layers[0], len(layers), len(batch)
                qs = np.ascontiguousarray(q[L0:L0 + nl][:, batch])
                qd = hip.to_device(qs)
                ks = hip.to_device(np.ascontiguousarray(k[L0:L0 + nl][:, batch]))
                vs = hip.to_device(np.ascontiguousarray(v[L0:L0 + nl][:, batch]))
                ctx.attn_layers(L0, nl, qd.ptr, ks.ptr, vs.ptr)
                ctx.sync()
                out = qd.download(np.float32, qs.size).reshape(qs.shape)
                for a, L in enumerate(layers):
                    for b, i in enumerate(batch):
                        ref, ex = refs[(L, i)]
                        check_out(out[a, b], ref, ex)
        finally:
            for s_ in seqs:
                s_.free()


def test_forward_host_matches_device_call(gpu_device):
    o = orc.Shape(3, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True)
    ctx_cap, pos = 200, 150
    with attn.Context(ashape(o)) as ctx:
        seq = DevSeq(ctx, o, ctx_cap)
        kc, vc = orc.alloc_kv(o, ctx_cap)
        try:
            kp = orc.normal(5, pos * o.nkv).reshape(pos, o.nkv)
            vp = orc.normal(6, pos * o.nkv).reshape(pos, o.nkv)
            seq.prefill(2, kp, vp)
            orc.kv_prefill(o, ctx_cap, 2, 0, kc, vc, kp, vp)
            q, k, v = orc.normal(7, o.nq), orc.normal(8, o.nkv), orc.normal(9, o.nkv)
            out, w = ctx.attn_forward_host(2, pos, ctx_cap, seq.k, seq.v, q, k, v, want_att=True)
            dk, dv = seq.download()
        finally:
            seq.free()
    ref, ratt = orc.attn_layer(o, ctx_cap, 2, pos, kc, vc, q, k, v)
    ex, wex = exact_attention(o, ctx_cap, 2, pos, kc, vc, q)
    check_out(out, ref, ex)
    check_weights(w[:, :pos + 1], ratt, wex)
    assert np.array_equal(dk, kc) and np.array_equal(dv, vc)


def test_errors_map_to_reference_conditions(gpu_device):
    o = orc.Shape(2, 4, 2, 64, 1e4, orc.ARCH_QWEN3, True)
    with attn.Context(ashape(o)) as ctx:
        k, v = ctx.kv_alloc(16)
        buf = hip.DeviceBuffer(o.nq * 4 * 4)
        try:
            with pytest.raises(attn.G2BError) as e:  # pos >= ctx (l5_model.c:469)
                ctx.attn_forward(0, 16, 16, k, v, buf.ptr, buf.ptr, buf.ptr)
            assert e.value.code == attn.G2B_EPOS
            with pytest.raises(attn.G2BError) as e:
                ctx.attn_forward(0, -1, 16, k, v, buf.ptr, buf.ptr, buf.ptr)
            assert e.value.code == attn.G2B_EPOS
            with pytest.raises(attn.G2BError) as e:  # no KV (l5_model.c:481)
                ctx.attn_forward(0, 3, 16, None, v, buf.ptr, buf.ptr, buf.ptr)
            assert e.value.code == attn.G2B_ENOKV
            with pytest.raises(attn.G2BError) as e:
                ctx.attn_forward(2, 3, 16, k, v, buf.ptr, buf.ptr, buf.ptr)
            assert e.value.code == attn.G2B_EINVAL
            with pytest.raises(attn.G2BError) as e:  # caches are read in 16-byte pieces
                ctx.attn_forward(0, 3, 16, k + 8, v, buf.ptr, buf.ptr, buf.ptr)
            assert e.value.code == attn.G2B_EINVAL
            with pytest.raises(attn.G2BError) as e:
                ctx.batch_begin([(3, 16, k, v + 4)])
            assert e.value.code == attn.G2B_EINVAL
            with pytest.raises(attn.G2BError) as e:
                ctx.batch_begin([(3, 16, k, v), (16, 16, k, v)])
            assert e.value.code == attn.G2B_EPOS
            ctx.batch_begin([(3, 16, k, v)])
            with pytest.raises(attn.G2BError) as e:  # att row shorter than pos+1
                ctx.attn_layers(0, 1, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 3)
            assert e.value.code == attn.G2B_EINVAL
            with pytest.raises(attn.G2BError) as e:
                ctx.kv_append_rows(k, v, 16, 0, 10, 7, buf.ptr, buf.ptr)
            assert e.value.code == attn.G2B_EPOS
            ctx.sync()
        finally:
            ctx.kv_free(k, v)


def test_synth_fill_matches_host_stream(gpu_device):
    """The device generator reproduces the host SplitMix64/Box-Muller stream
    (so bench inputs are the same distribution the oracle times), checked
    through the stored bytes of a small fill."""
    o = orc.Shape(2, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True)
    ctx_cap, n_pos, base, seq_id = 64, 50, 2024, 3
    with attn.Context(ashape(o)) as ctx:
        s = DevSeq(ctx, o, ctx_cap)
        try:
            ctx.synth_fill_kv(s.k, s.v, ctx_cap, 0, 2, 0, n_pos, base, seq_id, 1.0)
            ctx.sync()
            dk, dv = s.download()
        finally:
            s.free()
    kc, vc = orc.alloc_kv(o, ctx_cap)
    for L in range(2):
        kp = orc.normal(orc.stream_seed(base, seq_id, L, 0), n_pos * o.nkv).reshape(n_pos, o.nkv)
        vp = orc.normal(orc.stream_seed(base, seq_id, L, 1), n_pos * o.nkv).reshape(n_pos, o.nkv)
        sel = orc.normal(orc.stream_seed(base, seq_id, L, 5), n_pos)
        kp[sel > 1.0] *= np.float32(8.0)
        orc.kv_prefill(o, ctx_cap, L, 0, kc, vc, kp, vp)
    mism = np.count_nonzero(dk != kc) + np.count_nonzero(dv != vc)
    # double-precision log/cos/sin on the device may differ from glibc in the
    # last bit; after rounding to float that flips a value at most rarely
    assert mism <= 4, f"{mism} bytes differ"


def test_hbm_info_as_budget(gpu_device):
    """g2b_hbm_info reports the device's HBM, and g2b_auto_budget against the
    free HBM picks a plan whose KV then allocates (one sequence, c4 shape)."""
    s = attn.Shape(28, 16, 8, 128, 1e6, attn.ARCH_QWEN3, False)
    with attn.Context(s) as ctx:
        free, total = ctx.hbm_info()
        print(f"[hbm] free={free} total={total}", flush=True)
        assert 0 < free <= total
        q8, c, fits = attn.auto_budget(s, 40960, 1, free // 4)
        assert fits and c == 40960 and not q8  # 9.4 GB of F32 KV fits a quarter of HBM
        q8, c, fits = attn.auto_budget(s, 40960, 256, free // 4)
        assert fits and q8 and c < 40960  # 256 sequences need Q8_0 and a shorter context
        k, v = ctx.kv_alloc(c)
        ctx.kv_free(k, v)
