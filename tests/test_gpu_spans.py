"""k_short over several spans of 128 positions, which calls take only under
g2b_ctx_tune_kernel(3) (the automatic choice runs k_layer's splits past 128
positions; below 128 positions k_short is a single span): each span of a (sequence, layer, KV head) writes its partials, the last to
take a ticket merges them and writes the output; no combine launch.
Against the oracle on the same seeded inputs: K and V bytes bit-exact,
outputs within max-abs 1e-4 of float64 and of the oracle up to its own
float32 error (helpers.check_out).  Every specialised shape, ragged
batches (sequences of one span beside sequences of many), all layers in
one call and layer by layer, QK-RMSNorm, long single sequences, and the
counters: they must be zero again after every launch, which two identical
calls in a row check (a counter left over would stop the second call's
merge)."""
import zlib

import numpy as np
import pytest

from helpers import check_out, exact_attention
from oracle import orc
from test_gpu_parity import SHAPES, run_batch_case

from gguf2bin_amd import attn, hip

pytestmark = pytest.mark.gpu

SPAN_SHAPES = sorted(n for n in SHAPES if "generic" not in n)


def oshape(name, layers=2):
    nh, nkv, hd, arch, q8 = SHAPES[name]
    return orc.Shape(layers, nh, nkv, hd, 1e5 if arch == orc.ARCH_LLAMA else 1e6, arch, q8)


@pytest.mark.parametrize("name", SPAN_SHAPES)
@pytest.mark.parametrize("fused", [True, False])
def test_ragged_batch_vs_oracle(gpu_device, name, fused):
    o = oshape(name)
    caps = [1, 129, 130, 700, 2049, 256]
    poss = [0, 127, 129, 650, 2048, 255]  # one span; spans of 1 position; whole spans
    print(f"[spans] {name} fused={fused}", flush=True)
    run_batch_case(o, caps, poss, seed=zlib.crc32(name.encode()) % 1000, fused=fused,
                   want_att=False, kernel=3)


@pytest.mark.parametrize("name", ["qwen3_q8_g2", "smollm2_f32_g3", "llama3_q8_g4"])
def test_qk_norm_vs_oracle(gpu_device, name):
    o = oshape(name)
    hd = o.head_dim
    seed = zlib.crc32(name.encode()) % 1000 + 3
    qn = (1 + 0.25 * orc.normal(seed + 40, 2 * hd)).reshape(2, hd)
    kn = (1 + 0.25 * orc.normal(seed + 41, 2 * hd)).reshape(2, hd)
    print(f"[spans] qknorm {name}", flush=True)
    run_batch_case(o, [300, 1000, 129], [299, 640, 128], seed=seed, fused=True,
                   want_att=False, norms=(qn, kn, 1e-6), kernel=3)


@pytest.mark.parametrize("q8", [True, False])
def test_long_single_sequence(gpu_device, q8):
    """One sequence, layer by layer, at 20000 positions (157 spans, 1256
    workgroups: more than one round, so the automatic choice would take
    k_layer; asked for explicitly)."""
    o = orc.Shape(2, 16, 8, 128, 1e6, orc.ARCH_QWEN3, q8)
    print(f"[spans] single sequence q8={q8}", flush=True)
    run_batch_case(o, [20001], [20000], seed=91, fused=False, want_att=False, kernel=3)


@pytest.mark.parametrize("q8", [True, False])
def test_automatic_choice(gpu_device, q8):
    """Spans are taken only when asked for: the automatic choice for one layer
    of one sequence past 128 positions (2049: 17 spans) is k_layer's static
    splits, at least four per-lane wave-steps per wave, and the combine; below
    128 positions it is a single span writing the output itself.  Outputs
    against the oracle."""
    o = orc.Shape(1, 16, 8, 128, 1e6, orc.ARCH_QWEN3, q8)
    print(f"[spans] automatic q8={q8}", flush=True)
    sched = {}
    run_batch_case(o, [2049], [2048], seed=17, fused=False, want_att=False, sched=sched)
    assert sched["kernel"] == "k_layer" and sched["max_splits"] > 1, sched
    assert not sched["output_in_kernel"], sched
    run_batch_case(o, [128], [127], seed=18, fused=False, want_att=False, sched=sched)
    assert sched["kernel"] == "k_short" and sched["max_splits"] == 1, sched
    assert sched["output_in_kernel"], sched


@pytest.mark.parametrize("name", ["qwen3_q8_g2", "qwen3_f32_g2"])
def test_counters_reset_between_calls(gpu_device, name):
    """The same single-sequence call twice, then once more at another
    position: each call's last span must find the counter at zero."""
    nh, nkv, hd, arch, q8 = SHAPES[name]
    s = attn.Shape(1, nh, nkv, hd, 1e6, arch, q8)
    o = orc.Shape(1, nh, nkv, hd, 1e6, arch, q8)
    cap = 3000
    rng = np.random.default_rng(5)
    with attn.Context(s) as ctx:
        ctx.tune_kernel(3)
        kc, vc = ctx.kv_alloc(cap)
        host = orc.alloc_kv(o, cap)
        try:
            kp = rng.standard_normal((2000, o.nkv)).astype(np.float32)
            vp = rng.standard_normal((2000, o.nkv)).astype(np.float32)
            kd, vd = hip.to_device(kp), hip.to_device(vp)
            ctx.kv_append_rows(kc, vc, cap, 0, 0, 2000, kd.ptr, vd.ptr)
            orc.kv_prefill(o, cap, 0, 0, host[0], host[1], kp, vp)
            q = rng.standard_normal(o.nq).astype(np.float32)
            k = rng.standard_normal(o.nkv).astype(np.float32)
            v = rng.standard_normal(o.nkv).astype(np.float32)
            outs = []
            for rep in range(2):
                qd, kk, vv = hip.to_device(q), hip.to_device(k), hip.to_device(v)
                ctx.attn_forward(0, 2000, cap, kc, vc, qd.ptr, kk.ptr, vv.ptr)
                ctx.sync()
                outs.append(qd.download(np.float32, o.nq))
            assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
            ref, _ = orc.attn_layer(o, cap, 0, 2000, host[0], host[1], q, k, v)
            ex, _ = exact_attention(o, cap, 0, 2000, host[0], host[1], q)
            check_out(outs[0], ref, ex)
            # another position, fewer spans
            q2 = rng.standard_normal(o.nq).astype(np.float32)
            qd, kk, vv = hip.to_device(q2), hip.to_device(k), hip.to_device(v)
            ctx.attn_forward(0, 700, cap, kc, vc, qd.ptr, kk.ptr, vv.ptr)
            ctx.sync()
            out2 = qd.download(np.float32, o.nq)
            ref2, _ = orc.attn_layer(o, cap, 0, 700, host[0], host[1], q2, k, v)
            ex2, _ = exact_attention(o, cap, 0, 700, host[0], host[1], q2)
            check_out(out2, ref2, ex2)
        finally:
            ctx.kv_free(kc, vc)
