"""The headline config's own schedule at its real context length: Qwen3-0.6B
heads (16 q, 8 KV, head_dim 128, NEOX theta 1e6), Q8_0 KV, contexts of 8192
cached positions plus the new token (some ragged just below), through the
schedule the automatic choice gives the bench's c4 calls - k_layer's work
queue with KV chunks pulled straight into LDS (k_layer<1, 128, 32, 2, 2,
false, 1, true>) - layer by layer and all layers in one call.

32 sequences are enough for the automatic choice to take the work queue
(at most 64 waves per unit's counter: 32 units or more for one layer), as
c4's 256 do; nothing is tuned.  The KV comes from the device's seeded fill
(the bench's generator) and the oracle starts from those bytes: every byte
of both caches must equal the oracle's appends, and the outputs must be
within max-abs 1e-4 of the oracle (bit-exact with the compiled reference,
/root/reference/src/l5_model.c:513-578) and of a float64 evaluation of the
same bytes (helpers.check_out)."""
import numpy as np
import pytest

from helpers import check_out, exact_attention
from oracle import orc

from gguf2bin_amd import attn, hip

pytestmark = pytest.mark.gpu

C4_VARIANT = "k_layer<1, 128, 32, 2, 2, false, 1, true>"


@pytest.mark.parametrize("fused", [False, True])
def test_c4_schedule_at_ctx_8192(gpu_device, fused):
    L, n = 2, 32
    s = attn.Shape(L, 16, 8, 128, 1e6, attn.ARCH_QWEN3, True)
    o = orc.Shape(L, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True)
    poss = [8192] * n
    poss[3], poss[10], poss[17], poss[29] = 8191, 8000, 7777, 8189  # ragged just below
    caps = [8192 + 1] * n
    seed = 8192
    with attn.Context(s) as ctx:
        kvs = [ctx.kv_alloc(c) for c in caps]
        try:
            for i, (p, c) in enumerate(zip(poss, caps)):
                ctx.synth_fill_kv(kvs[i][0], kvs[i][1], c, 0, L, 0, p, seed, i)
            ctx.sync()
            host = [(hip.copy_d2h(k, np.uint8, attn.kv_bytes(s, c)),
                     hip.copy_d2h(v, np.uint8, attn.kv_bytes(s, c)))
                    for (k, v), c in zip(kvs, caps)]
            q = orc.normal(seed + 1, L * n * o.nq).reshape(L, n, o.nq)
            k = orc.normal(seed + 2, L * n * o.nkv).reshape(L, n, o.nkv)
            v = orc.normal(seed + 3, L * n * o.nkv).reshape(L, n, o.nkv)
            qd, kd, vd = hip.to_device(q), hip.to_device(k), hip.to_device(v)
            ctx.batch_begin([(p, c, kc, vc) for p, c, (kc, vc) in zip(poss, caps, kvs)])
            print(f"[c4] 32 sequences at ctx 8192, 2 layers, fused={fused}", flush=True)
            if fused:
                ctx.attn_layers(0, L, qd.ptr, kd.ptr, vd.ptr)
                sched = ctx.last_schedule()
            else:
                for layer in range(L):
                    ctx.attn_layers(layer, 1, qd.ptr + layer * n * o.nq * 4,
                                    kd.ptr + layer * n * o.nkv * 4,
                                    vd.ptr + layer * n * o.nkv * 4)
                    if layer == 0:
                        sched = ctx.last_schedule()
            ctx.sync()
            out = qd.download(np.float32, q.size).reshape(q.shape)
            dev = [(hip.copy_d2h(kc, np.uint8, attn.kv_bytes(s, c)),
                    hip.copy_d2h(vc, np.uint8, attn.kv_bytes(s, c)))
                   for (kc, vc), c in zip(kvs, caps)]
        finally:
            for kc, vc in kvs:
                ctx.kv_free(kc, vc)
    # c4's schedule: the work queue, chunks by LDS DMA, whole-block lanes
    assert sched["kernel"] == "k_layer", sched
    assert sched["piece_len"] > 0 and sched["staging"] == "LDS DMA", sched
    assert sched["variant"] == C4_VARIANT, sched
    worst = 0.0
    for i, (p, c) in enumerate(zip(poss, caps)):
        kc, vc = host[i]
        for layer in range(L):
            ref, _ = orc.attn_layer(o, c, layer, p, kc, vc, q[layer, i], k[layer, i],
                                    v[layer, i])
            if i % 4 == 0 or p != 8192:  # float64 on a quarter of the units and every ragged one
                ex, _ = exact_attention(o, c, layer, p, kc, vc, q[layer, i])
                check_out(out[layer, i], ref, ex)
            else:
                check_out(out[layer, i], ref, ref)
            worst = max(worst, float(np.max(np.abs(out[layer, i] - ref))))
        assert np.array_equal(dev[i][0], kc), f"K bytes of sequence {i}"
        assert np.array_equal(dev[i][1], vc), f"V bytes of sequence {i}"
    print(f"[c4] max |out - oracle| {worst:.3g}, schedule {sched}", flush=True)
