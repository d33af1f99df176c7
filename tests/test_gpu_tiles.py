"""k_tiles, the decode kernel whose K scores run on the int8 matrix cores
(Q8_0 KV, head_dim 128, 8 KV heads, 3 or 4 q heads per KV head), against
the oracle on the same seeded inputs: K and V bytes bit-exact, outputs
within max-abs 1e-4 of a float64 evaluation of the same bytes and of the
oracle up to the oracle's own float32 error (helpers.check_out; the oracle is
bit-exact with the compiled reference on the golden cases).  Every schedule
(static splits, the work queue, one call over all layers, layer by layer),
partial tiles and pieces, QK-RMSNorm, and the c5 shape at full context
length through the work queue.  k_layer runs the same cases
(g2b_ctx_tune_kernel(1)) so both kernels keep their coverage."""
import zlib

import numpy as np
import pytest

from helpers import check_out, exact_attention
from oracle import orc
from test_gpu_parity import MODES, run_batch_case

from gguf2bin_amd import attn, hip

pytestmark = pytest.mark.gpu

TILE_SHAPES = {
    # name: (n_heads, n_kv_heads, arch)
    "llama3_g4": (32, 8, orc.ARCH_LLAMA),
    "g3": (24, 8, orc.ARCH_QWEN3),
}


def oshape(name, layers=2):
    nh, nkv, arch = TILE_SHAPES[name]
    return orc.Shape(layers, nh, nkv, 128, 5e5 if arch == orc.ARCH_LLAMA else 1e6, arch, True)


@pytest.mark.parametrize("name", sorted(TILE_SHAPES))
@pytest.mark.parametrize("mode", ["fused", "layers", "wq", "wq_fused", "static"])
@pytest.mark.parametrize("kernel", [0, 1])
def test_ragged_batch_vs_oracle(gpu_device, name, mode, kernel):
    """Ragged sequences (pos 0, 1, mid-tile, a whole number of tiles, long):
    no weights output, so k_tiles runs unless kernel 1 asks for k_layer."""
    o = oshape(name)
    fused, tune = MODES[mode]
    caps = [1, 2, 40, 129, 700, 2049]
    poss = [0, 1, 39, 128, 650, 2048]
    print(f"[tiles] {name} mode={mode} kernel={kernel}", flush=True)
    run_batch_case(o, caps, poss, seed=zlib.crc32(name.encode()) % 1000, fused=fused,
                   want_att=False, tune=tune, kernel=kernel)


@pytest.mark.parametrize("name", sorted(TILE_SHAPES))
@pytest.mark.parametrize("kernel", [0, 1])
def test_qk_norm_vs_oracle(gpu_device, name, kernel):
    o = oshape(name)
    hd = o.head_dim
    seed = zlib.crc32(name.encode()) % 1000 + 5
    qn = (1 + 0.25 * orc.normal(seed + 40, 2 * hd)).reshape(2, hd)
    kn = (1 + 0.25 * orc.normal(seed + 41, 2 * hd)).reshape(2, hd)
    print(f"[tiles] qknorm {name} kernel={kernel}", flush=True)
    run_batch_case(o, [1, 37, 300, 129], [0, 36, 211, 64], seed=seed, fused=False,
                   want_att=False, norms=(qn, kn, 1e-5), kernel=kernel)


@pytest.mark.parametrize("mode", ["layers", "wq"])
def test_many_tiles_single_sequence(gpu_device, mode):
    """6000 positions of one sequence: hundreds of tiles and splits (or
    pieces claimed by many workgroups); the last tile of a split or piece
    partial."""
    o = oshape("llama3_g4", layers=1)
    print(f"[tiles] single sequence mode={mode}", flush=True)
    run_batch_case(o, [6000], [5999], seed=78, fused=False, want_att=False,
                   tune=(0, 0, 2, 12) if mode == "wq" else None)


def test_weights_output_takes_layer_kernel(gpu_device):
    """With the softmax weights requested the call runs k_layer (k_tiles
    writes no raw scores); outputs and weights within the bars."""
    o = oshape("llama3_g4")
    print("[tiles] weights output", flush=True)
    run_batch_case(o, [1, 300, 129], [0, 211, 64], seed=9, fused=True, want_att=True)


@pytest.mark.parametrize("fused", [False, True])
def test_c5_shape_work_queue(gpu_device, fused):
    """The c5 shape at full length: Llama-3-8B heads (32 q, 8 KV, head_dim
    128, theta 5e5, Q8_0), 4 sequences at contexts in [16384, 32767], 2
    layers, 1% of K rows scaled x8 before quantisation (the device's seeded
    fill, the bench's generator), through the work queue that the layer
    loop's calls take at this shape: every byte of both caches bit-exact
    with the oracle's appends, outputs against float64 and the oracle (whose
    own float32 drift at this length, ~4e-4, check_out accounts for)."""
    L = 2
    s = attn.Shape(L, 32, 8, 128, 5e5, attn.ARCH_LLAMA, True)
    o = orc.Shape(L, 32, 8, 128, 5e5, orc.ARCH_LLAMA, True)
    poss = [16384, 32766, 24001, 20000]
    caps = [p + 1 for p in poss]
    thr = float(np.float32(2.3263478740408408))  # N(0,1) quantile 0.99
    seed = 4242
    n = len(poss)
    with attn.Context(s) as ctx:
        kvs = [ctx.kv_alloc(c) for c in caps]
        try:
            for i, (p, c) in enumerate(zip(poss, caps)):
                ctx.synth_fill_kv(kvs[i][0], kvs[i][1], c, 0, L, 0, p, seed, i, thr)
            ctx.sync()
            # the oracle starts from the device's prefill bytes
            host = [(hip.copy_d2h(k, np.uint8, attn.kv_bytes(s, c)),
                     hip.copy_d2h(v, np.uint8, attn.kv_bytes(s, c)))
                    for (k, v), c in zip(kvs, caps)]
            q = orc.normal(seed + 1, L * n * o.nq).reshape(L, n, o.nq)
            k = orc.normal(seed + 2, L * n * o.nkv).reshape(L, n, o.nkv)
            v = orc.normal(seed + 3, L * n * o.nkv).reshape(L, n, o.nkv)
            qd, kd, vd = hip.to_device(q), hip.to_device(k), hip.to_device(v)
            ctx.batch_begin([(p, c, kc, vc) for p, c, (kc, vc) in zip(poss, caps, kvs)])
            print(f"[tiles] c5 shape fused={fused}", flush=True)
            if fused:
                ctx.attn_layers(0, L, qd.ptr, kd.ptr, vd.ptr)
            else:
                for layer in range(L):
                    ctx.attn_layers(layer, 1, qd.ptr + layer * n * o.nq * 4,
                                    kd.ptr + layer * n * o.nkv * 4,
                                    vd.ptr + layer * n * o.nkv * 4)
            ctx.sync()
            out = qd.download(np.float32, q.size).reshape(q.shape)
            dev = [(hip.copy_d2h(kc, np.uint8, attn.kv_bytes(s, c)),
                    hip.copy_d2h(vc, np.uint8, attn.kv_bytes(s, c)))
                   for (kc, vc), c in zip(kvs, caps)]
        finally:
            for kc, vc in kvs:
                ctx.kv_free(kc, vc)
    for i, (p, c) in enumerate(zip(poss, caps)):
        kc, vc = host[i]
        for layer in range(L):
            ref, _ = orc.attn_layer(o, c, layer, p, kc, vc, q[layer, i], k[layer, i],
                                    v[layer, i])
            ex, _ = exact_attention(o, c, layer, p, kc, vc, q[layer, i])
            check_out(out[layer, i], ref, ex)
        assert np.array_equal(dev[i][0], kc), f"K bytes of sequence {i}"
        assert np.array_equal(dev[i][1], vc), f"V bytes of sequence {i}"
