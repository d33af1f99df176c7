"""g2b_attn_forward_noalloc (include/g2b_attn.h): the single-sequence,
single-layer attention call over the library's fixed device scratch, which
allocates nothing.  Through the C ABI, against the allocating entry point
g2b_attn_forward on the same inputs and caches (KV bytes bit for bit,
outputs within 1e-4 - bit for bit where both take the same splits), and
against the oracle; two calls in a row on one context, the second at a
smaller position, so nothing the first left in the scratch leaks into the
second.  The contract itself: the first call on a fresh context leaves the
device's free memory unchanged, and a call captured into a HIP graph (kernel
nodes only) replays bit for bit like the direct call.  Also the refusals: a RoPE table that does not reach pos (nothing
may be allocated to extend it), and a shape whose partials need more than
the 2 MiB scratch."""
import numpy as np
import pytest

from helpers import check_out, exact_attention
from oracle import orc

from gguf2bin_amd import attn, hip

pytestmark = pytest.mark.gpu

CASES = {
    # name: (oracle shape, ctx_cap, positions of the two calls, same splits as forward?)
    # k_layer, static splits
    "qwen3_q8": (orc.Shape(1, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True), 6000, (5999, 700), True),
    # k_tiles, static splits; the first call's splits are lengthened to fit
    "llama3_q8_long": (orc.Shape(1, 32, 8, 128, 5e5, orc.ARCH_LLAMA, True), 32768,
                       (32767, 4000), False),
    # F32 rows
    "smollm2_f32": (orc.Shape(1, 9, 3, 64, 1e5, orc.ARCH_LLAMA, False), 3000, (2999, 500), True),
    # the generic kernels (rotated q in the scratch too)
    "generic_hd24": (orc.Shape(1, 4, 2, 24, 1e4, orc.ARCH_QWEN3, True), 3000, (2999, 40), True),
    # the short-context kernel: no scratch at all
    "short": (orc.Shape(1, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True), 200, (120, 10), True),
}


def ashape(o):
    return attn.Shape(o.n_layers, o.n_heads, o.n_kv_heads, o.head_dim, o.rope_theta, o.arch,
                      o.kv_q8)


@pytest.mark.parametrize("name", sorted(CASES))
def test_noalloc_matches_allocating_entry_point(gpu_device, name):
    o, cap, calls, same = CASES[name]
    rng = np.random.default_rng(sum(map(ord, name)))
    n_pre = calls[0]
    kp = rng.standard_normal((n_pre, o.nkv)).astype(np.float32)
    vp = rng.standard_normal((n_pre, o.nkv)).astype(np.float32)
    nbytes = attn.kv_bytes(ashape(o), cap)
    with attn.Context(ashape(o)) as ctx:
        a, b = ctx.kv_alloc(cap), ctx.kv_alloc(cap)  # forward's caches, noalloc's caches
        host = orc.alloc_kv(o, cap)
        try:
            kd, vd = hip.to_device(kp), hip.to_device(vp)
            for kc, vc in (a, b):
                ctx.kv_append_rows(kc, vc, cap, 0, 0, n_pre, kd.ptr, vd.ptr)
            ctx.sync()
            orc.kv_prefill(o, cap, 0, 0, host[0], host[1], kp, vp)
            for call, pos in enumerate(calls):
                print(f"[noalloc] {name} call {call} pos {pos}", flush=True)
                q = rng.standard_normal(o.nq).astype(np.float32)
                k = rng.standard_normal(o.nkv).astype(np.float32)
                v = rng.standard_normal(o.nkv).astype(np.float32)
                qa, qb = hip.to_device(q), hip.to_device(q)
                kk, vv = hip.to_device(k), hip.to_device(v)
                ctx.attn_forward(0, pos, cap, a[0], a[1], qa.ptr, kk.ptr, vv.ptr)
                ctx.attn_forward_noalloc(0, pos, cap, b[0], b[1], qb.ptr, kk.ptr, vv.ptr)
                ctx.sync()
                out_a = qa.download(np.float32, o.nq)
                out_b = qb.download(np.float32, o.nq)
                ref, _ = orc.attn_layer(o, cap, 0, pos, host[0], host[1], q, k, v)
                ex, _ = exact_attention(o, cap, 0, pos, host[0], host[1], q)
                check_out(out_b, ref, ex)
                if same:
                    assert np.array_equal(out_a.view(np.uint32), out_b.view(np.uint32))
                else:
                    assert float(np.max(np.abs(out_a - out_b))) <= 1e-4
                dk_a = hip.copy_d2h(a[0], np.uint8, nbytes)
                dk_b = hip.copy_d2h(b[0], np.uint8, nbytes)
                dv_b = hip.copy_d2h(b[1], np.uint8, nbytes)
                assert np.array_equal(dk_a, dk_b)
                assert np.array_equal(dk_b, host[0]) and np.array_equal(dv_b, host[1])
        finally:
            for kc, vc in (a, b):
                ctx.kv_free(kc, vc)


def test_noalloc_refusals(gpu_device):
    o = orc.Shape(1, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True)
    s = ashape(o)
    with attn.Context(s) as owner, attn.Context(s) as fresh:
        kc, vc = owner.kv_alloc(5000)  # extends owner's RoPE table, not fresh's
        try:
            q = hip.to_device(np.zeros(o.nq, np.float32))
            k = hip.to_device(np.zeros(o.nkv, np.float32))
            with pytest.raises(attn.G2BError) as e:
                fresh.attn_forward_noalloc(0, 4000, 5000, kc, vc, q.ptr, k.ptr, k.ptr)
            assert e.value.code == attn.G2B_EINVAL
            with pytest.raises(attn.G2BError) as e:
                fresh.attn_forward_noalloc(0, 5000, 5000, kc, vc, q.ptr, k.ptr, k.ptr)
            assert e.value.code == attn.G2B_EPOS
        finally:
            owner.kv_free(kc, vc)
    # a shape without a specialised kernel (group 8: the generic kernels, at
    # most 1024 positions per split): one split is 16 x 132 floats of
    # partials, so the 2 MiB scratch (524,288 floats, after the 1024 counter
    # words and the 2048 floats of rotated q) holds 246 splits, 251,904
    # positions; 259,999 need longer splits than the kernel takes
    big = attn.Shape(1, 16, 2, 128, 1e6, attn.ARCH_QWEN3, True)
    with attn.Context(big) as ctx:
        kc, vc = ctx.kv_alloc(260000)
        try:
            q = hip.to_device(np.zeros(big.nq, np.float32))
            k = hip.to_device(np.zeros(big.nkv, np.float32))
            with pytest.raises(attn.G2BError) as e:
                ctx.attn_forward_noalloc(0, 259999, 260000, kc, vc, q.ptr, k.ptr, k.ptr)
            assert e.value.code == attn.G2B_EUNSUP
            ctx.attn_forward_noalloc(0, 20000, 260000, kc, vc, q.ptr, k.ptr, k.ptr)
            ctx.sync()
        finally:
            ctx.kv_free(kc, vc)


def test_noalloc_allocates_nothing_and_replays_from_a_graph(gpu_device):
    """hipMemGetInfo around the first g2b_attn_forward_noalloc of a context
    that has only allocated its KV (k_layer's static splits: 50 splits of
    partials in the fixed scratch), then the same call captured on the
    context's stream and replayed three times, with eager calls and
    synchronisations between the replays, each replay bit for bit equal to
    the direct call (the append at pos rewrites the same bytes)."""
    o = orc.Shape(1, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True)
    s = ashape(o)
    cap, pos = 6000, 5999
    rng = np.random.default_rng(4711)
    kp = rng.standard_normal((pos, o.nkv)).astype(np.float32)
    vp = rng.standard_normal((pos, o.nkv)).astype(np.float32)
    q = rng.standard_normal(o.nq).astype(np.float32)
    k = rng.standard_normal(o.nkv).astype(np.float32)
    v = rng.standard_normal(o.nkv).astype(np.float32)
    with attn.Context(s) as warm:  # kernels loaded, runtime pools set up
        kc, vc = warm.kv_alloc(cap)
        qd, kd = hip.to_device(q), hip.to_device(k)
        warm.attn_forward_noalloc(0, pos, cap, kc, vc, qd.ptr, kd.ptr, kd.ptr)
        warm.sync()
        warm.kv_free(kc, vc)
    with attn.Context(s) as ctx:
        kc, vc = ctx.kv_alloc(cap)
        graph = None
        try:
            kpd, vpd = hip.to_device(kp), hip.to_device(vp)
            ctx.kv_append_rows(kc, vc, cap, 0, 0, pos, kpd.ptr, vpd.ptr)
            pristine, qd = hip.to_device(q), hip.to_device(q)
            kd, vd = hip.to_device(k), hip.to_device(v)
            ctx.sync()
            free0, _ = hip.mem_info()
            print("[noalloc] first call on a fresh context", flush=True)
            ctx.attn_forward_noalloc(0, pos, cap, kc, vc, qd.ptr, kd.ptr, vd.ptr)
            ctx.sync()
            free1, _ = hip.mem_info()
            assert free1 == free0, f"device free memory moved by {free0 - free1} bytes"
            assert ctx.last_schedule()["max_splits"] > 1  # the scratch holds partials
            direct = qd.download(np.float32, o.nq)
            host = orc.alloc_kv(o, cap)
            orc.kv_prefill(o, cap, 0, 0, host[0], host[1], kp, vp)
            ref, _ = orc.attn_layer(o, cap, 0, pos, host[0], host[1], q, k, v)
            ex, _ = exact_attention(o, cap, 0, pos, host[0], host[1], q)
            check_out(direct, ref, ex)

            hip.copy_d2d(qd.ptr, pristine.ptr, q.nbytes)
            hip.device_sync()
            print("[noalloc] capture into a graph", flush=True)
            graph = hip.Graph(ctx.stream, lambda: ctx.attn_forward_noalloc(
                0, pos, cap, kc, vc, qd.ptr, kd.ptr, vd.ptr))
            types = graph.node_types()
            assert types and all(t == hip.GRAPH_NODE_KERNEL for t in types), types
            for r in range(3):
                hip.copy_d2d(qd.ptr, pristine.ptr, q.nbytes)
                hip.device_sync()
                print(f"[noalloc] replay {r}", flush=True)
                graph.launch(ctx.stream)
                ctx.sync()
                got = qd.download(np.float32, o.nq)
                assert np.array_equal(got.view(np.uint32), direct.view(np.uint32)), r
                # eager work between replays
                hip.copy_d2d(qd.ptr, pristine.ptr, q.nbytes)
                hip.device_sync()
                ctx.attn_forward_noalloc(0, pos, cap, kc, vc, qd.ptr, kd.ptr, vd.ptr)
                ctx.sync()
                assert np.array_equal(qd.download(np.float32, o.nq).view(np.uint32),
                                      direct.view(np.uint32))
            nbytes = attn.kv_bytes(s, cap)
            assert np.array_equal(hip.copy_d2h(kc, np.uint8, nbytes), host[0])
            assert np.array_equal(hip.copy_d2h(vc, np.uint8, nbytes), host[1])
        finally:
            if graph is not None:
                graph.destroy()
            ctx.kv_free(kc, vc)
