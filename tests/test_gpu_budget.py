"""The HBM budget against what the device actually allocates.

g2b_hbm_bytes (include/g2b_attn.h) bounds the HBM one context takes for
n_seq sequences at context ctx in every call form; g2b_auto_budget plans with
it as model_auto_budget plans with est_for (/root/reference/src/l5_model.c:
174-187, :218-230).  Here the drop in free HBM (hipMemGetInfo) across a
context's whole life - KV allocation, a call over all layers at once, the
layer-serial calls, the weights output and the host entry point - must stay
within the bound.  Each case first runs the same calls on a throwaway context
so that the runtime's own one-time allocations (code objects, kernel scratch)
are not counted.
"""
import numpy as np
import pytest

from gguf2bin_amd import attn, hip

pytestmark = pytest.mark.gpu
Q3, LL = attn.ARCH_QWEN3, attn.ARCH_LLAMA

CASES = {
    # name: (shape, positions per sequence)
    "qwen3_q8_16seq": (attn.Shape(28, 16, 8, 128, 1e6, Q3, True), [2047] * 16),
    "qwen3_f32_1seq": (attn.Shape(28, 16, 8, 128, 1e6, Q3, False), [8191]),
    "smollm2_f32_64seq": (attn.Shape(30, 9, 3, 64, 1e5, LL, False),
                          [256 + (37 * i) % 768 for i in range(64)]),
    "llama3_q8_4seq": (attn.Shape(32, 32, 8, 128, 5e5, LL, True), [16383, 9000, 12000, 4000]),
    "generic_hd24": (attn.Shape(3, 6, 2, 24, 1e4, Q3, True), [2999, 100, 1500, 2000]),
}


def _exercise(shape, poss, ctx_cap, q, k, v, att, keep):
    """Every call form on a fresh context; returns it with its caches alive
    when keep is set (else frees everything)."""
    c = attn.Context(shape)
    kvs = [c.kv_alloc(ctx_cap) for _ in poss]
    c.batch_begin([(p, ctx_cap, kc, vc) for p, (kc, vc) in zip(poss, kvs)])
    L = shape.n_layers
    c.attn_layers(0, L, q.ptr, k.ptr, v.ptr)
    n, nq, nkv = len(poss), shape.nq, shape.nkv
    for layer in range(L):
        c.attn_layers(layer, 1, q.ptr + layer * n * nq * 4, k.ptr + layer * n * nkv * 4,
                      v.ptr + layer * n * nkv * 4)
    c.attn_layers(0, 1, q.ptr, k.ptr, v.ptr, att.ptr, ctx_cap)
    qh = np.zeros(nq, np.float32)
    kh = np.zeros(nkv, np.float32)
    c.attn_forward_host(0, poss[0], ctx_cap, kvs[0][0], kvs[0][1], qh, kh, kh.copy(),
                        want_att=True)
    c.sync()
    if keep:
        return c, kvs
    for kc, vc in kvs:
        c.kv_free(kc, vc)
    c.close()
    return None, None


@pytest.mark.parametrize("name", sorted(CASES))
def test_hbm_bytes_bounds_device_use(gpu_device, name):
    shape, poss = CASES[name]
    ctx_cap = max(poss) + 1
    n = len(poss)
    print(f"[budget] {name}: n_seq={n} ctx={ctx_cap} q8={shape.kv_q8}", flush=True)
    L, nq, nkv = shape.n_layers, shape.nq, shape.nkv
    # caller-owned buffers, allocated before the measurement
    q = hip.to_device(np.zeros(L * n * nq, np.float32))
    k = hip.to_device(np.zeros(L * n * nkv, np.float32))
    v = hip.to_device(np.zeros(L * n * nkv, np.float32))
    att = hip.DeviceBuffer(n * shape.n_heads * ctx_cap * 4)
    try:
        _exercise(shape, poss, ctx_cap, q, k, v, att, keep=False)
        free0, _ = hip.mem_info()
        c, kvs = _exercise(shape, poss, ctx_cap, q, k, v, att, keep=True)
        free1, _ = hip.mem_info()
        used = free0 - free1
        bound = attn.hbm_bytes(shape, ctx_cap, shape.kv_q8, n)
        kv = 2 * n * attn.kv_bytes(shape, ctx_cap)
        print(f"[budget] {name}: used {used} B, bound {bound} B, KV {kv} B "
              f"(bound - used = {(bound - used) / 2**20:.1f} MiB)", flush=True)
        assert used >= kv
        assert used <= bound
        for kc, vc in kvs:
            c.kv_free(kc, vc)
        c.close()
    finally:
        for b in (q, k, v, att):
            b.free()


def test_auto_budget_plan_fits_device(gpu_device):
    """A plan g2b_auto_budget accepts for a budget of 6 GiB, carried out:
    the HBM it takes stays within the budget."""
    shape = attn.Shape(28, 16, 8, 128, 1e6, Q3, False)
    n_seq, budget = 12, 6 << 30
    q8, ctx, fits = attn.auto_budget(shape, 40960, n_seq, budget)
    assert fits and q8  # F32 at 40960 does not fit, Q8_0 halved does
    run = attn.Shape(28, 16, 8, 128, 1e6, Q3, q8)
    print(f"[budget] plan: q8={q8} ctx={ctx}", flush=True)
    L = run.n_layers
    q = hip.to_device(np.zeros(L * n_seq * run.nq, np.float32))
    k = hip.to_device(np.zeros(L * n_seq * run.nkv, np.float32))
    v = hip.to_device(np.zeros(L * n_seq * run.nkv, np.float32))
    att = hip.DeviceBuffer(n_seq * run.n_heads * ctx * 4)
    poss = [ctx - 1] * n_seq
    try:
        _exercise(run, poss, ctx, q, k, v, att, keep=False)
        free0, _ = hip.mem_info()
        c, kvs = _exercise(run, poss, ctx, q, k, v, att, keep=True)
        used = free0 - hip.mem_info()[0]
        print(f"[budget] plan used {used} B of {budget} B", flush=True)
        assert used <= budget
        for kc, vc in kvs:
            c.kv_free(kc, vc)
        c.close()
    finally:
        for b in (q, k, v, att):
            b.free()
