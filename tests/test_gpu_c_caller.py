"""The ABI from a plain C99 program (tests/c_caller/g2b_c_caller.c, built with
gcc -std=c99 -Wall -Werror against include/g2b_attn.h and linked to
libg2b_attn.so): the reference's decode loop (/root/reference/src/
l5_model.c:493-578 with the attention block replaced by
g2b_attn_forward_host, KV from g2b_kv_alloc as alloc_rt would take it,
:113-149), token after token from an empty cache, against the oracle run
through the same sequence of calls.  Bar: both caches byte for byte, every
output within 1e-4 of the oracle (the oracle is bit-exact with the compiled
reference on the golden cases)."""
import os
import subprocess

import numpy as np
import pytest

from helpers import normed
from oracle import orc

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "c_caller", "g2b_c_caller")

CASES = {
    # name: (oracle shape, ctx_cap, tokens, with QK-RMSNorm)
    # Qwen3 head shape, Q8_0 KV, QK-RMSNorm: k_short below 128 positions,
    # the split kernel from 128 on
    "qwen3_q8_qkn": (orc.Shape(2, 16, 8, 128, 1e6, orc.ARCH_QWEN3, True), 320, 300, True),
    # SmolLM2 head shape, F32 KV, LLaMA rotation
    "smollm2_f32": (orc.Shape(2, 9, 3, 64, 1e5, orc.ARCH_LLAMA, False), 200, 180, False),
    # a shape without a specialised kernel (blocks spanning heads)
    "generic_hd24": (orc.Shape(1, 6, 2, 24, 1e4, orc.ARCH_QWEN3, True), 64, 60, False),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_c99_caller_decode_loop(gpu_device, tmp_path, name):
    assert os.path.exists(EXE), f"{EXE} is missing: build it with make -C tests/c_caller"
    o, cap, n_tok, with_norm = CASES[name]
    L, nq, nkv, hd = o.n_layers, o.nq, o.nkv, o.head_dim
    eps = 1e-6
    rng = np.random.default_rng(sum(map(ord, name)))
    q = rng.standard_normal((n_tok, L, nq)).astype(np.float32)
    k = rng.standard_normal((n_tok, L, nkv)).astype(np.float32)
    v = rng.standard_normal((n_tok, L, nkv)).astype(np.float32)
    norms = (rng.uniform(0.5, 1.5, (L, 2, hd)).astype(np.float32) if with_norm else None)
    head = np.array([L, o.n_heads, o.n_kv_heads, hd, o.arch, int(o.kv_q8), cap, n_tok,
                     int(with_norm)], np.int32).tobytes()
    head += np.array([o.rope_theta, eps], np.float32).tobytes()
    body = norms.tobytes() if with_norm else b""
    xs = np.concatenate([q, k, v], axis=2)  # [token][layer][nq + 2 nkv]
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    inp.write_bytes(head + body + xs.tobytes())
    print(f"[c_caller] {name}: {n_tok} tokens x {L} layers", flush=True)
    r = subprocess.run([EXE, str(inp), str(outp)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    raw = np.fromfile(outp, np.uint8)
    n_out = n_tok * L * nq * 4
    out = raw[:n_out].view(np.float32).reshape(n_tok, L, nq)
    kv_n = L * cap * o.row_bytes
    assert raw.size == n_out + 2 * kv_n
    k_dev, v_dev = raw[n_out:n_out + kv_n], raw[n_out + kv_n:]

    kc, vc = orc.alloc_kv(o, cap)
    worst = 0.0
    for t in range(n_tok):
        for layer in range(L):
            qq, kk = q[t, layer], k[t, layer]
            if with_norm:
                qq = normed(qq, norms[layer, 0], o.n_heads, hd, eps)
                kk = normed(kk, norms[layer, 1], o.n_kv_heads, hd, eps)
            ref, _ = orc.attn_layer(o, cap, layer, t, kc, vc, qq, kk, v[t, layer])
            worst = max(worst, float(np.max(np.abs(out[t, layer] - ref))))
    print(f"[c_caller] {name}: max |out - oracle| = {worst:.3g}", flush=True)
    assert np.array_equal(k_dev, kc), "K cache bytes differ from the oracle"
    assert np.array_equal(v_dev, vc), "V cache bytes differ from the oracle"
    assert worst <= 1e-4
