"""The C ABI without a GPU: the library loads, exports every symbol the
headers declare, and its host-side pieces (sizes, offsets, RoPE table,
stream seeds, argument validation) are right."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from helpers import bits, load_golden
from oracle import orc

import gguf2bin_amd as g
from gguf2bin_amd import attn

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in sorted(f for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h")):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(g2b_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    L = attn.lib()
    declared = declared_symbols()
    assert declared, "no declarations parsed"
    missing = [s for s in sorted(declared) if not hasattr(L, s)]
    assert not missing, missing
    assert declared == set(attn.EXPORTS)


def test_rope_table_bit_exact_with_reference():
    d = load_golden("rope_tables.npz")
    for a, th in enumerate(d["thetas"]):
        for b, hd in enumerate(d["hds"]):
            for c, p in enumerate(d["poss"]):
                got = g.rope_table(int(p), 1, int(hd), float(th))[0]
                assert np.array_equal(bits(got), bits(d["cs"][a, b, c, :hd])), (th, hd, p)


def test_rope_table_many_positions_equals_per_position():
    tab = g.rope_table(100, 50, 64, 1e4)
    for i in (0, 7, 49):
        assert np.array_equal(bits(tab[i]), bits(orc.rope_table(100 + i, 64, 1e4)))


def test_rope_table_errors():
    out = np.zeros(4096, np.float32)
    L = attn.lib()
    assert L.g2b_rope_table(0, 1, 7, 1e4, out.ctypes.data) == attn.G2B_EINVAL
    assert L.g2b_rope_table(0, 1, 2048, 1e4, out.ctypes.data) == attn.G2B_EUNSUP
    assert L.g2b_rope_table(-1, 1, 64, 1e4, out.ctypes.data) == attn.G2B_EINVAL


@pytest.mark.parametrize("nkv_heads,hd,q8", [(8, 128, True), (3, 64, True), (2, 16, True),
                                               (2, 24, True), (8, 128, False), (3, 64, False)])
def test_kv_sizes_match_reference_layout(nkv_heads, hd, q8):
    s = g.Shape(5, nkv_heads * 2, nkv_heads, hd, 1e6, 2, q8)
    o = orc.Shape(5, nkv_heads * 2, nkv_heads, hd, 1e6, 2, q8)
    nkv = nkv_heads * hd
    row = ((nkv + 31) // 32) * 34 if q8 else nkv * 4
    assert g.kv_row_bytes(s) == row == o.row_bytes
    assert g.kv_bytes(s, 300) == 5 * 300 * row
    for layer, pos in ((0, 0), (3, 17), (4, 299)):
        assert g.kv_offset(s, 300, layer, pos) == (layer * 300 + pos) * row
        assert g.kv_offset(s, 300, layer, pos) == orc.kv_offset(o, 300, layer, pos)


def test_stream_seed_matches_host_generator():
    for args in ((0, 0, 0, 0), (123, 4, 5, 1), (2**63 + 5, 255, 27, 5)):
        assert g.stream_seed(*args) == orc.stream_seed(*args)


@pytest.mark.parametrize("bad", [
    dict(n_heads=9, n_kv_heads=4),  # group must be integral
    dict(head_dim=7),               # RoPE pairs need an even head_dim
    dict(n_layers=0), dict(n_kv_heads=0), dict(head_dim=0),
])
def test_ctx_create_rejects_bad_shapes(bad):
    base = dict(n_layers=2, n_heads=8, n_kv_heads=4, head_dim=64, rope_theta=1e4, arch=2,
                kv_q8=True)
    base.update(bad)
    with pytest.raises(g.G2BError) as e:
        g.Context(g.Shape(**base))
    assert e.value.code == attn.G2B_EINVAL


def test_null_context_is_einval():
    L = attn.lib()
    assert L.g2b_sync(None) == attn.G2B_EINVAL
    assert L.g2b_ctx_destroy(None) == attn.G2B_EINVAL
    assert L.g2b_attn_layers(None, 0, 1, None, None, None, None, 0) == attn.G2B_EINVAL
    assert L.g2b_batch_begin(None, 1, None) == attn.G2B_EINVAL
    k = C.c_void_p()
    assert L.g2b_kv_alloc(None, 8, C.byref(k), C.byref(k)) == attn.G2B_EINVAL


def test_strerror_covers_every_code():
    texts = {attn.strerror(c) for c in range(0, -8, -1)}
    assert len(texts) == 8 and "unknown error" not in texts
