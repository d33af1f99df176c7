"""The G2BX container on the host (include/g2b_model.h: g2b_g2bx_open,
g2b_g2bx_slot) - no GPU.

Pins: the reference's own loader (model_load_g2bx, l5_model.c:393-408, run
from oracle/_ref) parses the same header, config and slot table from the
reference's tiny.g2bx (tests/golden/tiny.g2bx, a data file of the reference)
and from random files; the test writer (tests/helpers.write_g2bx) rewrites
tiny.g2bx byte for byte, so it lays files out as the reference's writer does.
"""
import os
import struct

import numpy as np
import pytest

from helpers import (F_QK_NORM, G2BX_CFG, R_ATTN_Q, R_FFN_DOWN, R_TOK_EMBD, random_model_slots,
                     require_ref, write_g2bx)
from oracle import orc
from gguf2bin_amd import attn

HERE = os.path.dirname(os.path.abspath(__file__))
TINY = os.path.join(HERE, "golden", "tiny.g2bx")


def cfg40(cfg: dict) -> bytes:
    return struct.pack("<8i2f", *[cfg[k] for k in G2BX_CFG])


def test_tiny_parse_matches_reference_loader():
    g = attn.g2bx_open(TINY)
    assert g["version"] == 1 and g["arch"] == attn.ARCH_QWEN3 and g["flags"] == 3
    assert g["cfg"]["dim"] == 64 and g["cfg"]["n_layers"] == 2 and g["cfg"]["head_dim"] == 16
    assert len(g["slots"]) == 24 and len(g["data"]) == 47616
    require_ref()
    c40, arch, flags, slots = orc.ref_g2bx_info(TINY)
    assert c40 == cfg40(g["cfg"])
    assert (arch, flags) == (g["arch"], g["flags"])
    assert slots == g["slots"]


def test_writer_rewrites_tiny_byte_for_byte(tmp_path):
    g = attn.g2bx_open(TINY)
    slots = [(r, l, t, g["data"][o:o + n]) for (r, l, t, n, o) in g["slots"]]
    out = tmp_path / "tiny2.g2bx"
    write_g2bx(str(out), g["cfg"], g["arch"], g["flags"], slots, g["version"])
    assert out.read_bytes() == open(TINY, "rb").read()


@pytest.mark.parametrize("seed", [1, 2])
def test_random_file_parse_matches_reference_loader(tmp_path, seed):
    rng = np.random.default_rng(seed)
    cfg = dict(dim=64, hidden_dim=96, n_layers=3, n_heads=4, n_kv_heads=2, vocab=50,
               seq_len=0 if seed == 2 else 128, head_dim=16, eps=1e-5, rope_theta=1e4)
    slots = random_model_slots(rng, cfg, F_QK_NORM, 8 if seed == 1 else 2, 0, 8)
    p = str(tmp_path / "m.g2bx")
    write_g2bx(p, cfg, attn.ARCH_LLAMA, F_QK_NORM, slots)
    g = attn.g2bx_open(p)
    # seq_len <= 0 in the file becomes 2048 (l5_model.c:375)
    assert g["cfg"]["seq_len"] == (2048 if seed == 2 else 128)
    for (r, l, t, n, o), s in zip(g["slots"], slots):
        assert (r, l, t, n) == (s[0], s[1], s[2], len(s[3]))
        assert g["data"][o:o + n] == s[3]
    require_ref()
    c40, arch, flags, rslots = orc.ref_g2bx_info(p)
    assert c40 == cfg40(g["cfg"]) and rslots == g["slots"]


def test_slot_lookup_follows_build_index(tmp_path):
    """slot_get over build_index (l5_model.c:27-45): a later duplicate wins,
    layers >= n_layers and roles >= R_COUNT are not indexed, layer < 0 is the
    global table."""
    import ctypes as C
    cfg = dict(dim=32, hidden_dim=32, n_layers=2, n_heads=1, n_kv_heads=1, vocab=4,
               seq_len=8, head_dim=32, eps=1e-5, rope_theta=1e4)
    s = [(R_TOK_EMBD, 0xFFFF, 0, bytes(512)), (R_ATTN_Q, 0, 0, bytes(64)),
         (R_ATTN_Q, 0, 0, bytes(128)), (R_ATTN_Q, 5, 0, bytes(32)), (R_FFN_DOWN, 1, 0, bytes(16)),
         (40, 0, 0, bytes(8))]
    p = str(tmp_path / "d.g2bx")
    write_g2bx(p, cfg, 0, 0, s)
    g = attn._G2bx()
    L = attn.lib()
    assert L.g2b_g2bx_open(p.encode(), C.byref(g)) == attn.G2B_OK
    try:
        def get(role, layer):
            r = L.g2b_g2bx_slot(C.byref(g), role, layer)
            return r.contents.nbytes if r else None
        assert get(R_ATTN_Q, 0) == 128       # the later duplicate
        assert get(R_ATTN_Q, 5) is None      # layer >= n_layers
        assert get(R_ATTN_Q, 1) is None
        assert get(R_FFN_DOWN, 1) == 16
        assert get(R_TOK_EMBD, -1) == 512 and get(R_TOK_EMBD, 0) is None
        assert get(40, 0) is None            # role >= R_COUNT
    finally:
        L.g2b_g2bx_close(C.byref(g))


def test_rejects_bad_files(tmp_path):
    """load_header_body's rejections (l5_model.c:288-293, :368-370)."""
    good = open(TINY, "rb").read()
    cases = {"magic": b"G2BY" + good[4:], "short_header": good[:30],
             "short_slots": good[:52 + 16 * 5], "truncated_blob": good[:-100]}
    for name, data in cases.items():
        p = tmp_path / f"{name}.g2bx"
        p.write_bytes(data)
        with pytest.raises(attn.G2BError) as e:
            attn.g2bx_open(str(p))
        assert e.value.code == attn.G2B_EINVAL, name
    with pytest.raises(attn.G2BError):
        attn.g2bx_open(str(tmp_path / "missing.g2bx"))


def test_rejects_wrapping_slot(tmp_path):
    """A slot whose off + nbytes wraps past 2^64 would leave the blob small
    and the slot pointing outside it; the parse refuses it (the reference
    trusts the file)."""
    good = bytearray(open(TINY, "rb").read())
    # first slot entry at 52: role, layer(2), type, nbytes(4), off(8)
    nbytes = struct.unpack_from("<I", good, 52 + 4)[0]
    assert nbytes > 0
    struct.pack_into("<Q", good, 52 + 8, (1 << 64) - nbytes // 2)
    p = tmp_path / "wrap.g2bx"
    p.write_bytes(bytes(good))
    with pytest.raises(attn.G2BError) as e:
        attn.g2bx_open(str(p))
    assert e.value.code == attn.G2B_EINVAL
