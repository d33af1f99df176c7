"""The CPU oracle against golden vectors written by the compiled reference
(tests/golden/make_golden.py).  Everything here is bit-exact: the oracle is
built with the reference's flags and follows its operation order."""
import numpy as np
import pytest

from helpers import (bits, fwd_cases, golden_shape, kv_rows, load_golden, oracle_run_case,
                     sha)
from oracle import orc


@pytest.fixture(scope="module")
def codec():
    return load_golden("codec_q8_fp16.npz")


def test_q8_special_blocks_bit_exact(codec):
    for row, q, deq in zip(codec["rows"], codec["q"], codec["deq"]):
        got = orc.q8_quant_row(row)
        assert np.array_equal(got, q), row
        assert np.array_equal(bits(orc.q8_dequant_row(q, 64)), bits(deq))


def test_q8_partial_block_bit_exact(codec):
    for row, q, deq in zip(codec["partial"], codec["q_partial"], codec["deq_partial"]):
        assert np.array_equal(orc.q8_quant_row(row), q)
        assert np.array_equal(bits(orc.q8_dequant_row(q, 45)), bits(deq))


def test_half_to_float_all_halves(codec):
    got = orc.half_to_float(np.arange(65536, dtype=np.uint16))
    assert np.array_equal(bits(got), bits(codec["h2f"]))


def test_f32_to_half_sweep(codec):
    stride = int(codec["f2h_stride"])
    f = np.arange(0, 1 << 32, stride, dtype=np.uint64).astype(np.uint32).view(np.float32)
    assert sha(orc.f32_to_half(f)) == codec["f2h_sha"].item().decode()


def test_rope_tables_bit_exact():
    d = load_golden("rope_tables.npz")
    for a, th in enumerate(d["thetas"]):
        for b, hd in enumerate(d["hds"]):
            for c, p in enumerate(d["poss"]):
                got = orc.rope_table(int(p), int(hd), float(th))
                assert np.array_equal(bits(got), bits(d["cs"][a, b, c, :hd])), (th, hd, p)
    got = orc.rope(orc.ARCH_LLAMA, d["llama_in"], 4321, 64, 1e5)
    assert np.array_equal(bits(got), bits(d["llama_out"]))


def test_qk_rmsnorm_bit_exact():
    """qk_rmsnorm (l3_math.c:107-114) on random heads at three sizes and on
    special heads (zero, subnormal, overflowing squares, Inf, NaN, -0)."""
    d = load_golden("qknorm.npz")
    for i in range(int(d["n_sets"])):
        nh, hd = [int(x) for x in d[f"meta{i}"]]
        got = orc.qk_rmsnorm(d[f"x{i}"], d[f"w{i}"], nh, hd, float(d[f"eps{i}"]))
        assert np.array_equal(bits(got), bits(d[f"y{i}"])), f"set {i}"


@pytest.mark.parametrize("name", fwd_cases())
def test_forward_case_bit_exact(name):
    """Prefill + model_forward steps: KV bytes, outputs and att weights."""
    d = load_golden(name)
    shape = golden_shape(d)
    outs, att, kc, vc = oracle_run_case(d)
    pos = int(d["n_pre"]) + int(d["n_fwd"]) - 1
    ctx_cap = int(d["ctx_cap"])
    kr, vr = kv_rows(shape, kc, ctx_cap, pos + 1), kv_rows(shape, vc, ctx_cap, pos + 1)
    assert sha(kr) == d["kc_sha"].item().decode()
    assert sha(vr) == d["vc_sha"].item().decode()
    assert np.array_equal(bits(outs), bits(d["out"]))
    if "att_sha" in d:
        assert sha(att) == d["att_sha"].item().decode()
        assert np.array_equal(bits(att[d["att_heads"]]), bits(d["att"]))
        rows = d["rows"]
        assert np.array_equal(kr[:, rows], d["kc_rows"])
        assert np.array_equal(vr[:, rows], d["vc_rows"])
    else:
        assert np.array_equal(bits(att), bits(d["att"]))
        assert np.array_equal(kr, d["kc"]) and np.array_equal(vr, d["vc"])


@pytest.mark.parametrize("arch", [orc.ARCH_LLAMA, orc.ARCH_QWEN3])
def test_rope_head_dim_over_1024_is_left_unrotated(arch):
    """rope_th_llama / rope_th_neox (/root/reference/src/l3_math.c:67,86)
    print a message and return when head_dim/2 > 512: the compiled
    reference's rope leaves x unchanged for head_dim 1026 and 2048 and
    rotates it at 1024; the oracle does the same, bit for bit."""
    from helpers import require_ref
    L = require_ref()
    for hd, rotated in ((1024, True), (1026, False), (2048, False)):
        x = orc.normal(61 + hd, 2 * hd)
        ref = x.copy()
        L.ref_rope(arch, ref, ref.size, 37, hd, 1e4)
        got = orc.rope(arch, x, 37, hd, 1e4)
        assert np.array_equal(bits(got), bits(ref)), hd
        assert np.array_equal(bits(got), bits(x)) != rotated, hd
