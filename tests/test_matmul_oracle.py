"""The weight-GEMV oracle (oracle/orc.py: matmul_scalar, matmul_exact) pinned
without a GPU:
  * bit-exact with the compiled reference's scalar matmul_q8_0 / matmul_q4_0 /
    matmul (l2_codec.c:306-340, l3_math.c:17-20; oracle/_ref scalar build),
    and with matmul_q's dequantising fallback (l2_codec.c:350-366) for F16
    and Q4_1 in both builds (the fallback is a serial fp32 loop in each);
  * within the serial-summation error bound of a float64 evaluation of the
    same (exactly dequantised) weights, as is the AVX2 reference;
  * the float64 evaluation itself against closed forms (one-hot x picks a
    column; constant nibble 8 gives zero weights; a block scale of 2^k scales
    the output by 2^k exactly).
"""
import numpy as np
import pytest

from helpers import require_ref
from oracle import orc
from gguf2bin_amd import attn

U = 2.0 ** -24
TYPES = [orc.T_Q8_0, orc.T_Q4_0, orc.T_F32, orc.T_F16, orc.T_Q4_1]
SHAPES = [(32, 1), (64, 5), (100, 9), (576, 33), (1024, 64), (3072, 17)]


def shape_ok(t, n):
    """Q4_1 rows must be whole blocks (the reference's fallback dequantises
    ceil(n/32) blocks into an n-element buffer otherwise)."""
    return t != orc.T_Q4_1 or n % 32 == 0


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n,d", SHAPES)
def test_scalar_restatement_bit_exact_with_reference(t, n, d):
    if not shape_ok(t, n):
        pytest.skip("Q4_1 needs whole blocks")
    require_ref("scalar")
    rng = np.random.default_rng(n * 7 + d + t)
    w = orc.random_weights(rng, t, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    a = orc.matmul_scalar(x, w, t, n, d)
    r = orc.ref_matmul(x, w, t, n, d, "scalar")
    assert np.array_equal(a.view(np.uint32), r.view(np.uint32))
    if t in (orc.T_F16, orc.T_Q4_1):  # the fallback: the same serial loop in the AVX2 build
        r2 = orc.ref_matmul(x, w, t, n, d, "avx2")
        assert np.array_equal(a.view(np.uint32), r2.view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n,d", SHAPES)
def test_oracle_and_avx2_reference_within_fp32_bound(t, n, d):
    if not shape_ok(t, n):
        pytest.skip("Q4_1 needs whole blocks")
    rng = np.random.default_rng(n * 11 + d + t)
    w = orc.random_weights(rng, t, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    ex, ab = orc.matmul_exact(x, w, t, n, d)
    terms = n if t in (orc.T_F32, orc.T_F16) else (n // 32) * 32
    bound = (terms + 2) * U * ab  # serial summation of terms products
    assert np.all(np.abs(orc.matmul_scalar(x, w, t, n, d) - ex) <= bound)
    if orc.ref_lib("avx2") is not None:
        assert np.all(np.abs(orc.ref_matmul(x, w, t, n, d, "avx2") - ex) <= bound)


@pytest.mark.parametrize("t", [orc.T_Q8_0, orc.T_Q4_0])
def test_exact_evaluation_closed_forms(t):
    n, d = 96, 4
    rng = np.random.default_rng(5)
    w = orc.random_weights(rng, t, n, d)
    bb = 34 if t == orc.T_Q8_0 else 18
    blk = w.reshape(d, n // 32, bb)
    # one-hot x at column j: the output is that column's dequantised weight
    for j in (0, 17, 31, 32, 95):
        x = np.zeros(n, np.float32)
        x[j] = 1.0
        ex, _ = orc.matmul_exact(x, w, t, n, d)
        b, e = divmod(j, 32)
        s = blk[:, b, :2].copy().view(np.float16).astype(np.float64).ravel()
        if t == orc.T_Q8_0:
            q = blk[:, b, 2 + e].view(np.int8).astype(np.float64)
        else:
            byte = blk[:, b, 2 + (e % 16)]
            q = ((byte & 0x0F) if e < 16 else (byte >> 4)).astype(np.float64) - 8
        assert np.array_equal(ex, s * q)
    # Q4_0 nibble 8 everywhere is the zero matrix
    if t == orc.T_Q4_0:
        z = blk.copy()
        z[:, :, 2:] = 0x88
        ex, ab = orc.matmul_exact(rng.standard_normal(n), z.ravel(), t, n, d)
        assert not ex.any() and not ab.any()
    # scale 2^k -> output x 2^k exactly
    x = rng.standard_normal(n).astype(np.float32)
    one = blk.copy()
    one[:, :, :2] = np.array([1.0], np.float16).view(np.uint8)
    four = blk.copy()
    four[:, :, :2] = np.array([4.0], np.float16).view(np.uint8)
    e1, _ = orc.matmul_exact(x, one.ravel(), t, n, d)
    e4, _ = orc.matmul_exact(x, four.ravel(), t, n, d)
    assert np.array_equal(e4, 4 * e1)


def test_fallback_types_closed_forms():
    """gguf_dequant's F16 (exact half_to_float) and Q4_1 (s*q + m, one fp32
    rounding) weights, independent of the C code: one-hot x picks a weight;
    a Q4_1 block of zero nibbles is its m; s = 1, m = 0 gives the nibbles."""
    n, d = 64, 3
    rng = np.random.default_rng(9)
    wh = orc.random_weights(rng, orc.T_F16, n, d)
    halves = wh.view(np.float16).reshape(d, n).astype(np.float64)
    w1 = orc.random_weights(rng, orc.T_Q4_1, n, d)
    blk = w1.reshape(d, n // 32, 20)
    for j in (0, 15, 16, 31, 33, 63):
        x = np.zeros(n, np.float32)
        x[j] = 1.0
        assert np.array_equal(orc.matmul_exact(x, wh, orc.T_F16, n, d)[0], halves[:, j])
        b, e = divmod(j, 32)
        s = blk[:, b, 0:2].copy().view(np.float16).astype(np.float32).ravel()
        m = blk[:, b, 2:4].copy().view(np.float16).astype(np.float32).ravel()
        byte = blk[:, b, 4 + (e % 16)]
        q = ((byte & 0x0F) if e < 16 else (byte >> 4)).astype(np.float32)
        want = (s * q + m).astype(np.float32).astype(np.float64)  # float32 rounding of s*q + m
        assert np.array_equal(orc.matmul_exact(x, w1, orc.T_Q4_1, n, d)[0], want)
    z = blk.copy()
    z[:, :, 4:] = 0
    x = rng.standard_normal(n).astype(np.float32)
    m = z[:, :, 2:4].copy().view(np.float16).astype(np.float64).reshape(d, n // 32)
    want = (m[:, :, None] * x.astype(np.float64).reshape(1, n // 32, 32)).sum(axis=(1, 2))
    np.testing.assert_allclose(orc.matmul_exact(x, z.ravel(), orc.T_Q4_1, n, d)[0], want,
                               rtol=1e-12)
    u = blk.copy()
    u[:, :, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    u[:, :, 2:4] = 0
    deq = orc.dequant_rows(u.ravel(), orc.T_Q4_1, n, d).reshape(d, n // 32, 32)
    assert np.array_equal(deq[:, :, :16], (u[:, :, 4:] & 0x0F).astype(np.float32))
    assert np.array_equal(deq[:, :, 16:], (u[:, :, 4:] >> 4).astype(np.float32))


@pytest.mark.parametrize("t", TYPES)
def test_row_bytes(t):
    for n in (0, 31, 32, 100, 1024, 14336):
        assert attn.matmul_row_bytes(t, n) == orc.matmul_row_bytes(t, n)
    assert attn.matmul_row_bytes(t, -1) == 0
    for kq in (orc.T_Q2_K, orc.T_Q3_K, orc.T_Q4_K, orc.T_Q5_K, orc.T_Q6_K, orc.T_Q8_K):
        assert attn.matmul_row_bytes(kq, 256) == 0  # K-quants: no device GEMV
