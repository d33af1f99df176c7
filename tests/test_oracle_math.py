"""Pins of the oracle that do not rely on the reference: independent
implementations (numpy's float16), closed forms, special cases fixed by the
definitions, float64 brute force, and invariants.  Each is chosen so that a
plausible slip (rounding instead of truncating, half-to-even instead of
half-away, swapped RoPE pairing, a dropped scale, an off-by-one in pos)
fails at least one of them."""
import numpy as np
import pytest

from oracle import orc


# ---------------------------------------------------------------- fp16

def test_half_to_float_matches_numpy_float16():
    h = np.arange(65536, dtype=np.uint16)
    got = orc.half_to_float(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_half_truncates_toward_zero():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 100,
        np.exp(rng.uniform(np.log(6.2e-5), np.log(65000), 200000)).astype(np.float32),
        np.array([6.103515625e-05, 65504.0, 65519.99, 1.0, -1.0, 0.1, -0.1], np.float32),
    ])
    h = orc.f32_to_half(x)
    back = h.view(np.float16).astype(np.float64)
    ax = np.abs(x.astype(np.float64))
    normal = (ax >= 2.0 ** -14) & (ax < 65536.0)
    # |back| <= |x| < next half above |back|, same sign
    nxt = (np.abs(h[normal].view(np.float16)).view(np.uint16) + 1).view(np.float16)
    assert np.all(np.abs(back[normal]) <= ax[normal])
    assert np.all(ax[normal] < nxt.astype(np.float64))
    assert np.all(np.signbit(back[normal]) == np.signbit(x[normal]))


def test_f32_to_half_special_ranges():
    x = np.array([1e-5, -1e-5, 6.1e-5, 0.0, -0.0, 65536.0, -7e4, 1e30, np.inf, -np.inf, np.nan],
                 np.float32)
    h = orc.f32_to_half(x)
    # below the normal range -> signed zero (no subnormals); overflow, Inf, NaN -> signed Inf
    assert list(h[:5]) == [0x0000, 0x8000, 0x0000, 0x0000, 0x8000]
    assert list(h[5:10]) == [0x7C00, 0xFC00, 0x7C00, 0x7C00, 0xFC00]
    assert h[10] & 0x7FFF == 0x7C00


# ---------------------------------------------------------------- Q8_0

def _blocks(row):
    return row.reshape(-1, 34)


def test_q8_tie_rounds_half_away_from_zero():
    # amax = 127 makes d = 1 exactly, so x/d = x and ties are exact
    row = np.zeros(32, np.float32)
    row[0] = 127.0
    row[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]
    q = orc.q8_quant_row(row).view(np.int8)[2:34]
    assert list(q[:9]) == [127, 1, 2, 3, -1, -2, -3, 127, -127]


def test_q8_scale_is_truncated_fp16_of_amax_over_127():
    rng = np.random.default_rng(2)
    for _ in range(200):
        x = (rng.standard_normal(32) * rng.uniform(0.01, 50)).astype(np.float32)
        b = orc.q8_quant_row(x)
        d = np.float32(np.abs(x).max()) / np.float32(127.0)
        s = b[:2].view(np.uint16)[0]
        sv = np.float64(np.uint16(s).view(np.float16))
        assert sv <= d and d < np.float64((np.uint16(s) + 1).view(np.float16))
        q = b[2:].view(np.int8).astype(np.int32)
        assert np.abs(q).max() == 127  # the largest element maps to +-127
        # dequantisation error bound: rounding (d/2) plus the truncated scale
        err = np.abs(x.astype(np.float64) - sv * q)
        assert np.all(err <= d / 2 * (1 + 1e-6) + 127 * (d - sv) + 1e-12)


def test_q8_zero_and_tiny_blocks():
    z = orc.q8_quant_row(np.zeros(64, np.float32))
    assert not z.any()  # fp16(1e-10) is 0x0000 and every q is 0
    tiny = np.linspace(-0.007, 0.007, 32).astype(np.float32)
    b = orc.q8_quant_row(tiny)
    assert b[0] == 0 and b[1] == 0  # scale below fp16's normal range
    assert np.abs(b[2:].view(np.int8)).max() == 127


def test_q8_partial_block_is_zero_padded():
    x = np.arange(1, 46, dtype=np.float32)
    b = _blocks(orc.q8_quant_row(x))
    assert b.shape == (2, 34)
    assert not b[1, 2 + 13:].any()
    deq = orc.q8_dequant_row(b.ravel(), 45)
    assert np.max(np.abs(deq - x)) < 0.5


# ---------------------------------------------------------------- RoPE

@pytest.mark.parametrize("arch", [orc.ARCH_LLAMA, orc.ARCH_QWEN3])
def test_rope_pos0_identity(arch):
    x = orc.normal(5, 4 * 128)
    assert np.array_equal(orc.rope(arch, x, 0, 128, 1e6).view(np.uint32), x.view(np.uint32))


@pytest.mark.parametrize("arch", [orc.ARCH_LLAMA, orc.ARCH_QWEN3])
def test_rope_preserves_pair_norms(arch):
    hd = 64
    x = orc.normal(6, 3 * hd).astype(np.float64)
    y = orc.rope(arch, x.astype(np.float32), 777, hd, 1e4).astype(np.float64)
    x3, y3 = x.reshape(3, hd), y.reshape(3, hd)
    if arch == orc.ARCH_LLAMA:
        nx = x3[:, 0::2] ** 2 + x3[:, 1::2] ** 2
        ny = y3[:, 0::2] ** 2 + y3[:, 1::2] ** 2
    else:
        nx = x3[:, :hd // 2] ** 2 + x3[:, hd // 2:] ** 2
        ny = y3[:, :hd // 2] ** 2 + y3[:, hd // 2:] ** 2
    np.testing.assert_allclose(ny, nx, rtol=2e-6, atol=1e-9)


def test_rope_pairing_neox_vs_llama():
    hd, pos, th = 16, 3, 100.0
    cs = orc.rope_table(pos, hd, th)
    c1, s1 = cs[2], cs[3]  # pair j = 1
    e = np.zeros(hd, np.float32)
    e[1] = 1.0
    neox = orc.rope(orc.ARCH_QWEN3, e, pos, hd, th)   # pair (1, 1+hd/2)
    assert neox[1] == c1 and neox[1 + hd // 2] == s1
    e2 = np.zeros(hd, np.float32)
    e2[2] = 1.0
    llama = orc.rope(orc.ARCH_LLAMA, e2, pos, hd, th)  # pair (2, 3)
    assert llama[2] == c1 and llama[3] == s1


def test_rope_table_matches_float64_angles():
    for hd, th in ((128, 1e6), (64, 1e5), (128, 5e5)):
        for pos in (1, 17, 2048, 8192, 32767):
            cs = orc.rope_table(pos, hd, th).astype(np.float64)
            j = np.arange(hd // 2)
            ang = pos * th ** (-2.0 * j / hd)
            # the serial fp32 frequency product drifts by a few ulp per step
            tol = 1e-6 + pos * 6e-8 * (1 + j)
            assert np.all(np.abs(cs[0::2] - np.cos(ang)) <= tol)
            assert np.all(np.abs(cs[1::2] - np.sin(ang)) <= tol)


# ---------------------------------------------------------------- softmax / attention

def test_softmax_matches_float64():
    x = orc.normal(9, 1000) * 4
    y = orc.softmax(x).astype(np.float64)
    r = np.exp(x.astype(np.float64) - x.max())
    r /= r.sum()
    np.testing.assert_allclose(y, r, rtol=2e-6)
    assert abs(y.sum() - 1) < 1e-5


def _brute_force(shape, ctx_cap, layer, pos, kc, vc, q):
    """float64 attention over the oracle's own cache bytes and RoPE table."""
    hd, nh = shape.head_dim, shape.n_heads
    group = nh // shape.n_kv_heads
    cs = orc.rope_table(pos, hd, shape.rope_theta).astype(np.float64)
    c, s = cs[0::2], cs[1::2]
    q64 = q.astype(np.float64).reshape(nh, hd)
    if shape.arch == orc.ARCH_LLAMA:
        a, b = q64[:, 0::2].copy(), q64[:, 1::2].copy()
        q64[:, 0::2], q64[:, 1::2] = a * c - b * s, a * s + b * c
    else:
        a, b = q64[:, :hd // 2].copy(), q64[:, hd // 2:].copy()
        q64[:, :hd // 2], q64[:, hd // 2:] = a * c - b * s, a * s + b * c
    rb = shape.row_bytes
    K = np.zeros((pos + 1, shape.nkv))
    V = np.zeros((pos + 1, shape.nkv))
    for t in range(pos + 1):
        off = orc.kv_offset(shape, ctx_cap, layer, t)
        if shape.kv_q8:
            K[t] = orc.q8_dequant_row(kc[off:off + rb], shape.nkv)
            V[t] = orc.q8_dequant_row(vc[off:off + rb], shape.nkv)
        else:
            K[t] = kc[off:off + rb].view(np.float32)
            V[t] = vc[off:off + rb].view(np.float32)
    out = np.zeros((nh, hd))
    W = np.zeros((nh, pos + 1))
    for h in range(nh):
        g = h // group
        sc = K[:, g * hd:(g + 1) * hd] @ q64[h] / np.sqrt(hd)
        w = np.exp(sc - sc.max())
        w /= w.sum()
        W[h] = w
        out[h] = w @ V[:, g * hd:(g + 1) * hd]
    return out.ravel(), W


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("arch,nh,nkv,hd", [(orc.ARCH_QWEN3, 16, 8, 128), (orc.ARCH_LLAMA, 9, 3, 64),
                                             (orc.ARCH_QWEN3, 4, 2, 16)])
def test_attention_layer_vs_float64(q8, arch, nh, nkv, hd):
    shape = orc.Shape(2, nh, nkv, hd, 1e5, arch, q8)
    ctx_cap, pos, layer = 80, 70, 1
    kc, vc = orc.alloc_kv(shape, ctx_cap)
    kp = orc.normal(31, pos * shape.nkv).reshape(pos, shape.nkv)
    vp = orc.normal(32, pos * shape.nkv).reshape(pos, shape.nkv)
    orc.kv_prefill(shape, ctx_cap, layer, 0, kc, vc, kp, vp)
    q, k, v = orc.normal(33, shape.nq), orc.normal(34, shape.nkv), orc.normal(35, shape.nkv)
    out, att = orc.attn_layer(shape, ctx_cap, layer, pos, kc, vc, q, k, v)
    ref, W = _brute_force(shape, ctx_cap, layer, pos, kc, vc, q)
    np.testing.assert_allclose(out, ref, atol=3e-6, rtol=0)
    np.testing.assert_allclose(att, W, rtol=1e-5, atol=0)
    # nothing of layer 0 was touched
    assert not kc[:ctx_cap * shape.row_bytes].any()


def test_attention_invariants():
    shape = orc.Shape(1, 4, 2, 32, 1e4, orc.ARCH_QWEN3, True)
    ctx_cap, pos = 40, 30
    kc, vc = orc.alloc_kv(shape, ctx_cap)
    kp = orc.normal(41, pos * shape.nkv).reshape(pos, shape.nkv)
    vrow = orc.normal(42, shape.nkv)
    orc.kv_prefill(shape, ctx_cap, 0, 0, kc, vc, kp, np.tile(vrow, (pos, 1)))
    # q = 0 -> every score is 0 -> uniform weights; constant V -> output = dequantised V
    out, att = orc.attn_layer(shape, ctx_cap, 0, pos, kc, vc, np.zeros(shape.nq, np.float32),
                              orc.normal(43, shape.nkv), vrow)
    assert np.all(att == np.float32(1.0) / np.float32(pos + 1))
    vdeq = orc.q8_dequant_row(orc.q8_quant_row(vrow), shape.nkv)
    group = shape.n_heads // shape.n_kv_heads
    for h in range(shape.n_heads):
        g = h // group
        np.testing.assert_allclose(out[h * 32:(h + 1) * 32], vdeq[g * 32:(g + 1) * 32],
                                   rtol=2e-6, atol=1e-7)


def test_pos_outside_ctx_is_rejected():
    shape = orc.Shape(1, 2, 1, 16, 1e4, orc.ARCH_QWEN3, False)
    kc, vc = orc.alloc_kv(shape, 8)
    with pytest.raises(ValueError):
        orc.attn_layer(shape, 8, 0, 8, kc, vc, np.zeros(32, np.float32),
                       np.zeros(16, np.float32), np.zeros(16, np.float32))
    assert not kc.any() and not vc.any()


# ---------------------------------------------------------------- QK-RMSNorm

def _rms_f64(x, w, nh, hd, eps):
    x = x.astype(np.float64).reshape(nh, hd)
    ms = (x * x).mean(axis=1, keepdims=True)
    return (w.astype(np.float64) * x / np.sqrt(ms + eps)).ravel()


@pytest.mark.parametrize("hd,nh,scale,eps", [(128, 16, 1.0, 1e-6), (64, 9, 1e-3, 1e-6),
                                             (24, 3, 30.0, 1e-5), (128, 2, 1e-3, 0.0)])
def test_qk_rmsnorm_matches_float64(hd, nh, scale, eps):
    """Within a few fp32 ulps of w*x/sqrt(mean(x^2)+eps) in float64.  At
    x ~ 1e-3, mean(x^2) ~ 1e-6 is the size of eps, so a dropped or misplaced
    eps, a sum instead of a mean, or a missing weight fails by far more."""
    x = (orc.normal(hd * 7 + nh, nh * hd) * scale).astype(np.float32)
    w = (1 + 0.25 * orc.normal(hd * 11 + nh, hd)).astype(np.float32)
    got = orc.qk_rmsnorm(x, w, nh, hd, eps).astype(np.float64)
    ref = _rms_f64(x, np.tile(w, 1), nh, hd, eps)
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) < 2e-6


def test_qk_rmsnorm_unit_weights_give_unit_rms():
    """w = 1, eps = 0: every head comes out with mean square 1."""
    nh, hd = 5, 64
    x = orc.normal(99, nh * hd) * np.float32(7.0)
    y = orc.qk_rmsnorm(x, np.ones(hd, np.float32), nh, hd, 0.0).astype(np.float64)
    ms = (y.reshape(nh, hd) ** 2).mean(axis=1)
    assert np.allclose(ms, 1.0, rtol=1e-5)


def test_qk_rmsnorm_heads_are_independent_and_weights_per_element():
    """Scaling one head by 2^k leaves the others unchanged and (eps = 0) its
    own output unchanged; weights multiply element by element."""
    nh, hd = 4, 32
    x = orc.normal(5, nh * hd)
    w = (1 + 0.5 * orc.normal(6, hd)).astype(np.float32)
    y = orc.qk_rmsnorm(x, w, nh, hd, 0.0)
    x2 = x.copy()
    x2[hd:2 * hd] *= np.float32(8.0)
    y2 = orc.qk_rmsnorm(x2, w, nh, hd, 0.0)
    assert np.array_equal(y, y2)
    y1 = orc.qk_rmsnorm(x, np.ones(hd, np.float32), nh, hd, 0.0)
    assert np.allclose(y.reshape(nh, hd), (y1.reshape(nh, hd) * w), rtol=3e-7, atol=0)


def test_qk_rmsnorm_zero_head_and_eps():
    """A zero head stays zero (0 * 1/sqrt(eps)); eps alone sets the scale of a
    head whose mean square is far below it."""
    hd = 16
    z = orc.qk_rmsnorm(np.zeros(hd, np.float32), np.ones(hd, np.float32), 1, hd, 1e-6)
    assert np.array_equal(z, np.zeros(hd, np.float32))
    x = np.full(hd, 1e-9, np.float32)
    y = orc.qk_rmsnorm(x, np.ones(hd, np.float32), 1, hd, 1e-2)
    assert np.allclose(y, 1e-9 / np.sqrt(1e-2 + 1e-18), rtol=1e-6)

