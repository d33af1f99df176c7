"""Device weight GEMVs (include/g2b_matmul.h) through the C ABI against the
oracle (tests/test_matmul_oracle.py pins it to the compiled reference).

Bar: fp32 arithmetic in another summation order than the reference, so
|out - exact| <= 64 * 2^-24 * sum_j |w_ij x_j| per output, with exact the
float64 product of the exactly dequantised weights; and, where the compiled
reference travelled with the tree, |out - reference| within the sum of the
two bounds.
"""
import numpy as np
import pytest

from oracle import orc
from gguf2bin_amd import attn, hip

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
TYPES = [orc.T_Q8_0, orc.T_Q4_0, orc.T_F32, orc.T_F16, orc.T_Q4_1]
# n covers every lane layout: 1, 2, 3 (+ tail), 18, 32, 48, 64, 96, 128 blocks
# (x of one or two blocks per lane in registers) and 256 / 448 blocks (x
# through the cache); d covers partial wave-steps and several grid passes
SHAPES = [(32, 1), (64, 3), (100, 7), (576, 257), (1024, 1000), (1536, 33), (2048, 4099),
          (3072, 64), (4096, 130), (8192, 70), (14336, 40)]
SHAPE = attn.Shape(1, 2, 1, 64, 1e4, attn.ARCH_QWEN3, False)


def check(out, x, w, t, n, d, what):
    ex, ab = orc.matmul_exact(x, w, t, n, d)
    err = np.abs(out.astype(np.float64) - ex)
    bad = err > 64 * U * ab
    assert not bad.any(), f"{what}: {bad.sum()} rows over the bound, worst {np.max(err / (ab + 1e-300))}"
    if orc.ref_lib("avx2") is not None and n * d <= 1 << 22:
        r = orc.ref_matmul(x, w, t, n, d, "avx2")
        assert np.all(np.abs(out - r) <= 64 * U * ab + (n + 2) * U * ab), what


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n,d", SHAPES)
def test_matmul_vs_exact(gpu_device, t, n, d):
    if t == orc.T_Q4_1 and n % 32:
        pytest.skip("Q4_1 rows are whole blocks (G2B_EINVAL otherwise)")
    rng = np.random.default_rng(1000 * n + d + t)
    w = orc.random_weights(rng, t, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    print(f"[gemv] type={t} n={n} d={d}", flush=True)
    with attn.Context(SHAPE) as ctx:
        wd = ctx.weights_upload(w)
        try:
            xd = hip.to_device(x)
            od = hip.DeviceBuffer(d * 4)
            ctx.matmul(od.ptr, xd.ptr, wd, t, n, d)
            ctx.sync()
            out = od.download(np.float32, d)
            host = ctx.matmul_host(x, wd, t, n, d)
        finally:
            ctx.weights_free(wd)
    check(out, x, w, t, n, d, f"type {t} n {n} d {d}")
    assert np.array_equal(out.view(np.uint32), host.view(np.uint32))


@pytest.mark.parametrize("t", [orc.T_Q8_0, orc.T_Q4_0, orc.T_Q4_1, orc.T_F16])
def test_matmul_unaligned_operands(gpu_device, t):
    """x at a 4-byte (not 16-byte) boundary takes the cached-x path; weights
    starting 2 bytes into an allocation put every other block at the other
    dword phase."""
    n, d = 1024, 300
    rng = np.random.default_rng(77 + t)
    w = orc.random_weights(rng, t, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    with attn.Context(SHAPE) as ctx:
        wd = ctx.weights_upload(np.concatenate([np.zeros(2, np.uint8), w, np.zeros(6, np.uint8)]))
        try:
            xd = hip.to_device(np.concatenate([np.zeros(1, np.float32), x]))
            od = hip.DeviceBuffer(d * 4)
            ctx.matmul(od.ptr, xd.ptr + 4, wd + 2, t, n, d)
            ctx.sync()
            out = od.download(np.float32, d)
        finally:
            ctx.weights_free(wd)
    check(out, x, w, t, n, d, "unaligned")


def test_matmul_guards_and_errors(gpu_device):
    """matmul_q's guard (l2_codec.c:343-346): null x or w, n <= 0 or d <= 0
    zero the output; unsupported types and odd weight pointers are errors."""
    n, d = 64, 10
    rng = np.random.default_rng(3)
    w = orc.random_weights(rng, orc.T_Q8_0, n, d)
    with attn.Context(SHAPE) as ctx:
        wd = ctx.weights_upload(w)
        try:
            xd = hip.to_device(rng.standard_normal(n).astype(np.float32))
            od = hip.to_device(np.full(d, 7.0, np.float32))
            for args in ((0, wd, n), (xd.ptr, 0, n), (xd.ptr, wd, 0), (xd.ptr, wd, -5)):
                hip.copy_h2d(od.ptr, np.full(d, 7.0, np.float32))
                ctx.matmul(od.ptr, args[0], args[1], orc.T_Q8_0, args[2], d)
                ctx.sync()
                assert not od.download(np.float32, d).any(), args
            ctx.matmul(od.ptr, xd.ptr, wd, orc.T_Q8_0, n, 0)  # d = 0: nothing to do
            for kq in (orc.T_Q2_K, orc.T_Q4_K, orc.T_Q6_K, orc.T_Q8_K):  # K-quants
                with pytest.raises(attn.G2BError) as e:
                    ctx.matmul(od.ptr, xd.ptr, wd, kq, 256, d)
                assert e.value.code == attn.G2B_EUNSUP
            with pytest.raises(attn.G2BError) as e:  # Q4_1 rows of whole blocks only
                ctx.matmul(od.ptr, xd.ptr, wd, orc.T_Q4_1, 48, d)
            assert e.value.code == attn.G2B_EINVAL
            with pytest.raises(attn.G2BError) as e:
                ctx.matmul(od.ptr, xd.ptr, wd + 1, orc.T_Q8_0, n, d)
            assert e.value.code == attn.G2B_EINVAL
            assert not ctx.matmul_host(np.zeros(0, np.float32), wd, orc.T_Q8_0, 0, d).any()
        finally:
            ctx.weights_free(wd)


@pytest.mark.parametrize("t", [orc.T_Q8_0, orc.T_Q4_0, orc.T_F16, orc.T_Q4_1])
def test_matmul_lm_head_full_size(gpu_device, t):
    """The measured shape: Qwen3-0.6B's output projection (vocab 151936 x
    dim 1024), every row against the float64 product."""
    n, d = 1024, 151936
    rng = np.random.default_rng(9 + t)
    w = orc.random_weights(rng, t, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    with attn.Context(SHAPE) as ctx:
        wd = ctx.weights_upload(w)
        try:
            out = ctx.matmul_host(x, wd, t, n, d)
        finally:
            ctx.weights_free(wd)
    check(out, x, w, t, n, d, "lm head")


@pytest.mark.parametrize("t", [orc.T_Q4_0, orc.T_Q4_1])
@pytest.mark.parametrize("case", ["normal", "outlier", "zero_blocks", "tiny", "huge"])
def test_q4_matrix_core_path(gpu_device, case, t):
    """Plain Q4_0 and Q4_1 products of 1024-element rows with at least 32768
    rows run on the int8 matrix cores (x as four int8 digit planes of a
    31-bit fixed point per block; Q4_1's m times each block's sum of x): the
    same bar as every GEMV, with x that stresses the digits - one channel
    3e4 x the others, whole blocks of zeros, x near the bottom of the normal
    range (1e-36) and near the top (1e35)."""
    n, d = 1024, 40000
    rng = np.random.default_rng(4321)
    w = orc.random_weights(rng, t, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    if case == "outlier":
        x[37] = np.float32(3e4)
    elif case == "zero_blocks":
        x[64:160] = 0
        x[1000:] = 0
    elif case == "tiny":
        x = (x * np.float32(1e-36)).astype(np.float32)
    elif case == "huge":
        x = (x * np.float32(1e30)).astype(np.float32)
    print(f"[gemv] q4 matrix cores type={t} {case}", flush=True)
    with attn.Context(SHAPE) as ctx:
        wd = ctx.weights_upload(w)
        try:
            xd = hip.to_device(x)
            od = hip.DeviceBuffer(d * 4)
            ctx.matmul(od.ptr, xd.ptr, wd, t, n, d)
            ctx.sync()
            out = od.download(np.float32, d)
        finally:
            ctx.weights_free(wd)
    check(out, x, w, t, n, d, f"q4 matrix cores type {t} {case}")


@pytest.mark.parametrize("n", [512, 1024, 2048, 3072])
@pytest.mark.parametrize("case", ["normal", "outlier", "zero_blocks", "tiny", "huge"])
def test_q8_digit_plane_path(gpu_device, n, case):
    """Q8_0 products over at least 32768 rows of 16-96 blocks take x as four
    int8 digit planes of a 31-bit fixed point per block: integer dot
    products against the quants on the VALU (16, 64 and 96 blocks: one and
    two blocks per lane) or on the int8 matrix cores (32 blocks).  The same
    bar as every GEMV, with the x that stresses the digits (one channel 3e4
    x the others, whole blocks of zeros, x near the bottom of the normal
    range and near the top)."""
    d, t = 33000, orc.T_Q8_0
    rng = np.random.default_rng(77 + n)
    w = orc.random_weights(rng, t, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    if case == "outlier":
        x[37] = np.float32(3e4)
    elif case == "zero_blocks":
        x[64:160] = 0
        x[n - 24:] = 0
    elif case == "tiny":
        x = (x * np.float32(1e-36)).astype(np.float32)
    elif case == "huge":
        x = (x * np.float32(1e30)).astype(np.float32)
    print(f"[gemv] q8 digit planes n={n} {case}", flush=True)
    with attn.Context(SHAPE) as ctx:
        wd = ctx.weights_upload(w)
        try:
            xd = hip.to_device(x)
            od = hip.DeviceBuffer(d * 4)
            ctx.matmul(od.ptr, xd.ptr, wd, t, n, d)
            ctx.sync()
            out = od.download(np.float32, d)
        finally:
            ctx.weights_free(wd)
    check(out, x, w, t, n, d, f"q8 digit planes n {n} {case}")


@pytest.mark.parametrize("t", [orc.T_Q8_0, orc.T_Q4_0, orc.T_Q4_1])
@pytest.mark.parametrize("case", ["outlier", "tiny", "huge"])
def test_vector_path_hard_x(gpu_device, case, t):
    """The VALU GEMVs (fewer rows than the matrix cores take) with the x that
    stresses a summation order: one channel 3e4 x the others, x near the
    bottom of the normal range and near the top - the same bar as every
    GEMV."""
    n, d = 1024, 4096
    rng = np.random.default_rng(99 + t)
    w = orc.random_weights(rng, t, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    if case == "outlier":
        x[37] = np.float32(3e4)
    elif case == "tiny":
        x = (x * np.float32(1e-36)).astype(np.float32)
    else:
        x = (x * np.float32(1e30)).astype(np.float32)
    print(f"[gemv] vector path type={t} {case}", flush=True)
    with attn.Context(SHAPE) as ctx:
        wd = ctx.weights_upload(w)
        try:
            xd = hip.to_device(x)
            od = hip.DeviceBuffer(d * 4)
            ctx.matmul(od.ptr, xd.ptr, wd, t, n, d)
            ctx.sync()
            out = od.download(np.float32, d)
        finally:
            ctx.weights_free(wd)
    check(out, x, w, t, n, d, f"vector path type {t} {case}")


@pytest.mark.parametrize("t", [orc.T_Q8_0, orc.T_Q4_0, orc.T_Q4_1])
@pytest.mark.parametrize("form", ["lds_dma", "direct"])
def test_matrix_core_ragged_rows(gpu_device, t, form):
    """The matrix-core GEMV at a row count that ends inside a trip: 32771
    rows are 8193 wave-steps of four, so the LDS-DMA form's last pair holds
    one real wave-step of three rows and one past the matrix (its loads run
    past the buffer's end and read zeros).  A 16-byte aligned matrix takes
    the LDS-DMA form, one 4 bytes off takes the direct loads.  Every row
    against the float64 product, and nothing stored past the last row."""
    n, d = 1024, 32771
    rng = np.random.default_rng(5150 + t)
    w = orc.random_weights(rng, t, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    pad = 0 if form == "lds_dma" else 4
    print(f"[gemv] ragged rows type={t} {form}", flush=True)
    with attn.Context(SHAPE) as ctx:
        wd = ctx.weights_upload(np.concatenate([np.zeros(pad, np.uint8), w]))
        try:
            xd = hip.to_device(x)
            od = hip.to_device(np.full(d + 64, 7.0, np.float32))
            ctx.matmul(od.ptr, xd.ptr, wd + pad, t, n, d)
            ctx.sync()
            full = od.download(np.float32, d + 64)
        finally:
            ctx.weights_free(wd)
    assert np.all(full[d:] == 7.0), "stores past the last row"
    check(full[:d], x, w, t, n, d, f"ragged rows type {t} {form}")
