"""ctypes wrapper for the CPU oracle (oracle/liborc.so) and, where it was
built, the compiled reference (oracle/_ref/libg2bref_*.so).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py may import this module, and only as the
checker or the timed CPU baseline; the product path never does.

The C functions restate /root/reference/src/l5_model.c:47-67,232-265,448-452,
513-578, src/l3_math.c:6-16,52-56,64-102 and src/l2_codec.c:35-54 (see
oracle/orc.h for the per-function citations and how each one is pinned).
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBORC = os.path.join(HERE, "liborc.so")
REF_DIR = os.path.join(HERE, "_ref")

ARCH_LLAMA, ARCH_QWEN2, ARCH_QWEN3 = 0, 1, 2

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


class OrcShape(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int32),
        ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("rope_theta", C.c_float),
        ("arch", C.c_int32),
        ("kv_q8", C.c_int32),
    ]


@dataclass(frozen=True)
class Shape:
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    rope_theta: float
    arch: int
    kv_q8: bool

    @property
    def nq(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def nkv(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def row_bytes(self) -> int:
        return q8_rowsize(self.nkv) if self.kv_q8 else self.nkv * 4

    def c(self) -> OrcShape:
        return OrcShape(self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim,
                        self.rope_theta, self.arch, 1 if self.kv_q8 else 0)


def q8_rowsize(nkv: int) -> int:
    return (nkv + 31) // 32 * 34


_lib = None


def lib() -> C.CDLL:
    """Load liborc.so (built by ``make -C oracle``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBORC):
            raise RuntimeError(f"{LIBORC} missing: run `make -C oracle`")
        L = C.CDLL(LIBORC)
        L.orc_splitmix64.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_splitmix64.restype = C.c_uint64
        L.orc_normal_f32.argtypes = [C.POINTER(C.c_uint64), _f32p, C.c_size_t]
        L.orc_f32_to_half_n.argtypes = [_f32p, _u16p, C.c_size_t]
        L.orc_half_to_float_n.argtypes = [_u16p, _f32p, C.c_size_t]
        L.orc_q8_quant_row.argtypes = [_f32p, _u8p, C.c_int32]
        L.orc_q8_dequant_row.argtypes = [_u8p, _f32p, C.c_int32]
        L.orc_rope_table.argtypes = [C.c_int32, C.c_int32, C.c_float, _f32p]
        L.orc_rope_table.restype = C.c_int
        L.orc_rope.argtypes = [C.c_int32, _f32p, C.c_int32, C.c_int32, C.c_int32, C.c_float]
        L.orc_softmax.argtypes = [_f32p, C.c_int32]
        L.orc_qk_rmsnorm.argtypes = [_f32p, _f32p, C.c_int32, C.c_int32, C.c_float]
        L.orc_kv_prefill.argtypes = [C.POINTER(OrcShape), C.c_int32, C.c_int32, C.c_int32,
                                     C.c_int32, _u8p, _u8p, _f32p, _f32p]
        L.orc_attn_layer.argtypes = [C.POINTER(OrcShape), C.c_int32, C.c_int32, C.c_int32,
                                     _u8p, _u8p, _f32p, _f32p, _f32p, _f32p, C.c_int]
        L.orc_attn_layer.restype = C.c_int
        L.orc_attn_batch.argtypes = [C.POINTER(OrcShape), C.c_int32, C.c_int32, C.c_int32,
                                     _i32p, _i32p, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p),
                                     _f32p, _f32p, _f32p, C.c_int]
        L.orc_attn_batch.restype = C.c_int
        L.orc_now_sec.restype = C.c_double
        L.orc_max_threads.restype = C.c_int
        _lib = L
    return _lib


# ---------------------------------------------------------------- RNG

def normal(seed: int, n: int) -> np.ndarray:
    """n float32 N(0,1) values of the SplitMix64/Box-Muller stream ``seed``."""
    st = C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)
    out = np.empty(n, np.float32)
    if n:
        lib().orc_normal_f32(C.byref(st), out, n)
    return out


def stream_seed(base: int, seq: int, layer: int, tensor: int) -> int:
    """Seed of the synthetic stream for (sequence, layer, tensor).

    tensor: 0 = K prefill rows, 1 = V prefill rows, 2 = new q, 3 = new k,
    4 = new v, 5 = row-scale selector.  Same formula as the device fill.
    """
    m = 0xFFFFFFFFFFFFFFFF

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        return z ^ (z >> 31)

    z = mix((base ^ (tensor * 0xD1B54A32D192ED03)) & m)
    z = mix((z + (seq + 1) * 0x9E3779B97F4A7C15) & m)
    return mix((z + (layer + 1) * 0xC2B2AE3D27D4EB4F) & m)


# ---------------------------------------------------------------- codec

def f32_to_half(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().orc_f32_to_half_n(x, out, x.size)
    return out


def half_to_float(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16).ravel()
    out = np.empty(h.size, np.float32)
    lib().orc_half_to_float_n(h, out, h.size)
    return out


def q8_quant_row(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(q8_rowsize(x.size), np.uint8)
    lib().orc_q8_quant_row(x, out, x.size)
    return out


def q8_dequant_row(b: np.ndarray, n: int) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint8).ravel()
    assert b.size >= q8_rowsize(n)
    out = np.empty(n, np.float32)
    lib().orc_q8_dequant_row(b, out, n)
    return out


def rope_table(pos: int, head_dim: int, theta: float) -> np.ndarray:
    cs = np.zeros(max(head_dim, 2), np.float32)
    rc = lib().orc_rope_table(pos, head_dim, theta, cs)
    if rc:
        raise ValueError("head_dim/2 > 512")
    return cs[:head_dim]


def rope(arch: int, x: np.ndarray, pos: int, head_dim: int, theta: float) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy().ravel()
    lib().orc_rope(arch, y, y.size, pos, head_dim, theta)
    return y


def qk_rmsnorm(x: np.ndarray, w: np.ndarray, n_heads: int, head_dim: int,
               eps: float) -> np.ndarray:
    """QK-RMSNorm of n_heads heads (l3_math.c:107-114); returns a new array."""
    y = np.ascontiguousarray(x, np.float32).copy().reshape(-1)
    ww = np.ascontiguousarray(w, np.float32).reshape(-1)
    assert y.size >= n_heads * head_dim and ww.size >= head_dim
    lib().orc_qk_rmsnorm(y, ww, n_heads, head_dim, eps)
    return y


def softmax(x: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy().ravel()
    lib().orc_softmax(y, y.size)
    return y


# ---------------------------------------------------------------- KV + attention

def alloc_kv(shape: Shape, ctx_cap: int):
    n = shape.n_layers * ctx_cap * shape.row_bytes
    return np.zeros(n, np.uint8), np.zeros(n, np.uint8)


def kv_offset(shape: Shape, ctx_cap: int, layer: int, pos: int) -> int:
    return (layer * ctx_cap + pos) * shape.row_bytes


def kv_prefill(shape: Shape, ctx_cap: int, layer: int, pos0: int, kc: np.ndarray,
               vc: np.ndarray, k_rows: np.ndarray, v_rows: np.ndarray):
    """RoPE + append rows [pos0, pos0+n) of one layer into kc/vc in place."""
    k_rows = np.ascontiguousarray(k_rows, np.float32)
    v_rows = np.ascontiguousarray(v_rows, np.float32)
    n = int(k_rows.shape[0]) if k_rows.ndim > 1 else 0
    if n:
        lib().orc_kv_prefill(C.byref(shape.c()), ctx_cap, layer, pos0, n, kc, vc,
                             k_rows.reshape(-1), v_rows.reshape(-1))


def attn_layer(shape: Shape, ctx_cap: int, layer: int, pos: int, kc: np.ndarray,
               vc: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray,
               avx2_order: bool = True):
    """One layer (RoPE, append into kc/vc in place, attention).

    Returns (out [nq], att [n_heads, pos+1]) or raises on a bad pos."""
    qo = np.ascontiguousarray(q, np.float32).copy().ravel()
    att = np.zeros(shape.n_heads * ctx_cap, np.float32)
    rc = lib().orc_attn_layer(C.byref(shape.c()), ctx_cap, layer, pos, kc, vc, qo,
                              np.ascontiguousarray(k, np.float32).ravel(),
                              np.ascontiguousarray(v, np.float32).ravel(), att,
                              1 if avx2_order else 0)
    if rc:
        raise ValueError(f"orc_attn_layer rc={rc} (pos={pos}, ctx_cap={ctx_cap})")
    return qo, att.reshape(shape.n_heads, ctx_cap)[:, : pos + 1].copy()


def attn_batch(shape: Shape, layer0: int, n_layers: int, pos: np.ndarray,
               ctx_cap: np.ndarray, kcs, vcs, q: np.ndarray, k: np.ndarray,
               v: np.ndarray, n_threads: int = 1) -> np.ndarray:
    """The CPU baseline: q/k/v are [n_layers][n_seq][...]; returns outputs."""
    n_seq = len(kcs)
    kp = (C.c_void_p * n_seq)(*[a.ctypes.data for a in kcs])
    vp = (C.c_void_p * n_seq)(*[a.ctypes.data for a in vcs])
    qo = np.ascontiguousarray(q, np.float32).copy()
    rc = lib().orc_attn_batch(C.byref(shape.c()), layer0, n_layers, n_seq,
                              np.ascontiguousarray(pos, np.int32),
                              np.ascontiguousarray(ctx_cap, np.int32), kp, vp,
                              qo.reshape(-1), np.ascontiguousarray(k, np.float32).reshape(-1),
                              np.ascontiguousarray(v, np.float32).reshape(-1), n_threads)
    if rc:
        raise RuntimeError(f"orc_attn_batch: {rc} failures")
    return qo


# ---------------------------------------------------------------- weight GEMVs
# numpy restatements of the scalar matmul kernels (the reference's build
# without AVX2, kvtest flags: no FMA contraction), vectorised over rows but
# in the reference's per-row operation order, so they are bit-exact with it.

T_F32, T_F16, T_Q4_0, T_Q4_1, T_Q8_0 = 0, 1, 2, 3, 8
# (the K-quant ids, include/g2b.h:14)
T_Q2_K, T_Q3_K, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_K = 10, 11, 12, 13, 14, 15
_BLOCK_BYTES = {T_Q8_0: 34, T_Q4_0: 18, T_Q4_1: 20}


def matmul_row_bytes(t: int, n: int) -> int:
    """row_stride (l2_codec.c:340): the fused types and the fallback's F16 / Q4_1."""
    if t == T_F32:
        return n * 4
    if t == T_F16:
        return n * 2
    return (n // 32) * _BLOCK_BYTES[t]


def _blocks(w: np.ndarray, t: int, n: int, d: int):
    nb, bb = n // 32, _BLOCK_BYTES[t]
    blk = np.ascontiguousarray(w[:d * nb * bb]).reshape(d, nb, bb)
    scale = half_to_float(blk[:, :, :2].copy().view(np.uint16)).reshape(d, nb)
    return nb, blk, scale


def dequant_rows(w: np.ndarray, t: int, n: int, d: int) -> np.ndarray:
    """gguf_dequant (l2_codec.c:186-199) of d rows, float32: F16 is exact
    half_to_float (:189); Q4_1 (deq_q4_1, :65-75) is s*q + m with q the low
    nibble of byte j for element j and the high nibble for j + 16, the
    product exact (fp16 x 4 bits) and the sum rounded to float32."""
    f = np.float32
    if t == T_F16:
        h = np.ascontiguousarray(w[:d * n * 2]).view(np.uint16).reshape(d, n)
        return half_to_float(h.reshape(-1)).reshape(d, n)
    assert t == T_Q4_1 and n % 32 == 0
    nb, blk, scale = _blocks(w, t, n, d)
    mn = half_to_float(blk[:, :, 2:4].copy().view(np.uint16)).reshape(d, nb)
    qs = blk[:, :, 4:]
    q = np.concatenate([(qs & 0x0F), (qs >> 4)], axis=2).astype(f)  # [d, nb, 32]
    out = (scale[:, :, None].astype(f) * q).astype(f) + mn[:, :, None].astype(f)
    return out.astype(f).reshape(d, nb * 32)


def matmul_scalar(x: np.ndarray, w: np.ndarray, t: int, n: int, d: int) -> np.ndarray:
    """matmul_q8_0 (l2_codec.c:306-320): sum += s*(f32)q*x[j] serially;
    matmul_q4_0 (:321-340): sum += s*((f32)(lo-8)*x[j] + (f32)(hi-8)*x[j+16]);
    matmul (l3_math.c:17-20): s += w*x serially.  float32, no contraction."""
    x = np.ascontiguousarray(x, np.float32)
    f = np.float32
    acc = np.zeros(d, np.float32)
    if t in (T_F16, T_Q4_1):
        # matmul_q's fallback (l2_codec.c:350-366): the row through
        # gguf_dequant, then s += tmp[j]*x[j] serially
        wf = dequant_rows(w, t, n, d)
        for j in range(n):
            acc = acc + wf[:, j] * x[j]
        return acc
    if t == T_F32:
        wf = np.ascontiguousarray(w[:d * n * 4]).view(np.float32).reshape(d, n)
        for j in range(n):
            acc = acc + wf[:, j] * x[j]
        return acc
    nb, blk, scale = _blocks(w, t, n, d)
    for b in range(nb):
        s = scale[:, b]
        xb = x[32 * b:32 * b + 32]
        if t == T_Q8_0:
            q = blk[:, b, 2:].view(np.int8).astype(np.float32)
            for j in range(32):
                acc = acc + (s * q[:, j]) * xb[j]
        else:
            qs = blk[:, b, 2:]
            lo = ((qs & 0x0F).astype(np.int32) - 8).astype(np.float32)
            hi = ((qs >> 4).astype(np.int32) - 8).astype(np.float32)
            for j in range(16):
                acc = acc + s * (lo[:, j] * xb[j] + hi[:, j] * xb[j + 16])
    assert acc.dtype == f
    return acc


def matmul_exact(x: np.ndarray, w: np.ndarray, t: int, n: int, d: int):
    """float64 W x of the same weights (dequantisation is exact: fp16 scale
    times a small integer), and sum_j |w_ij x_j| (for error bounds)."""
    x64 = np.asarray(x, np.float64)
    if t == T_F32:
        wf = np.ascontiguousarray(w[:d * n * 4]).view(np.float32).reshape(d, n).astype(np.float64)
    elif t in (T_F16, T_Q4_1):
        wf = dequant_rows(w, t, n, d).astype(np.float64)  # the reference's float32 weights
    else:
        nb, blk, scale = _blocks(w, t, n, d)
        if t == T_Q8_0:
            q = blk[:, :, 2:].view(np.int8).astype(np.float64)
        else:
            qs = blk[:, :, 2:]
            q = np.concatenate([(qs & 0x0F).astype(np.float64) - 8,
                                (qs >> 4).astype(np.float64) - 8], axis=2)
        wf = (q * scale.astype(np.float64)[:, :, None]).reshape(d, nb * 32)
        x64 = x64[:nb * 32]
    return wf @ x64, np.abs(wf) @ np.abs(x64)


def ref_matmul(x: np.ndarray, w: np.ndarray, t: int, n: int, d: int,
               variant: str = "avx2") -> np.ndarray:
    """The compiled reference's matmul_q8_0 / matmul_q4_0 / matmul, and
    matmul_q (its dequantising fallback) for the other types."""
    L = ref_lib(variant)
    if L is None:
        raise RuntimeError("compiled reference not built (make -C oracle ref)")
    out = np.zeros(d, np.float32)
    xx = np.ascontiguousarray(x, np.float32).copy()
    ww = np.ascontiguousarray(w, np.uint8)
    if t in (T_Q8_0, T_Q4_0, T_F32):
        fn = {T_Q8_0: L.matmul_q8_0, T_Q4_0: L.matmul_q4_0, T_F32: L.matmul}[t]
        fn.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32]
        fn.restype = None
        fn(out.ctypes.data, xx.ctypes.data, ww.ctypes.data, n, d)
        return out
    L.matmul_q.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_int32,
                           C.c_int32, C.c_void_p]
    L.matmul_q.restype = None
    L.matmul_q(out.ctypes.data, xx.ctypes.data, ww.ctypes.data, t, n, d, None)
    return out


def ref_gguf_dequant(t: int, src: np.ndarray, out: np.ndarray, ne: int, variant: str = "avx2"):
    """The compiled reference's gguf_dequant(t, src, out, ne) (l2_codec.c:
    186-199), writing into the caller's out (whatever it held stays where
    the reference does not write)."""
    L = ref_lib(variant)
    if L is None:
        raise RuntimeError("compiled reference not built (make -C oracle ref)")
    assert out.dtype == np.float32 and out.flags.c_contiguous
    ss = np.ascontiguousarray(src, np.uint8)
    L.gguf_dequant.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_uint64]
    L.gguf_dequant.restype = None
    L.gguf_dequant(t, ss.ctypes.data, out.ctypes.data, ne)


def ref_g2bx_info(path: str):
    """The compiled reference's model_load_g2bx on a file: (cfg40 bytes,
    arch, flags, slots as (role, layer, type, nbytes, off))."""
    L = ref_lib("avx2")
    if L is None:
        raise RuntimeError("compiled reference not built (make -C oracle ref)")
    fn = L.ref_g2bx_info
    fn.argtypes = [C.c_char_p, C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_int),
                   C.POINTER(C.c_uint32), C.c_void_p, C.c_uint32]
    fn.restype = C.c_int
    cfg = np.zeros(40, np.uint8)
    slots = np.zeros(16 * 4096, np.uint8)
    arch, flags, ns = C.c_int(), C.c_int(), C.c_uint32()
    if fn(path.encode(), cfg.ctypes.data, C.byref(arch), C.byref(flags), C.byref(ns),
          slots.ctypes.data, 4096):
        raise RuntimeError(f"reference loader rejected {path}")
    out = []
    for i in range(min(ns.value, 4096)):
        b = slots[16 * i:16 * i + 16].tobytes()
        out.append((b[0], int.from_bytes(b[1:3], "little"), b[3],
                    int.from_bytes(b[4:8], "little"), int.from_bytes(b[8:16], "little")))
    return cfg.tobytes(), arch.value, flags.value, out


def ref_model_forward(path: str, tokens, vocab: int, kv_q8: bool = False,
                      ctx: int = 0, timed: bool = False, variant: str = "avx2"):
    """The compiled reference's model_forward over tokens at positions
    0..n-1 of a G2BX file: logits [n][vocab]; with timed, (logits, seconds
    of the token loop alone, without the load).  variant "gpu": the
    reference with the maintainer's drop-in patch (oracle/refpatch.py;
    libg2bref_gpu.so), whose attention runs on the device (G2B_GPU is set
    for the call)."""
    L = ref_lib(variant)
    if L is None:
        raise RuntimeError(f"compiled reference '{variant}' not built (make -C oracle ref refgpu)")
    fn = L.ref_model_forward_g2bx
    fn.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                   C.POINTER(C.c_double)]
    fn.restype = C.c_int
    tok = np.ascontiguousarray(tokens, np.int32)
    out = np.zeros((len(tok), vocab), np.float32)
    secs = C.c_double(0.0)
    old = os.environ.get("G2B_GPU")
    if variant == "gpu":
        os.environ["G2B_GPU"] = "1"
    try:
        rc = fn(path.encode(), 1 if kv_q8 else 0, ctx, tok.ctypes.data, len(tok),
                out.ctypes.data, C.byref(secs))
    finally:
        if variant == "gpu":
            if old is None:
                del os.environ["G2B_GPU"]
            else:
                os.environ["G2B_GPU"] = old
    if rc:
        raise RuntimeError(f"reference forward failed ({rc})")
    return (out, secs.value) if timed else out


def ref_model_forward_kv(path: str, kv_q8: bool, ctx: int, kbytes: np.ndarray,
                         vbytes: np.ndarray, pos0: int, tokens, vocab: int):
    """The compiled reference's model_forward over tokens at positions
    pos0.. of a G2BX file whose KV positions [0, pos0) are the given cache
    bytes ([n_layers][ctx][row] each, ctx the model's effective context):
    (logits [n][vocab], seconds of the token loop)."""
    L = ref_lib("avx2")
    if L is None:
        raise RuntimeError("compiled reference not built (make -C oracle ref)")
    fn = L.ref_model_forward_g2bx_kv
    fn.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int,
                   C.c_void_p, C.c_int, C.c_void_p, C.POINTER(C.c_double)]
    fn.restype = C.c_int
    tok = np.ascontiguousarray(tokens, np.int32)
    kb = np.ascontiguousarray(kbytes, np.uint8)
    vb = np.ascontiguousarray(vbytes, np.uint8)
    out = np.zeros((len(tok), vocab), np.float32)
    secs = C.c_double(0.0)
    rc = fn(path.encode(), 1 if kv_q8 else 0, ctx, ctx, kb.ctypes.data, vb.ctypes.data, pos0,
            tok.ctypes.data, len(tok), out.ctypes.data, C.byref(secs))
    if rc:
        raise RuntimeError(f"reference forward failed ({rc})")
    return out, secs.value


def random_weights(rng: np.random.Generator, t: int, n: int, d: int) -> np.ndarray:
    """d rows of random blocks: fp16 scales in [2^-10, 2^-4), int8 quants in
    [-128, 127] (Q8_0) or nibbles (Q4_0); N(0,1) floats for F32."""
    if t == T_F32:
        return rng.standard_normal(d * n).astype(np.float32).view(np.uint8).copy()
    if t == T_F16:
        return (rng.standard_normal(d * n) * 0.1).astype(np.float16).view(np.uint8).copy()
    nb, bb = n // 32, _BLOCK_BYTES[t]
    blk = rng.integers(0, 256, (d, nb, bb), dtype=np.uint8)
    sc = np.exp2(rng.uniform(-10, -4, (d, nb))).astype(np.float16)
    blk[:, :, :2] = sc.view(np.uint8).reshape(d, nb, 2)
    if t == T_Q4_1:  # the block minimum: about -8 scales (q in 0..15 centred)
        mn = (-8.0 * sc.astype(np.float32) * rng.uniform(0.5, 1.5, (d, nb))).astype(np.float16)
        blk[:, :, 2:4] = mn.view(np.uint8).reshape(d, nb, 2)
    return blk.reshape(-1).copy()


# ---------------------------------------------------------------- budgeting
# Pure-Python restatements (small integer arithmetic).


def est_for_ram(dim: int, hid: int, n_layers: int, n_heads: int, n_kv_heads: int, vocab: int,
                head_dim: int, ctx: int, q8: int) -> int:
    """est_for (l5_model.c:174-187) of a Model without tokenizer: K and V at
    ctx positions (kv_q8_rowsize or nkv*4 per row) plus the f32 runtime
    buffer of alloc_rt (:124-125)."""
    nkv = n_kv_heads * head_dim
    row = (nkv + 31) // 32 * 34 if q8 else nkv * 4
    kv = 2 * n_layers * ctx * row
    maxn = dim if dim > hid else hid
    if vocab > maxn:
        maxn = vocab
    nbuf = dim * 3 + hid * 2 + n_heads * head_dim + nkv * 2 + n_heads * ctx + maxn
    return kv + nbuf * 4


def auto_budget(est, seq_len: int, q8: int, budget: int):
    """model_auto_budget (l5_model.c:218-230) followed by model_set_ctx's
    clamp (:166-169), for an estimator est(ctx, q8).  Returns (ctx, q8,
    fits): Q8_0 first if F32 at the starting context does not fit, then
    integer halving while ctx > 256 and the estimate exceeds the budget."""
    q8 = 1 if q8 else 0
    ctx = seq_len if seq_len > 0 else 2048
    if not q8 and est(ctx, 0) > budget:
        q8 = 1
    while ctx > 256 and est(ctx, q8) > budget:
        ctx //= 2
    fits = est(ctx, q8) <= budget
    if ctx <= 0:
        ctx = 256
    if seq_len > 0 and ctx > seq_len:
        ctx = seq_len
    return ctx, q8, fits


def now() -> float:
    return lib().orc_now_sec()


def max_threads() -> int:
    return lib().orc_max_threads()


# ---------------------------------------------------------------- compiled reference

_ref = {}


def ref_lib(variant: str = "avx2"):
    """The compiled reference driver, or None where it was not built."""
    if variant in _ref:
        return _ref[variant]
    path = os.path.join(REF_DIR, f"libg2bref_{variant}.so")
    if not os.path.exists(path):
        _ref[variant] = None
        return None
    L = C.CDLL(path)
    L.ref_q8_quant_row.argtypes = [_f32p, _u8p, C.c_int32]
    L.ref_q8_dequant_row.argtypes = [_u8p, _f32p, C.c_int32]
    L.ref_f32_to_half_n.argtypes = [_f32p, _u16p, C.c_size_t]
    L.ref_half_to_float_n.argtypes = [_u16p, _f32p, C.c_size_t]
    L.ref_softmax.argtypes = [_f32p, C.c_int32]
    L.ref_qk_rmsnorm.argtypes = [_f32p, _f32p, C.c_int32, C.c_int32, C.c_float]
    L.ref_rope.argtypes = [C.c_int32, _f32p, C.c_int32, C.c_int32, C.c_int32, C.c_float]
    L.ref_forward_case.argtypes = [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                                   C.c_int32, C.c_int32, C.c_int32,
                                   C.c_int32, _f32p, _f32p, C.c_int32, _f32p,
                                   _f32p, _f32p, _f32p, _u8p, _u8p]
    L.ref_forward_case.restype = C.c_int
    _vp = C.c_void_p  # nullable float arrays
    L.ref_forward_case_qkn.argtypes = [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                                       C.c_int32, C.c_int32, C.c_int32,
                                       C.c_int32, _f32p, _f32p, C.c_int32, _f32p,
                                       _vp, _vp, C.c_float,
                                       _f32p, _f32p, _f32p, _u8p, _u8p]
    L.ref_forward_case_qkn.restype = C.c_int
    L.ref_est_for.argtypes = [C.c_int32] * 9 + [C.c_int]
    L.ref_est_for.restype = C.c_uint64
    L.ref_auto_budget.argtypes = ([C.c_int32] * 8 + [C.c_int, C.c_uint64,
                                  C.POINTER(C.c_int32), C.POINTER(C.c_int32)])
    L.ref_auto_budget.restype = C.c_int
    _ref[variant] = L
    return L


def ref_qk_rmsnorm(x: np.ndarray, w: np.ndarray, n_heads: int, head_dim: int,
                   eps: float) -> np.ndarray:
    """The compiled reference's qk_rmsnorm (l3_math.c:107-114)."""
    L = ref_lib("avx2")
    if L is None:
        raise RuntimeError("compiled reference not built (make -C oracle ref)")
    y = np.ascontiguousarray(x, np.float32).copy().reshape(-1)
    ww = np.ascontiguousarray(w, np.float32).reshape(-1)
    L.ref_qk_rmsnorm(y, ww, n_heads, head_dim, eps)
    return y


def ref_forward_case(shape: Shape, ctx_cap: int, k_pre: np.ndarray, v_pre: np.ndarray,
                     x_rows: np.ndarray, variant: str = "avx2", q_norm: np.ndarray = None,
                     k_norm: np.ndarray = None, eps: float = 1e-6):
    """Run the reference model_forward on a selector model (oracle/ref_driver.c).

    q_norm / k_norm ([n_layers, head_dim] or None) add attn_q_norm /
    attn_k_norm slots and F_QK_NORM.
    Returns dict(xb [n_fwd, dim], out [n_fwd, nq], att [n_heads, ctx_cap],
    kc, vc [n_layers*ctx_cap*row])."""
    L = ref_lib(variant)
    if L is None:
        raise RuntimeError("compiled reference not built (make -C oracle ref)")
    nq, nkv = shape.nq, shape.nkv
    dim = nq + 2 * nkv
    n_pre = 0 if k_pre is None else int(k_pre.shape[0])
    n_fwd = int(x_rows.shape[0])
    kp = np.ascontiguousarray(k_pre if n_pre else np.zeros((1, nkv)), np.float32)
    vp = np.ascontiguousarray(v_pre if n_pre else np.zeros((1, nkv)), np.float32)
    xr = np.ascontiguousarray(x_rows, np.float32)
    assert xr.shape[1] == dim
    xb = np.zeros((n_fwd, dim), np.float32)
    out = np.zeros((n_fwd, nq), np.float32)
    att = np.zeros((shape.n_heads, ctx_cap), np.float32)
    nbytes = shape.n_layers * ctx_cap * shape.row_bytes
    kc = np.zeros(nbytes, np.uint8)
    vc = np.zeros(nbytes, np.uint8)
    norms = []
    for w in (q_norm, k_norm):
        if w is None:
            norms.append(None)
        else:
            a = np.ascontiguousarray(w, np.float32).reshape(-1)
            assert a.size == shape.n_layers * shape.head_dim
            norms.append(a)
    ptr = [None if a is None else a.ctypes.data for a in norms]
    rc = L.ref_forward_case_qkn(shape.n_layers, shape.n_heads, shape.n_kv_heads,
                                shape.head_dim, shape.rope_theta, shape.arch,
                                1 if shape.kv_q8 else 0, ctx_cap, n_pre, kp.reshape(-1),
                                vp.reshape(-1), n_fwd, xr.reshape(-1), ptr[0], ptr[1], eps,
                                xb.reshape(-1), out.reshape(-1), att.reshape(-1), kc, vc)
    if rc:
        raise RuntimeError(f"ref_forward_case rc={rc}")
    return dict(xb=xb, out=out, att=att, kc=kc, vc=vc)
