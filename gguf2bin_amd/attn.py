"""Python mirror of the C ABI in include/g2b_attn.h and include/g2b_synth.h.

It follows the reference's own seam (/root/reference/src/l5_model.c:513-578
plus the KV allocation of alloc_rt/free_rt, :113-149): a context per model
shape, KV buffers in the reference [layer][ctx][row] layout, and a per-layer
call that rotates q and k, appends k/v at `pos`, and writes the attention
output over q.  Errors come back as ``G2BError`` carrying the C code; the
library never falls back to the CPU and this module refuses to load without
the compiled library.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBPATH = os.path.join(HERE, "libg2b_attn.so")
# The phase-stamp build (make -C gguf2bin_amd stamps): the same library with
# per-workgroup wall-clock stamps in static k_layer launches and their
# combine; loaded instead of LIBPATH only by bench.py --phases.
STAMPS_LIBPATH = os.path.join(HERE, "libg2b_attn_stamps.so")
STAMP_WORDS = 8

G2B_OK, G2B_EINVAL, G2B_EPOS, G2B_ENOKV, G2B_ENOMEM, G2B_EDEVICE, G2B_ESWAP, G2B_EUNSUP = (
    0, -1, -2, -3, -4, -5, -6, -7)
ARCH_LLAMA, ARCH_QWEN2, ARCH_QWEN3 = 0, 1, 2

# Every symbol the headers declare (checked by tests/test_abi.py).
EXPORTS = [
    "g2b_ctx_create", "g2b_ctx_destroy", "g2b_ctx_set_stream", "g2b_ctx_stream",
    "g2b_strerror", "g2b_ctx_last_error", "g2b_kv_row_bytes", "g2b_kv_bytes",
    "g2b_kv_offset", "g2b_kv_alloc", "g2b_kv_free", "g2b_kv_read", "g2b_kv_append_rows",
    "g2b_set_qk_norm",
    "g2b_model_kv_bytes", "g2b_clamp_ctx", "g2b_hbm_bytes", "g2b_auto_budget", "g2b_hbm_info",
    "g2b_matmul_row_bytes", "g2b_matmul", "g2b_matmul_host", "g2b_weights_upload",
    "g2b_weights_free", "g2b_g2bx_open", "g2b_g2bx_close", "g2b_g2bx_slot",
    "g2b_model_load_g2bx", "g2b_model_free", "g2b_model_info", "g2b_model_ctx", "g2b_model_kv",
    "g2b_model_forward", "g2b_model_use_graph", "g2b_model_set_fused",
    "g2b_batch_begin", "g2b_attn_layers", "g2b_attn_forward", "g2b_attn_forward_host",
    "g2b_attn_forward_noalloc",
    "g2b_rope_table", "g2b_sync",
    "g2b_stream_seed", "g2b_synth_normal", "g2b_synth_fill_kv", "g2b_synth_copy",
    "g2b_ctx_profile", "g2b_ctx_profile_read", "g2b_ctx_tune", "g2b_ctx_tune_kernel",
    "g2b_ctx_last_schedule",
]


class G2BError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (code {code})")
        self.code = code


class _Shape(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("rope_theta", C.c_float), ("arch", C.c_int32),
                ("kv_q8", C.c_int32)]


class _Seq(C.Structure):
    _fields_ = [("pos", C.c_int32), ("ctx_cap", C.c_int32), ("kcache", C.c_void_p),
                ("vcache", C.c_void_p)]


class _ModelCfg(C.Structure):
    _fields_ = [("dim", C.c_int32), ("hidden_dim", C.c_int32), ("n_layers", C.c_int32),
                ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("vocab", C.c_int32),
                ("seq_len", C.c_int32), ("head_dim", C.c_int32), ("eps", C.c_float),
                ("rope_theta", C.c_float)]


class _Slot(C.Structure):
    _fields_ = [("role", C.c_uint8), ("layer", C.c_uint16), ("type", C.c_uint8),
                ("nbytes", C.c_uint32), ("off", C.c_uint64)]


class _G2bx(C.Structure):
    _fields_ = [("version", C.c_uint16), ("arch", C.c_uint8), ("flags", C.c_uint8),
                ("cfg", _ModelCfg), ("n_slots", C.c_uint32), ("slots", C.POINTER(_Slot)),
                ("data", C.POINTER(C.c_uint8)), ("data_size", C.c_uint64)]


@dataclass(frozen=True)
class Shape:
    """ModelCfg fields the path reads (include/g2b.h:51-55) plus F_KV_Q8."""
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

    def c(self) -> _Shape:
        return _Shape(self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim,
                      self.rope_theta, self.arch, 1 if self.kv_q8 else 0)


_lib = None


def lib() -> C.CDLL:
    """Load the in-tree libg2b_attn.so; fail loudly when it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBPATH):
            raise RuntimeError(f"{LIBPATH} is missing: build it with `make -C gguf2bin_amd` "
                               "(or __graft_entry__.build())")
        L = C.CDLL(LIBPATH)
        vp, i32, u64 = C.c_void_p, C.c_int32, C.c_uint64
        fp = C.c_void_p
        sig = {
            "g2b_ctx_create": ([C.POINTER(vp), i32, C.POINTER(_Shape)], C.c_int),
            "g2b_ctx_destroy": ([vp], C.c_int),
            "g2b_ctx_set_stream": ([vp, vp], C.c_int),
            "g2b_ctx_stream": ([vp], vp),
            "g2b_strerror": ([i32], C.c_char_p),
            "g2b_ctx_last_error": ([vp], C.c_char_p),
            "g2b_kv_row_bytes": ([C.POINTER(_Shape)], C.c_size_t),
            "g2b_kv_bytes": ([C.POINTER(_Shape), i32], u64),
            "g2b_kv_offset": ([C.POINTER(_Shape), i32, i32, i32], u64),
            "g2b_model_kv_bytes": ([C.POINTER(_Shape), i32, i32], u64),
            "g2b_clamp_ctx": ([i32, i32], i32),
            "g2b_hbm_bytes": ([C.POINTER(_Shape), i32, i32, i32], u64),
            "g2b_auto_budget": ([C.POINTER(_Shape), i32, i32, u64, C.POINTER(i32),
                                 C.POINTER(i32)], C.c_int),
            "g2b_hbm_info": ([vp, C.POINTER(u64), C.POINTER(u64)], C.c_int),
            "g2b_g2bx_open": ([C.c_char_p, C.POINTER(_G2bx)], C.c_int),
            "g2b_g2bx_close": ([C.POINTER(_G2bx)], None),
            "g2b_g2bx_slot": ([C.POINTER(_G2bx), i32, i32], C.POINTER(_Slot)),
            "g2b_model_load_g2bx": ([C.POINTER(vp), i32, C.c_char_p, i32, i32], C.c_int),
            "g2b_model_free": ([vp], C.c_int),
            "g2b_model_info": ([vp, C.POINTER(_ModelCfg), C.POINTER(i32), C.POINTER(i32),
                                C.POINTER(i32)], C.c_int),
            "g2b_model_ctx": ([vp], vp),
            "g2b_model_kv": ([vp, C.POINTER(vp), C.POINTER(vp), C.POINTER(i32)], C.c_int),
            "g2b_model_forward": ([vp, i32, i32, fp], C.c_int),
            "g2b_model_use_graph": ([vp, i32], C.c_int),
            "g2b_model_set_fused": ([vp, i32], C.c_int),
            "g2b_matmul_row_bytes": ([i32, i32], C.c_size_t),
            "g2b_matmul": ([vp, fp, fp, vp, i32, i32, i32], C.c_int),
            "g2b_matmul_host": ([vp, fp, fp, vp, i32, i32, i32], C.c_int),
            "g2b_weights_upload": ([vp, vp, u64, C.POINTER(vp)], C.c_int),
            "g2b_weights_free": ([vp, vp], C.c_int),
            "g2b_kv_alloc": ([vp, i32, C.POINTER(vp), C.POINTER(vp)], C.c_int),
            "g2b_kv_free": ([vp, vp, vp], C.c_int),
            "g2b_kv_read": ([vp, vp, u64, u64, vp], C.c_int),
            "g2b_kv_append_rows": ([vp, vp, vp, i32, i32, i32, i32, fp, fp], C.c_int),
            "g2b_set_qk_norm": ([vp, i32, vp, vp, C.c_float], C.c_int),
            "g2b_batch_begin": ([vp, i32, C.POINTER(_Seq)], C.c_int),
            "g2b_attn_layers": ([vp, i32, i32, fp, fp, fp, fp, i32], C.c_int),
            "g2b_attn_forward": ([vp, i32, i32, i32, vp, vp, fp, fp, fp, fp], C.c_int),
            "g2b_attn_forward_host": ([vp, i32, i32, i32, vp, vp, fp, fp, fp, fp], C.c_int),
            "g2b_attn_forward_noalloc": ([vp, i32, i32, i32, vp, vp, fp, fp, fp], C.c_int),
            "g2b_rope_table": ([i32, i32, i32, C.c_float, fp], C.c_int),
            "g2b_sync": ([vp], C.c_int),
            "g2b_stream_seed": ([u64, i32, i32, i32], u64),
            "g2b_synth_normal": ([vp, fp, u64, u64], C.c_int),
            "g2b_synth_fill_kv": ([vp, vp, vp, i32, i32, i32, i32, i32, u64, i32, C.c_float],
                                  C.c_int),
            "g2b_synth_copy": ([vp, vp, vp, u64], C.c_int),
            "g2b_ctx_profile": ([vp, i32], C.c_int),
            "g2b_ctx_tune": ([vp, i32, i32, i32, i32], C.c_int),
            "g2b_ctx_tune_kernel": ([vp, i32], C.c_int),
            "g2b_ctx_last_schedule": ([vp, C.POINTER(C.c_int32)], C.c_int),
            "g2b_ctx_profile_read": ([vp, C.POINTER(C.c_double), C.POINTER(C.c_int64)],
                                     C.c_int),
        }
        for name, (args, res) in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        if hasattr(L, "g2b_stamps_enable"):  # (the phase-stamp build only)
            L.g2b_stamps_enable.argtypes = [vp, i32, i32]
            L.g2b_stamps_enable.restype = C.c_int
            L.g2b_stamps_read.argtypes = [vp, vp, i32]
            L.g2b_stamps_read.restype = C.c_int
        _lib = L
    return _lib


def strerror(code: int) -> str:
    return lib().g2b_strerror(code).decode()


def kv_row_bytes(shape: Shape) -> int:
    return int(lib().g2b_kv_row_bytes(C.byref(shape.c())))


def kv_bytes(shape: Shape, ctx_cap: int) -> int:
    return int(lib().g2b_kv_bytes(C.byref(shape.c()), ctx_cap))


def kv_offset(shape: Shape, ctx_cap: int, layer: int, pos: int) -> int:
    return int(lib().g2b_kv_offset(C.byref(shape.c()), ctx_cap, layer, pos))


T_F32, T_F16, T_Q4_0, T_Q4_1, T_Q8_0 = 0, 1, 2, 3, 8  # GGML type ids of the device GEMVs
CFG_FIELDS = ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab", "seq_len",
              "head_dim", "eps", "rope_theta")


def g2bx_open(path: str) -> dict:
    """Parse a G2BX container on the host (g2b_g2bx_open): header, config,
    slots (role, layer, type, nbytes, off) and the weight blob (bytes)."""
    g = _G2bx()
    rc = lib().g2b_g2bx_open(path.encode(), C.byref(g))
    if rc:
        raise G2BError(rc, f"g2b_g2bx_open({path}): {strerror(rc)}")
    try:
        cfg = {f: getattr(g.cfg, f) for f in CFG_FIELDS}
        slots = [(g.slots[i].role, g.slots[i].layer, g.slots[i].type, g.slots[i].nbytes,
                  g.slots[i].off) for i in range(g.n_slots)]
        data = C.string_at(g.data, g.data_size)
        return {"version": g.version, "arch": g.arch, "flags": g.flags, "cfg": cfg,
                "slots": slots, "data": data}
    finally:
        lib().g2b_g2bx_close(C.byref(g))


class Model:
    """A G2BX model on the device (g2b_model_*): weights in HBM, the decode
    step (model_forward, l5_model.c:461-606) as device kernels."""

    def __init__(self, path: str, device: int = 0, kv_q8: bool = False, ctx: int = 0):
        self.h = C.c_void_p()
        rc = lib().g2b_model_load_g2bx(C.byref(self.h), device, path.encode(),
                                       1 if kv_q8 else 0, ctx)
        if rc:
            raise G2BError(rc, f"g2b_model_load_g2bx({path}): {strerror(rc)}")
        c, arch, flags, cc = _ModelCfg(), C.c_int32(), C.c_int32(), C.c_int32()
        lib().g2b_model_info(self.h, C.byref(c), C.byref(arch), C.byref(flags), C.byref(cc))
        self.cfg = {f: getattr(c, f) for f in CFG_FIELDS}
        self.arch, self.flags, self.ctx_cap = arch.value, flags.value, cc.value

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.zeros(self.cfg["vocab"], np.float32)
        rc = lib().g2b_model_forward(self.h, token, pos, out.ctypes.data)
        if rc:
            raise G2BError(rc, f"g2b_model_forward: {strerror(rc)}")
        return out

    def kv(self):
        """(K cache, V cache, ctx_cap): the model's device caches."""
        k, v, cap = C.c_void_p(), C.c_void_p(), C.c_int32()
        rc = lib().g2b_model_kv(self.h, C.byref(k), C.byref(v), C.byref(cap))
        if rc:
            raise G2BError(rc, f"g2b_model_kv: {strerror(rc)}")
        return k.value, v.value, cap.value

    def use_graph(self, on: bool):
        """Capture the step once and replay it (on), or launch every step
        eagerly with the attention sized for its position (off, the default)."""
        lib().g2b_model_use_graph(self.h, 1 if on else 0)

    def set_fused(self, on: bool):
        """Fused GEMV launches (rmsnorm, SiLU x up and the residual inside
        them; default) or every step as separate launches."""
        lib().g2b_model_set_fused(self.h, 1 if on else 0)

    def forward_rc(self, token: int, pos: int):
        """(return code, logits) without raising."""
        out = np.full(self.cfg["vocab"], 7.0, np.float32)
        rc = lib().g2b_model_forward(self.h, token, pos, out.ctypes.data)
        return rc, out

    def close(self):
        if self.h:
            lib().g2b_model_free(self.h)
            self.h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def matmul_row_bytes(t: int, n: int) -> int:
    """Bytes of one weight row (row_stride, l2_codec.c:340)."""
    return int(lib().g2b_matmul_row_bytes(t, n))


def model_kv_bytes(shape: Shape, seq_len: int, kv_q8: bool) -> int:
    """model_kv_bytes (l5_model.c:195-203): K+V bytes at the full seq_len."""
    return int(lib().g2b_model_kv_bytes(C.byref(shape.c()), seq_len, 1 if kv_q8 else 0))


def clamp_ctx(ctx: int, seq_len: int) -> int:
    """model_set_ctx's clamp (l5_model.c:166-169)."""
    return int(lib().g2b_clamp_ctx(ctx, seq_len))


def hbm_bytes(shape: Shape, ctx: int, kv_q8: bool, n_seq: int) -> int:
    """HBM of n_seq sequences at context ctx: KV, RoPE table, partial scratch."""
    return int(lib().g2b_hbm_bytes(C.byref(shape.c()), ctx, 1 if kv_q8 else 0, n_seq))


def auto_budget(shape: Shape, seq_len: int, n_seq: int, budget: int):
    """model_auto_budget (l5_model.c:218-230) against an HBM budget.
    Returns (kv_q8, ctx, fits); raises G2BError for invalid arguments."""
    q8, ctx = C.c_int32(), C.c_int32()
    rc = lib().g2b_auto_budget(C.byref(shape.c()), seq_len, n_seq, budget, C.byref(q8),
                               C.byref(ctx))
    if rc not in (G2B_OK, G2B_ENOMEM):
        raise G2BError(rc, f"g2b_auto_budget: {strerror(rc)}")
    return bool(q8.value), int(ctx.value), rc == G2B_OK


def rope_table(pos0: int, n_pos: int, head_dim: int, theta: float) -> np.ndarray:
    out = np.zeros((max(n_pos, 1), max(head_dim, 2)), np.float32)
    rc = lib().g2b_rope_table(pos0, n_pos, head_dim, theta, out.ctypes.data)
    if rc:
        raise G2BError(rc, f"g2b_rope_table: {strerror(rc)}")
    return out[:n_pos, :head_dim]


SCHED_FIELDS = 9  # G2B_SCHED_FIELDS
KERNEL_NAMES = {1: "k_layer", 2: "k_tiles", 3: "k_short", 4: "k_decode_generic"}


def schedule_dict(shape: Shape, a) -> dict:
    """g2b_ctx_last_schedule's fields as a dict, with "variant": the kernel
    instance they name for this shape (include/g2b_synth.h)."""
    kernel = KERNEL_NAMES.get(a[0], "none")
    wq = "true" if a[2] > 0 else "false"
    if kernel == "k_layer":
        variant = (f"k_layer<{1 if shape.kv_q8 else 0}, {shape.head_dim}, {a[7]}, "
                   f"{shape.n_heads // shape.n_kv_heads}, 2, {'true' if a[8] else 'false'}, "
                   f"{a[6]}, {wq}>")
    elif kernel == "k_tiles":
        variant = f"k_tiles<{shape.n_heads // shape.n_kv_heads}, {wq}>"
    elif kernel == "k_short":
        variant = f"k_short<{1 if shape.kv_q8 else 0}, {shape.head_dim}>"
    else:
        variant = kernel
    return {"kernel": kernel, "split_len": a[1], "piece_len": a[2], "max_splits": a[3],
            "workgroups": a[4], "output_in_kernel": bool(a[5]),
            "staging": {0: "per-lane loads", 1: "LDS DMA", 2: "register staging"}.get(a[6], "?"),
            "chunk": a[7], "weights": bool(a[8]), "variant": variant}


def stream_seed(base: int, seq: int, layer: int, tensor: int) -> int:
    return int(lib().g2b_stream_seed(base & 0xFFFFFFFFFFFFFFFF, seq, layer, tensor))


class Context:
    """One g2b_ctx: a model shape on one device (include/g2b_attn.h)."""

    def __init__(self, shape: Shape, device: int = 0):
        self.shape = shape
        h = C.c_void_p()
        rc = lib().g2b_ctx_create(C.byref(h), device, C.byref(shape.c()))
        if rc:
            raise G2BError(rc, f"g2b_ctx_create: {strerror(rc)}")
        self.h = h.value

    def _check(self, rc: int, what: str):
        if rc:
            detail = lib().g2b_ctx_last_error(self.h).decode()
            raise G2BError(rc, f"{what}: {strerror(rc)}: {detail}")

    def close(self):
        if self.h:
            lib().g2b_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return lib().g2b_ctx_stream(self.h) or 0

    def set_stream(self, stream: Optional[int]):
        self._check(lib().g2b_ctx_set_stream(self.h, stream), "g2b_ctx_set_stream")

    def sync(self):
        self._check(lib().g2b_sync(self.h), "g2b_sync")

    # ---- weight GEMVs (matmul_q, l2_codec.c:342-360) ----
    def weights_upload(self, host: np.ndarray) -> int:
        """Copy a host byte array into HBM; returns the device pointer."""
        h = np.ascontiguousarray(host).view(np.uint8)
        dev = C.c_void_p()
        self._check(lib().g2b_weights_upload(self.h, h.ctypes.data, h.nbytes, C.byref(dev)),
                     "g2b_weights_upload")
        return int(dev.value)

    def weights_free(self, dev: int):
        self._check(lib().g2b_weights_free(self.h, dev), "g2b_weights_free")

    def matmul(self, out: int, x: int, w: int, t: int, n: int, d: int):
        """Device pointers; asynchronous on the context's stream."""
        self._check(lib().g2b_matmul(self.h, out, x, w, t, n, d), "g2b_matmul")

    def matmul_host(self, x: np.ndarray, w: int, t: int, n: int, d: int) -> np.ndarray:
        """x in host memory, w a device pointer; returns out (host)."""
        out = np.zeros(max(d, 1), np.float32)
        xx = np.ascontiguousarray(x, np.float32)
        self._check(lib().g2b_matmul_host(self.h, out.ctypes.data, xx.ctypes.data, w, t, n, d),
                     "g2b_matmul_host")
        return out[:d]

    def hbm_info(self):
        """(free, total) HBM bytes of the context's device."""
        fr, tot = C.c_uint64(), C.c_uint64()
        self._check(lib().g2b_hbm_info(self.h, C.byref(fr), C.byref(tot)), "g2b_hbm_info")
        return int(fr.value), int(tot.value)

    # ---- KV (alloc_rt / free_rt) ----
    def kv_alloc(self, ctx_cap: int):
        k, v = C.c_void_p(), C.c_void_p()
        self._check(lib().g2b_kv_alloc(self.h, ctx_cap, C.byref(k), C.byref(v)), "g2b_kv_alloc")
        return k.value, v.value

    def kv_free(self, k: int, v: int):
        self._check(lib().g2b_kv_free(self.h, k, v), "g2b_kv_free")

    def kv_read(self, cache: int, offset: int, nbytes: int) -> np.ndarray:
        """nbytes of a device cache from byte offset, as host uint8."""
        out = np.empty(nbytes, np.uint8)
        self._check(lib().g2b_kv_read(self.h, cache, offset, nbytes, out.ctypes.data),
                    "g2b_kv_read")
        return out

    def kv_append_rows(self, kc: int, vc: int, ctx_cap: int, layer: int, pos0: int,
                       n_rows: int, k_dev: int, v_dev: int):
        self._check(lib().g2b_kv_append_rows(self.h, kc, vc, ctx_cap, layer, pos0, n_rows,
                                             k_dev, v_dev), "g2b_kv_append_rows")

    def set_qk_norm(self, layer: int, q_norm=None, k_norm=None, eps: float = 1e-6):
        """QK-RMSNorm weights of one layer (host arrays of head_dim floats, or
        None), as model_forward applies them under F_QK_NORM."""
        keep = []
        ptrs = []
        for w in (q_norm, k_norm):
            if w is None:
                ptrs.append(None)
                continue
            a = np.ascontiguousarray(w, np.float32).reshape(-1)
            if a.size != self.shape.head_dim:
                raise ValueError(f"norm weights: {a.size} floats, head_dim {self.shape.head_dim}")
            keep.append(a)
            ptrs.append(a.ctypes.data)
        self._check(lib().g2b_set_qk_norm(self.h, layer, ptrs[0], ptrs[1], eps),
                    "g2b_set_qk_norm")

    # ---- the path ----
    def batch_begin(self, seqs: Sequence[tuple]):
        arr = (_Seq * len(seqs))(*[_Seq(int(p), int(c), k, v) for (p, c, k, v) in seqs])
        self._check(lib().g2b_batch_begin(self.h, len(seqs), arr), "g2b_batch_begin")

    def attn_layers(self, layer0: int, n_layers: int, q: int, k: int, v: int,
                    att: Optional[int] = None, att_stride: int = 0):
        self._check(lib().g2b_attn_layers(self.h, layer0, n_layers, q, k, v, att, att_stride),
                    "g2b_attn_layers")

    def attn_forward(self, layer: int, pos: int, ctx_cap: int, kc: int, vc: int, q: int,
                     k: int, v: int, att: Optional[int] = None):
        self._check(lib().g2b_attn_forward(self.h, layer, pos, ctx_cap, kc, vc, q, k, v, att),
                    "g2b_attn_forward")

    def attn_forward_noalloc(self, layer: int, pos: int, ctx_cap: int, kc: int, vc: int, q: int,
                             k: int, v: int):
        """g2b_attn_forward over the library's fixed scratch (allocates nothing)."""
        self._check(lib().g2b_attn_forward_noalloc(self.h, layer, pos, ctx_cap, kc, vc, q, k, v),
                    "g2b_attn_forward_noalloc")

    def attn_forward_host(self, layer: int, pos: int, ctx_cap: int, kc: int, vc: int,
                          q: np.ndarray, k: np.ndarray, v: np.ndarray, want_att: bool = False):
        """Host-memory variant; returns (out, att or None).  q is not modified."""
        qo = np.ascontiguousarray(q, np.float32).copy()
        kk = np.ascontiguousarray(k, np.float32)
        vv = np.ascontiguousarray(v, np.float32)
        att = np.zeros(self.shape.n_heads * ctx_cap, np.float32) if want_att else None
        self._check(lib().g2b_attn_forward_host(
            self.h, layer, pos, ctx_cap, kc, vc, qo.ctypes.data, kk.ctypes.data,
            vv.ctypes.data, att.ctypes.data if att is not None else None),
            "g2b_attn_forward_host")
        return qo, (att.reshape(self.shape.n_heads, ctx_cap) if att is not None else None)

    # ---- synthetic inputs (bench / full-size tests) ----
    def synth_normal(self, out: int, n: int, seed: int):
        self._check(lib().g2b_synth_normal(self.h, out, n, seed & 0xFFFFFFFFFFFFFFFF),
                    "g2b_synth_normal")

    def synth_copy(self, dst: int, src: int, nbytes: int):
        self._check(lib().g2b_synth_copy(self.h, dst, src, nbytes), "g2b_synth_copy")

    def tune(self, split_len: int = 0, chunk: int = 0, stage: int = 0, piece: int = 0):
        """Decode-kernel tuning (0 = automatic): static split length, Q8 chunk,
        KV row path (-1 per-lane HBM loads, 1 / 2 staged through LDS), schedule
        (-1 static splits, > 0 work-queue piece length in positions)."""
        self._check(lib().g2b_ctx_tune(self.h, split_len, chunk, stage, piece), "g2b_ctx_tune")

    def tune_kernel(self, kernel: int):
        """0 automatic, 1 k_layer only, 2 k_tiles where it applies, 3 spanned k_short."""
        self._check(lib().g2b_ctx_tune_kernel(self.h, kernel), "g2b_ctx_tune_kernel")

    KERNEL_NAMES = KERNEL_NAMES

    def last_schedule(self) -> dict:
        """The last decode call's schedule (g2b_ctx_last_schedule)."""
        a = (C.c_int32 * SCHED_FIELDS)()
        self._check(lib().g2b_ctx_last_schedule(self.h, a), "g2b_ctx_last_schedule")
        return schedule_dict(self.shape, a)

    def profile(self, enable: bool):
        self._check(lib().g2b_ctx_profile(self.h, 1 if enable else 0), "g2b_ctx_profile")

    def stamps_enable(self, cap: int, launches: int = 1):
        """Room for the phase stamps of `launches` decode calls of up to cap
        workgroups each (the phase-stamp build only)."""
        if not hasattr(lib(), "g2b_stamps_enable"):
            raise RuntimeError(f"{LIBPATH} has no phase stamps: load {STAMPS_LIBPATH} "
                               "(make -C gguf2bin_amd stamps) instead")
        self._check(lib().g2b_stamps_enable(self.h, cap, launches), "g2b_stamps_enable")
        self._stamp_cap, self._stamp_launches = cap, launches

    def stamps_read(self, clear: bool = True) -> np.ndarray:
        """The stamps of the decode calls since the last read:
        [launches][2][cap][STAMP_WORDS] uint64 (call i's decode kernel
        workgroups, then its combine's), zeroed afterwards when clear."""
        out = np.zeros((self._stamp_launches, 2, self._stamp_cap, STAMP_WORDS), np.uint64)
        self._check(lib().g2b_stamps_read(self.h, out.ctypes.data, 1 if clear else 0),
                    "g2b_stamps_read")
        return out

    def profile_read(self):
        """(summed decode-kernel milliseconds, launches) since the last read."""
        ms, n = C.c_double(0), C.c_int64(0)
        self._check(lib().g2b_ctx_profile_read(self.h, C.byref(ms), C.byref(n)),
                    "g2b_ctx_profile_read")
        return ms.value, n.value

    def synth_fill_kv(self, kc: int, vc: int, ctx_cap: int, layer0: int, n_layers: int,
                      pos0: int, n_pos: int, base_seed: int, seq: int,
                      sel_threshold: float = float("inf")):
        self._check(lib().g2b_synth_fill_kv(self.h, kc, vc, ctx_cap, layer0, n_layers, pos0,
                                            n_pos, base_seed & 0xFFFFFFFFFFFFFFFF, seq,
                                            sel_threshold), "g2b_synth_fill_kv")
