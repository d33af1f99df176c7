"""Minimal HIP runtime bindings (ctypes over libamdhip64.so): device memory,
copies and events.  Plumbing for tests and the benchmark; the product is the
C ABI in libg2b_attn.so."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_H2D, _D2H, _D2D = 1, 2, 3
_lib = None


class HipError(RuntimeError):
    pass


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        cands = ["libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"]
        rocm = os.environ.get("ROCM_PATH")
        if rocm:
            cands.insert(0, os.path.join(rocm, "lib", "libamdhip64.so"))
        last = None
        for p in cands:
            try:
                _lib = C.CDLL(p)
                break
            except OSError as e:  # pragma: no cover - depends on the image
                last = e
        if _lib is None:
            raise HipError(f"cannot load libamdhip64.so: {last}")
        L = _lib
        L.hipGetErrorString.restype = C.c_char_p
        L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        L.hipFree.argtypes = [C.c_void_p]
        L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        L.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        L.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
        L.hipSetDevice.argtypes = [C.c_int]
        L.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        L.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        L.hipEventSynchronize.argtypes = [C.c_void_p]
        L.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        L.hipEventDestroy.argtypes = [C.c_void_p]
        L.hipStreamSynchronize.argtypes = [C.c_void_p]
        L.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        L.hipDeviceGetAttribute.argtypes = [C.POINTER(C.c_int), C.c_int, C.c_int]
    return _lib


def check(rc: int, what: str):
    if rc != 0:
        msg = lib().hipGetErrorString(rc).decode()
        raise HipError(f"{what}: {msg} ({rc})")


def device_count() -> int:
    n = C.c_int(0)
    try:
        rc = lib().hipGetDeviceCount(C.byref(n))
    except HipError:
        return 0
    return n.value if rc == 0 else 0


def set_device(d: int):
    check(lib().hipSetDevice(d), "hipSetDevice")


HIP_ATTR_WALL_CLOCK_RATE = 10017  # hipDeviceAttributeWallClockRate (kHz)


def wall_clock_khz(d: int = 0) -> int:
    """Frequency of the device's constant wall clock (wall_clock64), kHz."""
    v = C.c_int(0)
    check(lib().hipDeviceGetAttribute(C.byref(v), HIP_ATTR_WALL_CLOCK_RATE, d),
          "hipDeviceGetAttribute")
    return v.value


def mem_info():
    f, t = C.c_size_t(0), C.c_size_t(0)
    check(lib().hipMemGetInfo(C.byref(f), C.byref(t)), "hipMemGetInfo")
    return f.value, t.value


class DeviceBuffer:
    """Owning device allocation of `nbytes`."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().hipMalloc(C.byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    def free(self):
        if self.ptr:
            check(lib().hipFree(self.ptr), "hipFree")
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, _H2D), "H2D")

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes, _D2H), "D2H")
        return out


def to_device(a: np.ndarray) -> DeviceBuffer:
    a = np.ascontiguousarray(a)
    b = DeviceBuffer(a.nbytes)
    b.upload(a)
    return b


def copy_d2h(ptr: int, dtype, count: int, offset: int = 0) -> np.ndarray:
    out = np.empty(count, dtype)
    if out.nbytes:
        check(lib().hipMemcpy(out.ctypes.data, ptr + offset, out.nbytes, _D2H), "D2H")
    return out


def copy_h2d(ptr: int, a: np.ndarray, offset: int = 0):
    a = np.ascontiguousarray(a)
    if a.nbytes:
        check(lib().hipMemcpy(ptr + offset, a.ctypes.data, a.nbytes, _H2D), "H2D")


def copy_d2d(dst: int, src: int, nbytes: int):
    check(lib().hipMemcpy(dst, src, nbytes, _D2D), "D2D")


def device_sync():
    """hipDeviceSynchronize: every stream of the device has drained (a
    device-to-device hipMemcpy may return before it completes, and the null
    stream does not order work on non-blocking streams)."""
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(lib().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.e = e.value

    def record(self, stream):
        check(lib().hipEventRecord(self.e, stream), "hipEventRecord")

    def synchronize(self):
        check(lib().hipEventSynchronize(self.e), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0.0)
        check(lib().hipEventElapsedTime(C.byref(ms), self.e, end.e), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.e:
                lib().hipEventDestroy(self.e)
        except Exception:
            pass


GRAPH_NODE_KERNEL = 0  # hipGraphNodeTypeKernel


class Graph:
    """A stream capture (hipStreamBeginCapture in thread-local mode ..
    hipStreamEndCapture) instantiated for replay: fn() issues the work on
    `stream` while it is captured."""

    def __init__(self, stream, fn):
        L = lib()
        for name, args in (("hipStreamBeginCapture", [C.c_void_p, C.c_int]),
                           ("hipStreamEndCapture", [C.c_void_p, C.POINTER(C.c_void_p)]),
                           ("hipGraphInstantiate", [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p,
                                                    C.c_char_p, C.c_size_t]),
                           ("hipGraphLaunch", [C.c_void_p, C.c_void_p]),
                           ("hipGraphGetNodes", [C.c_void_p, C.POINTER(C.c_void_p),
                                                 C.POINTER(C.c_size_t)]),
                           ("hipGraphNodeGetType", [C.c_void_p, C.POINTER(C.c_int)]),
                           ("hipGraphExecDestroy", [C.c_void_p]),
                           ("hipGraphDestroy", [C.c_void_p])):
            getattr(L, name).argtypes = args
        self.graph = self.exec = None
        check(L.hipStreamBeginCapture(stream, 1), "hipStreamBeginCapture")
        g = C.c_void_p()
        try:
            fn()
        finally:
            rc = L.hipStreamEndCapture(stream, C.byref(g))
            self.graph = g.value
        check(rc, "hipStreamEndCapture")
        ex = C.c_void_p()
        check(L.hipGraphInstantiate(C.byref(ex), self.graph, None, None, 0), "hipGraphInstantiate")
        self.exec = ex.value

    def node_types(self):
        L = lib()
        n = C.c_size_t(0)
        check(L.hipGraphGetNodes(self.graph, None, C.byref(n)), "hipGraphGetNodes")
        nodes = (C.c_void_p * max(n.value, 1))()
        check(L.hipGraphGetNodes(self.graph, nodes, C.byref(n)), "hipGraphGetNodes")
        out = []
        for i in range(n.value):
            t = C.c_int(-1)
            check(L.hipGraphNodeGetType(nodes[i], C.byref(t)), "hipGraphNodeGetType")
            out.append(t.value)
        return out

    def launch(self, stream):
        check(lib().hipGraphLaunch(self.exec, stream), "hipGraphLaunch")

    def destroy(self):
        L = lib()
        if self.exec:
            L.hipGraphExecDestroy(self.exec)
            self.exec = None
        if self.graph:
            L.hipGraphDestroy(self.graph)
            self.graph = None
