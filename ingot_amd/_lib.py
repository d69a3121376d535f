"""ctypes binding of libingot_hip.so (the C ABI in include/ingot_hip.h).

The library is the product: there is no Python or CPU fallback. Loading fails loudly when the built library is
missing (run ``python -m ingot_amd.build`` first).
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libingot_hip.so"
HEADER = HERE.parent / "include" / "ingot_hip.h"

IH_OK, IH_EINVAL, IH_EDEVICE, IH_ENOMEM, IH_ESTATE = 0, 1, 2, 3, 4
_NAMES = {1: "IH_EINVAL", 2: "IH_EDEVICE", 3: "IH_ENOMEM", 4: "IH_ESTATE"}


class IngotError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_NAMES.get(code, code)}: {msg}")
        self.code = code


_lib = None


def lib() -> C.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m ingot_amd.build`")
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


def declared_symbols() -> list[str]:
    """Function names declared in include/ingot_hip.h."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ih_[a-z0-9_]+)\s*\(", text)))


vp = C.c_void_p
i32 = C.c_int
u64 = C.c_uint64
sz = C.c_size_t
P = C.POINTER


def _declare(L: C.CDLL) -> None:
    sig = {
        "ih_last_error": (C.c_char_p, []),
        "ih_version": (i32, []),
        "ih_init": (i32, [i32, P(vp)]),
        "ih_ctx_free": (i32, [vp]),
        "ih_sync": (i32, [vp]),
        "ih_stream": (vp, [vp]),
        "ih_cu_count": (i32, [vp]),
        "ih_malloc": (i32, [vp, sz, P(vp)]),
        "ih_free": (i32, [vp, vp]),
        "ih_memcpy_htod": (i32, [vp, vp, vp, sz]),
        "ih_memcpy_dtoh": (i32, [vp, vp, vp, sz]),
        "ih_memcpy_dtod": (i32, [vp, vp, vp, sz]),
        "ih_fill": (i32, [vp, vp, i32, sz]),
        "ih_qmat_int4_create": (i32, [vp, vp, vp, vp, i32, i32, i32, P(vp)]),
        "ih_qmat_int4_create_dev": (i32, [vp, vp, vp, vp, i32, i32, i32, P(vp)]),
        "ih_qmat_free": (i32, [vp]),
        "ih_qmat_bytes": (sz, [vp]),
        "ih_qmm_int4": (i32, [vp, vp, vp, i32, i32, vp, i32, i32]),
    }
    for name, (res, args) in sig.items():
        if hasattr(L, name):
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args


def check(code: int) -> None:
    if code != IH_OK:
        raise IngotError(code, lib().ih_last_error().decode())


def ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class DeviceBuffer:
    """A device allocation owned by the library's context."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx, self.nbytes = ctx, int(nbytes)
        p = vp()
        check(lib().ih_malloc(ctx.handle, self.nbytes, C.byref(p)))
        self.ptr = p.value

    def upload(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().ih_memcpy_htod(self.ctx.handle, self.ptr, ptr(a), a.nbytes))
        return self

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(lib().ih_memcpy_dtoh(self.ctx.handle, ptr(out), self.ptr, out.nbytes))
        return out

    def fill(self, byte: int = 0) -> "DeviceBuffer":
        check(lib().ih_fill(self.ctx.handle, self.ptr, byte, self.nbytes))
        return self

    def free(self) -> None:
        if self.ptr:
            check(lib().ih_free(self.ctx.handle, self.ptr))
            self.ptr = None


class Context:
    def __init__(self, device: int = 0):
        h = vp()
        check(lib().ih_init(device, C.byref(h)))
        self.handle = h.value

    def sync(self) -> None:
        check(lib().ih_sync(self.handle))

    @property
    def stream(self) -> int:
        return lib().ih_stream(self.handle)

    def buffer(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        return DeviceBuffer(self, max(a.nbytes, 1)).upload(a)

    def close(self) -> None:
        if self.handle:
            lib().ih_ctx_free(self.handle)
            self.handle = None


class QMat:
    """A quantized matrix owned by the library (MLX int4 g64 source format)."""

    def __init__(self, ctx: Context, handle: int, N: int, K: int, E: int = 1):
        self.ctx, self.handle, self.N, self.K, self.E = ctx, handle, N, K, E

    @classmethod
    def int4(cls, ctx: Context, w: np.ndarray, s: np.ndarray, b: np.ndarray) -> "QMat":
        w = np.ascontiguousarray(w, dtype=np.uint32)
        s = np.ascontiguousarray(s, dtype=np.uint16)
        b = np.ascontiguousarray(b, dtype=np.uint16)
        E = 1 if w.ndim == 2 else w.shape[0]
        N, K = w.shape[-2], w.shape[-1] * 8
        h = vp()
        check(lib().ih_qmat_int4_create(ctx.handle, ptr(w), ptr(s), ptr(b), E, N, K, C.byref(h)))
        return cls(ctx, h.value, N, K, E)

    @property
    def nbytes(self) -> int:
        return lib().ih_qmat_bytes(self.handle)

    def free(self) -> None:
        if self.handle:
            lib().ih_qmat_free(self.handle)
            self.handle = None


class HipEvents:
    """HIP events recorded on the library context's stream (libamdhip64 through ctypes)."""

    _hip = None

    @classmethod
    def hip(cls):
        if cls._hip is None:
            h = C.CDLL("libamdhip64.so")
            h.hipEventCreate.argtypes = [P(vp)]
            h.hipEventRecord.argtypes = [vp, vp]
            h.hipEventSynchronize.argtypes = [vp]
            h.hipEventElapsedTime.argtypes = [P(C.c_float), vp, vp]
            h.hipEventDestroy.argtypes = [vp]
            cls._hip = h
        return cls._hip

    def __init__(self, ctx: Context, n: int):
        self.stream = ctx.stream
        self.ev = []
        for _ in range(n):
            e = vp()
            if self.hip().hipEventCreate(C.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.ev.append(e.value)

    def record(self, i: int) -> None:
        if self.hip().hipEventRecord(self.ev[i], self.stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_ms(self, a: int, b: int) -> float:
        self.hip().hipEventSynchronize(self.ev[b])
        t = C.c_float()
        if self.hip().hipEventElapsedTime(C.byref(t), self.ev[a], self.ev[b]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return t.value

    def close(self) -> None:
        for e in self.ev:
            self.hip().hipEventDestroy(e)
        self.ev = []
