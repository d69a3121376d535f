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
        "ih_argmax_rows": (i32, [vp, vp, i32, i32, vp]),
        "ih_argmax_rows_noalloc": (i32, [vp, vp, i32, i32, vp]),
        "ih_accept": (i32, [vp, vp, i32, vp]),
        "ih_spec_accept_dev": (i32, [vp, vp, vp, vp, vp, i32, i32]),
        "ih_model_create_synthetic": (i32, [vp, vp, C.c_uint64, P(vp)]),
        "ih_model_free": (i32, [vp]),
        "ih_model_weight_bytes": (sz, [vp]),
        "ih_kv_create": (i32, [vp, i32, P(vp)]),
        "ih_kv_free": (i32, [vp]),
        "ih_kv_fill_synthetic": (i32, [vp, i32, C.c_uint64]),
        "ih_kv_pos": (i32, [vp]),
        "ih_kv_set_pos": (i32, [vp, i32]),
        "ih_kv_commit": (i32, [vp, i32]),
        "ih_kv_chunk": (i32, [vp]),
        "ih_verify_step": (i32, [vp, vp, vp, i32, vp, vp]),
        "ih_verify_step_dev": (i32, [vp, vp, vp, i32, vp]),
        "ih_verify_and_accept": (i32, [vp, vp, vp, i32, vp]),
        "ih_model_logits_dev": (vp, [vp]),
        "ih_kv_create_chunked": (i32, [vp, i32, i32, P(vp)]),
        "ih_model_moe_union": (i32, [vp, vp]),
        "ih_qmat_mxfp4_create": (i32, [vp, vp, vp, i32, i32, i32, P(vp)]),
        "ih_qmat_mxfp4_create_dev": (i32, [vp, vp, vp, i32, i32, i32, P(vp)]),
        "ih_qmat_format": (i32, [vp]),
        "ih_qmm_expert": (i32, [vp, vp, i32, vp, i32, i32, vp, i32]),
        "ih_moe_route": (i32, [vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp]),
        "ih_qmm_gathered": (i32, [vp, vp, vp, i32, i32, i32, vp, vp, vp, vp, i32]),
        "ih_copy_index_create": (i32, [i32, i32, i32, P(vp)]),
        "ih_copy_index_free": (i32, [vp]),
        "ih_copy_index_append": (i32, [vp, vp, i32]),
        "ih_copy_index_sync": (i32, [vp, vp, i32]),
        "ih_copy_index_reset": (i32, [vp]),
        "ih_copy_index_len": (i32, [vp]),
        "ih_copy_index_propose": (i32, [vp, i32, vp, P(i32), P(i32)]),
        "ih_copy_lookup_dev": (i32, [vp, vp, i32, i32, i32, i32, vp, vp, i32]),
        "ih_verify_step_chained": (i32, [vp, vp, vp, i32, vp, vp, i32, i32]),
        "ih_kv_capacity": (i32, [vp]),
        "ih_decode_greedy": (i32, [vp, vp, vp, i32, C.c_uint32, vp, vp, i32, P(i32), vp]),
        "ih_model_load_mlx": (i32, [vp, C.c_char_p, P(vp)]),
        "ih_mlx_describe": (i32, [C.c_char_p, vp]),
        "ih_topk64_dev": (i32, [vp, vp, i32, i32, i32, C.c_float, vp, vp, vp]),
        "ih_spec_accept_sample_dev": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32]),
        "ih_spec_rows_choose_dev": (i32, [vp, vp, vp, vp]),
        "ih_decode_sample": (i32, [vp, vp, vp, i32, C.c_uint32, vp, vp, C.c_uint64, vp, i32, P(i32), vp]),
        "ih_drafter_create_synthetic": (i32, [vp, vp, C.c_uint64, P(vp)]),
        "ih_drafter_load_mlx": (i32, [vp, C.c_char_p, P(vp)]),
        "ih_drafter_describe": (i32, [vp, vp]),
        "ih_quantize_int4_g64": (i32, [vp, i32, i32, vp, vp, vp]),
        "ih_drafter_free": (i32, [vp]),
        "ih_model_set_drafter": (i32, [vp, vp]),
        "ih_drafter_captures_dev": (vp, [vp]),
        "ih_drafter_context": (i32, [vp, i32, i32, i32, vp]),
        "ih_drafter_block": (i32, [vp, vp, i32, vp, vp]),
        "ih_drafter_block_rows": (i32, [vp]),
        "ih_timing_enable": (i32, [vp, i32]),
        "ih_qmm_shape_override": (i32, [vp, i32, i32, i32, i32, i32]),
        "ih_timing_read": (i32, [vp, i32, P(C.c_double), P(C.c_int), P(C.c_double)]),
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

    @classmethod
    def mxfp4(cls, ctx: Context, w: np.ndarray, s: np.ndarray) -> "QMat":
        """MLX mxfp4: codes uint32 [(E,) N, K/8], e8m0 scales uint8 [(E,) N, K/32]."""
        w = np.ascontiguousarray(w, dtype=np.uint32)
        s = np.ascontiguousarray(s, dtype=np.uint8)
        E = 1 if w.ndim == 2 else w.shape[0]
        N, K = w.shape[-2], w.shape[-1] * 8
        h = vp()
        check(lib().ih_qmat_mxfp4_create(ctx.handle, ptr(w), ptr(s), E, N, K, C.byref(h)))
        return cls(ctx, h.value, N, K, E)

    @property
    def format(self) -> int:
        return lib().ih_qmat_format(self.handle)

    def expert(self, x_dev: "DeviceBuffer", M: int, expert: int = 0) -> np.ndarray:
        """y = x[M, K] (bf16 on the device) · W[expert]ᵀ, fp32 [M, N]."""
        y = self.ctx.buffer(M * self.N * 4)
        check(lib().ih_qmm_expert(self.ctx.handle, self.handle, expert, x_dev.ptr, self.K, M, y.ptr, self.N))
        out = y.download(np.float32, (M, self.N))
        y.free()
        return out

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


MAX_ROWS = 17


class AcceptResult(C.Structure):
    _fields_ = [("m", C.c_int), ("n_emitted", C.c_int), ("tokens", C.c_uint32 * MAX_ROWS)]

    @property
    def emitted(self) -> list[int]:
        return list(self.tokens[: self.n_emitted])


class ModelDesc(C.Structure):
    """ih_model_desc (include/ingot_hip.h)."""

    _fields_ = [
        ("n_layers", C.c_int), ("hidden", C.c_int), ("n_q_heads", C.c_int), ("n_kv_heads", C.c_int),
        ("head_dim", C.c_int), ("intermediate", C.c_int), ("vocab", C.c_int), ("rope_theta", C.c_float),
        ("rms_eps", C.c_float), ("n_experts", C.c_int), ("top_k", C.c_int), ("expert_intermediate", C.c_int),
        ("expert_format", C.c_int), ("router_bias", C.c_int), ("expert_bias", C.c_int), ("act", C.c_int),
        ("swiglu_limit", C.c_float), ("sliding_window", C.c_int), ("sinks", C.c_int), ("hadamard_k", C.c_int),
        ("qk_norm", C.c_int), ("qkv_bias", C.c_int), ("iid_routing", C.c_int), ("rotary_dims", C.c_int),
        ("attn_gate", C.c_int), ("o_bias", C.c_int), ("rope_type", C.c_int), ("rope_factor", C.c_float),
        ("rope_orig_max", C.c_float), ("rope_beta_fast", C.c_float), ("rope_beta_slow", C.c_float),
        ("rope_mscale", C.c_float), ("rope_attn_factor", C.c_float), ("rope_no_truncate", C.c_int),
        ("rope_partial", C.c_float), ("router_int4", C.c_int),
    ]

    @classmethod
    def make(cls, **kw) -> "ModelDesc":
        d = cls(rope_theta=1e6, rms_eps=1e-6, hadamard_k=1, swiglu_limit=7.0)
        for k, v in kw.items():
            setattr(d, k, v)
        return d

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}


class DecodeOpts(C.Structure):
    """ih_decode_opts (include/ingot_hip.h)."""

    _fields_ = [("max_tokens", C.c_int), ("stop_tokens", vp), ("n_stop", C.c_int), ("rows", C.c_int),
                ("min_match", C.c_int), ("max_match", C.c_int), ("inflight", C.c_int), ("drafter", vp),
                ("rows_params", vp)]


class DrafterDesc(C.Structure):
    """ih_drafter_desc (include/ingot_hip.h)."""

    _fields_ = [("n_layers", C.c_int), ("hidden", C.c_int), ("n_q_heads", C.c_int), ("head_dim", C.c_int),
                ("intermediate", C.c_int), ("block", C.c_int), ("window", C.c_int), ("n_targets", C.c_int),
                ("target_layers", C.c_int * 8), ("rank", C.c_int), ("dyn_conv", C.c_int), ("mask_token", C.c_uint32),
                ("rope_theta", C.c_float), ("rms_eps", C.c_float)]

    @classmethod
    def make(cls, targets=(), **kw) -> "DrafterDesc":
        d = cls(rope_theta=1e6, rms_eps=1e-6, dyn_conv=1)
        for k, v in kw.items():
            setattr(d, k, v)
        d.n_targets = len(targets)
        for i, t in enumerate(targets):
            d.target_layers[i] = t
        return d


class Drafter:
    """A synthetic-weight DFlash2 drafter for a model (ih_drafter_*)."""

    def __init__(self, model: "Model", desc: DrafterDesc, seed: int):
        self.model, self.desc, self.seed = model, desc, seed
        h = vp()
        check(lib().ih_drafter_create_synthetic(model.handle, C.byref(desc), seed, C.byref(h)))
        self.handle = h.value

    @classmethod
    def load_mlx(cls, model: "Model", directory) -> "Drafter":
        """A trained drafter from its checkpoint directory (ih_drafter_load_mlx)."""
        self = cls.__new__(cls)
        self.model, self.seed = model, None
        h = vp()
        check(lib().ih_drafter_load_mlx(model.handle, str(directory).encode(), C.byref(h)))
        self.handle = h.value
        self.desc = DrafterDesc()
        check(lib().ih_drafter_describe(self.handle, C.byref(self.desc)))
        return self

    def attach(self) -> None:
        check(lib().ih_model_set_drafter(self.model.handle, self.handle))

    def captures(self, rows: int) -> np.ndarray:
        ctx = self.model.ctx
        n = rows * self.desc.n_targets * self.model.desc.hidden
        out = np.empty(n, np.uint16)
        check(lib().ih_memcpy_dtoh(ctx.handle, ptr(out), lib().ih_drafter_captures_dev(self.handle), n * 2))
        return out.reshape(rows, -1)

    def context(self, rows: int, nvalid: int, pos0: int) -> None:
        check(lib().ih_drafter_context(self.handle, rows, nvalid, pos0, None))

    def block(self, anchor: int, P: int):
        """(drafts [block − 1], conf [block − 1]) for the anchor at P."""
        ctx = self.model.ctx
        B = self.desc.block
        vt = ctx.to_device(np.full(B, anchor, np.uint32))
        cf = ctx.buffer(4 * B)
        check(lib().ih_drafter_block(self.handle, vt.ptr, P, None, cf.ptr))
        out = vt.download(np.uint32, (B,))[1:], cf.download(np.float32, (B - 1,))
        vt.free()
        cf.free()
        return out

    def free(self) -> None:
        if self.handle:
            lib().ih_drafter_free(self.handle)
            self.handle = None


class DecodeStats(C.Structure):
    _fields_ = [("rounds", C.c_int), ("drafted", C.c_int), ("accepted", C.c_int), ("emitted", C.c_int),
                ("finish", C.c_int)]


FINISH_LENGTH, FINISH_STOP, FINISH_CONTEXT = 0, 1, 2
TOPK, RND_PER_ROUND = 64, 34


class SampleParams(C.Structure):
    """ih_sample_params: temperature → top-k → min-p → top-p."""

    _fields_ = [("temp", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int), ("min_p", C.c_float)]


class RowsParams(C.Structure):
    """ih_rows_params: Platt (a, b) per draft depth group, cost per rows, kmin, kmax."""

    _fields_ = [("a", C.c_float * 4), ("b", C.c_float * 4), ("cost", C.c_float * 18), ("kmin", C.c_int),
                ("kmax", C.c_int)]


def accept(vtok, top1) -> AcceptResult:
    vtok = np.ascontiguousarray(vtok, np.uint32)
    top1 = np.ascontiguousarray(top1, np.uint32)
    r = AcceptResult()
    check(lib().ih_accept(ptr(vtok), ptr(top1), len(vtok), C.byref(r)))
    return r


class Model:
    """A synthetic-weight model and its KV cache owned by the library."""

    def __init__(self, ctx: Context, desc: ModelDesc, seed: int):
        self.ctx, self.desc, self.seed = ctx, desc, seed
        h = vp()
        check(lib().ih_model_create_synthetic(ctx.handle, C.byref(desc), seed, C.byref(h)))
        self.handle = h.value

    @classmethod
    def load_mlx(cls, ctx: Context, directory) -> "Model":
        """An mlx-lm 4-bit checkpoint directory (ih_model_load_mlx)."""
        d = describe_mlx(directory)
        self = cls.__new__(cls)
        self.ctx, self.desc, self.seed = ctx, d, None
        h = vp()
        check(lib().ih_model_load_mlx(ctx.handle, str(directory).encode(), C.byref(h)))
        self.handle = h.value
        return self

    @property
    def weight_bytes(self) -> int:
        return lib().ih_model_weight_bytes(self.handle)

    def free(self) -> None:
        if self.handle:
            lib().ih_model_free(self.handle)
            self.handle = None


def quantize_int4_g64(w_bf16: np.ndarray):
    """(w uint32 [N, K/8], scales, biases bf16 [N, K/64]) of a bf16 matrix (ih_quantize_int4_g64; host only)."""
    a = np.ascontiguousarray(w_bf16, np.uint16)
    N, K = a.shape
    w = np.empty((N, K // 8), np.uint32)
    s = np.empty((N, K // 64), np.uint16)
    b = np.empty((N, K // 64), np.uint16)
    check(lib().ih_quantize_int4_g64(ptr(a), N, K, ptr(w), ptr(s), ptr(b)))
    return w, s, b


def describe_mlx(directory) -> ModelDesc:
    """The model description of an mlx-lm checkpoint directory (ih_mlx_describe; host only)."""
    d = ModelDesc()
    check(lib().ih_mlx_describe(str(directory).encode(), C.byref(d)))
    return d


class KVCache:
    def __init__(self, model: Model, capacity: int, chunk: int = 0):
        self.model = model
        h = vp()
        check(lib().ih_kv_create_chunked(model.handle, capacity, chunk, C.byref(h)))
        self.handle = h.value

    def fill_synthetic(self, P: int, seed: int) -> None:
        check(lib().ih_kv_fill_synthetic(self.handle, P, seed))

    @property
    def pos(self) -> int:
        return lib().ih_kv_pos(self.handle)

    def set_pos(self, p: int) -> None:
        check(lib().ih_kv_set_pos(self.handle, p))

    def commit(self, n: int) -> None:
        check(lib().ih_kv_commit(self.handle, n))

    @property
    def chunk(self) -> int:
        return lib().ih_kv_chunk(self.handle)

    def verify(self, tokens, want_logits: bool = False):
        t = np.ascontiguousarray(tokens, np.uint32)
        top1 = np.zeros(len(t), np.uint32)
        logits = np.zeros((len(t), self.model.desc.vocab), np.float32) if want_logits else None
        check(lib().ih_verify_step(self.model.handle, self.handle, ptr(t), len(t),
                                   ptr(logits) if logits is not None else None, ptr(top1)))
        return (top1, logits) if want_logits else top1

    @property
    def capacity(self) -> int:
        return lib().ih_kv_capacity(self.handle)

    def decode_greedy(self, first: int, max_tokens: int, rows: int = 1, history=None, stop=(), inflight: int = 2,
                      min_match: int = 3, max_match: int = 64, drafter: "Drafter | None" = None,
                      rows_params: "RowsParams | None" = None):
        """Chained greedy decoding (ih_decode_greedy): (emitted tokens, DecodeStats)."""
        stop_a = np.ascontiguousarray(np.asarray(stop, np.uint32).reshape(-1))
        o = DecodeOpts(max_tokens=max_tokens, stop_tokens=ptr(stop_a) if stop_a.size else None, n_stop=stop_a.size,
                       rows=rows, min_match=min_match, max_match=max_match, inflight=inflight,
                       drafter=drafter.handle if drafter is not None else None,
                       rows_params=C.addressof(rows_params) if rows_params is not None else None)
        hist = None if history is None else np.ascontiguousarray(np.asarray(history, np.uint32))
        out = np.zeros(max_tokens, np.uint32)
        n = C.c_int()
        st = DecodeStats()
        check(lib().ih_decode_greedy(self.model.handle, self.handle, ptr(hist) if hist is not None else None,
                                     0 if hist is None else hist.size, first, C.byref(o), ptr(out), max_tokens,
                                     C.byref(n), C.byref(st)))
        return [int(x) for x in out[: n.value]], st

    def decode_sample(self, first: int, max_tokens: int, params: "SampleParams", seed: int, rows: int = 1,
                      history=None, stop=(), inflight: int = 2, min_match: int = 3, max_match: int = 64,
                      drafter: "Drafter | None" = None, rows_params: "RowsParams | None" = None):
        """Chained decoding with temperature sampling (ih_decode_sample): (emitted tokens, DecodeStats)."""
        stop_a = np.ascontiguousarray(np.asarray(stop, np.uint32).reshape(-1))
        o = DecodeOpts(max_tokens=max_tokens, stop_tokens=ptr(stop_a) if stop_a.size else None, n_stop=stop_a.size,
                       rows=rows, min_match=min_match, max_match=max_match, inflight=inflight,
                       drafter=drafter.handle if drafter is not None else None,
                       rows_params=C.addressof(rows_params) if rows_params is not None else None)
        hist = None if history is None else np.ascontiguousarray(np.asarray(history, np.uint32))
        out = np.zeros(max_tokens, np.uint32)
        n = C.c_int()
        st = DecodeStats()
        check(lib().ih_decode_sample(self.model.handle, self.handle, ptr(hist) if hist is not None else None,
                                     0 if hist is None else hist.size, first, C.byref(o), C.byref(params), seed,
                                     ptr(out), max_tokens, C.byref(n), C.byref(st)))
        return [int(x) for x in out[: n.value]], st

    def verify_and_accept(self, tokens) -> AcceptResult:
        t = np.ascontiguousarray(tokens, np.uint32)
        r = AcceptResult()
        check(lib().ih_verify_and_accept(self.model.handle, self.handle, ptr(t), len(t), C.byref(r)))
        return r

    def free(self) -> None:
        if self.handle:
            lib().ih_kv_free(self.handle)
            self.handle = None


class CopyIndex:
    """Host trigram index of a token history (ih_copy_index_*; CopyIndex, Sources/Ingot/CopySpec.swift:15-139)."""

    def __init__(self, min_match: int = 3, max_match: int = 64, capacity: int = 1 << 16):
        h = vp()
        check(lib().ih_copy_index_create(min_match, max_match, capacity, C.byref(h)))
        self.handle = h.value
        self.last_match = 0

    def append(self, tokens) -> None:
        a = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))
        check(lib().ih_copy_index_append(self.handle, ptr(a), a.size))

    def sync(self, tokens) -> None:
        a = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))
        check(lib().ih_copy_index_sync(self.handle, ptr(a), a.size))

    def reset(self) -> None:
        check(lib().ih_copy_index_reset(self.handle))

    def __len__(self) -> int:
        return lib().ih_copy_index_len(self.handle)

    def propose(self, max_k: int) -> list[int]:
        out = np.zeros(max(max_k, 1), np.uint32)
        n, m = C.c_int(), C.c_int()
        check(lib().ih_copy_index_propose(self.handle, max_k, ptr(out), C.byref(n), C.byref(m)))
        self.last_match = m.value
        return [int(x) for x in out[: n.value]]

    def free(self) -> None:
        if self.handle:
            lib().ih_copy_index_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:  # noqa: BLE001
            pass


def copy_lookup_dev(ctx: "Context", hist_dev: "DeviceBuffer", n: int, max_k: int, min_match: int = 3,
                    max_match: int = 64, vtok_dev: "DeviceBuffer | None" = None, rows: int = 0):
    """Device scan (ih_copy_lookup_dev): returns (proposal, match, end p or -1)."""
    out = ctx.buffer((4 + max_k) * 4)
    check(lib().ih_copy_lookup_dev(ctx.handle, hist_dev.ptr, n, max_k, min_match, max_match, out.ptr,
                                   vtok_dev.ptr if vtok_dev is not None else None, rows))
    o = out.download(np.uint32, (4 + max_k,))
    out.free()
    cnt = int(o[0])
    end = int(o[2]) if cnt else -1
    return [int(x) for x in o[4: 4 + cnt]], int(o[1]), end


class Routing:
    """Device outputs of ih_moe_route for `rows` rows and top-k."""

    def __init__(self, ctx: Context, rows: int, K: int, E: int):
        self.ctx, self.rows, self.K, self.E = ctx, rows, K, E
        n = rows * K
        self.nent = ctx.buffer(4)
        self.entries = ctx.buffer(3 * max(E, 1) * 4)
        self.x_row = ctx.buffer(n * 4)
        self.pair_w = ctx.buffer(n * 4)
        self.row_pair = ctx.buffer(n * 4)

    def route(self, logits_dev: "DeviceBuffer", ldl: int, bias_dev=None, pes_dev=None) -> "Routing":
        check(lib().ih_moe_route(self.ctx.handle, logits_dev.ptr, ldl, self.rows, self.E, self.K,
                                 bias_dev.ptr if bias_dev is not None else None,
                                 pes_dev.ptr if pes_dev is not None else None, self.nent.ptr, self.entries.ptr,
                                 self.x_row.ptr, self.pair_w.ptr, self.row_pair.ptr))
        return self

    def download(self):
        U = int(self.nent.download(np.int32, (1,))[0])
        n = self.rows * self.K
        return dict(U=U, entries=self.entries.download(np.int32, (self.E, 3))[:U],
                    x_row=self.x_row.download(np.int32, (n,)), pair_w=self.pair_w.download(np.float32, (n,)),
                    row_pair=self.row_pair.download(np.int32, (self.rows, self.K)))

    def gathered(self, W: QMat, x_dev: "DeviceBuffer") -> np.ndarray:
        """y [rows·k, N] fp32 of ih_qmm_gathered (by pair)."""
        n = self.rows * self.K
        y = self.ctx.buffer(n * W.N * 4).fill(0)
        check(lib().ih_qmm_gathered(self.ctx.handle, W.handle, x_dev.ptr, W.K, self.rows, self.K, self.nent.ptr,
                                    self.entries.ptr, self.x_row.ptr, y.ptr, W.N))
        out = y.download(np.float32, (n, W.N))
        y.free()
        return out

    def free(self) -> None:
        for b in (self.nent, self.entries, self.x_row, self.pair_w, self.row_pair):
            b.free()
