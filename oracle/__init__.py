"""CPU oracle — TEST INFRASTRUCTURE ONLY.

ctypes front end of oracle/liboracle.so (oracle.cpp, a C++17 restatement of the reference's verify-step semantics).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, as the checker or the
timed CPU baseline; the product (ingot_amd) never does.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None

f32p = C.POINTER(C.c_float)
u32p = C.POINTER(C.c_uint32)
u16p = C.POINTER(C.c_uint16)
u8p = C.POINTER(C.c_uint8)
i32p = C.POINTER(C.c_int32)
vp = C.c_void_p
i32 = C.c_int


def build() -> Path:
    """Compiles liboracle.so with the committed Makefile."""
    r = subprocess.run(["make", "-s", "-C", str(HERE)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run `make -C oracle`")
        _lib = C.CDLL(str(LIB_PATH))
        for name, res, args in _SIGS:
            if hasattr(_lib, name):
                f = getattr(_lib, name)
                f.restype, f.argtypes = res, args
    return _lib


_SIGS = [
    ("or_bf16_to_f32", C.c_float, [C.c_uint16]),
    ("or_f32_to_bf16", C.c_uint16, [C.c_float]),
    ("or_fp4_e2m1", C.c_float, [C.c_uint32]),
    ("or_e8m0", C.c_float, [C.c_uint8]),
    ("or_dequant_int4", None, [vp, vp, vp, i32, i32, vp]),
    ("or_dequant_mxfp4", None, [vp, vp, i32, i32, vp]),
    ("or_qmm_int4", None, [vp, i32, vp, vp, vp, i32, i32, vp]),
    ("or_qmm_mxfp4", None, [vp, i32, vp, vp, i32, i32, vp]),
    ("or_argmax_rows", None, [vp, i32, i32, vp]),
    ("or_accept", i32, [vp, vp, i32, vp]),
    ("or_num_threads", i32, []),
    ("or_sm_at", C.c_uint64, [C.c_uint64, C.c_uint64]),
    ("or_sm_key", C.c_uint64, [C.c_uint64, C.c_uint64]),
    ("or_sm_normal", C.c_float, [C.c_uint64, C.c_uint64]),
    ("or_synth_int4", None, [C.c_uint64, C.c_uint64, i32, i32, C.c_float, vp, vp, vp]),
    ("or_synth_mxfp4", None, [C.c_uint64, C.c_uint64, i32, i32, vp, vp]),
    ("or_synth_bf16", None, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, C.c_float, vp]),
    ("or_synth_f32", None, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, C.c_float, vp]),
    ("or_f32_to_f16", C.c_uint16, [C.c_float]),
    ("or_f16_to_f32", C.c_float, [C.c_uint16]),
    ("or_synth_kv", None, [C.c_uint64, C.c_uint64, i32, i32, i32, i32, vp, vp, vp, vp]),
    ("or_rmsnorm", None, [vp, i32, i32, vp, C.c_float, vp]),
    ("or_rms_split", None, [vp, i32, i32, vp, C.c_float, vp, vp]),
    ("or_glu", C.c_float, [C.c_float, C.c_float, i32, C.c_float]),
    ("or_fwht", None, [vp, i32]),
    ("or_rope_wht", None, [vp, i32, i32, C.c_float, i32]),
    ("or_rope_wht_ex", None, [vp, i32, i32, i32, C.c_float, vp, C.c_float, i32]),
    ("or_rope_table", C.c_float, [i32, C.c_double, i32, C.c_double, C.c_double, C.c_double, C.c_double, C.c_double,
                                  C.c_double, i32, C.c_double, vp]),
    ("or_attention", None, [vp, i32, i32, i32, i32, i32, vp, vp, vp, vp, i32, i32, vp, vp]),
    ("or_verify_dense", i32, [vp, C.c_uint64, C.c_uint64, i32, vp, i32, vp, vp]),
    ("or_model_create", vp, [vp, C.c_uint64, C.c_uint64, i32, i32]),
    ("or_model_verify", i32, [vp, vp, i32, vp, vp]),
    ("or_model_free", None, [vp]),
    ("or_route", None, [vp, i32, i32, i32, i32, vp, vp, vp, C.c_float, C.c_float, vp, vp]),
    ("or_expert_union", i32, [vp, i32, i32, i32, vp, vp]),
    ("or_copy_naive", i32, [vp, i32, i32, i32, i32, vp, vp]),
    ("or_copy_index_new", vp, [i32]),
    ("or_copy_index_free", None, [vp]),
    ("or_copy_index_append", None, [vp, vp, i32]),
    ("or_copy_index_propose", i32, [vp, i32, vp, vp]),
    ("or_splitmix64", None, [C.c_uint64, i32, vp]),
    ("or_model_set_capture", None, [vp, i32, vp]),
    ("or_model_tie_head", None, [vp]),
    ("or_set_attn_p16", None, [i32]),
    ("or_model_captures", None, [vp, vp]),
    ("or_drafter_create", vp, [vp, C.c_uint64, vp, C.c_uint64]),
    ("or_drafter_free", None, [vp]),
    ("or_drafter_context", None, [vp, vp, i32, i32, i32]),
    ("or_drafter_block", None, [vp, C.c_uint32, i32, vp, vp]),
    ("or_topk64", None, [vp, i32, i32, C.c_float, vp, vp, vp]),
    ("or_sample_dist", i32, [vp, vp, C.c_float, C.c_float, vp, vp]),
    ("or_accept_sample", i32, [vp, i32, vp, vp, vp, vp, vp, vp]),
    ("or_rows_choose", i32, [vp, vp, vp, vp, i32, i32]),
]


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be contiguous"
    return a.ctypes.data


# ---- number formats ----------------------------------------------------------------------------------------------

def bf16_to_f32(v: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) → float32 (exact)."""
    return (np.asarray(v, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 → bf16 bit patterns, round to nearest even (Loader/Quant.swift:121-125)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(x))


def fp4_e2m1(q: int) -> float:
    return float(lib().or_fp4_e2m1(q))


def e8m0(s: int) -> float:
    return float(lib().or_e8m0(s))


def dequant_int4(w: np.ndarray, s: np.ndarray, b: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint32)
    s = np.ascontiguousarray(s, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    N, K = w.shape[0], w.shape[1] * 8
    out = np.empty((N, K), np.float32)
    lib().or_dequant_int4(_p(w), _p(s), _p(b), N, K, _p(out))
    return out


def dequant_mxfp4(w: np.ndarray, s: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint32)
    s = np.ascontiguousarray(s, np.uint8)
    N, K = w.shape[0], w.shape[1] * 8
    out = np.empty((N, K), np.float32)
    lib().or_dequant_mxfp4(_p(w), _p(s), N, K, _p(out))
    return out


# ---- kernels of the verify step ----------------------------------------------------------------------------------

def qmm_int4(x: np.ndarray, w: np.ndarray, s: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Y[M, N] = X[M, K] · dequant(W)ᵀ in fp32 (X given as float values)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.uint32)
    s = np.ascontiguousarray(s, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape[1] * 8 == K
    y = np.empty((M, N), np.float32)
    lib().or_qmm_int4(_p(x), M, _p(w), _p(s), _p(b), N, K, _p(y))
    return y


def qmm_mxfp4(x: np.ndarray, w: np.ndarray, s: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.uint32)
    s = np.ascontiguousarray(s, np.uint8)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float32)
    lib().or_qmm_mxfp4(_p(x), M, _p(w), _p(s), N, K, _p(y))
    return y


def argmax_rows(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, N = x.shape
    out = np.empty(rows, np.uint32)
    lib().or_argmax_rows(_p(x), rows, N, _p(out))
    return out


def accept(vtok: np.ndarray, top1: np.ndarray) -> tuple[int, np.ndarray]:
    """Greedy acceptance: (m, emitted tokens [m + 1])."""
    vtok = np.ascontiguousarray(vtok, np.uint32)
    top1 = np.ascontiguousarray(top1, np.uint32)
    B = len(vtok)
    em = np.zeros(B, np.uint32)
    m = lib().or_accept(_p(vtok), _p(top1), B, _p(em))
    return m, em[: m + 1].copy()


def num_threads() -> int:
    return int(lib().or_num_threads())


# ---- synthetic data and the whole verify step ---------------------------------------------------------------------

def synth_int4(seed: int, tensor: int, N: int, K: int, sd: float = 0.02):
    w = np.empty((N, K // 8), np.uint32)
    s = np.empty((N, K // 64), np.uint16)
    b = np.empty((N, K // 64), np.uint16)
    lib().or_synth_int4(seed, tensor, N, K, sd, _p(w), _p(s), _p(b))
    return w, s, b


def synth_kv(seed: int, tensor: int, KVH: int, HD: int, pos0: int, npos: int):
    k = np.empty((KVH, npos, HD), np.int8)
    v = np.empty((KVH, npos, HD), np.int8)
    ks = np.empty((KVH, npos), np.uint16)
    vs = np.empty((KVH, npos), np.uint16)
    lib().or_synth_kv(seed, tensor, KVH, HD, pos0, npos, _p(k), _p(v), _p(ks), _p(vs))
    return k, v, ks, vs


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def rmsnorm(x: np.ndarray, w_bf16: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w_bf16, np.uint16)
    out = np.empty_like(x)
    lib().or_rmsnorm(_p(x), x.shape[0], x.shape[1], _p(w), eps, _p(out))
    return out


def fwht(v: np.ndarray) -> np.ndarray:
    v = np.array(v, np.float32)
    lib().or_fwht(_p(v), len(v))
    return v


def rope_wht(x: np.ndarray, pos: int, theta: float, hadk: int) -> np.ndarray:
    x = np.array(x, np.float32)
    lib().or_rope_wht(_p(x), len(x), pos, theta, hadk)
    return x


ROPE_KINDS = {"default": 0, "linear": 1, "yarn": 2, "proportional": 3}


def rope_table(params: dict, theta: float, dims: int):
    """(inv_freq fp32 [dims/2], mscale) of a RoPE parameter dict (rope_type/type, factor, original_max_position_embeddings,
    beta_fast, beta_slow, mscale, attention_factor, truncate, partial_rotary_factor), as RopeTable.make."""
    kind = ROPE_KINDS[params.get("rope_type", params.get("type", "default"))]
    inv = np.zeros(dims // 2, np.float32)
    if kind == 0:
        inv[:] = (1.0 / np.power(float(theta), 2.0 * np.arange(dims // 2) / dims)).astype(np.float32)
        return inv, 1.0
    ms = lib().or_rope_table(kind, theta, dims, float(params.get("factor", 1.0)),
                             float(params.get("original_max_position_embeddings", 0.0)),
                             float(params.get("beta_fast", 32.0)), float(params.get("beta_slow", 1.0)),
                             float(params.get("mscale", 1.0)), float(params.get("attention_factor", 0.0)),
                             int(params.get("truncate", True)), float(params.get("partial_rotary_factor", 1.0)),
                             _p(inv))
    return inv, float(ms)


def rope_wht_ex(x: np.ndarray, rot: int, pos: int, theta: float, inv, mscale: float, hadk: int) -> np.ndarray:
    x = np.array(x, np.float32)
    inv = None if inv is None else np.ascontiguousarray(inv, np.float32)
    lib().or_rope_wht_ex(_p(x), len(x), rot, pos, theta, None if inv is None else _p(inv), mscale, hadk)
    return x


def attention(q, P, QH, KVH, k, v, ks, vs, window=0, sinks=None):
    """q fp32 [B][QH][HD]; k/v int8 [KVH][npos][HD]; ks/vs fp16 bits [KVH][npos] → [B][QH·HD]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.int8)
    v = np.ascontiguousarray(v, np.int8)
    ks = np.ascontiguousarray(ks, np.uint16)
    vs = np.ascontiguousarray(vs, np.uint16)
    B, _, HD = q.shape
    out = np.empty((B, QH * HD), np.float32)
    sk = None if sinks is None else np.ascontiguousarray(sinks, np.float32)
    lib().or_attention(_p(q), B, P, QH, KVH, HD, _p(k), _p(v), _p(ks), _p(vs), k.shape[1], window,
                       _p(sk) if sk is not None else None, _p(out))
    return out


def verify_dense(desc, seed: int, kv_seed: int, P: int, tokens):
    """(logits [B][V], top1 [B]) of the synthetic dense model; desc: ingot_amd._lib.ModelDesc (same layout)."""
    t = np.ascontiguousarray(tokens, np.uint32)
    B = len(t)
    logits = np.empty((B, desc.vocab), np.float32)
    top1 = np.empty(B, np.uint32)
    rc = lib().or_verify_dense(C.addressof(desc), seed, kv_seed, P, _p(t), B, _p(logits), _p(top1))
    assert rc == 0
    return logits, top1


class attn_p16:
    """Context manager: inside it, the oracle's attention rounds each probability × V scale to fp16, as the
    reference's attention does (verify_attn_pf.metal:268-276); outside, it is fp32."""

    def __enter__(self):
        lib().or_set_attn_p16(1)
        return self

    def __exit__(self, *exc):
        lib().or_set_attn_p16(0)
        return False


def attn_rounding_spread(desc, seed: int, kv_seed: int, P: int, tokens, ref_logits=None) -> float:
    """Max-abs change of the oracle's logits when its attention rounds p·vs to fp16 (the reference's and the GPU's
    rounding point): the scale of the difference that rounding point alone makes."""
    if ref_logits is None:
        ref_logits, _ = verify_dense(desc, seed, kv_seed, P, tokens)
    with attn_p16():
        alt, _ = verify_dense(desc, seed, kv_seed, P, tokens)
    return float(np.abs(alt - ref_logits).max())


class OracleModel:
    """The synthetic dense model held in host memory (weights and KV history), for repeated CPU verify steps."""

    def __init__(self, desc, seed: int, kv_seed: int, P: int, max_rows: int = 17):
        self.desc = desc
        self.h = lib().or_model_create(C.addressof(desc), seed, kv_seed, P, max_rows)

    def verify(self, tokens):
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty((len(t), self.desc.vocab), np.float32)
        top1 = np.empty(len(t), np.uint32)
        assert lib().or_model_verify(self.h, _p(t), len(t), _p(logits), _p(top1)) == 0
        return logits, top1

    def tie_head(self):
        """The head becomes the embedding table (tie_word_embeddings)."""
        lib().or_model_tie_head(self.h)

    def set_capture(self, layers):
        self.cap_layers = np.ascontiguousarray(layers, np.int32)
        lib().or_model_set_capture(self.h, len(self.cap_layers), _p(self.cap_layers))

    def captures(self, rows):
        out = np.empty((rows, len(self.cap_layers) * self.desc.hidden), np.uint16)
        lib().or_model_captures(self.h, _p(out))
        return out

    def free(self):
        if self.h:
            lib().or_model_free(self.h)
            self.h = None


# ---- MoE routing and copy-from-context ----------------------------------------------------------------------------

def route(logits, K, sigmoid=False, sel_bias=None, logit_bias=None, pes=None, scale=1.0, eps=0.0):
    """(expert ids [rows][K] int32, weights [rows][K] fp32)."""
    lg = np.ascontiguousarray(logits, np.float32)
    rows, E = lg.shape
    inds = np.empty((rows, K), np.int32)
    wts = np.empty((rows, K), np.float32)

    def opt(a):
        return None if a is None else np.ascontiguousarray(a, np.float32)

    sb, lb, pe = opt(sel_bias), opt(logit_bias), opt(pes)
    lib().or_route(_p(lg), rows, E, K, int(sigmoid), _p(sb) if sb is not None else None,
                   _p(lb) if lb is not None else None, _p(pe) if pe is not None else None, scale, eps, _p(inds), _p(wts))
    return inds, wts


def expert_union(inds, E):
    """(entries [U][3] = (expert, start, count), pairs [rows·K][2] = (row, slot))."""
    inds = np.ascontiguousarray(inds, np.int32)
    rows, K = inds.shape
    entries = np.empty((rows * K, 3), np.int32)
    pairs = np.empty((rows * K, 2), np.int32)
    U = lib().or_expert_union(_p(inds), rows, K, E, _p(entries), _p(pairs))
    return entries[:U].copy(), pairs


def copy_naive(h, maxK, min_match=3, max_match=64):
    """(proposal, match length) of the reference's copy rule by brute force."""
    h = np.ascontiguousarray(h, np.uint32)
    out = np.empty(max(maxK, 1), np.uint32)
    m = C.c_int()
    n = lib().or_copy_naive(_p(h), len(h), maxK, min_match, max_match, _p(out), C.byref(m))
    return out[:n].copy(), m.value


class CopyIndexRef:
    """The reference's trigram index, restated (test infrastructure)."""

    def __init__(self, capacity=1 << 16):
        self.h = lib().or_copy_index_new(capacity)

    def append(self, toks):
        t = np.ascontiguousarray(np.atleast_1d(toks), np.uint32)
        lib().or_copy_index_append(self.h, _p(t), len(t))

    def propose(self, maxK):
        out = np.empty(max(maxK, 1), np.uint32)
        m = C.c_int()
        n = lib().or_copy_index_propose(self.h, maxK, _p(out), C.byref(m))
        return out[:n].copy(), m.value

    def free(self):
        if self.h:
            lib().or_copy_index_free(self.h)
            self.h = None


def splitmix64(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().or_splitmix64(seed, n, _p(out))
    return out


# ---- sampling -------------------------------------------------------------------------------------------------

class SampleParams(C.Structure):
    _fields_ = [("temp", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int), ("min_p", C.c_float)]


def topk64(x, temp):
    """(idx [rows][64] uint32, val [rows][64] f32, z [rows][2] = (max, Σ exp((x − max)/T)))."""
    x = np.ascontiguousarray(x, np.float32)
    rows, V = x.shape
    idx = np.empty((rows, 64), np.uint32)
    val = np.empty((rows, 64), np.float32)
    z = np.empty((rows, 2), np.float32)
    lib().or_topk64(_p(x), rows, V, temp, _p(idx), _p(val), _p(z))
    return idx, val, z


def sample_dist(idx_row, val_row, M, Z, p: SampleParams):
    """(n, probabilities of the first n candidates)."""
    ci = np.ascontiguousarray(idx_row, np.uint32)
    cv = np.ascontiguousarray(val_row, np.float32)
    pr = np.zeros(64, np.float32)
    n = lib().or_sample_dist(_p(ci), _p(cv), M, Z, C.addressof(p), _p(pr))
    return n, pr[:n].copy()


def accept_sample(vtok, idx, val, z, u, p: SampleParams):
    """(m, emitted [m + 1]) of the rejection acceptance with uniforms u [2·rows]."""
    vtok = np.ascontiguousarray(vtok, np.uint32)
    idx = np.ascontiguousarray(idx, np.uint32)
    val = np.ascontiguousarray(val, np.float32)
    z = np.ascontiguousarray(z, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    em = np.zeros(len(vtok), np.uint32)
    m = lib().or_accept_sample(_p(vtok), len(vtok), _p(idx), _p(val), _p(z), _p(u), C.addressof(p), _p(em))
    return m, em[: m + 1].copy()


def rows_choose(conf, a, b, cost, kmin, kmax) -> int:
    conf = np.ascontiguousarray(conf, np.float32)
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    cost = np.ascontiguousarray(cost, np.float32)
    return int(lib().or_rows_choose(_p(conf), _p(a), _p(b), _p(cost), kmin, kmax))


# ---- DFlash2 drafter ------------------------------------------------------------------------------------------

class OracleDrafter:
    """The drafter with the synthetic weights of `desc` (ingot_amd._lib.DrafterDesc, same layout) for the target
    model `tdesc` (seed `tseed`): its window rings in host memory."""

    def __init__(self, desc, seed: int, tdesc, tseed: int):
        self.desc = desc
        self.h = lib().or_drafter_create(C.addressof(desc), seed, C.addressof(tdesc), tseed)

    def context(self, caps, nvalid: int, pos0: int):
        caps = np.ascontiguousarray(caps, np.uint16)
        lib().or_drafter_context(self.h, _p(caps), caps.shape[0], nvalid, pos0)

    def block(self, anchor: int, P: int):
        M = self.desc.block - 1
        drafts = np.empty(M, np.uint32)
        conf = np.empty(M, np.float32)
        lib().or_drafter_block(self.h, anchor, P, _p(drafts), _p(conf))
        return drafts, conf

    def free(self):
        if self.h:
            lib().or_drafter_free(self.h)
            self.h = None
