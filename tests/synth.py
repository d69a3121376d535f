"""Seeded synthetic tensors for the tests (numpy; not the product's synthetic-model generator)."""
from __future__ import annotations

import numpy as np

from oracle import f32_to_bf16, bf16_to_f32


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def int4_matrix(g: np.random.Generator, N: int, K: int, E: int | None = None, scale_sd: float = 0.02):
    """MLX int4 g64: uniform codes, bf16 scale ~ |N(0, scale_sd)|, bias = -8·scale (benchmark configuration 0)."""
    shape = (N, K) if E is None else (E, N, K)
    q = g.integers(0, 16, size=shape, dtype=np.uint32)
    w = pack_nibbles(q)
    gs = shape[:-1] + (K // 64,)
    s = f32_to_bf16(np.abs(g.normal(0, scale_sd, size=gs)).astype(np.float32))
    b = f32_to_bf16(-8.0 * bf16_to_f32(s))
    return w, s, b


def pack_nibbles(q: np.ndarray) -> np.ndarray:
    """Codes [..., K] (0..15) → uint32 [..., K/8], value j in bits 4j (low nibble first)."""
    q = q.astype(np.uint32)
    sh = q.reshape(q.shape[:-1] + (q.shape[-1] // 8, 8))
    out = np.zeros(sh.shape[:-1], np.uint32)
    for j in range(8):
        out |= sh[..., j] << np.uint32(4 * j)
    return out


def bf16_normal(g: np.random.Generator, shape, sd: float = 1.0):
    """(bf16 bits, their float values)."""
    v = f32_to_bf16(g.normal(0, sd, size=shape).astype(np.float32))
    return v, bf16_to_f32(v)


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def zipf_context(seed: int, n: int = 131072, vocab: int = 151936, s: float = 1.1, spans: int = 64,
                 span_len: int = 32, tail: int = 8):
    """Config 2's context: int32 ids drawn Zipf(s) over the vocab (rank r has weight r^-s, id = rank - 1), with
    `spans` repeated spans of `span_len` tokens (each copied from an earlier position to a later one), ending with
    the first `tail` tokens of one more copy of the last planted span, so the trailing trigram has a long earlier
    match. Returns (context uint32 [n], the span's source position)."""
    g = np.random.default_rng(seed)
    w = np.arange(1, vocab + 1, dtype=np.float64) ** -s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    h = np.searchsorted(cdf, g.random(n), side="right").astype(np.uint32)
    h = np.minimum(h, vocab - 1)
    body = n - tail
    src = 0
    for _ in range(spans):
        src = int(g.integers(0, body // 2 - span_len))
        dst = int(g.integers(body // 2, body - span_len))
        h[dst:dst + span_len] = h[src:src + span_len]
    h[body:] = h[src:src + tail]
    return h, src


def mxfp4_matrix(g: np.random.Generator, N: int, K: int, E: int | None = None, lo: int = 119, hi: int = 125):
    """MLX mxfp4: uniform e2m1 codes (8 per uint32, low nibble first), e8m0 scales uniform in [lo, hi]
    (2^-8 … 2^-2 by default: benchmark configuration 4)."""
    shape = (N, K) if E is None else (E, N, K)
    q = g.integers(0, 16, size=shape, dtype=np.uint32)
    s = g.integers(lo, hi + 1, size=shape[:-1] + (K // 32,), dtype=np.uint8)
    return pack_nibbles(q), s
