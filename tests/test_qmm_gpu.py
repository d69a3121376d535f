"""int4 g64 few-row qmm on the GPU against the CPU oracle (fp32 dequant + matmul).

Reference cases: the verify qmv (Sources/Ingot/Shaders/verify_nax.metal:102-176) is checked in the reference against a
CPU matmul of the dequantised weights (Tests/IngotTests/KernelHarness.swift:95-115,189-195) and for row invariance
(KernelCaseTests.swift:66-86, qmv4-rows at :614-621).
"""
import numpy as np
import pytest

import oracle
from ingot_amd._lib import QMat, lib, check
from synth import rng, int4_matrix, bf16_normal, cosine

pytestmark = pytest.mark.gpu

# fp32 accumulation on both sides: the GPU sums per group of 64 on MFMA, the oracle in 16 interleaved lanes.
REL_TOL = 2e-5


def run_qmm(ctx, W, xb, M, out_mode=0, y0=None):
    K = W.K
    dx = ctx.to_device(xb)
    if out_mode == 2:
        dy = ctx.buffer(M * W.N * 2)
    else:
        dy = ctx.to_device(y0.astype(np.float32)) if y0 is not None else ctx.buffer(M * W.N * 4).fill(0)
    check(lib().ih_qmm_int4(ctx.handle, W.handle, dx.ptr, K, M, dy.ptr, W.N, out_mode))
    ctx.sync()
    out = dy.download(np.uint16 if out_mode == 2 else np.float32, (M, W.N))
    dx.free()
    dy.free()
    return out


@pytest.mark.parametrize(
    "M,N,K,seed",
    [
        (8, 4096, 4096, 0),      # benchmark configuration 0
        (1, 256, 2048, 1),
        (5, 512, 4096, 2),
        (16, 1024, 1024, 3),
        (17, 6144, 4096, 4),     # config 1 qkv at k = 16
        (32, 256, 768, 5),
        (18, 512, 1024, 8),      # token 16 on VALU, tokens 17+ on the second MFMA tile
        (17, 1000, 2880, 6),     # K % 128 == 64 (config 4 hidden), N not a multiple of 16
        (17, 5120, 2880, 9),     # 23 K-blocks in one split of 8 waves × 3: the last wave's third block is past K
        (5, 32768, 2880, 10),    # the same with 4 row tiles per wave (vocabulary-sized N)
        (32, 512, 2880, 12),     # the same with two 16-token tiles (M = 32)
        (3, 4096, 14336, 7),     # down projection K
    ],
)
def test_qmm_matches_oracle(ctx, M, N, K, seed):
    g = rng(seed)
    w, s, b = int4_matrix(g, N, K)
    xb, xf = bf16_normal(g, (M, K))
    W = QMat.int4(ctx, w, s, b)
    try:
        got = run_qmm(ctx, W, xb, M)
    finally:
        W.free()
    ref = oracle.qmm_int4(xf, w, s, b)
    err = np.abs(got - ref).max()
    assert np.isfinite(got).all()
    assert err <= REL_TOL * np.abs(ref).max() + 1e-6, f"max-abs {err} vs scale {np.abs(ref).max()}"
    assert cosine(got, ref) >= 0.999999


def test_qmm_bf16_out_and_accumulate(ctx):
    g = rng(11)
    M, N, K = 8, 512, 2048
    w, s, b = int4_matrix(g, N, K)
    xb, xf = bf16_normal(g, (M, K))
    y0 = g.normal(0, 3, size=(M, N)).astype(np.float32)
    W = QMat.int4(ctx, w, s, b)
    try:
        got16 = run_qmm(ctx, W, xb, M, out_mode=2)
        gotacc = run_qmm(ctx, W, xb, M, out_mode=1, y0=y0)
    finally:
        W.free()
    ref = oracle.qmm_int4(xf, w, s, b)
    # bf16 output: within one bf16 ulp of the fp32 reference (plus the fp32 accumulation difference).
    g16 = oracle.bf16_to_f32(got16)
    assert np.all(np.abs(g16 - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-4)
    assert np.abs(gotacc - (y0 + ref)).max() <= REL_TOL * np.abs(ref).max() + 1e-5


def test_qmm_row_invariance(ctx):
    """Row r gives the same bits whatever M and whatever its neighbours (KernelCaseTests.swift:66-86)."""
    g = rng(21)
    N, K = 2048, 4096
    w, s, b = int4_matrix(g, N, K)
    xb, _ = bf16_normal(g, (17, K))
    other, _ = bf16_normal(g, (17, K))
    W = QMat.int4(ctx, w, s, b)
    try:
        full = run_qmm(ctx, W, xb, 17)
        for m in (1, 2, 8, 16):
            part = run_qmm(ctx, W, np.ascontiguousarray(xb[:m]), m)
            assert np.array_equal(part.view(np.uint32), full[:m].view(np.uint32)), f"M={m}"
        mixed = xb.copy()
        mixed[5:] = other[5:]
        got = run_qmm(ctx, W, mixed, 17)
        assert np.array_equal(got[:5].view(np.uint32), full[:5].view(np.uint32))
        # Repeated launches give the same bits (fixed split-K order).
        again = run_qmm(ctx, W, xb, 17)
        assert np.array_equal(again.view(np.uint32), full.view(np.uint32))
    finally:
        W.free()


def test_qmm_rejects_bad_shapes(ctx):
    g = rng(3)
    w, s, b = int4_matrix(g, 64, 128)
    W = QMat.int4(ctx, w, s, b)
    try:
        dx = ctx.buffer(33 * 128 * 2)
        dy = ctx.buffer(33 * 64 * 4)
        assert lib().ih_qmm_int4(ctx.handle, W.handle, dx.ptr, 128, 33, dy.ptr, 64, 0) == 1
        assert lib().ih_qmm_int4(ctx.handle, W.handle, dx.ptr, 64, 4, dy.ptr, 64, 0) == 1
        assert lib().ih_qmm_int4(ctx.handle, W.handle, dx.ptr, 128, 4, dy.ptr, 64, 7) == 1
        dx.free()
        dy.free()
    finally:
        W.free()


# Every launch shape the verify step of config 1 uses (qkv, o, gate|up, down, head) at B = 1, 8 and 17.
CFG1_SHAPES = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336), (151936, 4096)]


@pytest.mark.parametrize("N,K", CFG1_SHAPES)
def test_qmm_config1_shapes(ctx, N, K):
    g = rng(N + K)
    w, s, b = int4_matrix(g, N, K)
    xb, xf = bf16_normal(g, (17, K))
    W = QMat.int4(ctx, w, s, b)
    try:
        ref = oracle.qmm_int4(xf, w, s, b)
        full = run_qmm(ctx, W, xb, 17)
        assert np.isfinite(full).all()
        err = np.abs(full - ref).max()
        assert err <= REL_TOL * np.abs(ref).max() + 1e-6, err
        for m in (1, 8, 16):
            part = run_qmm(ctx, W, np.ascontiguousarray(xb[:m]), m)
            assert np.array_equal(part.view(np.uint32), full[:m].view(np.uint32)), m
    finally:
        W.free()
