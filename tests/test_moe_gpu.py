"""MoE pieces on the GPU against the oracle and the reference's fixtures: the MXFP4 matmul (MXFP4ReferenceTests vectors,
Tests/IngotTests/KernelCaseMXFP4.swift:142-158), the router (ref/router_vectors.json, mlx-lm 0.32.2; the engine's tie
rule, KernelCaseRouter.swift:6-12,54-80), the expert union (vmoe_route, verify.metal:262-318) and the gathered
per-expert product (MoEPipeline, Tests/IngotTests/KernelHarness.swift:630-652)."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from ingot_amd._lib import QMat, Routing
from synth import bf16_normal, int4_matrix, mxfp4_matrix, rng

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def close(got, ref, rel):
    err = np.abs(got - ref).max()
    return err <= rel * max(np.abs(ref).max(), 1e-30), err


@pytest.mark.parametrize("N,K", [(300, 2880), (256, 128), (17, 96)])
@pytest.mark.parametrize("M", [1, 9, 17])
def test_mxfp4_qmm_matches_oracle(ctx, N, K, M):
    """bf16 x (used as fp16) · MXFP4 W: only the fp32 summation order differs from the oracle."""
    g = rng(N + K + M)
    w, s = mxfp4_matrix(g, N, K)
    xb, xf = bf16_normal(g, (M, K))
    W = QMat.mxfp4(ctx, w, s)
    assert W.format == 1
    dx = ctx.to_device(xb)
    got = W.expert(dx, M)
    ref = oracle.qmm_mxfp4(xf, w, s)
    ok, err = close(got, ref, 2e-5)
    assert ok, err
    dx.free()
    W.free()


def test_mxfp4_decode_matches_reference_vectors(ctx):
    """The 128 values of MXFP4ReferenceTests (mx.dequantize(mode="mxfp4")) out of the GPU product with one-hot x."""
    fx = json.loads((GOLD / "mxfp4_reference.json").read_text())
    words = np.array(fx["words"], np.uint32).reshape(1, 16)
    scales = np.array(fx["scales"], np.uint8).reshape(1, 4)
    want = np.array(fx["values"], np.float32)
    W = QMat.mxfp4(ctx, words, scales)
    from oracle import f32_to_bf16
    got = np.zeros(128, np.float32)
    for b in range(0, 128, 16):
        x = np.zeros((16, 128), np.float32)
        x[np.arange(16), b + np.arange(16)] = 1.0
        dx = ctx.to_device(f32_to_bf16(x))
        got[b:b + 16] = W.expert(dx, 16)[:, 0]
        dx.free()
    W.free()
    assert np.array_equal(got, want)


def test_int4_expert_of_a_stack(ctx):
    g = rng(5)
    w, s, b = int4_matrix(g, 272, 512, E=4)
    W = QMat.int4(ctx, w, s, b)
    xb, xf = bf16_normal(g, (17, 512))
    dx = ctx.to_device(xb)
    for e in (0, 3):
        ok, err = close(W.expert(dx, 17, e), oracle.qmm_int4(xf, w[e], s[e], b[e]), 1e-5)
        assert ok, (e, err)
    dx.free()
    W.free()


def _route_case(ctx, logits, K, bias=None, pes=None):
    rows, E = logits.shape
    dl = ctx.to_device(np.ascontiguousarray(logits, np.float32))
    db = ctx.to_device(np.asarray(bias, np.float32)) if bias is not None else None
    dp = ctx.to_device(np.asarray(pes, np.float32)) if pes is not None else None
    R = Routing(ctx, rows, K, E).route(dl, E, db, dp)
    out = R.download()
    R.free()
    for d in (dl, db, dp):
        if d is not None:
            d.free()
    # Back to (row, slot) form.
    inds = np.zeros((rows, K), np.int32)
    wts = np.zeros((rows, K), np.float32)
    for e, start, cnt in out["entries"]:
        for p in range(start, start + cnt):
            r = out["x_row"][p]
            slot = list(out["row_pair"][r]).index(p)
            inds[r, slot] = e
            wts[r, slot] = out["pair_w"][p]
    return inds, wts, out


@pytest.mark.parametrize("name", ["gpt-oss-e32", "gpt-oss-e32-bias", "gemma4-e128-k8"])
def test_route_against_mlx_lm_vectors(ctx, name):
    """Softmax routers of ref/router_vectors.json (configs 3 and 4 are softmax top-k): expert sets and weights of rows
    2… against mlx-lm (maxRel 1e-5); rows 0–1 hold exact ties and follow the lower-index rule, brute-forced."""
    c = {x["name"]: x for x in json.loads((GOLD / "router_vectors.json").read_text())["cases"]}[name]
    E, K, R = int(c["experts"]), int(c["topK"]), int(c["rows"])
    logits = np.array(c["logits"], np.float32).reshape(R, E)
    lb = np.array(c["logitBias"], np.float32) if c.get("logitBias") is not None else None
    pes = np.array(c["perExpertScale"], np.float32) if c.get("perExpertScale") is not None else None
    inds, wts, _ = _route_case(ctx, logits, K, lb, pes)
    dense = np.zeros((R, E), np.float32)
    for r in range(R):
        dense[r, inds[r]] += wts[r]
    mlx = np.array(c["weights"], np.float32).reshape(R, E)
    assert np.array_equal(dense[2:] != 0, mlx[2:] != 0)
    assert np.abs(dense[2:] - mlx[2:]).max() <= 1e-5 * np.abs(mlx[2:]).max()
    for r in (0, 1):
        l = logits[r] + (lb if lb is not None else 0)
        assert list(inds[r]) == sorted(range(E), key=lambda e: (-l[e], e))[:K]


@pytest.mark.parametrize("rows,E,K", [(17, 128, 8), (9, 32, 4), (1, 8, 2), (32, 256, 16)])
def test_route_and_union_match_oracle(ctx, rows, E, K):
    g = rng(rows * E + K)
    logits = g.normal(0, 1, size=(rows, E)).astype(np.float32)
    logits[0, 3] = np.nan                      # NaN never wins
    logits[min(1, rows - 1), :4] = 2.5         # exact ties → lower index
    inds, wts, out = _route_case(ctx, logits, K)
    ri, rw = oracle.route(logits, K)
    assert np.array_equal(inds, ri)
    assert np.abs(wts - rw).max() <= 2e-6
    entries, pairs = oracle.expert_union(ri, E)
    assert out["U"] == len(entries)
    assert np.array_equal(out["entries"], entries)
    assert list(out["x_row"]) == list(pairs[:, 0])
    for p, (r, slot) in enumerate(pairs):
        assert out["row_pair"][r, slot] == p


@pytest.mark.parametrize("fmt", ["int4", "mxfp4"])
@pytest.mark.parametrize("rows,E,K", [(17, 32, 4), (9, 8, 2), (17, 4, 4)])
def test_gathered_product_matches_oracle(ctx, fmt, rows, E, K):
    """Every pair's row through its expert, one launch; (17, 4, 4): each expert takes all 17 rows (two token tiles)."""
    g = rng(rows + E + K + (fmt == "mxfp4"))
    N, D = 160, 384
    if fmt == "int4":
        w, s, b = int4_matrix(g, N, D, E=E)
        W = QMat.int4(ctx, w, s, b)
        ref_e = lambda x, e: oracle.qmm_int4(x, w[e], s[e], b[e])  # noqa: E731
    else:
        w, s = mxfp4_matrix(g, N, D, E=E)
        W = QMat.mxfp4(ctx, w, s)
        ref_e = lambda x, e: oracle.qmm_mxfp4(x, w[e], s[e])  # noqa: E731
    xb, xf = bf16_normal(g, (rows, D))
    logits = g.normal(0, 1, size=(rows, E)).astype(np.float32)
    dl, dx = ctx.to_device(logits), ctx.to_device(xb)
    R = Routing(ctx, rows, K, E).route(dl, E)
    y = R.gathered(W, dx)
    out = R.download()
    for e, start, cnt in out["entries"]:
        rws = out["x_row"][start:start + cnt]
        ok, err = close(y[start:start + cnt], ref_e(xf[rws], e), 2e-5)
        assert ok, (e, err)
    R.free()
    for d in (dl, dx):
        d.free()
    W.free()


@pytest.mark.parametrize("fmt,rows,E,K,N,D,umin", [
    ("int4", 17, 128, 8, 1536, 2048, 60),    # config 3's gate|up: 2·768 rows over hidden 2048
    ("int4", 17, 128, 8, 2048, 768, 60),     # config 3's down
    ("mxfp4", 9, 32, 4, 5760, 2880, 14),     # config 4's gate|up: 2·2880 rows over hidden 2880 (23 K-blocks)
    ("mxfp4", 9, 32, 4, 2880, 2880, 14),     # config 4's down
], ids=["cfg3-gate-up", "cfg3-down", "cfg4-gate-up", "cfg4-down"])
def test_gathered_product_at_config_expert_shapes(ctx, fmt, rows, E, K, N, D, umin):
    """The gathered per-expert product at configs 3 and 4's real expert shapes, under the configurations' routing
    (router logits ~N(0,1): U ≈ 85 of 128 and ≈ 22 of 32 distinct experts), every pair against the oracle's fp32
    dequant + matmul of its row through its expert (MoE.swift:346-428 gathered qmv; KernelHarness.swift:720-766)."""
    g = rng(N + D + E)
    if fmt == "int4":
        w, s, b = int4_matrix(g, N, D, E=E)
        W = QMat.int4(ctx, w, s, b)
        ref_e = lambda x, e: oracle.qmm_int4(x, w[e], s[e], b[e])  # noqa: E731
    else:
        w, s = mxfp4_matrix(g, N, D, E=E)
        W = QMat.mxfp4(ctx, w, s)
        ref_e = lambda x, e: oracle.qmm_mxfp4(x, w[e], s[e])  # noqa: E731
    xb, xf = bf16_normal(g, (rows, D))
    logits = g.normal(0, 1, size=(rows, E)).astype(np.float32)
    dl, dx = ctx.to_device(logits), ctx.to_device(xb)
    R = Routing(ctx, rows, K, E).route(dl, E)
    y = R.gathered(W, dx)
    out = R.download()
    ri, _ = oracle.route(logits, K)
    entries, _ = oracle.expert_union(ri, E)
    assert np.array_equal(out["entries"], entries)
    print(f"[gathered {fmt} {N}x{D}] U = {len(entries)} of {E}", flush=True)
    assert len(entries) >= umin
    worst = 0.0
    for e, start, cnt in out["entries"]:
        rws = out["x_row"][start:start + cnt]
        ok, err = close(y[start:start + cnt], ref_e(xf[rws], e), 2e-5)
        worst = max(worst, err)
        assert ok, (e, err)
    print(f"[gathered {fmt} {N}x{D}] worst relative error {worst:.2e}", flush=True)
    R.free()
    for d_ in (dl, dx):
        d_.free()
    W.free()
