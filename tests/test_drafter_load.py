"""Trained DFlash2 drafter checkpoints (ih_drafter_load_mlx) and the load-time quantization of their bf16 projections
(ih_quantize_int4_g64).

Reference: DFlash2Drafter.init (Sources/Ingot/Drafter.swift:114-256: bf16 weights quantized to 4 bits at load, names
and config), DenseQ.quantizeAffine (Sources/Ingot/Layers/Linear.swift:592-628). The quantizer is checked on the CPU
against a restatement of that text and against what affine quantization must satisfy; the GPU tests load checkpoints
written from the synthetic drafter's streams (tests/golden/make_drafter_checkpoint.py) and require drafts and
confidences bit-identical to the synthetic drafter (int4 files), and bf16 files to load exactly as the restated
quantizer's int4 output of the same weights.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from ingot_amd._lib import Drafter, DrafterDesc, KVCache, Model, ModelDesc, quantize_int4_g64

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
from make_drafter_checkpoint import write_drafter  # noqa: E402


def quantize_ref(wb: np.ndarray):
    """quantizeAffine restated (Linear.swift:592-628): per row and group of 64, sb = bf16((max − min)/15),
    bb = bf16(min), q = round((v − bias)/scale) half away from zero, clamped to 0…15, 0 where the scale is 0."""
    N, K = wb.shape
    v = oracle.bf16_to_f32(wb).reshape(N, K // 64, 64)
    mn, mx = v.min(axis=2), v.max(axis=2)
    sb = oracle.f32_to_bf16(((mx - mn) / np.float32(15)).astype(np.float32))
    bb = oracle.f32_to_bf16(mn.astype(np.float32))
    sc, bi = oracle.bf16_to_f32(sb)[..., None], oracle.bf16_to_f32(bb)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        x = ((v - bi) / sc).astype(np.float32)
    q = np.where(sc > 0, np.clip(np.sign(x) * np.floor(np.abs(x) + np.float32(0.5)), 0, 15), 0).astype(np.uint32)
    q = q.reshape(N, K // 8, 8)
    w = np.bitwise_or.reduce(q << (4 * np.arange(8, dtype=np.uint32)), axis=2).astype(np.uint32)
    return w, sb, bb


def dequant(w, s, b):
    sh = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    q = ((w[:, :, None] >> sh) & 15).reshape(w.shape[0], -1).astype(np.float64)
    return q * np.repeat(oracle.bf16_to_f32(s), 64, axis=1) + np.repeat(oracle.bf16_to_f32(b), 64, axis=1)


def test_quantize_int4_g64_matches_the_restated_quantizer():
    g = np.random.default_rng(1)
    wb = oracle.f32_to_bf16(g.normal(0, 0.05, size=(24, 256)).astype(np.float32))
    wb[0, :64] = oracle.f32_to_bf16(np.full(64, 0.37, np.float32))      # constant group: scale 0, codes 0
    wb[1, 64:128] = oracle.f32_to_bf16(np.float32(-1.0) * np.ones(64, np.float32))
    wb[2, :64] = oracle.f32_to_bf16((np.arange(64) % 16 * 0.25 - 2).astype(np.float32))  # exactly on a 16-level grid
    wb[3, :64] = oracle.f32_to_bf16(np.linspace(-1, 1, 64).astype(np.float32))  # ties at half levels
    got = quantize_int4_g64(wb)
    want = quantize_ref(wb)
    for x, y in zip(got, want):
        assert np.array_equal(x, y)
    w, s, b = got
    # Closed forms: a constant group dequantizes to its value's bf16 bias with scale 0; a group on a 16-level grid
    # with bf16-exact levels comes back exactly; every weight is within half a step (plus the bias's bf16 rounding).
    assert oracle.bf16_to_f32(s[0, 0]) == 0 and np.all(((w[0, :8, None] >> (4 * np.arange(8))) & 15) == 0)
    v = oracle.bf16_to_f32(wb).astype(np.float64)
    r = dequant(w, s, b)
    assert np.array_equal(r[2, :64], v[2, :64])
    step = np.repeat(oracle.bf16_to_f32(s), 64, axis=1)
    bias_err = np.repeat(np.abs(oracle.bf16_to_f32(b) - v.reshape(24, 4, 64).min(axis=2)), 64, axis=1)
    assert np.all(np.abs(r - v) <= step / 2 + bias_err + 1e-6 + 16 * step * 2 ** -8)


SMALL = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, vocab=1000)
DF2 = dict(n_layers=2, hidden=256, n_q_heads=8, head_dim=64, intermediate=256, block=8, window=32, rank=64,
           dyn_conv=1, mask_token=999)


def _drafts(model, kv, dr, toks):
    """Three context writes of the verify step's own captures, then blocks at two anchors."""
    dr.attach()
    kv.verify(toks)
    out = []
    for pos0 in (0, 17, 34):
        dr.context(17, 17, pos0)
    for anchor, P in ((int(toks[3]), 51), (17, 51), (int(toks[9]), 40)):
        out.append(dr.block(anchor, P))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int4", "bf16"])
def test_loaded_drafter_drafts_like_its_weights(ctx, tmp_path, fmt):
    """int4 file: the same drafts and confidences (bit-exact) as the synthetic drafter with the same seed. bf16 file:
    quantized at load, the same as loading the restated quantizer's int4 output of those bf16 weights."""
    d = ModelDesc.make(**SMALL)
    m = Model(ctx, d, 7)
    kv = KVCache(m, 512)
    spec = dict(DF2, targets=(0, 1))
    toks = np.random.default_rng(4).integers(0, d.vocab, size=17).astype(np.uint32)
    if fmt == "int4":
        path = write_drafter(tmp_path / "dr", spec, SMALL["hidden"], SMALL["vocab"], seed=5, fmt="int4")
        ref = Drafter(m, DrafterDesc.make(targets=(0, 1), **DF2), 5)
    else:
        path = write_drafter(tmp_path / "dr", spec, SMALL["hidden"], SMALL["vocab"], seed=5, fmt="bf16")
        qpath = write_drafter(tmp_path / "q", spec, SMALL["hidden"], SMALL["vocab"], seed=5, fmt="bf16",
                              quantizer=quantize_ref)
        ref = Drafter.load_mlx(m, qpath)
    dr = Drafter.load_mlx(m, path)
    try:
        for k in ("n_layers", "hidden", "n_q_heads", "head_dim", "intermediate", "block", "window", "rank",
                  "dyn_conv", "mask_token", "n_targets"):
            assert getattr(dr.desc, k) == getattr(ref.desc, k), k
        kv.fill_synthetic(100, 11)
        got = _drafts(m, kv, dr, toks)
        kv.set_pos(100)
        want = _drafts(m, kv, ref, toks)
        for (gd, gc), (wd, wc) in zip(got, want):
            assert list(gd) == list(wd)
            assert np.array_equal(gc.view(np.uint32), wc.view(np.uint32))
    finally:
        dr.free()
        ref.free()
        kv.free()
        m.free()


@pytest.mark.gpu
def test_drafter_load_refuses_what_it_cannot_run(ctx, tmp_path):
    import json
    from ingot_amd._lib import IngotError
    d = ModelDesc.make(**SMALL)
    m = Model(ctx, d, 7)
    try:
        spec = dict(DF2, targets=(0, 1))
        p = write_drafter(tmp_path / "a", spec, SMALL["hidden"], SMALL["vocab"], seed=5)
        cfg = json.loads((p / "config.json").read_text())
        for edit, word in (({"attention_bias": True}, "biases"), ({"num_key_value_heads": 4}, "8 KV heads"),
                           ({"rope_scaling": {"rope_type": "yarn", "factor": 4.0}}, "RoPE"),
                           ({"hidden_size": 512}, "hidden")):
            (p / "config.json").write_text(json.dumps({**cfg, **edit}))
            with pytest.raises(IngotError) as e:
                Drafter.load_mlx(m, p)
            assert word in str(e.value), str(e.value)
    finally:
        m.free()
