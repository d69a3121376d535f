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

import oracle
import pytest

from ingot_amd._lib import IngotError, KVCache, Model, ModelDesc, describe_mlx

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
from make_mlx_checkpoint import pack_nibbles, write_checkpoint  # noqa: E402

DENSE = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, vocab=1000)
QWEN = dict(DENSE, qk_norm=1, qkv_bias=1)
MOE = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=0, vocab=1000, n_experts=8,
           top_k=2, expert_intermediate=128, expert_format=0)
MOEX = dict(MOE, expert_format=1, hidden=192, n_q_heads=8, head_dim=64, expert_intermediate=96)
# gpt-oss's layout at a small size: mlp.router (int4, with bias) in front of MXFP4 experts with biases, q|k|v|o biases,
# sinks, alternating 16-key window, swiglu_oai and its YaRN (ModelSpec.swift:27-33; GptOssSpecTests.swift:36-76).
GPTOSS = dict(MOEX, qkv_bias=1, o_bias=1, sinks=1, sliding_window=16, act=1, router_bias=1, expert_bias=1,
              router_int4=1, rope_type=2, rope_factor=32.0, rope_orig_max=4096.0, rope_no_truncate=1,
              rope_theta=150000.0)
# Qwen3-Next attention: [q | gate] q_proj rows per head, partial RoPE (partial_rotary_factor 0.25), QK-norm.
GATED = dict(DENSE, attn_gate=1, rotary_dims=32, qk_norm=1)
# Linear and proportional RoPE scaling.
LINEAR = dict(DENSE, rope_type=1, rope_factor=4.0)
PROP = dict(DENSE, rope_type=3, rope_factor=1.0, rope_partial=0.25)
FAMILY = {id(GPTOSS): "gpt_oss"}


def fields(d: ModelDesc) -> dict:
    return d.as_dict()


@pytest.mark.parametrize("shape,shards", [(DENSE, 1), (QWEN, 3), (MOE, 2), (MOEX, 1), (GPTOSS, 2), (GATED, 1),
                                          (LINEAR, 1), (PROP, 1)],
                         ids=["dense", "qwen-sharded", "moe-int4", "moe-mxfp4", "gpt-oss", "gated-partial-rope",
                              "rope-linear", "rope-proportional"])
def test_describe(tmp_path, shape, shards):
    write_checkpoint(tmp_path, shape, seed=7, shards=shards, family=FAMILY.get(id(shape), ""))
    got = fields(describe_mlx(tmp_path))
    want = fields(ModelDesc.make(**shape))
    for k in ("n_layers", "hidden", "n_q_heads", "n_kv_heads", "head_dim", "intermediate", "vocab", "n_experts",
              "top_k", "expert_intermediate", "expert_format", "qk_norm", "qkv_bias", "hadamard_k", "o_bias", "sinks",
              "sliding_window", "act", "router_bias", "expert_bias", "router_int4", "attn_gate", "rotary_dims",
              "rope_type", "rope_no_truncate"):
        assert got[k] == want[k], k
    for k in ("rope_theta", "rope_factor", "rope_orig_max", "rope_partial"):
        assert got[k] == pytest.approx(want[k]), k
    assert got["rms_eps"] == pytest.approx(1e-6)


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
    # Rope scaling other than default / linear / yarn / proportional (RopeTableTests.unsupportedTypesThrow,
    # Tests/IngotTests/RopeTableTests.swift:61-74), and the malformed ones of the kinds that run.
    for i, (rs, words) in enumerate([({"rope_type": "llama3", "factor": 8.0}, ["rope_scaling", "llama3"]),
                                     ({"rope_type": "dynamic", "factor": 2.0}, ["dynamic"]),
                                     ({"rope_type": "longrope", "short_factor": [1.0]}, ["longrope"]),
                                     ({"rope_type": "yarn", "factor": 4.0}, ["original_max_position_embeddings"]),
                                     ({"rope_type": "yarn", "factor": 40.0, "original_max_position_embeddings": 4096,
                                       "mscale_all_dim": 1.0}, ["mscale_all_dim"]),
                                     ({"rope_type": "linear"}, ["factor"]),
                                     ({"rope_type": "proportional", "partial_rotary_factor": 1.5}, ["proportional"])]):
        q = write_checkpoint(tmp_path / f"b{i}", DENSE, seed=7, extra_config={"rope_scaling": rs})
        expect_error(q, *words)
    # A partial RoPE that does not give an even number of dims.
    q = write_checkpoint(tmp_path / "b9", DENSE, seed=7, extra_config={"partial_rotary_factor": 0.3})
    expect_error(q, "partial_rotary_factor")
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
@pytest.mark.parametrize("shape,shards,pad", [(DENSE, 1, None), (QWEN, 3, None), (MOE, 2, None), (MOEX, 1, None),
                                              (DENSE, 1, 3), (MOEX, 2, 1), (GPTOSS, 1, 3), (GATED, 1, None),
                                              (LINEAR, 1, None), (PROP, 1, 3)],
                         ids=["dense", "qwen-sharded", "moe-int4", "moe-mxfp4", "dense-misaligned",
                              "moe-mxfp4-misaligned", "gpt-oss-misaligned", "gated-partial-rope", "rope-linear",
                              "rope-proportional-misaligned"])
def test_loaded_model_equals_synthetic(ctx, tmp_path, shape, shards, pad):
    """A checkpoint written from the synthetic streams loads into the same model: logits bit-identical to
    ih_model_create_synthetic's. pad = 1 or 3 writes odd-length headers (every tensor at an unaligned offset, like
    the real packs and FormatTests.safetensorsQuantizedLayer, Tests/IngotTests/FormatTests.swift:33-69)."""
    write_checkpoint(tmp_path, shape, seed=7, shards=shards, family=FAMILY.get(id(shape), ""), pad=pad)
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
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        assert np.array_equal(ta, tb)
    finally:
        for x in (kv_a, kv_b, loaded, syn):
            x.free()


@pytest.mark.gpu
def test_tied_head_is_the_embedding(ctx, tmp_path):
    """tie_word_embeddings: the head is the embedding table. The tied checkpoint's logits match the oracle with its
    head replaced by the embedding (within the dense tolerance, top-1 equal outside near ties), and the same checkpoint
    with lm_head written as an explicit copy of embed_tokens loads into bit-identical logits."""
    write_checkpoint(tmp_path / "tied", DENSE, seed=7, tied=True)
    untied = write_checkpoint(tmp_path / "copy", DENSE, seed=7, tied=False)
    raw = (untied / "model.safetensors").read_bytes()
    import struct
    n = struct.unpack("<Q", raw[:8])[0]
    head = json.loads(raw[8:8 + n])
    body = bytearray(raw[8 + n:])
    for part in ("weight", "scales", "biases"):
        e0, e1 = head["model.embed_tokens." + part]["data_offsets"]
        h0, h1 = head["lm_head." + part]["data_offsets"]
        assert e1 - e0 == h1 - h0
        body[h0:h1] = body[e0:e1]
    (untied / "model.safetensors").write_bytes(raw[:8 + n] + bytes(body))
    a = Model.load_mlx(ctx, tmp_path / "tied")
    b = Model.load_mlx(ctx, untied)
    c = Model(ctx, ModelDesc.make(**DENSE), 7)
    kvs = [KVCache(x, 256) for x in (a, b, c)]
    try:
        for kv in kvs:
            kv.fill_synthetic(100, 11)
        toks = np.random.default_rng(4).integers(0, DENSE["vocab"], size=9).astype(np.uint32)
        la, lb, lc = (kv.verify(toks, want_logits=True)[1] for kv in kvs)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        assert not np.array_equal(la, lc)
        # Tolerance: 2.5 × how far the oracle moves when its attention rounds p·vs to fp16 as the reference and the
        # GPU do (measured 0.059 here, GPU error 0.129); the untied synthetic model shows the same ratio (0.053, 0.090).
        om = oracle.OracleModel(ModelDesc.make(**DENSE), 7, 11, 100)
        om.tie_head()
        ol, ot = om.verify(toks)
        with oracle.attn_p16():
            ol16, _ = om.verify(toks)
        om.free()
        err = float(np.abs(la - ol).max())
        spread = float(np.abs(ol16 - ol).max())
        assert err <= max(0.02, 2.5 * spread), (err, spread)
        srt = np.sort(ol, axis=1)
        sure = (srt[:, -1] - srt[:, -2]) > 2 * err
        assert np.array_equal(np.argmax(la, axis=1)[sure], ot[sure])
    finally:
        for x in kvs + [a, b, c]:
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


def test_nibble_order_and_misaligned_header(tmp_path):
    """FormatTests.safetensorsQuantizedLayer (Tests/IngotTests/FormatTests.swift:33-69): MLX packs element j of a word
    in bits 4j..4j+3 (packQ([1…8]) = 0x87654321), and a header of odd length leaves the tensors unaligned; the
    description still reads."""
    assert pack_nibbles([1, 2, 3, 4, 5, 6, 7, 8]).tolist() == [0x87654321]
    q = np.array([(j * 7 + 3) % 16 for j in range(256)], np.uint32).reshape(2, 128)
    w = pack_nibbles(q)
    assert all(((int(w[r, j // 8]) >> (4 * (j % 8))) & 15) == q[r, j] for r in range(2) for j in range(128))
    import struct
    p = write_checkpoint(tmp_path, DENSE, seed=7, pad=3)
    raw = (p / "model.safetensors").read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    assert (8 + n) % 4 == 3
    assert fields(describe_mlx(p))["hidden"] == DENSE["hidden"]


def test_describe_rejects_mismatched_scales(tmp_path):
    """A quantized layer's scales and biases must have the weight's leading dims (out rows, experts) and the same
    shape as each other; a header that disagrees is refused, naming the tensor, before any upload sizes a copy by it."""
    import struct
    for i, (name, shape) in enumerate([("model.layers.0.self_attn.o_proj.scales", [128, 4]),
                                       ("model.layers.0.mlp.down_proj.biases", [256, 4])]):
        p = write_checkpoint(tmp_path / str(i), DENSE, seed=7)
        f = p / "model.safetensors"
        raw = f.read_bytes()
        n = struct.unpack("<Q", raw[:8])[0]
        head = json.loads(raw[8:8 + n])
        o0, _ = head[name]["data_offsets"]
        head[name]["shape"] = shape
        head[name]["data_offsets"] = [o0, o0 + 2 * shape[0] * shape[1]]
        h = json.dumps(head).encode()
        h += b" " * ((8 - len(h) % 8) % 8)
        f.write_bytes(struct.pack("<Q", len(h)) + h + raw[8 + n:])
        expect_error(p, name.rsplit(".", 1)[0], "does not match")


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
