"""Writes a small mlx-lm-format checkpoint (config.json + model.safetensors, optionally sharded) whose tensors are the
synthetic model's (the same SplitMix64 streams the library's synthetic generator and the oracle use), so a model loaded
from it must give bit-identical results to ih_model_create_synthetic with the same seed.

Layout of an mlx-lm quantized pack: separate q/k/v and gate/up projections (weight u32 [out, in/8], scales and biases
bf16 [out, in/64]), model.layers.N.{input,post_attention}_layernorm.weight, model.embed_tokens.*, model.norm.weight,
lm_head.*; MoE: mlp.gate (router) and mlp.switch_mlp.{gate,up,down}_proj stacked over experts; MXFP4 experts with
uint8 e8m0 scales and no biases, the other layers named in the quantization dict as affine 4-bit g64.

gpt-oss packs (family="gpt_oss") name the router mlp.router and the experts mlp.experts.*, carry the router's and
the experts' biases, q|k|v|o biases and self_attn.sinks, and declare swiglu_limit, alternating layer_types and YaRN.
The header can be written with an odd length (pad), as the reference's FormatTests and real packs have it, so that
every tensor starts at an unaligned offset.

Usage: python tests/golden/make_mlx_checkpoint.py OUT_DIR [--moe|--moe-mxfp4|--qwen] [--shards N]
(the tests call write_checkpoint() directly).
"""
from __future__ import annotations

import argparse
import json
import struct
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402  (the synthetic streams; test infrastructure)

W_SD = 0.02


def layer_tensor(l: int, kind: int) -> int:
    return 1000 + 100 * l + kind


def expert_tensor(l: int, kind: int, e: int) -> int:
    return 3000000 + 10000 * l + 1000 * kind + e


def bf16_vec(seed, tensor, n, base, amp) -> np.ndarray:
    out = np.empty(n, np.uint16)
    oracle.lib().or_synth_bf16(seed, tensor, n, base, amp, out.ctypes.data)
    return out


def f32_vec(seed, tensor, n, base, amp) -> np.ndarray:
    out = np.empty(n, np.float32)
    oracle.lib().or_synth_f32(seed, tensor, n, base, amp, out.ctypes.data)
    return out


def mxfp4_mat(seed, tensor, N, K):
    w = np.empty((N, K // 8), np.uint32)
    s = np.empty((N, K // 32), np.uint8)
    oracle.lib().or_synth_mxfp4(seed, tensor, N, K, w.ctypes.data, s.ctypes.data)
    return w, s


def pack_nibbles(q) -> np.ndarray:
    """Codes 0..15 [..., K] → uint32 [..., K/8], element j in bits 4j..4j+3 (MLX: low nibble first)."""
    q = np.asarray(q, np.uint32).reshape(*np.shape(q)[:-1], -1, 8)
    return np.bitwise_or.reduce(q << (4 * np.arange(8, dtype=np.uint32)), axis=-1).astype(np.uint32)


def write_safetensors(path: Path, tensors: dict, pad=None) -> None:
    """tensors: name → (dtype string, numpy array); little-endian u64 header length, JSON header, raw data. pad=None
    pads the header to 8 bytes; pad=p pads it so that (8 + length) % 4 == p (FormatTests.writeSafetensors: p = 3
    leaves every tensor misaligned)."""
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        dt, a = tensors[name]
        a = np.ascontiguousarray(a)
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    h = json.dumps(header).encode()
    if pad is None:
        h += b" " * ((8 - len(h) % 8) % 8)
    else:
        while (8 + len(h)) % 4 != pad:
            h += b" "
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def write_checkpoint(out: Path, desc: dict, seed: int, shards: int = 1, tied: bool = False, extra_config=None,
                     family: str = "", pad=None) -> Path:
    """desc: the ih_model_desc fields (n_layers, hidden, n_q_heads, n_kv_heads, head_dim, intermediate, vocab, …)."""
    out = Path(out)
    out.mkdir(parents=True, exist_ok=True)
    d = dict(desc)
    L, H, QH, KVH, HD, V = d["n_layers"], d["hidden"], d["n_q_heads"], d["n_kv_heads"], d["head_dim"], d["vocab"]
    E, K, IE, fmt = d.get("n_experts", 0), d.get("top_k", 0), d.get("expert_intermediate", 0), d.get("expert_format", 0)
    QS = HD * (2 if d.get("attn_gate") else 1)  # a gated q head is [q | gate]
    QP = QH * QS + 2 * KVH * HD
    gpt = family == "gpt_oss"
    router_name, experts_name = ("mlp.router", "mlp.experts.") if gpt else ("mlp.gate", "mlp.switch_mlp.")
    t = {}
    overrides = {}

    def q4(name, tensor, N, Kd, rows=None):
        w, s, b = oracle.synth_int4(seed, tensor, N, Kd, W_SD)
        if rows is not None:
            w, s, b = w[rows], s[rows], b[rows]
        t[name + ".weight"] = ("U32", w)
        t[name + ".scales"] = ("BF16", s)
        t[name + ".biases"] = ("BF16", b)
        if fmt == 1:
            overrides[name] = {"group_size": 64, "bits": 4}

    q4("model.embed_tokens", 1, V, H)
    t["model.norm.weight"] = ("BF16", bf16_vec(seed, 2, H, 1.0, 0.125))
    if not tied:
        q4("lm_head", 3, V, H)
    for l in range(L):
        p = f"model.layers.{l}."
        t[p + "input_layernorm.weight"] = ("BF16", bf16_vec(seed, layer_tensor(l, 0), H, 1.0, 0.125))
        t[p + "post_attention_layernorm.weight"] = ("BF16", bf16_vec(seed, layer_tensor(l, 3), H, 1.0, 0.125))
        q4(p + "self_attn.q_proj", layer_tensor(l, 1), QP, H, slice(0, QH * QS))
        q4(p + "self_attn.k_proj", layer_tensor(l, 1), QP, H, slice(QH * QS, QH * QS + KVH * HD))
        q4(p + "self_attn.v_proj", layer_tensor(l, 1), QP, H, slice(QH * QS + KVH * HD, QP))
        q4(p + "self_attn.o_proj", layer_tensor(l, 2), H, QH * HD)
        if d.get("o_bias"):
            t[p + "self_attn.o_proj.bias"] = ("F32", f32_vec(seed, layer_tensor(l, 14), H, 0.0, 0.1))
        if d.get("sinks"):
            t[p + "self_attn.sinks"] = ("F32", f32_vec(seed, layer_tensor(l, 9), QH, 0.0, 1.0))
        if d.get("qk_norm"):
            t[p + "self_attn.q_norm.weight"] = ("BF16", bf16_vec(seed, layer_tensor(l, 10), HD, 1.0, 0.125))
            t[p + "self_attn.k_norm.weight"] = ("BF16", bf16_vec(seed, layer_tensor(l, 11), HD, 1.0, 0.125))
        if d.get("qkv_bias"):
            b = f32_vec(seed, layer_tensor(l, 12), QP, 0.0, 0.1)
            t[p + "self_attn.q_proj.bias"] = ("F32", b[: QH * QS])
            t[p + "self_attn.k_proj.bias"] = ("F32", b[QH * QS: QH * QS + KVH * HD])
            t[p + "self_attn.v_proj.bias"] = ("F32", b[QH * QS + KVH * HD:])
        if not E:
            I = d["intermediate"]
            q4(p + "mlp.gate_proj", layer_tensor(l, 4), 2 * I, H, slice(0, I))
            q4(p + "mlp.up_proj", layer_tensor(l, 4), 2 * I, H, slice(I, 2 * I))
            q4(p + "mlp.down_proj", layer_tensor(l, 5), H, I)
            continue
        xp = p + experts_name
        if fmt == 0 or d.get("router_int4"):
            q4(p + router_name, layer_tensor(l, 6), E, H)
        else:
            w, s = mxfp4_mat(seed, layer_tensor(l, 6), E, H)
            t[p + router_name + ".weight"], t[p + router_name + ".scales"] = ("U32", w), ("U8", s)
        if fmt == 0:
            gu = [oracle.synth_int4(seed, expert_tensor(l, 0, e), 2 * IE, H, W_SD) for e in range(E)]
            dn = [oracle.synth_int4(seed, expert_tensor(l, 1, e), H, IE, W_SD) for e in range(E)]
            for j, nm in enumerate(("weight", "scales", "biases")):
                dt = "U32" if j == 0 else "BF16"
                t[xp + f"gate_proj.{nm}"] = (dt, np.stack([x[j][:IE] for x in gu]))
                t[xp + f"up_proj.{nm}"] = (dt, np.stack([x[j][IE:] for x in gu]))
                t[xp + f"down_proj.{nm}"] = (dt, np.stack([x[j] for x in dn]))
        else:
            gu = [mxfp4_mat(seed, expert_tensor(l, 0, e), 2 * IE, H) for e in range(E)]
            dn = [mxfp4_mat(seed, expert_tensor(l, 1, e), H, IE) for e in range(E)]
            for j, nm in enumerate(("weight", "scales")):
                dt = "U32" if j == 0 else "U8"
                t[xp + f"gate_proj.{nm}"] = (dt, np.stack([x[j][:IE] for x in gu]))
                t[xp + f"up_proj.{nm}"] = (dt, np.stack([x[j][IE:] for x in gu]))
                t[xp + f"down_proj.{nm}"] = (dt, np.stack([x[j] for x in dn]))
        if d.get("router_bias"):
            t[p + router_name + ".bias"] = ("F32", f32_vec(seed, layer_tensor(l, 7), E, 0.0, 0.5))
        if d.get("expert_bias"):
            gub = np.stack([bf16_vec(seed, expert_tensor(l, 2, e), 2 * IE, 0.0, 0.1) for e in range(E)])
            t[xp + "gate_proj.bias"] = ("BF16", gub[:, :IE])
            t[xp + "up_proj.bias"] = ("BF16", gub[:, IE:])
            t[xp + "down_proj.bias"] = ("BF16", np.stack([bf16_vec(seed, expert_tensor(l, 3, e), H, 0.0, 0.1)
                                                          for e in range(E)]))
    cfg = {"model_type": "gpt_oss" if gpt else "qwen3_moe" if E else ("qwen3" if d.get("qk_norm") else "llama"),
           "hidden_size": H, "num_hidden_layers": L, "num_attention_heads": QH, "num_key_value_heads": KVH,
           "head_dim": HD, "vocab_size": V, "rope_theta": d.get("rope_theta", 1e6), "rms_norm_eps": d.get("rms_eps", 1e-6),
           "tie_word_embeddings": tied}
    if gpt:
        cfg.update(num_local_experts=E, experts_per_token=K, num_experts_per_tok=K, intermediate_size=IE,
                   swiglu_limit=d.get("swiglu_limit", 7.0), attention_bias=bool(d.get("qkv_bias") and d.get("o_bias")),
                   layer_types=["sliding_attention" if i % 2 == 0 else "full_attention" for i in range(L)],
                   sliding_window=d.get("sliding_window", 128))
    elif E:
        cfg.update(num_experts=E, num_experts_per_tok=K, moe_intermediate_size=IE, norm_topk_prob=True)
    else:
        cfg["intermediate_size"] = d["intermediate"]
    if d.get("rotary_dims"):
        cfg["partial_rotary_factor"] = d["rotary_dims"] / HD
    if d.get("rope_type"):
        kinds = {1: "linear", 2: "yarn", 3: "proportional"}
        rs = {"rope_type": kinds[d["rope_type"]], "factor": d.get("rope_factor", 1.0)}
        if d["rope_type"] == 2:
            rs.update(original_max_position_embeddings=d["rope_orig_max"], beta_fast=d.get("rope_beta_fast") or 32.0,
                      beta_slow=d.get("rope_beta_slow") or 1.0, truncate=not d.get("rope_no_truncate", 0))
        if d["rope_type"] == 3:
            rs["partial_rotary_factor"] = d.get("rope_partial", 1.0)
        cfg["rope_scaling"] = rs
    cfg["quantization"] = {"group_size": 64, "bits": 4} if fmt == 0 else {"group_size": 32, "bits": 4, "mode": "mxfp4",
                                                                         **overrides}
    cfg.update(extra_config or {})
    (out / "config.json").write_text(json.dumps(cfg, indent=1))
    names = sorted(t)
    if shards <= 1:
        write_safetensors(out / "model.safetensors", t, pad)
    else:
        wm = {}
        for i in range(shards):
            part = {n: t[n] for n in names[i::shards]}
            fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            write_safetensors(out / fn, part, pad)
            wm.update({n: fn for n in part})
        (out / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("out")
    ap.add_argument("--shards", type=int, default=1)
    ap.add_argument("--seed", type=int, default=7)
    g = ap.add_mutually_exclusive_group()
    g.add_argument("--moe", action="store_true")
    g.add_argument("--moe-mxfp4", action="store_true")
    g.add_argument("--qwen", action="store_true")
    a = ap.parse_args()
    base = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, vocab=1000)
    if a.moe or a.moe_mxfp4:
        base.update(intermediate=0, n_experts=8, top_k=2, expert_intermediate=128, expert_format=int(a.moe_mxfp4))
    if a.qwen:
        base.update(qk_norm=1, qkv_bias=1)
    write_checkpoint(Path(a.out), base, a.seed, a.shards)
