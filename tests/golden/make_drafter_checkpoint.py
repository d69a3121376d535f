"""Writes a small DFlash2 (or DFlash v1) drafter checkpoint directory whose tensors are the synthetic drafter's (the
same SplitMix64 streams as ih_drafter_create_synthetic and oracle.OracleDrafter), in the layout DFlash2Drafter reads
(Sources/Ingot/Drafter.swift:114-256): config.json with dflash_config, layers.N.* without a model prefix, fc,
hidden_norm, norm, {attention,mlp}_conv.{kernel_projection,base_kernel} and candidate_selector.*.

fmt="int4": projections as MLX int4 g64 (weight/scales/biases), exactly the synthetic drafter's, so a drafter loaded
from it must draft bit-identically. fmt="bf16": projections as bf16 (the synthetic weights dequantized and rounded to
bf16), which the loader quantizes itself; with quantizer=f, the same bf16 matrices quantized by f written as int4
instead (the expected result of that quantization).
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
from make_mlx_checkpoint import bf16_vec, write_safetensors  # noqa: E402

import oracle  # noqa: E402  (the synthetic streams; test infrastructure)

KVH = 8
D_N1, D_N2, D_QN, D_KN, D_QKV, D_O, D_GU, D_DOWN, D_APROJ, D_MPROJ, D_ABASE, D_MBASE = range(12)
D_FC, D_HNORM, D_FNORM, D_HPROJ, D_PRED, D_SUCC = 1, 2, 3, 4, 5, 6


def dl_tensor(l, kind):
    return 7000000 + 1000 * l + kind


def dg_tensor(kind):
    return 7900000 + kind


def dequant_bf16(w, s, b) -> np.ndarray:
    """bf16 bits of s·q + b (fp32, rounded to nearest even)."""
    sh = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    q = ((w[:, :, None] >> sh) & 15).reshape(w.shape[0], -1).astype(np.float32)
    sc = np.repeat(oracle.bf16_to_f32(s), 64, axis=1)
    bi = np.repeat(oracle.bf16_to_f32(b), 64, axis=1)
    return oracle.f32_to_bf16((sc * q + bi).astype(np.float32))


def write_drafter(out: Path, desc: dict, target_hidden: int, vocab: int, seed: int, fmt: str = "int4",
                  quantizer=None) -> Path:
    """desc: n_layers, hidden, n_q_heads, head_dim, intermediate, block, window, rank, dyn_conv, mask_token,
    targets (the target layer ids)."""
    out = Path(out)
    out.mkdir(parents=True, exist_ok=True)
    L, H, QH, HD, I = desc["n_layers"], desc["hidden"], desc["n_q_heads"], desc["head_dim"], desc["intermediate"]
    rank, conv, targets = desc.get("rank", 0), desc.get("dyn_conv", 0), list(desc["targets"])
    QP, DYN = (QH + 2 * KVH) * HD, 4 * (H // 16)
    t = {}

    def mat(name, tensor, N, K, rows=None):
        w, s, b = oracle.synth_int4(seed, tensor, N, K, 0.02)
        if rows is not None:
            w, s, b = w[rows], s[rows], b[rows]
        if fmt == "int4":
            t[name + ".weight"], t[name + ".scales"], t[name + ".biases"] = ("U32", w), ("BF16", s), ("BF16", b)
            return
        wb = dequant_bf16(w, s, b)
        if quantizer is None:
            t[name + ".weight"] = ("BF16", wb)
        else:
            qw, qs, qb = quantizer(wb)
            t[name + ".weight"], t[name + ".scales"], t[name + ".biases"] = ("U32", qw), ("BF16", qs), ("BF16", qb)

    for l in range(L):
        p, a = f"layers.{l}.", f"layers.{l}.self_attn."
        t[p + "input_layernorm.weight"] = ("BF16", bf16_vec(seed, dl_tensor(l, D_N1), H, 1.0, 0.125))
        t[p + "post_attention_layernorm.weight"] = ("BF16", bf16_vec(seed, dl_tensor(l, D_N2), H, 1.0, 0.125))
        t[a + "q_norm.weight"] = ("BF16", bf16_vec(seed, dl_tensor(l, D_QN), HD, 1.0, 0.125))
        t[a + "k_norm.weight"] = ("BF16", bf16_vec(seed, dl_tensor(l, D_KN), HD, 1.0, 0.125))
        mat(a + "q_proj", dl_tensor(l, D_QKV), QP, H, slice(0, QH * HD))
        mat(a + "k_proj", dl_tensor(l, D_QKV), QP, H, slice(QH * HD, (QH + KVH) * HD))
        mat(a + "v_proj", dl_tensor(l, D_QKV), QP, H, slice((QH + KVH) * HD, QP))
        mat(a + "o_proj", dl_tensor(l, D_O), H, QH * HD)
        mat(p + "mlp.gate_proj", dl_tensor(l, D_GU), 2 * I, H, slice(0, I))
        mat(p + "mlp.up_proj", dl_tensor(l, D_GU), 2 * I, H, slice(I, 2 * I))
        mat(p + "mlp.down_proj", dl_tensor(l, D_DOWN), H, I)
        if conv:
            mat(p + "attention_conv.kernel_projection", dl_tensor(l, D_APROJ), DYN, H)
            mat(p + "mlp_conv.kernel_projection", dl_tensor(l, D_MPROJ), DYN, H)
            for nm, kind in (("attention_conv", D_ABASE), ("mlp_conv", D_MBASE)):
                base = np.stack([bf16_vec(seed, dl_tensor(l, kind) + 100 * k, H, 0.0 if k % 2 else 1.0, 0.1)
                                 for k in range(4)]).reshape(2, 2, H)
                t[p + nm + ".base_kernel"] = ("BF16", base)
    mat("fc", dg_tensor(D_FC), H, len(targets) * target_hidden)
    t["hidden_norm.weight"] = ("BF16", bf16_vec(seed, dg_tensor(D_HNORM), H, 1.0, 0.125))
    t["norm.weight"] = ("BF16", bf16_vec(seed, dg_tensor(D_FNORM), H, 1.0, 0.125))
    if rank:
        mat("candidate_selector.hidden_projection", dg_tensor(D_HPROJ), rank, H)
        t["candidate_selector.predecessor_codebook.weight"] = (
            "BF16", bf16_vec(seed, dg_tensor(D_PRED), vocab * rank, 0.0, 0.25).reshape(vocab, rank))
        t["candidate_selector.successor_codebook.weight"] = (
            "BF16", bf16_vec(seed, dg_tensor(D_SUCC), vocab * rank, 0.0, 0.25).reshape(vocab, rank))
    cfg = {"model_type": "qwen3", "hidden_size": H, "num_hidden_layers": L, "num_attention_heads": QH,
           "num_key_value_heads": KVH, "head_dim": HD, "intermediate_size": I, "rms_norm_eps": 1e-6,
           "rope_theta": 1e6, "sliding_window": desc["window"],
           "dflash_config": {"target_layer_ids": targets, "mask_token_id": desc["mask_token"],
                             "block_size": desc["block"]}}
    (out / "config.json").write_text(json.dumps(cfg, indent=1))
    write_safetensors(out / "model.safetensors", t, pad=3)
    return out
