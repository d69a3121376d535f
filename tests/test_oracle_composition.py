"""The oracle's composition of the verify step (or_model_verify, moe_forward, or_rms_split) against an independent
float64 forward written from the reference's text (tests/ref64.py), on tiny shapes, CPU only.

The comparison is relative (the oracle rounds activations to bf16/fp16 and the KV to int8 at the points the GPU does;
the float64 forward rounds only the cache), and each mutation of the float64 forward — a dropped residual, the two
RMSNorm weights swapped, a wrong GQA head map, MoE weights not renormalised over the chosen experts — must land
outside the tolerance, so the check is known to catch those mistakes.
"""
import numpy as np
import pytest

import oracle
import ref64
from ingot_amd._lib import ModelDesc

DENSE = dict(n_layers=2, hidden=128, n_q_heads=4, n_kv_heads=2, head_dim=64, intermediate=192, vocab=300,
             rope_theta=1e4)
MOE = dict(n_layers=2, hidden=128, n_q_heads=4, n_kv_heads=2, head_dim=64, intermediate=0, vocab=300, n_experts=8,
           top_k=2, expert_intermediate=64, expert_format=0, rope_theta=1e4)
MOEX = dict(n_layers=2, hidden=128, n_q_heads=8, n_kv_heads=2, head_dim=64, intermediate=0, vocab=300, n_experts=8,
            top_k=4, expert_intermediate=64, expert_format=1, router_bias=1, expert_bias=1, act=1, sinks=1,
            sliding_window=8, rope_theta=1e4)
QWEN = dict(DENSE, qk_norm=1, qkv_bias=1)
# Qwen3-Next-style attention: gated output, partial RoPE over a quarter of the head, QK-norm.
GATED = dict(DENSE, attn_gate=1, rotary_dims=16, qk_norm=1)
# gpt-oss-style attention: q|k|v|o biases, YaRN (gpt-oss's parameters, no truncation), sinks and the window.
YARN = dict(DENSE, qkv_bias=1, o_bias=1, sinks=1, sliding_window=8, rope_type=2, rope_factor=32.0,
            rope_orig_max=4096.0, rope_no_truncate=1, rope_theta=150000.0)
# The synthetic i.i.d. routing of the benchmark MoE configurations.
MOEIID = dict(MOE, iid_routing=1, n_experts=16, top_k=4)
P = 24
TOKS = np.array([5, 17, 250, 3, 9, 101, 77], np.uint32)


def rel_err(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


# Tolerance (max-abs error over max |logit|): measured 0.007 for the int4 shapes and 0.02 for the MXFP4 one, whose
# expert weights (up to 1.5, against int4's ~0.02 scale) amplify the rounding of the activations through the router's
# softmax and the experts; every mutation lands at ≥ 0.1. (With top-4 of 8 experts under such a sharp router the
# renormalisation changes little, so the MXFP4 shape checks the slot order instead.)
@pytest.mark.parametrize("shape,tol,muts", [(DENSE, 0.015, ["residual", "norm", "gqa"]),
                                            (MOE, 0.015, ["residual", "norm", "gqa", "renorm", "slots"]),
                                            (MOEX, 0.03, ["residual", "norm", "gqa", "slots"]),
                                            (dict(MOEX, router_int4=1), 0.03, ["residual", "slots"]),
                                            (QWEN, 0.015, ["residual", "gqa", "qknorm", "qkvbias"]),
                                            (GATED, 0.015, ["residual", "gqa", "gate", "rot"]),
                                            (YARN, 0.015, ["residual", "obias", "qkvbias", "rope"]),
                                            (MOEIID, 0.015, ["residual", "renorm", "route"])],
                         ids=["dense", "moe-int4", "moe-mxfp4-sinks-swa", "moe-mxfp4-int4-router", "qknorm-qkvbias",
                              "gated-partial-rope",
                              "yarn-obias-sinks", "moe-iid-routing"])
def test_oracle_composition_matches_float64_forward(shape, tol, muts):
    d = ModelDesc.make(**shape)
    logits, _ = oracle.verify_dense(d, 7, 11, P, TOKS)
    ref = ref64.forward(d, 7, 11, P, TOKS)
    err = rel_err(logits, ref)
    assert err <= tol, err
    for m in muts:
        bad = ref64.forward(d, 7, 11, P, TOKS, mutate=m)
        assert rel_err(logits, bad) > 2 * tol, (m, rel_err(logits, bad))


def test_rms_split_times_factor_is_the_norm():
    """or_rms_split's input bf16(h ⊙ w) times its row factor r equals or_rmsnorm up to the bf16 rounding point."""
    g = np.random.default_rng(2)
    h = g.normal(0, 3, size=(5, 256)).astype(np.float32)
    w = oracle.f32_to_bf16(g.normal(1, 0.125, size=256).astype(np.float32))
    x = np.empty_like(h)
    r = np.empty(5, np.float32)
    oracle.lib().or_rms_split(h.ctypes.data, 5, 256, w.ctypes.data, 1e-6, x.ctypes.data, r.ctypes.data)
    full = oracle.rmsnorm(h, w, 1e-6)
    want = h.astype(np.float64) / np.sqrt(np.mean(h.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6)
    want = want * oracle.bf16_to_f32(w)
    assert np.abs(x * r[:, None] - want).max() <= 2 ** -7 * np.abs(want).max()
    assert np.abs(full - want).max() <= 2 ** -7 * np.abs(want).max()
    assert np.allclose(r, 1 / np.sqrt(np.mean(h.astype(np.float64) ** 2, axis=1) + 1e-6), rtol=1e-6)
