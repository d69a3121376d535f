"""An independent float64 forward of the synthetic verify step, written from the reference's text — TEST ONLY.

It shares nothing with the C++ oracle but the weight and KV generators (whose streams are pinned by their own known
answers): dequantisation, RMSNorm, RoPE, the Walsh–Hadamard rotation, the int8 KV of the block's own rows, attention,
the SwiGLU / swiglu_oai FFN, the MoE router and combine and the head are restated here in numpy float64, from

* the round skeleton, HybridModel.encodeVerify (Sources/Ingot/ModelRound.swift:48-82): embed → per layer (norm →
  attention → o_proj into the residual → norm → FFN into the residual) → final norm → head → argmax;
* the dense FFN, DenseMLP.encode (Sources/Ingot/Layers/Dense.swift:55-72): gate|up → act(g)·u → down, accumulated;
* the MoE layer, MoEReference (Tests/IngotTests/KernelHarness.swift:720-766): y[r] = Σ_k w·(down_e(act(gate_e x +
  bg_e, up_e x + bu_e)) + bd_e), with swiglu_oai as CPU.swigluOAI (:185-188);
* the int8 KV scheme, ref/kv8_ref.py:63-103 (had(kv8(had(x))) for keys: scale = amax/127, round half to even, clip
  ±127; the scale stored in fp16 as the benchmark configuration states) and the attention fixture
  AttnFixture.reference (KernelHarness.swift:420-501).

No intermediate is rounded to bf16 here (the oracle and the GPU round the activations at the same points), so the
comparison tolerance is relative, and the mutation switches (`mutate=`) show it is tight enough to fail a dropped
residual, a swapped norm weight, a wrong GQA head map, MoE weights renormalised over all experts or combined in the
wrong slot order.
"""
from __future__ import annotations

import numpy as np
from scipy.linalg import hadamard

import oracle

T_EMBED, T_FINAL_NORM, T_HEAD = 1, 2, 3
L_ATTN_NORM, L_QKV, L_O, L_MLP_NORM, L_GATE_UP, L_DOWN, L_ROUTER, L_ROUTER_BIAS, L_SINKS = 0, 1, 2, 3, 4, 5, 6, 7, 9
L_Q_NORM, L_K_NORM, L_QKV_BIAS, L_ROUTE_IID, L_O_BIAS = 10, 11, 12, 13, 14
X_GATE_UP, X_DOWN, X_GU_BIAS, X_DOWN_BIAS = 0, 1, 2, 3


def layer_tensor(l: int, kind: int) -> int:
    return 1000 + 100 * l + kind


def expert_tensor(l: int, kind: int, e: int) -> int:
    return 3000000 + 10000 * l + 1000 * kind + e


# ---- generators (the model's streams) and closed-form dequantisation ---------------------------------------------

def bf16(seed, tensor, n, base, amp) -> np.ndarray:
    out = np.empty(n, np.uint16)
    oracle.lib().or_synth_bf16(seed, tensor, n, base, amp, out.ctypes.data)
    return oracle.bf16_to_f32(out).astype(np.float64)


def f32(seed, tensor, n, base, amp) -> np.ndarray:
    out = np.empty(n, np.float32)
    oracle.lib().or_synth_f32(seed, tensor, n, base, amp, out.ctypes.data)
    return out.astype(np.float64)


def nibbles(w: np.ndarray) -> np.ndarray:
    """uint32 [N, K/8] → codes [N, K], low nibble first (Loader/Quant.swift:4-12)."""
    sh = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    return ((w[:, :, None] >> sh) & 15).reshape(w.shape[0], -1).astype(np.float64)


def int4_dense(seed, tensor, N, K) -> np.ndarray:
    """W[N, K] = s·q + b per group of 64 (MLX affine)."""
    w, s, b = oracle.synth_int4(seed, tensor, N, K)
    g = np.repeat(oracle.bf16_to_f32(s).astype(np.float64), 64, axis=1)
    o = np.repeat(oracle.bf16_to_f32(b).astype(np.float64), 64, axis=1)
    return nibbles(w) * g + o


E2M1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6], np.float64)


def mxfp4_dense(seed, tensor, N, K) -> np.ndarray:
    """W[N, K] = 2^(e − 127)·e2m1(q) per group of 32 (Loader/Quant.swift:190-202)."""
    w = np.empty((N, K // 8), np.uint32)
    s = np.empty((N, K // 32), np.uint8)
    oracle.lib().or_synth_mxfp4(seed, tensor, N, K, w.ctypes.data, s.ctypes.data)
    q = nibbles(w).astype(np.int64)
    return E2M1[q] * np.repeat(np.exp2(s.astype(np.float64) - 127), 32, axis=1)


def expert_matrix(fmt, seed, tensor, N, K):
    return int4_dense(seed, tensor, N, K) if fmt == 0 else mxfp4_dense(seed, tensor, N, K)


# ---- the pieces --------------------------------------------------------------------------------------------------

def rmsnorm(h, w, eps):
    return h / np.sqrt(np.mean(h * h, axis=-1, keepdims=True) + eps) * w


def rope(x, pos, theta, rot=None, inv=None, mscale=1.0):
    """Non-interleaved halves over the first `rot` dims (angle pos·θ^(−i/(rot/2)), or pos·inv[i] from a scaled RoPE's
    table with the rotated dims × mscale); the other dims are kept (AT_ROT, verify_attn_nax.metal:92-98)."""
    HD = x.shape[-1]
    rot = rot or HD
    RH = rot // 2
    ang = pos * (theta ** (-np.arange(RH) / RH) if inv is None else np.asarray(inv, np.float64))
    c, s = np.cos(ang) * mscale, np.sin(ang) * mscale
    a, b = x[..., :RH], x[..., RH:rot]
    return np.concatenate([a * c - b * s, b * c + a * s, x[..., rot:]], axis=-1)


def rope_scaling(desc):
    """The RoPE parameter dict a model description stands for (None for the default RoPE)."""
    kinds = {1: "linear", 2: "yarn", 3: "proportional"}
    if desc.rope_type == 0:
        return None
    p = {"rope_type": kinds[desc.rope_type], "factor": desc.rope_factor or 1.0}
    if desc.rope_type == 2:
        p.update(original_max_position_embeddings=desc.rope_orig_max, beta_fast=desc.rope_beta_fast or 32.0,
                 beta_slow=desc.rope_beta_slow or 1.0, mscale=desc.rope_mscale or 1.0,
                 truncate=not desc.rope_no_truncate)
        if desc.rope_attn_factor:
            p["attention_factor"] = desc.rope_attn_factor
    if desc.rope_type == 3:
        p["partial_rotary_factor"] = desc.rope_partial or 1.0
    return p


def had(x):
    HD = x.shape[-1]
    return x @ (hadamard(HD).astype(np.float64) / np.sqrt(HD))


def kv8(x):
    """Symmetric int8 of one vector with its scale rounded to fp16: (dequantised values)."""
    amax = np.max(np.abs(x))
    sc = np.float64(np.float16(amax / 127.0 if amax > 0 else 1.0))
    return np.clip(np.round(x / sc), -127, 127) * sc


def silu_glu(g, u):
    return g / (1 + np.exp(-g)) * u


def swiglu_oai(g, u, limit):
    g = np.minimum(g, limit)
    u = np.clip(u, -limit, limit)
    return (u + 1) * (g / (1 + np.exp(-1.702 * g)))


def attention(q, K, V, P, G, window, sinks, mutate):
    """q [B][QH][HD]; K/V [KVH][n][HD] (dequantised, rotated keys); causal key ≤ P + t, window q − k < W."""
    B, QH, HD = q.shape
    out = np.zeros((B, QH, HD))
    for t in range(B):
        n = P + t + 1
        lo = max(0, n - window) if window else 0
        for h in range(QH):
            kvh = (h % (QH // G)) if mutate == "gqa" else h // G
            s = K[kvh, lo:n] @ q[t, h] / np.sqrt(HD)
            mx = s.max() if sinks is None else max(s.max(), sinks[h])
            p = np.exp(s - mx)
            den = p.sum() + (np.exp(sinks[h] - mx) if sinks is not None else 0.0)
            out[t, h] = p @ V[kvh, lo:n] / den
    return out.reshape(B, QH * HD)


def iid_logits(seed, l, P, B, E):
    key = oracle.lib().or_sm_key(seed, layer_tensor(l, L_ROUTE_IID))
    return np.array([[oracle.lib().or_sm_normal(key, (P + r) * E + e) for e in range(E)] for r in range(B)],
                    np.float64)


def route(logits, k):
    """Top-k by logit (ties to the lower index), weights = softmax over the chosen logits."""
    inds = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    ch = np.take_along_axis(logits, inds, axis=1)
    w = np.exp(ch - ch[:, :1])
    return inds, w / w.sum(axis=1, keepdims=True)


def forward(desc, seed: int, kv_seed: int, P: int, tokens, mutate: str | None = None):
    """Logits [B][vocab] in float64. mutate ∈ {None, "residual", "norm", "gqa", "renorm", "slots", "qknorm", "qkvbias",
    "gate", "obias", "rot", "rope", "route"} breaks one piece."""
    d = desc
    H, QH, KVH, HD, V = d.hidden, d.n_q_heads, d.n_kv_heads, d.head_dim, d.vocab
    G = QH // KVH
    toks = np.asarray(tokens, np.int64)
    B = len(toks)
    QS = HD * (2 if d.attn_gate else 1)
    QP = QH * QS + 2 * KVH * HD
    rot = d.rotary_dims or HD
    if mutate == "rot":  # the whole head rotated instead of the first rotary_dims
        rot = HD
    inv, msc = None, 1.0
    if rope_scaling(d) is not None and mutate != "rope":  # the table from the restated formula (mlx-lm vectors)
        inv, msc = oracle.rope_table(rope_scaling(d), d.rope_theta, rot)
    emb = int4_dense(seed, T_EMBED, V, H)
    h = emb[toks].copy()
    for l in range(d.n_layers):
        wa = bf16(seed, layer_tensor(l, L_ATTN_NORM), H, 1.0, 0.125)
        wm = bf16(seed, layer_tensor(l, L_MLP_NORM), H, 1.0, 0.125)
        if mutate == "norm":
            wa, wm = wm, wa
        x = rmsnorm(h, wa, d.rms_eps)
        proj = x @ int4_dense(seed, layer_tensor(l, L_QKV), QP, H).T
        if d.qkv_bias and mutate != "qkvbias":
            proj = proj + f32(seed, layer_tensor(l, L_QKV_BIAS), QP, 0.0, 0.1)
        qg = proj[:, : QH * QS].reshape(B, QH, QS)
        q = qg[:, :, :HD]
        gate = qg[:, :, HD:] if d.attn_gate else None
        k = proj[:, QH * QS: QH * QS + KVH * HD].reshape(B, KVH, HD)
        if d.qk_norm and mutate != "qknorm":  # per-head RMSNorm before RoPE (Qwen3's q_norm / k_norm)
            q = rmsnorm(q, bf16(seed, layer_tensor(l, L_Q_NORM), HD, 1.0, 0.125), d.rms_eps)
            k = rmsnorm(k, bf16(seed, layer_tensor(l, L_K_NORM), HD, 1.0, 0.125), d.rms_eps)
        v = proj[:, QH * QS + KVH * HD:].reshape(B, KVH, HD)
        pos = P + np.arange(B)
        qr = np.stack([rope(q[t], pos[t], d.rope_theta, rot, inv, msc) for t in range(B)])
        kr = np.stack([rope(k[t], pos[t], d.rope_theta, rot, inv, msc) for t in range(B)])
        if d.hadamard_k:
            qr, kr = had(qr), had(kr)
        # History from the generator (int8 and fp16 scales), then the block's own rows quantised as the cache stores them.
        kh, vh, ksh, vsh = oracle.synth_kv(kv_seed, 500000 + l, KVH, HD, 0, P)
        Kc = np.zeros((KVH, P + B, HD))
        Vc = np.zeros((KVH, P + B, HD))
        Kc[:, :P] = kh * oracle.f16_to_f32(ksh)[..., None]
        Vc[:, :P] = vh * oracle.f16_to_f32(vsh)[..., None]
        for t in range(B):
            for j in range(KVH):
                Kc[j, P + t] = kv8(kr[t, j])
                Vc[j, P + t] = kv8(v[t, j])
        window = d.sliding_window if (d.sliding_window > 0 and l % 2 == 0) else 0
        sinks = f32(seed, layer_tensor(l, L_SINKS), QH, 0.0, 1.0) if d.sinks else None
        att = attention(qr, Kc, Vc, P, G, window, sinks, mutate)
        if gate is not None and mutate != "gate":  # gated output (at_gate, verify_attn.metal:94-99)
            att = att * (1 / (1 + np.exp(-gate.reshape(B, QH * HD))))
        y = att @ int4_dense(seed, layer_tensor(l, L_O), H, QH * HD).T
        if d.o_bias and mutate != "obias":
            y = y + f32(seed, layer_tensor(l, L_O_BIAS), H, 0.0, 0.1)
        h = h + y if mutate != "residual" else y
        x = rmsnorm(h, wm, d.rms_eps)
        act = (lambda g, u: swiglu_oai(g, u, d.swiglu_limit)) if d.act == 1 else silu_glu
        if d.n_experts == 0:
            I = d.intermediate
            gu = x @ int4_dense(seed, layer_tensor(l, L_GATE_UP), 2 * I, H).T
            a = act(gu[:, :I], gu[:, I:])
            h = h + a @ int4_dense(seed, layer_tensor(l, L_DOWN), H, I).T
            continue
        E, Kt, IE, fmt = d.n_experts, d.top_k, d.expert_intermediate, d.expert_format
        lg = x @ expert_matrix(0 if d.router_int4 else fmt, seed, layer_tensor(l, L_ROUTER), E, H).T
        if d.iid_routing and mutate != "route":
            # Synthetic i.i.d. routing: logit (row, expert) = draw (position·E + expert) of the layer's N(0,1) stream.
            lg = iid_logits(seed, l, P, B, E)
        if d.router_bias:
            lg = lg + f32(seed, layer_tensor(l, L_ROUTER_BIAS), E, 0.0, 0.5)
        inds, w = route(lg, Kt)
        if mutate == "renorm":  # weights from a softmax over all experts instead of the chosen ones
            full = np.exp(lg - lg.max(axis=1, keepdims=True))
            w = np.take_along_axis(full / full.sum(axis=1, keepdims=True), inds, axis=1)
        if mutate == "slots":  # each row's weights applied to its experts in reverse slot order
            w = w[:, ::-1]
        y = np.zeros_like(h)
        for e in np.unique(inds):
            rows, slots = np.nonzero(inds == e)
            Wgu = expert_matrix(fmt, seed, expert_tensor(l, X_GATE_UP, e), 2 * IE, H)
            Wd = expert_matrix(fmt, seed, expert_tensor(l, X_DOWN, e), H, IE)
            g = x[rows] @ Wgu[:IE].T
            u = x[rows] @ Wgu[IE:].T
            if d.expert_bias:
                bgu = bf16(seed, expert_tensor(l, X_GU_BIAS, e), 2 * IE, 0.0, 0.1)
                g, u = g + bgu[:IE], u + bgu[IE:]
            o = act(g, u) @ Wd.T
            if d.expert_bias:
                o = o + bf16(seed, expert_tensor(l, X_DOWN_BIAS, e), H, 0.0, 0.1)
            y[rows] += w[rows, slots][:, None] * o
        h = h + y if mutate != "residual" else y
    x = rmsnorm(h, bf16(seed, T_FINAL_NORM, H, 1.0, 0.125), d.rms_eps)
    return x @ int4_dense(seed, T_HEAD, V, H).T
