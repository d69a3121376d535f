"""Pins the oracle's DFlash2 drafter restatement (oracle.OracleDrafter) with an independent numpy float64 restatement
written from the reference's text — CPU only.

Reference text followed here:
* DFlash2Drafter.encodeContext / encodeBlock (Sources/Ingot/Drafter.swift:300-550): captures → fc → hidden_norm → the
  K/V of each layer into its window ring; the block [anchor, mask × (block − 1)] at position P → per layer (norm →
  dynamic conv → q|k|v → attention → o_proj → conv-finish into the residual → norm → conv → gate|up → SwiGLU → down →
  conv-finish) → final norm of rows 1 … block − 1 → the target's lm_head → top-16 → selector;
* dconv_prep / dconv_fin_add (Shaders/yy_model.metal:159-182): two taps over the block rows, x₋₁ = 0, per-group (16
  channels) dynamic offsets on the base kernels;
* dnorm_rope / dattn_prework / dctx_write (:246-335): per-head RMSNorm with weight, then RoPE on halves; block k and
  v at slots window + t, context rows at slot position mod window;
* dvisible (:337-342): a window slot holds the latest position k ≡ slot (mod window) below P, visible to row t when
  P + t − k < window; the block's slots are visible to every row (non-causal block);
* topk16_rows (:503-560, ties to the lower index), dselect (:580-619): greedy chain, score = logit + Σ_r pred[prev][r]
  · hp[t][r] · succ[cand][r], first maximum kept, confidence 1 / Σ_j exp((s_j − s_best)/1.5); dpick_top1 (:563-578)
  for DFlash v1 (rank 0, no conv).

Shared with the oracle: only the synthetic weight generators (their streams are pinned by known answers in
test_oracle.py) and the rounding points this build chose for the GPU path (bf16 inputs to every projection, fp16 q and
ring K/V; the reference keeps them in half). Every other step is restated here in float64. Mutation switches show that
the comparison fails a window off by one, a causal block, swapped conv taps, a missing hidden_norm, a selector without
its low-rank term and a wrong GQA map.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from ingot_amd._lib import DrafterDesc, ModelDesc
from ref64 import bf16, int4_dense

T_EMBED, T_HEAD = 1, 3


def dl(l: int, kind: int) -> int:
    return 7000000 + 1000 * l + kind


def dg(kind: int) -> int:
    return 7900000 + kind


def rb(x):
    """Round to bf16 (round to nearest even) and back, in float64."""
    return oracle.round_bf16(np.asarray(x, np.float32)).astype(np.float64)


def rh(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def rmsn(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def norm_rope(x, w, pos, eps, theta):
    """Per-head RMSNorm with weight, then RoPE on the halves of the head (dnorm_rope)."""
    y = rmsn(x, w, eps)
    HD = y.shape[-1]
    RH = HD // 2
    ang = pos * theta ** (-(np.arange(HD) % RH) / RH)
    rot = np.concatenate([-y[..., RH:], y[..., :RH]], axis=-1)
    return y * np.cos(ang) + rot * np.sin(ang)


class NumpyDrafter:
    def __init__(self, d: DrafterDesc, seed: int, td: ModelDesc, tseed: int, mutate: str | None = None):
        self.d, self.mut = d, mutate
        self.H, self.HD, self.QH, self.I = d.hidden, d.head_dim, d.n_q_heads, d.intermediate
        self.Ht, self.V = td.hidden, td.vocab
        H, HD, QH, I = self.H, self.HD, self.QH, self.I
        self.GC = H // 16
        self.embed = int4_dense(tseed, T_EMBED, self.V, self.Ht)
        self.head = int4_dense(tseed, T_HEAD, self.V, self.Ht)
        self.fc = int4_dense(seed, dg(1), H, d.n_targets * self.Ht)
        self.hnorm = bf16(seed, dg(2), H, 1.0, 0.125)
        self.fnorm = bf16(seed, dg(3), H, 1.0, 0.125)
        if d.rank > 0:
            self.hproj = int4_dense(seed, dg(4), d.rank, H)
            self.pred = bf16(seed, dg(5), self.V * d.rank, 0.0, 0.25).reshape(self.V, d.rank)
            self.succ = bf16(seed, dg(6), self.V * d.rank, 0.0, 0.25).reshape(self.V, d.rank)
        self.L = []
        for l in range(d.n_layers):
            L = dict(n1=bf16(seed, dl(l, 0), H, 1.0, 0.125), n2=bf16(seed, dl(l, 1), H, 1.0, 0.125),
                     qn=bf16(seed, dl(l, 2), HD, 1.0, 0.125), kn=bf16(seed, dl(l, 3), HD, 1.0, 0.125),
                     qkv=int4_dense(seed, dl(l, 4), (QH + 16) * HD, H), o=int4_dense(seed, dl(l, 5), H, QH * HD),
                     gu=int4_dense(seed, dl(l, 6), 2 * I, H), down=int4_dense(seed, dl(l, 7), H, I))
            if d.dyn_conv:
                L["aproj"] = int4_dense(seed, dl(l, 8), 4 * self.GC, H)
                L["mproj"] = int4_dense(seed, dl(l, 9), 4 * self.GC, H)
                L["abase"] = np.stack([bf16(seed, dl(l, 10) + 100 * k, H, 0.0 if k % 2 else 1.0, 0.1) for k in range(4)])
                L["mbase"] = np.stack([bf16(seed, dl(l, 11) + 100 * k, H, 0.0 if k % 2 else 1.0, 0.1) for k in range(4)])
            # The window ring of each KV head: position → (k, v); the block's rows are kept apart.
            L["ring_k"] = {}
            L["ring_v"] = {}
            self.L.append(L)

    def context(self, caps_bf16: np.ndarray, nvalid: int, pos0: int):
        d = self.d
        c = oracle.bf16_to_f32(caps_bf16).astype(np.float64)
        e = c @ self.fc.T
        e = rb(rmsn(e, self.hnorm, d.rms_eps) if self.mut != "no_hnorm" else e)
        HD, QH = self.HD, self.QH
        for L in self.L:
            kv = e @ L["qkv"][QH * HD:].T  # the k | v rows of q | k | v
            for t in range(nvalid):
                pos = pos0 + t
                k = kv[t, :8 * HD].reshape(8, HD)
                v = kv[t, 8 * HD:].reshape(8, HD)
                L["ring_k"][pos % d.window] = (pos, rh(norm_rope(k, L["kn"], pos, d.rms_eps, d.rope_theta)))
                L["ring_v"][pos % d.window] = (pos, rh(v))

    def _visible(self, k: int, t: int, P: int) -> bool:
        W = self.d.window
        if self.mut == "window_off_by_one":
            return P + t - k <= W
        return P + t - k < W

    def _conv(self, x, base, dyn, taps):
        """out_t = (base[a] + dyn_t[a][g]) ⊙ x_t + (base[b] + dyn_t[b][g]) ⊙ x_{t−1}, x₋₁ = 0."""
        a, b = taps
        if self.mut == "swap_taps":
            a, b = b, a
        g = np.repeat(np.arange(self.GC), 16)
        k0 = base[a][None, :] + dyn[:, a * self.GC:(a + 1) * self.GC][:, g]
        k1 = base[b][None, :] + dyn[:, b * self.GC:(b + 1) * self.GC][:, g]
        prev = np.vstack([np.zeros((1, x.shape[1])), x[:-1]])
        return k0 * x + k1 * prev

    def block(self, anchor: int, P: int):
        d = self.d
        B, M, H, HD, QH, I = d.block, d.block - 1, self.H, self.HD, self.QH, self.I
        G = QH // 8
        conv = d.dyn_conv != 0
        toks = [anchor] + [d.mask_token] * M
        x = self.embed[toks].copy()
        for L in self.L:
            xn = rb(rmsn(x, L["n1"], d.rms_eps))
            if conv:
                dyn = xn @ L["aproj"].T
                a = rb(self._conv(xn, L["abase"], dyn, (0, 1)))
            else:
                a = xn
            qkv = a @ L["qkv"].T
            q = np.zeros((B, QH, HD))
            kb = np.zeros((B, 8, HD))
            vb = np.zeros((B, 8, HD))
            for t in range(B):
                heads = qkv[t].reshape(QH + 16, HD)
                q[t] = rh(norm_rope(heads[:QH], L["qn"], P + t, d.rms_eps, d.rope_theta))
                kb[t] = rh(norm_rope(heads[QH:QH + 8], L["kn"], P + t, d.rms_eps, d.rope_theta))
                vb[t] = rh(heads[QH + 8:])
            att = np.zeros((B, QH, HD))
            ctx = [(pos, L["ring_k"][s][1], L["ring_v"][s][1]) for s, (pos, _) in L["ring_k"].items() if pos < P]
            for t in range(B):
                for h in range(QH):
                    kvh = h % 8 if self.mut == "gqa" else h // G
                    keys, vals = [], []
                    for pos, kk, vv in ctx:
                        if self._visible(pos, t, P):
                            keys.append(kk[kvh])
                            vals.append(vv[kvh])
                    for u in range(B):
                        if self.mut == "causal_block" and u > t:
                            continue
                        keys.append(kb[u, kvh])
                        vals.append(vb[u, kvh])
                    s = np.array(keys) @ q[t, h] / np.sqrt(HD)
                    p = np.exp(s - s.max())
                    att[t, h] = p @ np.array(vals) / p.sum()
            y = rb(att.reshape(B, QH * HD)) @ L["o"].T
            x = x + (self._conv(y, L["abase"], dyn, (2, 3)) if conv else y)
            xn = rb(rmsn(x, L["n2"], d.rms_eps))
            if conv:
                dyn = xn @ L["mproj"].T
                a = rb(self._conv(xn, L["mbase"], dyn, (0, 1)))
            else:
                a = xn
            gu = a @ L["gu"].T
            g, u = gu[:, :I], gu[:, I:]
            hb = rb(g / (1 + np.exp(-g)) * u)
            y = hb @ L["down"].T
            x = x + (self._conv(y, L["mbase"], dyn, (2, 3)) if conv else y)
        hid = rb(rmsn(x[1:], self.fnorm, d.rms_eps))
        logits = hid @ self.head.T
        drafts = np.zeros(M, np.int64)
        conf = np.zeros(M)
        prev = anchor
        for t in range(M):
            cand = np.lexsort((np.arange(self.V), -logits[t]))[:16]  # descending, ties to the lower index
            sc = logits[t, cand].copy()
            if d.rank > 0 and self.mut != "no_lowrank":
                hp = hid[t] @ self.hproj.T
                sc = sc + (self.pred[prev] * hp) @ self.succ[cand].T
            best = int(np.argmax(sc))  # the first maximum
            drafts[t] = cand[best]
            conf[t] = 1.0 / np.sum(np.exp((sc - sc[best]) / 1.5))
            prev = int(drafts[t])
        return drafts, conf


TD = dict(n_layers=1, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=64, intermediate=256, vocab=1000)
DF2 = dict(n_layers=2, hidden=256, n_q_heads=16, head_dim=64, intermediate=256, block=8, window=32, rank=64,
           dyn_conv=1, mask_token=999)
DF1 = dict(DF2, rank=0, dyn_conv=0, n_q_heads=8, block=4)


def run(impl_cls, dd, td, mutate=None):
    """Two context passes (the second wraps the window ring), then two blocks."""
    rng = np.random.default_rng(4)
    caps = oracle.f32_to_bf16(rng.standard_normal((2, 24, dd.n_targets * td.hidden)).astype(np.float32))
    d = impl_cls(dd, 5, td, 7) if impl_cls is oracle.OracleDrafter else impl_cls(dd, 5, td, 7, mutate)
    out = []
    try:
        d.context(caps[0], 24, 0)
        out.append(d.block(123, 24))
        d.context(caps[1], 20, 24)
        out.append(d.block(456, 44))
    finally:
        if impl_cls is oracle.OracleDrafter:
            d.free()
    return out


def agree(a, b, conf_rtol):
    return all(np.array_equal(np.asarray(x[0], np.int64), np.asarray(y[0], np.int64)) and
               np.allclose(x[1], y[1], rtol=conf_rtol, atol=0) for x, y in zip(a, b))


@pytest.mark.parametrize("shape,muts", [(DF2, ["window_off_by_one", "causal_block", "swap_taps", "no_hnorm",
                                                 "no_lowrank", "gqa"]),
                                        (DF1, ["window_off_by_one", "causal_block", "no_hnorm"])],
                         ids=["dflash2", "dflash-v1"])
def test_oracle_drafter_matches_float64_restatement(shape, muts):
    dd = DrafterDesc.make(targets=(0, 1), **shape)
    td = ModelDesc.make(**TD)
    want = run(NumpyDrafter, dd, td)
    got = run(oracle.OracleDrafter, dd, td)
    # The oracle accumulates in fp32 where this restatement uses float64, at the same rounding points. A bf16 rounding
    # that lands on the other side of a boundary moves that element by 2^-8 and the block's two conv taps, residual and
    # attention carry it on: perturbing the inputs of this restatement's roundings by 3e-7 relative moves a confidence
    # by up to 0.75 %. Hence 3 % on the confidences (the drafts agree exactly: no selector near-tie in these blocks),
    # and every mutation must move some confidence by more than twice that or change a draft.
    for (gd, gc), (wd, wc) in zip(got, want):
        np.testing.assert_array_equal(gd.astype(np.int64), wd)
        np.testing.assert_allclose(gc, wc, rtol=0.03)
    assert min(np.ptp(w[1]) for w in want) > 1e-3, "confidences too flat to discriminate"
    for m in muts:
        assert not agree(run(NumpyDrafter, dd, td, m), want, 0.06), f"mutation {m} not detected"
