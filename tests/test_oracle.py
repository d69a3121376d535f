"""Pins of the CPU oracle (oracle/oracle.cpp) before it is trusted as the checker of the GPU path.

Each oracle function is checked against the reference's golden vectors (tests/golden, from the reference's own tests),
a known answer, an independent float64 formulation of the textbook definition, or brute force on tiny inputs, chosen
so that a plausible mistake (a dropped term, a sign, an index, a transposed operand) fails one of them. CPU only.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from synth import bf16_normal, int4_matrix, pack_nibbles, rng

GOLD = Path(__file__).resolve().parent / "golden"


# ---- number formats ----------------------------------------------------------------------------------------------

def test_bf16_round_to_nearest_even():
    # Exact halfway cases go to the even mantissa; values computed with exact rationals.
    one = 0x3F80
    cases = {1.0: one, 1 + 2 ** -8: one, 1 + 3 * 2 ** -8: one + 2, 1 + 2 ** -7: one + 1, -2.5: 0xC020,
             1 + 2 ** -8 + 2 ** -20: one + 1}
    for x, want in cases.items():
        assert int(oracle.f32_to_bf16(np.array([x], np.float32))[0]) == want, x
    # Round trip of every bf16 value in a sample is exact.
    bits = np.arange(0, 0x7F80, 97, dtype=np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(oracle.bf16_to_f32(bits)), bits)


def test_fp4_and_e8m0_known_answers():
    """KernelCaseMXFP4.swift:176-180: the e2m1 table with −0, and e8m0 116 → 2⁻¹¹, 135 → 256, 255 → NaN."""
    table = [oracle.fp4_e2m1(q) for q in range(16)]
    assert table == [0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6]
    assert np.signbit(table[8]) and not np.signbit(table[0])
    assert oracle.e8m0(116) == 2.0 ** -11 and oracle.e8m0(135) == 256.0 and np.isnan(oracle.e8m0(255))
    assert oracle.e8m0(127) == 1.0


def test_mxfp4_dequant_matches_mlx_golden_vectors():
    """MXFP4ReferenceTests (KernelCaseMXFP4.swift:142-158): bit for bit, the sign of zero included."""
    g = json.loads((GOLD / "mxfp4_reference.json").read_text())
    w = np.array(g["words"], np.uint32).reshape(2, 8)
    s = np.array(g["scales"], np.uint8).reshape(2, 2)
    got = oracle.dequant_mxfp4(w, s).reshape(-1)
    assert np.array_equal(got.view(np.uint32), np.array(g["value_bits"], np.uint32))


def test_int4_dequant_layout_and_closed_form():
    """w = scale·q + bias with value j of a row in bits 4j … 4j+3 of word j/8 (Loader/Quant.swift:4-12)."""
    N, K = 3, 128
    q = np.zeros((N, K), np.uint32)
    q[0, 0] = 1          # low nibble of word 0
    q[1, 9] = 15         # second word, second nibble
    q[2, :] = np.arange(K) % 16
    w = pack_nibbles(q)
    assert w[0, 0] == 1 and w[1, 1] == 15 << 4
    s = oracle.f32_to_bf16(np.array([[0.5, 0.25], [1.0, 2.0], [0.125, 4.0]], np.float32))
    b = oracle.f32_to_bf16(np.array([[1.0, -1.0], [0.0, 3.0], [-0.5, 0.25]], np.float32))
    got = oracle.dequant_int4(w, s, b)
    sf, bf = oracle.bf16_to_f32(s), oracle.bf16_to_f32(b)
    want = sf[:, np.arange(K) // 64] * q + bf[:, np.arange(K) // 64]
    assert np.array_equal(got, want.astype(np.float32))
    assert got[0, 0] == 1.5 and got[1, 9] == 15.0 and got[2, 64 + 5] == 4 * 5 + 0.25


def test_qmm_int4_against_float64_matmul():
    g = rng(1)
    w, s, b = int4_matrix(g, 96, 256)
    _, x = bf16_normal(g, (5, 256))
    W = oracle.dequant_int4(w, s, b).astype(np.float64)
    want = x.astype(np.float64) @ W.T
    got = oracle.qmm_int4(x, w, s, b)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_qmm_mxfp4_against_float64_matmul():
    g = rng(2)
    w = g.integers(0, 2 ** 32, size=(64, 256 // 8), dtype=np.uint64).astype(np.uint32)
    s = g.integers(127 - 11, 127 + 9, size=(64, 256 // 32)).astype(np.uint8)
    _, x = bf16_normal(g, (3, 256), sd=0.05)
    W = oracle.dequant_mxfp4(w, s).astype(np.float64)
    want = x.astype(np.float64) @ W.T
    got = oracle.qmm_mxfp4(x, w, s)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


# ---- row operations ----------------------------------------------------------------------------------------------

def test_argmax_ties_and_nan():
    x = np.array([[1, 3, 3, 2], [np.nan, 1, np.nan, 1], [-np.inf] * 4, [0, -0.0, 0, 0]], np.float32)
    assert list(oracle.argmax_rows(x)) == [1, 1, 0, 0]
    # -inf never takes an index (a scan from (-inf, 0) with a strict >, verify.metal:537): NaN mixed with -inf gives 0,
    # a finite value behind -inf and NaN wins.
    z = np.array([[np.nan, -np.inf, np.nan, -np.inf], [-np.inf, np.nan, -5.0, -np.inf]], np.float32)
    assert list(oracle.argmax_rows(z)) == [0, 2]
    g = rng(4)
    y = g.normal(size=(7, 1000)).astype(np.float32)
    assert np.array_equal(oracle.argmax_rows(y), np.argmax(y, axis=1))


def test_rmsnorm_against_definition():
    g = rng(5)
    x = g.normal(0, 3, size=(4, 512)).astype(np.float32)
    wb, wf = bf16_normal(g, 512, sd=1.0)
    got = oracle.rmsnorm(x, wb, 1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * wf
    assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max()   # output is rounded to bf16
    assert np.array_equal(got, oracle.round_bf16(got))


def test_glu_activations():
    """SiLU(g)·u and swiglu_oai (clip(u, ±7) + 1)·g·σ(1.702 g), g = min(gate, 7) (KernelHarness.swift:185-188)."""
    L = oracle.lib()
    for gv, uv in [(0.5, 2.0), (-3.0, 1.5), (9.0, 8.0), (6.9, -9.0), (-20.0, 0.1)]:
        silu = gv / (1 + np.exp(-gv)) * uv
        assert abs(L.or_glu(gv, uv, 0, 7.0) - silu) <= 1e-6 * max(1, abs(silu))
        gc, uc = min(gv, 7.0), min(max(uv, -7.0), 7.0)
        oai = (uc + 1) * gc / (1 + np.exp(-1.702 * gc))
        assert abs(L.or_glu(gv, uv, 1, 7.0) - oai) <= 1e-6 * max(1, abs(oai))


def sylvester(n):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


def test_fwht_is_sylvester_hadamard():
    g = rng(6)
    for n in (64, 128):
        v = g.normal(size=n).astype(np.float32)
        got = oracle.fwht(v)
        want = sylvester(n) @ v.astype(np.float64)
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
        # Orthonormal form is an involution.
        assert np.abs(oracle.fwht(got / np.sqrt(n)) / np.sqrt(n) - v).max() < 1e-5


def rope64(x, pos, theta):
    x = x.astype(np.float64)
    n = len(x)
    h = n // 2
    inv = theta ** (-np.arange(h) / h)
    c, s = np.cos(pos * inv), np.sin(pos * inv)
    return np.concatenate([x[:h] * c - x[h:] * s, x[h:] * c + x[:h] * s])


def test_rope_and_hadamard_rotation():
    g = rng(7)
    theta = 1e6
    for hd in (64, 128):
        q = g.normal(size=hd).astype(np.float32)
        k = g.normal(size=hd).astype(np.float32)
        assert np.allclose(oracle.rope_wht(q, 0, theta, 0), q, atol=1e-7)
        for pos in (1, 37, 8191):
            r = oracle.rope_wht(q, pos, theta, 0)
            assert np.abs(r - rope64(q, pos, theta)).max() < 1e-5
            assert abs(np.linalg.norm(r) - np.linalg.norm(q)) < 1e-4
            rh = oracle.rope_wht(q, pos, theta, 1)
            assert np.abs(rh - sylvester(hd) @ rope64(q, pos, theta) / np.sqrt(hd)).max() < 1e-5
        # Relative positions: ⟨R_m q, R_n k⟩ depends on m − n only; the Hadamard leaves the product unchanged.
        a = np.dot(oracle.rope_wht(q, 40, theta, 1), oracle.rope_wht(k, 33, theta, 1))
        b = np.dot(oracle.rope_wht(q, 107, theta, 0), oracle.rope_wht(k, 100, theta, 0))
        assert abs(a - b) < 1e-4 * max(1.0, abs(a))


def test_synthetic_kv_quantisation():
    """Symmetric int8 per (token, head) with an fp16 scale: |q| ≤ 127, the largest |x| maps to ±127, and
    q·scale is within half a step of x (CPU.quantI8, KernelHarness.swift:249-254)."""
    k, v, ks, vs = oracle.synth_kv(11, 500000, 2, 128, 5, 9)
    key = oracle.lib().or_sm_key(11, 2 * 500000)
    for h in range(2):
        for p in range(9):
            x = np.array([oracle.lib().or_sm_normal(key, ((h << 24) + 5 + p) * 128 + d) for d in range(128)],
                         np.float32)
            sc = oracle.f16_to_f32(ks[h, p])
            assert sc == np.float32(np.float16(np.abs(x).max() / 127))
            q = k[h, p].astype(np.float32)
            assert np.abs(q).max() <= 127 and np.abs(q).max() >= 126
            assert np.abs(q * sc - x).max() <= sc * 0.5 + 1e-6 or np.abs(q).max() == 127


def attention64(q, P, QH, KVH, k, v, ks, vs, window, sinks):
    """Textbook softmax attention in float64 (causal, sliding window, optional sink logits)."""
    B, _, HD = q.shape
    G = QH // KVH
    kf = k.astype(np.float64) * oracle.f16_to_f32(ks).astype(np.float64)[..., None]
    vf = v.astype(np.float64) * oracle.f16_to_f32(vs).astype(np.float64)[..., None]
    out = np.zeros((B, QH * HD))
    for t in range(B):
        n = P + t + 1
        lo = max(0, n - window) if window else 0
        for h in range(QH):
            s = kf[h // G, lo:n] @ q[t, h].astype(np.float64) / np.sqrt(HD)
            z = np.exp(s - max(s.max(), sinks[h] if sinks is not None else -np.inf))
            den = z.sum() + (np.exp(sinks[h] - max(s.max(), sinks[h])) if sinks is not None else 0.0)
            out[t, h * HD:(h + 1) * HD] = (z / den) @ vf[h // G, lo:n]
    return out


@pytest.mark.parametrize("window,use_sinks", [(0, False), (24, False), (0, True), (16, True)])
def test_attention_against_float64_softmax(window, use_sinks):
    g = rng(8)
    B, P, QH, KVH, HD = 3, 40, 4, 2, 64
    npos = P + B
    k = g.integers(-127, 128, size=(KVH, npos, HD)).astype(np.int8)
    v = g.integers(-127, 128, size=(KVH, npos, HD)).astype(np.int8)
    ks = np.float16(g.uniform(0.01, 0.02, size=(KVH, npos))).view(np.uint16)
    vs = np.float16(g.uniform(0.01, 0.02, size=(KVH, npos))).view(np.uint16)
    q = g.normal(size=(B, QH, HD)).astype(np.float32)
    sinks = g.normal(size=QH).astype(np.float32) if use_sinks else None
    got = oracle.attention(q, P, QH, KVH, k, v, ks, vs, window, sinks)
    want = attention64(q, P, QH, KVH, k, v, ks, vs, window, sinks)
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()


# ---- routing, union, copy ----------------------------------------------------------------------------------------

def _vec(c, key):
    v = c.get(key)
    return None if v is None else np.array(v, np.float32)


def test_router_against_mlx_lm_vectors():
    """ref/router_vectors.json (mlx-lm 0.32.2): rows 2… against mlx-lm's weights (maxRel 1e-5); rows 0–1 carry exact
    ties and follow the engine's lower-index rule (KernelCaseRouter.swift:6-12,54-80)."""
    cases = json.loads((GOLD / "router_vectors.json").read_text())["cases"]
    assert len(cases) >= 7
    for c in cases:
        E, K, R = int(c["experts"]), int(c["topK"]), int(c["rows"])
        logits = np.array(c["logits"], np.float32).reshape(R, E)
        inds, wts = oracle.route(logits, K, sigmoid=c["score"] == "sigmoid", sel_bias=_vec(c, "bias"),
                                 logit_bias=_vec(c, "logitBias"), pes=_vec(c, "perExpertScale"),
                                 scale=float(c["scale"]), eps=float(c["eps"]))
        dense = np.zeros((R, E), np.float32)
        for r in range(R):
            dense[r, inds[r]] += wts[r]
        mlx = np.array(c["weights"], np.float32).reshape(R, E)
        assert np.array_equal(dense[2:] != 0, mlx[2:] != 0), c["name"]
        rel = np.abs(dense[2:] - mlx[2:]).max() / np.abs(mlx[2:]).max()
        assert rel <= 1e-5, (c["name"], rel)
        # Rows 0–1: ties to the lower index, by brute force over the scores.
        for r in (0, 1):
            l = logits[r] + (_vec(c, "logitBias") if c.get("logitBias") is not None else 0)
            p = 1 / (1 + np.exp(-l)) if c["score"] == "sigmoid" else l
            sel = p + (_vec(c, "bias") if c.get("bias") is not None else 0)
            order = sorted(range(E), key=lambda e: (-sel[e], e))[:K]
            assert list(inds[r]) == order, c["name"]


def test_expert_union_counting_sort():
    g = rng(9)
    for _ in range(20):
        rows, E, K = int(g.integers(1, 18)), 32, 4
        inds = np.array([g.choice(E, K, replace=False) for _ in range(rows)], np.int32)
        entries, pairs = oracle.expert_union(inds, E)
        assert list(entries[:, 0]) == sorted(set(inds.ravel().tolist()))
        off = 0
        for e, start, cnt in entries:
            assert start == off
            want = [(r, k) for r in range(rows) for k in range(K) if inds[r, k] == e]
            assert [tuple(x) for x in pairs[start:start + cnt]] == want
            off += cnt
        assert off == rows * K


def test_splitmix64_known_answer():
    assert [hex(int(x)) for x in oracle.splitmix64(0, 3)] == [
        "0xe220a8397b1dcdaf", "0x6e789e6aa1b965f4", "0x6c45d188009454f"]


def naive_py(h, maxK):
    """CopySpecTests.naive written in plain Python (Tests/IngotTests/CopySpecTests.swift:9-28)."""
    n = len(h)
    if n < 4:
        return [], 0
    cur = n - 1
    occ = [p for p in range(cur - 1, 1, -1) if h[p] == h[cur] and h[p - 1] == h[cur - 1] and h[p - 2] == h[cur - 2]]
    cand = ([cur] + occ)[:4][1:]
    best_end, best_len = 0, 0
    for p in cand:
        ln = 0
        while ln < 64 and ln <= p and h[p - ln] == h[cur - ln]:
            ln += 1
        if ln > best_len:
            best_len, best_end = ln, p
    if best_len < 3:
        return [], 0
    return list(h[best_end + 1: min(cur, best_end + maxK) + 1]), best_len


class SplitMix:
    def __init__(self, seed):
        self.buf = list(oracle.splitmix64(seed, 400000))
        self.i = 0

    def next(self):
        v = int(self.buf[self.i])
        self.i += 1
        return v


def test_copy_index_matches_naive_like_the_reference():
    """CopySpecTests.proposeMatchesNaive (Tests/IngotTests/CopySpecTests.swift:30-59): SplitMix64(seed 3), 20 trials of
    1500 tokens with spans copied from earlier, vocab 6 / 40, a capacity-64 index that rebuilds as it grows."""
    g = SplitMix(3)
    for trial in range(20):
        ci = oracle.CopyIndexRef(64)
        h = []
        vocab = 6 if trial % 2 == 0 else 40
        for _ in range(1500):
            if len(h) > 50 and g.next() % 4 == 0:
                s = g.next() % (len(h) - 20)
                ln = g.next() % 20 + 1
                span = h[s:s + ln]
                h += span
                ci.append(span)
            else:
                t = g.next() % vocab
                h.append(t)
                ci.append([t])
            k = g.next() % 16 + 1
            exp, m = naive_py(h, k)
            got, gm = ci.propose(k)
            assert list(got) == exp and gm == m, (trial, len(h))
            nv, nm = oracle.copy_naive(np.array(h, np.uint32), k)
            assert list(nv) == exp and nm == m
        ci.free()


# ---- whole verify step -------------------------------------------------------------------------------------------

def test_oracle_model_row_causality():
    """Row r of a block depends only on rows ≤ r (causal attention, per-row norms and matmuls): the oracle's logits of
    the first rows are the same with more rows after them."""
    from ingot_amd._lib import ModelDesc

    d = ModelDesc.make(n_layers=2, hidden=128, n_q_heads=2, n_kv_heads=1, head_dim=64, intermediate=128, vocab=300)
    toks = np.array([5, 17, 250, 3, 9], np.uint32)
    l5, t5 = oracle.verify_dense(d, 7, 11, 20, toks)
    l2, t2 = oracle.verify_dense(d, 7, 11, 20, toks[:2])
    assert np.abs(l5[:2] - l2).max() <= 1e-5 * np.abs(l2).max()
    assert list(t5[:2]) == list(t2)
    m = oracle.OracleModel(d, 7, 11, 20)
    la, ta = m.verify(toks)
    m.free()
    assert np.array_equal(la, l5) and np.array_equal(ta, t5)


def test_moe_oracle_sensitivity_to_last_bit_changes():
    """The MoE model's logits move by a few hundredths under a one-part-in-10^7 change of RoPE θ (rounding flips of the
    bf16 activations and int8 KV, amplified by the softmax router across two layers), while the dense model's move less:
    the measured basis of the wider tolerance of the two-layer MoE GPU test."""
    from ingot_amd._lib import ModelDesc

    shape = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=0, vocab=1000,
                 n_experts=8, top_k=2, expert_intermediate=128, expert_format=0)
    toks = np.random.default_rng(17).integers(0, 1000, size=17).astype(np.uint32)
    a, _ = oracle.verify_dense(ModelDesc.make(**shape), 7, 11, 100, toks)
    b, _ = oracle.verify_dense(ModelDesc.make(**shape, rope_theta=1e6 * (1 + 1e-7)), 7, 11, 100, toks)
    d = np.abs(a - b).max()
    assert 0.02 < d < 0.05 + 0.03 * np.abs(a).max(), d


# ---- RoPE frequency tables (RopeTable.make) ----------------------------------------------------------------------

def _ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def test_rope_table_matches_mlx_lm_vectors():
    """RopeTableTests.matchesMlxLm (Tests/IngotTests/RopeTableTests.swift:17-38) on ref/rope/rope_ref.json: the table
    within 1 ulp of the float64 formula, within 8 ulp of mlx-lm's float32 steps, mscale within 1 ulp (yarn with and
    without truncate, gpt-oss's, yarn with mscale, linear, default)."""
    cases = json.loads((GOLD / "rope_ref.json").read_text())["cases"]
    assert len(cases) >= 5
    for c in cases:
        inv, ms = oracle.rope_table(c["params"], c["theta"], c["dims"])
        assert len(inv) == c["dims"] // 2
        assert _ulps(inv, c["inv_freq_f64"]).max() <= 1, c["name"]
        assert _ulps(inv, c["inv_freq"]).max() <= 8, c["name"]
        assert _ulps(np.float32(ms), np.float32(c["mscale"])) <= 1, (c["name"], ms, c["mscale"])


def test_rope_table_proportional_and_linear_closed_forms():
    """RopeTableTests.proportionalTable (RopeTable.swift:109-113): the first int(dims·partial)/2 pairs at period
    factor·θ^(2i/dims), the rest exactly 0; linear = default / factor."""
    inv, ms = oracle.rope_table({"rope_type": "proportional", "partial_rotary_factor": 0.25}, 1e6, 512)
    want = (1 / np.power(1e6, 2.0 * np.arange(64) / 512)).astype(np.float32)
    assert ms == 1.0 and _ulps(inv[:64], want).max() <= 1 and np.all(inv[64:] == 0)
    inv2, _ = oracle.rope_table({"rope_type": "proportional", "factor": 2.0}, 1e4, 256)
    assert _ulps(inv2, (1 / (2 * np.power(1e4, 2.0 * np.arange(128) / 256))).astype(np.float32)).max() <= 1
    lin, _ = oracle.rope_table({"rope_type": "linear", "factor": 4.0}, 1e4, 128)
    dflt, _ = oracle.rope_table({"rope_type": "default"}, 1e4, 128)
    assert _ulps(lin, dflt / 4).max() <= 1


def test_yarn_table_ends_are_original_and_interpolated():
    """YaRN: pairs below the correction range keep θ^(−2i/d), pairs above it are divided by the factor, and without an
    attention_factor mscale = 0.1·mscale·ln(factor) + 1."""
    p = {"rope_type": "yarn", "factor": 32.0, "original_max_position_embeddings": 4096, "beta_fast": 32.0,
         "beta_slow": 1.0, "truncate": False}
    inv, ms = oracle.rope_table(p, 150000.0, 64)
    base = 1 / np.power(150000.0, 2.0 * np.arange(32) / 64)
    assert _ulps(inv[:3], base[:3].astype(np.float32)).max() <= 1
    assert _ulps(inv[-3:], (base[-3:] / 32).astype(np.float32)).max() <= 1
    assert abs(ms - (0.1 * np.log(32.0) + 1)) < 1e-6
    assert np.all(np.diff(inv) < 0)  # monotone through the ramp


def test_partial_rope_rotates_only_the_first_dims():
    """AT_ROT < head_dim: dims from rot on are untouched, the rotated ones equal a whole-head RoPE of width rot
    (pairs d, d + rot/2), and the rotation keeps the norm of each pair."""
    g = np.random.default_rng(5)
    x = g.normal(size=128).astype(np.float32)
    y = oracle.rope_wht_ex(x, 64, 1234, 1e7, None, 1.0, 0)
    assert np.array_equal(y[64:], x[64:])
    z = oracle.rope_wht(x[:64], 1234, 1e7, 0)
    assert np.array_equal(y[:64], z)
    assert np.allclose(y[:32] ** 2 + y[32:64] ** 2, x[:32] ** 2 + x[32:64] ** 2, rtol=1e-5)
    # A table and mscale: the rotated dims scale by mscale, the others not.
    inv, _ = oracle.rope_table({"rope_type": "default"}, 1e7, 64)
    w = oracle.rope_wht_ex(x, 64, 1234, 1e7, inv, 2.0, 0)
    # (the table holds fp32 frequencies, the default path forms the angle from θ in double: angles agree to ~1e-4)
    assert np.allclose(w[:64], 2 * y[:64], atol=2e-3) and np.array_equal(w[64:], x[64:])


def test_attention_p16_rounds_probability_times_v_scale():
    """oracle.attn_p16 (the reference's rounding point half(p·vs), verify_attn_pf.metal:268-276): the oracle's
    attention then equals a float64 restatement in which each exp(s − max)·vs is rounded to fp16 before it weights V
    and the denominator sums the unrounded probabilities; and it differs from the fp32 attention by about one fp16
    rounding (relative 2^-11), not more."""
    g = rng(9)
    B, P, QH, KVH, HD = 2, 30, 4, 2, 64
    npos = P + B
    k = g.integers(-127, 128, size=(KVH, npos, HD)).astype(np.int8)
    v = g.integers(-127, 128, size=(KVH, npos, HD)).astype(np.int8)
    ks = np.float16(g.uniform(0.01, 0.02, size=(KVH, npos))).view(np.uint16)
    vs = np.float16(g.uniform(0.01, 0.02, size=(KVH, npos))).view(np.uint16)
    q = g.normal(size=(B, QH, HD)).astype(np.float32)
    with oracle.attn_p16():
        got = oracle.attention(q, P, QH, KVH, k, v, ks, vs, 0, None)
    plain = oracle.attention(q, P, QH, KVH, k, v, ks, vs, 0, None)
    G = QH // KVH
    want = np.zeros((B, QH * HD))
    for t in range(B):
        n = P + t + 1
        for h in range(QH):
            kf = k[h // G, :n].astype(np.float64) * oracle.f16_to_f32(ks[h // G, :n]).astype(np.float64)[:, None]
            s = kf @ q[t, h].astype(np.float64) / np.sqrt(HD)
            p = np.exp(s - s.max())
            pv = (p * oracle.f16_to_f32(vs[h // G, :n]).astype(np.float64)).astype(np.float16).astype(np.float64)
            want[t, h * HD:(h + 1) * HD] = (pv @ v[h // G, :n].astype(np.float64)) / p.sum()
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 2e-5 * scale
    d = np.abs(got - plain).max() / scale
    assert 1e-6 < d <= 2e-3
