"""Temperature > 0 verification: the oracle's restatement of topk64, sample_dist, spec_accept_sample and
spec_rows_choose (Sources/Ingot/Shaders/zz_sample.metal:1-281, yy_model.metal:644-675, SpecRows.swift:93-105) pinned
on the CPU by what the mathematics fixes: the top-64 against a full sort, the filtered distribution against a float64
restatement and its closed forms, and — the property the reference states for the rejection scheme — the emitted
token's distribution equals the target row's, whatever the draft (Monte Carlo, chi-square)."""
import numpy as np
import pytest

import oracle
from oracle import SampleParams


def ref_dist(vals, M, Z, temp, top_k, min_p, top_p):
    """float64 temperature → top-k → min-p → top-p over sorted candidate logits."""
    e = np.exp((np.asarray(vals, np.float64) - M) / temp)
    n = len(vals)
    if top_k > 0:
        n = min(n, top_k)
        p = e[:n] / e[:n].sum()
    else:
        p = e[:n] / Z
    if min_p > 0:
        k = 1
        while k < n and p[k] >= min_p * p[0]:
            k += 1
        n = k
        p = p[:n] / p[:n].sum()
    if top_p < 1:
        c = np.cumsum(p[:n])
        hit = np.nonzero(c >= top_p)[0]
        n = int(hit[0]) + 1 if len(hit) else n
    p = p[:n]
    return p / p.sum()


def test_topk64_against_sort_with_ties_and_nan():
    g = np.random.default_rng(0)
    x = np.round(g.normal(size=(5, 5000)) * 3).astype(np.float32)  # many ties
    x[1, ::13] = np.nan
    x[2, :] = -np.inf
    x[2, 100:110] = np.arange(10)
    idx, val, z = oracle.topk64(x, 0.8)
    for r in (0, 1, 3, 4):
        row = x[r]
        ok = ~np.isnan(row)
        order = sorted(np.nonzero(ok)[0], key=lambda i: (-row[i], i))[:64]
        assert list(idx[r]) == order
        assert np.array_equal(val[r], row[order])
        m = np.nanmax(row)
        assert z[r, 0] == m
        assert z[r, 1] == pytest.approx(np.nansum(np.exp((row[ok].astype(np.float64) - m) / 0.8)), rel=1e-6)
    # −inf logits are never candidates (they rank below the empty entry): 10 real candidates, then empties.
    assert list(idx[2, :10]) == list(range(109, 99, -1)) and np.all(idx[2, 10:] == 0xFFFFFFFF)


@pytest.mark.parametrize("temp,top_k,min_p,top_p", [(1.0, 0, 0.0, 1.0), (0.7, 20, 0.0, 1.0), (1.3, 0, 0.05, 1.0),
                                                    (0.9, 0, 0.0, 0.8), (0.6, 40, 0.02, 0.9), (2.0, 64, 0.1, 0.5)])
def test_sample_dist_against_float64(temp, top_k, min_p, top_p):
    g = np.random.default_rng(int(temp * 10) + top_k)
    x = g.normal(0, 2, size=(1, 3000)).astype(np.float32)
    idx, val, z = oracle.topk64(x, temp)
    p = SampleParams(temp=temp, top_p=top_p, top_k=top_k, min_p=min_p)
    n, pr = oracle.sample_dist(idx[0], val[0], z[0, 0], z[0, 1], p)
    want = ref_dist(val[0], z[0, 0], float(np.exp((x.astype(np.float64) - z[0, 0]) / temp).sum()), temp, top_k, min_p,
                    top_p)
    assert n == len(want)
    assert np.allclose(pr, want, rtol=1e-4, atol=1e-7)


def test_sample_dist_closed_forms():
    x = np.array([[5.0, 4.0, 4.0, 1.0] + [-30.0] * 96], np.float32)
    idx, val, z = oracle.topk64(x, 1.0)
    n, pr = oracle.sample_dist(idx[0], val[0], z[0, 0], z[0, 1], SampleParams(temp=1.0, top_p=1.0, top_k=1))
    assert n == 1 and pr[0] == 1.0  # top-k 1 is greedy
    n, pr = oracle.sample_dist(idx[0], val[0], z[0, 0], z[0, 1], SampleParams(temp=1.0, top_p=1e-6, top_k=0))
    assert n == 1  # a tiny nucleus keeps the best token
    n, pr = oracle.sample_dist(idx[0], val[0], z[0, 0], z[0, 1], SampleParams(temp=1.0, top_p=1.0, top_k=0,
                                                                             min_p=np.exp(-1.0) - 1e-6))
    assert n == 3 and pr[1] == pr[2]  # min-p e^-1 keeps the logits within 1 of the max (the tie kept in id order)


@pytest.mark.parametrize("draft_rank", [0, 1, 5, 63, -1])
def test_rejection_acceptance_emits_the_target_distribution(draft_rank):
    """First emitted token over many uniforms: its frequencies match p_0 (chi-square), whatever the draft — the
    accepted draft or, on rejection, a token of p_0 without the draft renormalised."""
    g = np.random.default_rng(11)
    x = g.normal(0, 1.5, size=(2, 200)).astype(np.float32)
    temp = 0.9
    idx, val, z = oracle.topk64(x, temp)
    p = SampleParams(temp=temp, top_p=0.95, top_k=0, min_p=0.0)
    n, pr = oracle.sample_dist(idx[0], val[0], z[0, 0], z[0, 1], p)
    draft = int(idx[0, draft_rank]) if draft_rank >= 0 else 199 if 199 not in idx[0, :n] else 198
    vtok = np.array([7, draft], np.uint32)
    N = 40000
    counts = {}
    u = g.random((N, 4)).astype(np.float32)
    for i in range(N):
        m, em = oracle.accept_sample(vtok, idx, val, z, u[i], p)
        t = int(em[0])
        counts[t] = counts.get(t, 0) + 1
    obs = np.array([counts.get(int(t), 0) for t in idx[0, :n]], np.float64)
    assert obs.sum() == N  # nothing outside the filtered set
    exp = pr.astype(np.float64) * N
    keep = exp >= 5
    chi2 = (((obs - exp) ** 2) / exp)[keep].sum()
    dof = keep.sum() - 1
    assert chi2 < dof + 6 * np.sqrt(2 * dof), (chi2, dof)


def test_rows_choose_against_brute_force():
    g = np.random.default_rng(5)
    for _ in range(300):
        kmax = int(g.integers(2, 18))
        kmin = int(g.integers(2, kmax + 1))
        conf = g.random(16).astype(np.float32)
        a = g.normal(1, 0.3, 4).astype(np.float32)
        b = g.normal(0, 0.5, 4).astype(np.float32)
        cost = np.concatenate([[1e9, 1e9], 1 + np.cumsum(g.random(16))]).astype(np.float32)
        got = oracle.rows_choose(conf, a, b, cost, kmin, kmax)
        # Expected tokens E(k) = 1 + Σ_{i<k−1} Π_{t≤i} q_t, best E(k)/cost(k), first maximum.
        c = np.clip(conf.astype(np.float64), 1e-6, 1 - 1e-6)
        q = np.array([1 / (1 + np.exp(-(a[min(t, 3)] * np.log(c[t] / (1 - c[t])) + b[min(t, 3)]))) for t in range(16)])
        E = {k: 1 + sum(np.prod(q[: i + 1]) for i in range(k - 1)) for k in range(2, kmax + 1)}
        score = {k: E[k] / cost[k] for k in range(kmin, kmax + 1)}
        best = max(score.values())
        close = [k for k in score if score[k] >= best * (1 - 1e-5)]
        assert got in close, (got, score)
    # q = 1 for every draft (confident drafts): E(k) = k, so with a flat cost the most rows win.
    assert oracle.rows_choose(np.ones(16, np.float32), np.ones(4, np.float32), np.full(4, 20, np.float32),
                              np.ones(18, np.float32), 2, 9) == 9
