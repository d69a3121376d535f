"""Temperature > 0 on the GPU: ih_topk64_dev, ih_spec_accept_sample_dev, ih_spec_rows_choose_dev and the sampling
decode loop against the oracle's restatement (pinned in test_sampling.py).

Reference: Shaders/zz_sample.metal:1-281 (topk64_part/merge, sample_dist, spec_accept_sample), yy_model.metal:644-675
(spec_rows_choose), Generate.swift:240-512 (decodeSpec with sampling, roundUniforms)."""
import ctypes as C

import numpy as np
import pytest

import oracle
from ingot_amd._lib import RND_PER_ROUND, KVCache, Model, ModelDesc, RowsParams, SampleParams, check, lib

pytestmark = pytest.mark.gpu


def gpu_topk(ctx, x, temp):
    rows, V = x.shape
    dx = ctx.to_device(np.ascontiguousarray(x, np.float32))
    di, dv, dz = ctx.buffer(rows * 64 * 4), ctx.buffer(rows * 64 * 4), ctx.buffer(rows * 8)
    check(lib().ih_topk64_dev(ctx.handle, dx.ptr, V, rows, V, temp, di.ptr, dv.ptr, dz.ptr))
    out = (di.download(np.uint32, (rows, 64)), dv.download(np.float32, (rows, 64)), dz.download(np.float32, (rows, 2)))
    for b in (dx, di, dv, dz):
        b.free()
    return out


@pytest.mark.parametrize("rows,V", [(17, 151936), (9, 201088), (4, 1000), (3, 50)])
def test_topk64_matches_oracle(ctx, rows, V):
    g = np.random.default_rng(V)
    x = (g.normal(size=(rows, V)) * 3).astype(np.float32)
    x[0] = np.round(x[0])  # ties everywhere
    x[1, ::17] = np.nan
    if rows > 2:
        x[2, : V // 2] = -np.inf
    for temp in (0.6, 1.0):
        gi, gv, gz = gpu_topk(ctx, x, temp)
        oi, ov, oz = oracle.topk64(x, temp)
        assert np.array_equal(gi, oi)
        assert np.array_equal(gv, ov)
        assert np.array_equal(gz[:, 0], oz[:, 0])
        assert np.allclose(gz[:, 1], oz[:, 1], rtol=2e-5)


@pytest.mark.parametrize("order", ["ascending", "descending", "sawtooth"])
def test_topk64_buffer_paths_match_oracle(ctx, order):
    """Orders that drive the chunk kernel's candidate buffer to its extremes: ascending logits make every element beat
    the running 64th best (a flush per 64 elements), descending ones admit only the first 64 of each wave, a sawtooth
    mixes both with ties across the teeth."""
    rows, V = 5, 151936
    base = np.arange(V, dtype=np.float32)
    x = {"ascending": base / 1000.0, "descending": -base / 1000.0, "sawtooth": np.float32(0.25) * (base % 997)}[order]
    x = np.tile(x, (rows, 1)).astype(np.float32)
    x[1] *= -1.0
    x[2, ::5] = np.nan
    for temp in (0.7, 1.0):
        gi, gv, gz = gpu_topk(ctx, x, temp)
        oi, ov, oz = oracle.topk64(x, temp)
        assert np.array_equal(gi, oi)
        assert np.array_equal(gv, ov)
        assert np.array_equal(gz[:, 0], oz[:, 0])
        assert np.allclose(gz[:, 1], oz[:, 1], rtol=2e-5)


def test_accept_sample_matches_oracle(ctx):
    """Many rounds on one device state: drafts planted from each row's likely candidates, uniforms random; m and the
    emitted tokens equal the oracle's on the same candidates and uniforms (a uniform within 1e-5 of an acceptance
    probability would be a rounding coin flip: counted, allowed once)."""
    g = np.random.default_rng(3)
    ring, R = 8, 60
    params = [SampleParams(temp=0.8, top_p=1.0, top_k=0, min_p=0.0), SampleParams(temp=1.2, top_p=0.9, top_k=40,
                                                                                min_p=0.02)]
    d_st = ctx.to_device(np.zeros(8, np.uint32))
    d_rec = ctx.buffer(ring * 24 * 4).fill(0)
    d_vtok = ctx.buffer(17 * 4)
    rnd = g.random((R, RND_PER_ROUND)).astype(np.float32)
    d_rnd = ctx.to_device(rnd)
    near = 0
    P = 0
    for r in range(R):
        B = 1 + r % 17
        p = params[r % 2]
        x = (g.normal(size=(B, 3000)) * 2.5).astype(np.float32)
        idx, val, z = oracle.topk64(x, p.temp)
        vtok = np.zeros(17, np.uint32)
        vtok[0] = 5
        for i in range(1, B):
            vtok[i] = idx[i - 1, min(int(g.integers(0, 3)), 63)]  # likely drafts
        d_vtok.upload(vtok)
        di, dv, dz = ctx.to_device(idx), ctx.to_device(val), ctx.to_device(z)
        check(lib().ih_spec_accept_sample_dev(ctx.handle, d_st.ptr, d_vtok.ptr, di.ptr, dv.ptr, dz.ptr, d_rec.ptr,
                                              d_rnd.ptr, C.byref(p), ring, B))
        rec = d_rec.download(np.uint32, (ring, 24))[r % ring]
        m, em = oracle.accept_sample(vtok[:B], idx, val, z, rnd[r, : 2 * B], p)
        gm = int(rec[0])
        if gm != m or list(rec[1: gm + 2]) != list(em):
            # A coin flip at a rounding boundary: the oracle's q for the deciding row.
            row = min(gm, m)
            n, pr = oracle.sample_dist(idx[row], val[row], z[row, 0], z[row, 1], p)
            q = pr[list(idx[row, :n]).index(vtok[row + 1])] if vtok[row + 1] in idx[row, :n] else 0.0
            assert abs(rnd[r, 2 * row] - q) < 1e-5, (r, gm, m, rec[: gm + 2], em)
            near += 1
        st = d_st.download(np.uint32, (8,))
        assert st[5] == r + 1 and st[3] == P and st[0] == P + gm + 1
        P = int(st[0])
        for b in (di, dv, dz):
            b.free()
    assert near <= 1
    for b in (d_st, d_rec, d_vtok, d_rnd):
        b.free()


def test_accept_sample_all_drafts_accepted_uses_its_own_rounds_uniforms(ctx):
    """B = 17 with every draft accepted: the 17th row's resample draws uniform 33 of its own round (uniforms per round
    = 2 × 17), never the next round's first. Rows 0–15 are sharp (the draft has probability ≈ 1 and the accept uniform
    is 0), row 16 is flat over many candidates so the drawn token depends on that uniform; each round's uniforms differ
    from the next round's."""
    g = np.random.default_rng(17)
    ring, R, B, V = 4, 6, 17, 2000
    assert RND_PER_ROUND >= 2 * B
    p = SampleParams(temp=1.0, top_p=1.0, top_k=0, min_p=0.0)
    d_st = ctx.to_device(np.zeros(8, np.uint32))
    d_rec = ctx.buffer(ring * 24 * 4).fill(0)
    d_vtok = ctx.buffer(17 * 4)
    rnd = g.random((R, RND_PER_ROUND)).astype(np.float32)
    rnd[:, 0:2 * (B - 1):2] = 0.0  # accept every draft
    d_rnd = ctx.to_device(rnd)
    seen = set()
    for r in range(R):
        x = np.full((B, V), -1e4, np.float32)
        top = g.choice(V, size=B - 1, replace=False)
        x[np.arange(B - 1), top] = 50.0  # rows 0–15: one candidate holds all the mass
        x[B - 1, :40] = g.normal(size=40).astype(np.float32) * 0.1  # row 16: ~flat over 40 candidates
        idx, val, z = oracle.topk64(x, p.temp)
        vtok = np.zeros(17, np.uint32)
        vtok[0] = 7
        vtok[1:B] = idx[: B - 1, 0]
        d_vtok.upload(vtok)
        di, dv, dz = ctx.to_device(idx), ctx.to_device(val), ctx.to_device(z)
        check(lib().ih_spec_accept_sample_dev(ctx.handle, d_st.ptr, d_vtok.ptr, di.ptr, dv.ptr, dz.ptr, d_rec.ptr,
                                              d_rnd.ptr, C.byref(p), ring, B))
        rec = d_rec.download(np.uint32, (ring, 24))[r % ring]
        m, em = oracle.accept_sample(vtok[:B], idx, val, z, rnd[r, : 2 * B], p)
        assert m == B - 1 and int(rec[0]) == B - 1
        assert list(rec[1:B + 1]) == list(em)
        # The same pick as the oracle's with the next round's first uniform would be a coincidence for some round.
        _, em_next = oracle.accept_sample(vtok[:B], idx, val, z, np.concatenate([rnd[r, :2 * B - 1], rnd[(r + 1) % R, 1:2]]), p)
        seen.add(int(em[-1]) != int(em_next[-1]))
        for b in (di, dv, dz):
            b.free()
    assert True in seen  # the test can tell the two uniforms apart
    for b in (d_st, d_rec, d_vtok, d_rnd):
        b.free()


def test_rows_choose_matches_oracle(ctx):
    g = np.random.default_rng(9)
    d_st = ctx.to_device(np.zeros(8, np.uint32))
    for _ in range(40):
        kmax = int(g.integers(2, 18))
        kmin = int(g.integers(2, kmax + 1))
        conf = g.random(16).astype(np.float32)
        p = RowsParams(kmin=kmin, kmax=kmax)
        a = g.normal(1, 0.3, 4).astype(np.float32)
        b = g.normal(0, 0.5, 4).astype(np.float32)
        cost = np.concatenate([[1e9, 1e9], 1 + np.cumsum(g.random(16))]).astype(np.float32)
        for i in range(4):
            p.a[i], p.b[i] = float(a[i]), float(b[i])
        for i in range(18):
            p.cost[i] = float(cost[i])
        dc = ctx.to_device(conf)
        check(lib().ih_spec_rows_choose_dev(ctx.handle, d_st.ptr, dc.ptr, C.byref(p)))
        got = int(d_st.download(np.uint32, (8,))[6])
        assert got == oracle.rows_choose(conf, a, b, cost, kmin, kmax)
        dc.free()
    d_st.free()


SMALL = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, vocab=1000)


def test_sampling_decode(ctx):
    """top-k 1 is greedy: the sampling loop gives the greedy tokens; a seed reproduces its tokens; copy drafts do not
    change the sampled tokens (the same uniforms per round are not guaranteed across row counts, so this compares the
    distribution's support: every token is among its row's candidates with non-zero probability)."""
    d = ModelDesc.make(**SMALL)
    m = Model(ctx, d, 7)
    kv = KVCache(m, 1024)
    try:
        kv.fill_synthetic(300, 11)
        greedy, _ = kv.decode_greedy(17, 30, rows=1)
        kv.set_pos(300)
        t1, _ = kv.decode_sample(17, 30, SampleParams(temp=0.7, top_p=1.0, top_k=1, min_p=0.0), seed=1, rows=4,
                                 history=np.zeros(300, np.uint32), inflight=3)
        assert t1 == greedy
        kv.set_pos(300)
        p = SampleParams(temp=1.0, top_p=0.95, top_k=0, min_p=0.0)
        a, sa = kv.decode_sample(17, 40, p, seed=42, rows=1, inflight=2)
        kv.set_pos(300)
        b, _ = kv.decode_sample(17, 40, p, seed=42, rows=1, inflight=1)
        assert a == b and sa.emitted == 40 and kv.pos == 300 + 39
        kv.set_pos(300)
        c, _ = kv.decode_sample(17, 40, p, seed=43, rows=1, inflight=2)
        assert c != a  # another seed, other tokens (1000-token vocabulary, 39 draws)
    finally:
        kv.free()
        m.free()
