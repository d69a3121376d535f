"""Device argmax and device acceptance, called directly through the C ABI, against the oracle and brute force.

argmax_rows: Sources/Ingot/Shaders/verify.metal:525-547 (scan from (−inf, 0) with a strict >, so ties go to the lowest
index, NaN never wins and a row of only −inf/NaN gives 0). spec_accept: Sources/Ingot/Shaders/yy_model.metal:616-642
(st = [P, nacc, pend, pendPos, anchor, round, rows], rec[round % ring] = m, tokens, [20] = P before, [21] = rows).
"""
import numpy as np
import pytest

import oracle
from ingot_amd._lib import check, lib

pytestmark = pytest.mark.gpu

CHUNKS = 16  # chunks per row of the device argmax (argmax_chunk_kernel)


def gpu_argmax(ctx, x: np.ndarray) -> np.ndarray:
    rows, N = x.shape
    dx = ctx.to_device(np.ascontiguousarray(x, np.float32))
    out = ctx.buffer(rows * 4)
    check(lib().ih_argmax_rows(ctx.handle, dx.ptr, rows, N, out.ptr))
    r = out.download(np.uint32, (rows,))
    dx.free()
    out.free()
    return r


def planted_rows(N: int, rows: int, seed: int) -> np.ndarray:
    """N(0,1) rows with the edge cases the reduction order could get wrong, one per row (cycling)."""
    g = np.random.default_rng(seed)
    x = g.normal(0, 1, size=(rows, N)).astype(np.float32)
    per = (N + CHUNKS - 1) // CHUNKS
    for r in range(rows):
        case = r % 9
        row = x[r]
        if case == 0:  # tie across a chunk boundary: the earlier chunk's index wins
            i = per * 3 - 1
            row[i] = row[i + 1] = 9.0
        elif case == 1:  # tie inside one chunk, 4 apart (same lane, different 16-byte loads) and 1 apart
            i = per * 5 + 17
            row[[i, i + 1, i + 4]] = 7.5
        elif case == 2:  # NaN everywhere except one value
            row[:] = np.nan
            row[N // 2 + 3] = -1e30
        elif case == 3:  # all −inf: index 0
            row[:] = -np.inf
        elif case == 4:  # NaN mixed with −inf: index 0 (−inf never takes an index)
            row[:] = -np.inf
            row[::7] = np.nan
        elif case == 5:  # +0 and −0 the maximum of a negative row: the lowest of them
            row[:] = -np.abs(row) - 1.0
            row[N - 1] = 0.0
            row[per * 9 + 2] = -0.0
            row[per * 12] = 0.0
        elif case == 6:  # the maximum at the very last index, +inf elsewhere absent
            row[N - 1] = 50.0
        elif case == 7:  # +inf twice: the first
            row[per * 2 + 40] = np.inf
            row[per * 14 + 1] = np.inf
        else:  # the maximum at index 0 behind a NaN at index 1
            row[0] = 20.0
            row[1] = np.nan
    return x


@pytest.mark.parametrize("rows,N", [(8, 32000), (17, 151936), (9, 201088), (9, 1000)])
def test_argmax_rows_edge_cases(ctx, rows, N):
    x = planted_rows(N, rows, seed=N + rows)
    got = gpu_argmax(ctx, x)
    want = oracle.argmax_rows(x)
    assert np.array_equal(got, want), (got, want)
    # The oracle against the closed form on the finite rows (no NaN / ±inf): numpy's first maximum.
    finite = np.all(np.isfinite(x), axis=1)
    assert np.array_equal(want[finite], np.argmax(x[finite], axis=1).astype(np.uint32))


@pytest.mark.parametrize("rows,N", [(3, 17), (2, 1), (17, 5), (4, 63)])
def test_argmax_rows_short_rows(ctx, rows, N):
    """Rows shorter than the 16 chunks (empty chunks) with NaN, ±inf, −0 and ties drawn at random, many seeds."""
    g = np.random.default_rng(N)
    for _ in range(20):
        x = g.choice(np.array([np.nan, -np.inf, np.inf, -0.0, 0.0, 1.0, 2.0, -1.0], np.float32), size=(rows, N))
        assert np.array_equal(gpu_argmax(ctx, x), oracle.argmax_rows(x))


def test_argmax_rows_random_full_vocab(ctx):
    """Config 1's head output shape [17, 151936] on random rows with many exact ties (values on a coarse grid)."""
    g = np.random.default_rng(1)
    x = np.round(g.normal(0, 1, size=(17, 151936)) * 4).astype(np.float32)
    assert np.array_equal(gpu_argmax(ctx, x), oracle.argmax_rows(x))
    assert np.array_equal(gpu_argmax(ctx, x), np.argmax(x, axis=1).astype(np.uint32))


REC_STRIDE, REC_P, REC_ROWS = 24, 20, 21


def brute_accept(vtok, top1, nr):
    m = 0
    for j in range(nr):
        if all(vtok[i + 1] == top1[i] for i in range(j)):
            m = j
    return m


@pytest.mark.parametrize("ring", [4, 64])
def test_spec_accept_dev_chained_rounds(ctx, ring):
    """Rounds of device acceptance on one state: B = 1…17 (and rows = 0, read from st[6]) with planted agreeing
    prefixes; st, rec[round % ring] (through the ring's wrap) and vtok[0] after every round against brute force and
    oracle.accept."""
    g = np.random.default_rng(ring)
    st = np.zeros(8, np.uint32)
    st[0] = 1000
    d_st = ctx.to_device(st)
    d_vtok = ctx.buffer(17 * 4)
    d_top1 = ctx.buffer(17 * 4)
    d_rec = ctx.buffer(ring * REC_STRIDE * 4).fill(0)
    want_rec = np.zeros((ring, REC_STRIDE), np.uint32)
    try:
        for rnd in range(40):
            B = 1 + rnd % 17
            use_state_rows = rnd % 3 == 2
            top1 = g.integers(0, 50, size=17).astype(np.uint32)
            vtok = g.integers(0, 50, size=17).astype(np.uint32)
            L = int(g.integers(0, B))  # drafts 1..L agree
            vtok[1 : L + 1] = top1[:L]
            if L + 1 < 17:
                vtok[L + 1] = (top1[L] + 1) % 50
            d_vtok.upload(vtok)
            d_top1.upload(top1)
            if use_state_rows:
                st[6] = B
                d_st.upload(st)
            check(lib().ih_spec_accept_dev(ctx.handle, d_st.ptr, d_vtok.ptr, d_top1.ptr, d_rec.ptr, ring,
                                           0 if use_state_rows else B))
            m = brute_accept(vtok, top1, B)
            om, em = oracle.accept(vtok[:B], top1[:B])
            assert m == om == min(L, B - 1)
            rec_row = want_rec[st[5] % ring]
            # Words past the emitted tokens keep what an earlier round of this slot left (the kernel writes only these).
            rec_row[0] = m
            rec_row[1 : m + 2] = em
            rec_row[REC_P] = st[0]
            rec_row[REC_ROWS] = B
            st[3] = st[0]
            st[2] = m + 1
            st[0] += m + 1
            st[1] = m + 1
            st[4] = top1[m]
            st[5] += 1
            got_st = d_st.download(np.uint32, (8,))
            assert np.array_equal(got_st, st), (rnd, got_st, st)
            got_vtok = d_vtok.download(np.uint32, (17,))
            assert got_vtok[0] == top1[m]
            assert np.array_equal(got_vtok[1:], vtok[1:])
            got_rec = d_rec.download(np.uint32, (ring, REC_STRIDE))
            assert np.array_equal(got_rec, want_rec), (rnd, got_rec[(st[5] - 1) % ring], want_rec[(st[5] - 1) % ring])
    finally:
        for b in (d_st, d_vtok, d_top1, d_rec):
            b.free()


def test_spec_accept_dev_state_rows_are_clamped(ctx):
    """rows = 0 with st[6] beyond IH_MAX_ROWS (or 0) is clamped to 1…17: nothing past the 17 rows is read or written."""
    for bad, nr in ((1000, 17), (0, 1)):
        st = np.zeros(8, np.uint32)
        st[6] = bad
        top1 = np.arange(17, dtype=np.uint32)
        vtok = np.concatenate([[99], top1[:16]]).astype(np.uint32)  # all 16 drafts agree
        d_st, d_vtok, d_top1 = ctx.to_device(st), ctx.to_device(vtok), ctx.to_device(top1)
        d_rec = ctx.buffer(2 * REC_STRIDE * 4).fill(0xAB)
        check(lib().ih_spec_accept_dev(ctx.handle, d_st.ptr, d_vtok.ptr, d_top1.ptr, d_rec.ptr, 1, 0))
        rec = d_rec.download(np.uint32, (2, REC_STRIDE))
        got = d_st.download(np.uint32, (8,))
        assert rec[0][0] == nr - 1 and rec[0][REC_ROWS] == nr
        assert got[0] == nr and got[4] == top1[nr - 1]
        assert np.all(rec[1] == 0xABABABAB)  # the next record is untouched
        for b in (d_st, d_vtok, d_top1, d_rec):
            b.free()
