"""Chained greedy decoding with the round state on the device (ih_decode_greedy, ih_verify_step_chained) against
plain one-row greedy decoding on the host path.

Reference behaviour: decodeSpec (Sources/Ingot/Generate.swift:240-504) enqueues round N+1 before round N's acceptance is
read; its output is exactly greedy decoding (docs/adr/0002; gen --check), and the rounds enqueued past the stop are
rolled back (rewindExtraRound, Generate.swift:515-540) so the next call continues from the last emitted token.
"""
import numpy as np
import pytest

from ingot_amd._lib import FINISH_CONTEXT, FINISH_LENGTH, FINISH_STOP, KVCache, Model, ModelDesc, check, lib

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, vocab=1000)
SWA = dict(n_layers=2, hidden=512, n_q_heads=8, n_kv_heads=1, head_dim=64, intermediate=256, vocab=777, sinks=1,
           sliding_window=16)
P0 = 300


def setup(ctx, shape, cap=1024, chunk=0):
    d = ModelDesc.make(**shape)
    m = Model(ctx, d, 7)
    kv = KVCache(m, cap, chunk)
    kv.fill_synthetic(P0, 11)
    return d, m, kv


def plain(kv, first, n):
    """n greedy tokens after `first` by one-row verify + accept + commit, from P0; leaves the cache at P0."""
    kv.set_pos(P0)
    toks, t = [], first
    for _ in range(n):
        t = kv.verify_and_accept([t]).tokens[0]
        toks.append(int(t))
    kv.set_pos(P0)
    return toks


@pytest.mark.parametrize("shape", [SMALL, SWA], ids=["gqa2", "swa16-sinks"])
@pytest.mark.parametrize("inflight", [1, 3])
def test_chained_plain_rounds_equal_plain_decode(ctx, shape, inflight):
    d, m, kv = setup(ctx, shape)
    try:
        first = 17
        ref = plain(kv, first, 24)
        out, st = kv.decode_greedy(first, 25, rows=1, inflight=inflight)
        assert out == [first] + ref
        assert st.finish == FINISH_LENGTH and st.rounds == 24 and st.emitted == 25
        assert kv.pos == P0 + 24  # the last emitted token is the next anchor, its K/V not committed
        # The next call continues from it.
        out2, _ = kv.decode_greedy(out[-1], 6, rows=1, inflight=inflight)
        kv.set_pos(P0)
        more = plain(kv, first, 29)
        assert out2 == [out[-1]] + more[24:29]
    finally:
        kv.free()
        m.free()


@pytest.mark.parametrize("shape", [SMALL, SWA], ids=["gqa2", "swa16-sinks"])
@pytest.mark.parametrize("rows,inflight", [(8, 1), (8, 3), (17, 2)])
def test_chained_copy_rounds_equal_plain_decode(ctx, shape, rows, inflight):
    """Copy drafts from a history in which the greedy continuation was planted: drafts are accepted (fewer rounds than
    tokens) and the output is still exactly greedy decoding; a history with nothing to copy gives the same tokens."""
    d, m, kv = setup(ctx, shape)
    try:
        first = 23
        ref = plain(kv, first, 40)
        g = np.random.default_rng(rows)
        hist = g.integers(0, d.vocab, size=P0).astype(np.uint32)
        q = 120
        hist[q - 2], hist[q - 1], hist[q] = hist[P0 - 2], hist[P0 - 1], first
        hist[q + 1: q + 1 + 40] = ref
        out, st = kv.decode_greedy(first, 41, rows=rows, history=hist, inflight=inflight)
        assert out == [first] + ref
        assert st.accepted > 0 and st.rounds < 40, (st.rounds, st.accepted)
        assert kv.pos == P0 + 40
        kv.set_pos(P0)
        noise = g.integers(0, d.vocab, size=P0).astype(np.uint32)
        out2, _ = kv.decode_greedy(first, 41, rows=rows, history=noise, inflight=inflight)
        assert out2 == out
    finally:
        kv.free()
        m.free()


def test_stop_token_and_context_end(ctx):
    d, m, kv = setup(ctx, SMALL, cap=P0 + 40)
    try:
        first = 5
        ref = plain(kv, first, 20)
        stop = ref[6]
        j = ref.index(stop)  # the first occurrence ends the output
        out, st = kv.decode_greedy(first, 30, rows=4, history=np.zeros(P0, np.uint32), stop=[stop], inflight=3)
        assert out == [first] + ref[: j + 1] and st.finish == FINISH_STOP
        assert kv.pos == P0 + j + 1
        # Context end: the cache holds P0 + 40 positions.
        kv.set_pos(P0)
        out, st = kv.decode_greedy(first, 100, rows=1, inflight=2)
        assert st.finish == FINISH_CONTEXT
        assert out[: 21] == [first] + ref
        assert kv.pos <= kv.capacity
    finally:
        kv.free()
        m.free()


def test_chained_step_flags_a_position_outside_its_range(ctx):
    """ih_verify_step_chained launched for [pos_min, pos_max] with the device position beyond it: st[7] = 1 and the
    cache is not written past its end."""
    d, m, kv = setup(ctx, SMALL, cap=P0 + 40)
    try:
        st = np.zeros(8, np.uint32)
        st[0] = P0 + 39  # beyond pos_max; P + B would pass the capacity
        dst = ctx.to_device(st)
        tok = ctx.to_device(np.full(4, 3, np.uint32))
        top = ctx.buffer(16)
        check(lib().ih_verify_step_chained(m.handle, kv.handle, tok.ptr, 4, top.ptr, dst.ptr, P0, P0 + 8))
        ctx.sync()
        assert dst.download(np.uint32, (8,))[7] == 1
        for b in (dst, tok, top):
            b.free()
    finally:
        kv.free()
        m.free()
