"""The DFlash2 drafter behind the C ABI (ih_drafter_*) and the verify step's hidden-state captures, against the
oracle's restatement (oracle.OracleDrafter) on the same synthetic weights and the same captured rows.

Reference: DFlash2Drafter.encodeContext / encodeBlock (Sources/Ingot/Drafter.swift:300-550), capture_rows, dctx_write,
dattn_*, dconv_*, topk16_rows, dselect, dpick_top1 (Shaders/yy_model.metal:94-104,151-614); the chained DFlash2 rounds of
decodeSpec (Generate.swift:240-504), whose output is exactly greedy decoding whatever the drafts.
"""
import numpy as np
import pytest

import oracle
from ingot_amd._lib import Drafter, DrafterDesc, KVCache, Model, ModelDesc
from synth import cosine

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, vocab=1000)
DF2 = dict(n_layers=2, hidden=256, n_q_heads=8, head_dim=64, intermediate=256, block=8, window=32, rank=64,
           dyn_conv=1, mask_token=999)
DF1 = dict(DF2, rank=0, dyn_conv=0, n_q_heads=16, head_dim=128, block=4, window=64)


def bf16f(a):
    return oracle.bf16_to_f32(a).astype(np.float64)


def test_captures_match_oracle(ctx):
    d = ModelDesc.make(**SMALL)
    m = Model(ctx, d, 7)
    kv = KVCache(m, 512)
    dr = Drafter(m, DrafterDesc.make(targets=(0, 1), **DF2), 5)
    try:
        kv.fill_synthetic(100, 11)
        dr.attach()
        toks = np.random.default_rng(2).integers(0, d.vocab, size=17).astype(np.uint32)
        kv.verify(toks)
        got = dr.captures(17)
        om = oracle.OracleModel(d, 7, 11, 100)
        om.set_capture([0, 1])
        om.verify(toks)
        want = om.captures(17)
        om.free()
        g, w = bf16f(got), bf16f(want)
        assert np.abs(g - w).max() <= 1e-2 * np.abs(w).max() and cosine(g, w) >= 0.9999
    finally:
        dr.free()
        kv.free()
        m.free()


@pytest.mark.parametrize("shape", [DF2, DF1], ids=["dflash2", "dflash-v1"])
def test_drafter_block_matches_oracle(ctx, shape):
    """The GPU's own captures as context (three writes of 17 rows: the 32-position window wraps), then a block at
    P = 51: drafts bit-exact, confidences within 1e-2 (a confidence is softmax(score/1.5) over the 16 candidates,
    and the scores carry the head's logit error, ~0.02 at bf16 activations: ∂conf/∂s ≤ 1/(4·1.5) per candidate)."""
    d = ModelDesc.make(**SMALL)
    m = Model(ctx, d, 7)
    kv = KVCache(m, 512)
    dd = DrafterDesc.make(targets=(0, 1), **shape)
    dr = Drafter(m, dd, 5)
    od = oracle.OracleDrafter(dd, 5, d, 7)
    try:
        kv.fill_synthetic(100, 11)
        dr.attach()
        toks = np.random.default_rng(4).integers(0, d.vocab, size=17).astype(np.uint32)
        kv.verify(toks)
        caps = dr.captures(17)
        for pos0 in (0, 17, 34):
            dr.context(17, 17, pos0)
            od.context(caps, 17, pos0)
        for anchor, P in ((int(toks[3]), 51), (17, 51), (int(toks[9]), 40)):
            gd, gc = dr.block(anchor, P)
            odr, oc = od.block(anchor, P)
            assert list(gd) == list(odr), (anchor, P, gd, odr)
            assert np.abs(gc - oc).max() <= 1e-2, (gc, oc)
    finally:
        od.free()
        dr.free()
        kv.free()
        m.free()


@pytest.mark.parametrize("inflight", [1, 3])
def test_drafter_rounds_equal_plain_decode(ctx, inflight):
    """Chained DFlash2 rounds (context of the last accepted rows → block → verify → accept, all on the device state)
    emit exactly the greedy tokens."""
    d = ModelDesc.make(**SMALL)
    m = Model(ctx, d, 7)
    kv = KVCache(m, 1024)
    dr = Drafter(m, DrafterDesc.make(targets=(0, 1), **DF2), 5)
    try:
        kv.fill_synthetic(300, 11)
        ref = []
        t = 17
        for _ in range(30):
            t = kv.verify_and_accept([t]).tokens[0]
            ref.append(int(t))
        kv.set_pos(300)
        dr.attach()
        out, st = kv.decode_greedy(17, 31, rows=8, inflight=inflight, drafter=dr)
        assert out == [17] + ref
        assert st.drafted == 7 * st.rounds and kv.pos == 330
    finally:
        dr.free()
        kv.free()
        m.free()


@pytest.mark.parametrize("kmin,kmax", [(4, 4), (2, 8)])
def test_row_chooser_rounds_equal_plain_decode(ctx, kmin, kmax):
    """DFlash2 rounds whose verify rows are chosen on the device from the drafts' confidences (spec_rows_choose,
    yy_model.metal:644-675) still emit exactly the greedy tokens; the rounds' records carry the chosen rows (a fixed
    choice k gives k − 1 drafts a round), and temperature sampling at top-k 1 is the same greedy output."""
    from ingot_amd._lib import RowsParams, SampleParams
    d = ModelDesc.make(**SMALL)
    m = Model(ctx, d, 7)
    kv = KVCache(m, 1024)
    dr = Drafter(m, DrafterDesc.make(targets=(0, 1), **DF2), 5)
    rp = RowsParams(kmin=kmin, kmax=kmax)
    for g in range(4):
        rp.a[g], rp.b[g] = 1.0, 0.5 - 0.25 * g
    for k in range(18):
        rp.cost[k] = 1.0 + 0.15 * k
    try:
        kv.fill_synthetic(300, 11)
        ref = []
        t = 17
        for _ in range(30):
            t = kv.verify_and_accept([t]).tokens[0]
            ref.append(int(t))
        kv.set_pos(300)
        dr.attach()
        out, st = kv.decode_greedy(17, 31, rows=8, inflight=2, drafter=dr, rows_params=rp)
        assert out == [17] + ref and kv.pos == 330
        assert (kmin - 1) * st.rounds <= st.drafted <= (kmax - 1) * st.rounds
        if kmin == kmax:
            assert st.drafted == (kmin - 1) * st.rounds
        kv.set_pos(300)
        out2, _ = kv.decode_sample(17, 31, SampleParams(temp=0.8, top_p=1.0, top_k=1, min_p=0.0), seed=3, rows=8,
                                   inflight=2, drafter=dr, rows_params=rp)
        assert out2 == out
    finally:
        dr.free()
        kv.free()
        m.free()


def test_drafter_outliving_its_model_refuses_work(ctx):
    """Freeing the target model first orphans its drafters: their calls return IH_EINVAL instead of touching the freed
    model, and freeing them afterwards is still fine."""
    from ingot_amd._lib import IngotError
    d = ModelDesc.make(**SMALL)
    m = Model(ctx, d, 7)
    dr = Drafter(m, DrafterDesc.make(targets=(0, 1), **DF2), 5)
    dr.attach()
    m.free()
    with pytest.raises(IngotError) as e:
        dr.context(4, 4, 0)
    assert "freed" in str(e.value)
    dr.free()
