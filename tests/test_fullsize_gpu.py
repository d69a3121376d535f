"""The whole verify step at the benchmark configurations' full sizes on the GPU against the CPU oracle.

Config 1 exactly (32 layers, hidden 4096, vocab 151936, B = 17, P = 8192), config 2's verify (the same model at
P = 32768) and full-width two-layer slices of configs 3 (E128 top-8 int4 MoE, P = 16384) and 4 (MXFP4 MoE with sinks
and the alternating 128-key window, B = 9, P = 65536). Logits against the oracle's fp32 within the stated tolerance,
top-1 bit-exact on every row whose oracle top-2 margin exceeds twice the logit error (the rows inside it are counted
and reported), and the accepted prefix of a greedy chain planted as drafts bit-exact against oracle.accept on the
oracle's own top-1. The reference's own checks of these properties: the attention round vs CPU
(Tests/IngotTests/KernelCaseTests.swift:178-206) and rowscheck / gen --check (Sources/ingot-dev/Checks/RowsCheck.swift).
"""
import json
import os
import time

import numpy as np
import pytest

import oracle
from ingot_amd._lib import Drafter, DrafterDesc, KVCache, Model, ModelDesc, accept, check, lib
from synth import cosine

pytestmark = pytest.mark.gpu

DENSE8B = dict(n_layers=32, hidden=4096, n_q_heads=32, n_kv_heads=8, head_dim=128, intermediate=14336, vocab=151936)
# The MoE configurations' routing: router logits ~N(0,1) per layer and row (iid_routing), U ≈ 85 of 128 / ≈ 22 of 32.
MOE3 = dict(n_layers=2, hidden=2048, n_q_heads=32, n_kv_heads=4, head_dim=128, intermediate=0, vocab=151936,
            n_experts=128, top_k=8, expert_intermediate=768, expert_format=0, iid_routing=1)
MOE4 = dict(n_layers=2, hidden=2880, n_q_heads=64, n_kv_heads=8, head_dim=64, intermediate=0, vocab=201088,
            n_experts=32, top_k=4, expert_intermediate=2880, expert_format=1, router_bias=1, expert_bias=1, act=1,
            sinks=1, sliding_window=128, iid_routing=1)
CASES = {
    "cfg1-dense8b-P8192": (DENSE8B, 8192, 17),
    "cfg2-dense8b-P32768": (DENSE8B, 32768, 17),
    "cfg3-moe-e128-2L-P16384": (MOE3, 16384, 17),
    "cfg4-mxfp4-moe-2L-P65536": (MOE4, 65536, 9),
}
SEED, KV_SEED = 2026, 11

# Logits tolerance. Dense: max-abs ≤ 1% of max |ref| and cosine ≥ 0.9999. Both sides round the activations to bf16
# at the same points, so the difference is the occasional one-ulp flip of a bf16 (2^-8 relative) or of an int8 KV
# level where the pre-rounding values differ in the last fp32 bits; at config 1's logit scale (~70) one bf16 ulp of a
# logit is 0.25–0.5.
# MoE (the configurations' i.i.d. routing, identical on both sides): cosine ≥ 0.9999 and max-abs ≤ 1e-3 of the scale
# or, where the function itself is less well conditioned than that, 1.5 × how far the oracle's own logits move when
# RoPE θ changes by one part in 10^7 (which flips the same kind of last-bit roundings). Config 4's MXFP4 experts
# (weights up to 1.5 over 2880 inputs) move the oracle by 3–5e-3 of the scale that way; config 3's by ~5e-4.
TOL = {"dense": (0.01, 0.9999), "moe": (1e-3, 0.9999)}


def oracle_sensitivity(d, shape, P, toks, ref_logits):
    """Max-abs change of the oracle's logits under RoPE θ·(1 ± 1e-7)."""
    sens = 0.0
    for eps in (1e-7, -1e-7):
        alt = ModelDesc.make(**shape)
        alt.rope_theta = d.rope_theta * (1 + eps)
        om = oracle.OracleModel(alt, SEED, KV_SEED, P)
        other, _ = om.verify(toks)
        om.free()
        sens = max(sens, float(np.abs(other - ref_logits).max()))
    return sens


def report(name, **kv):
    """Measured figures of a case, printed and appended to gpurun_out/fullsize.jsonl when that folder exists."""
    line = json.dumps({"case": name, **kv})
    print(line, flush=True)
    if os.path.isdir("gpurun_out"):
        with open("gpurun_out/fullsize.jsonl", "a") as f:
            f.write(line + "\n")


@pytest.mark.parametrize("name", list(CASES))
def test_fullsize_verify_matches_oracle(ctx, name):
    shape, P, B = CASES[name]
    print(f"[fullsize] {name}: building", flush=True)
    d = ModelDesc.make(**shape)
    m = Model(ctx, d, SEED)
    kv = KVCache(m, P + 2 * B)
    try:
        kv.fill_synthetic(P, KV_SEED)
        toks = np.random.default_rng(P + B).integers(0, d.vocab, size=B).astype(np.uint32)
        top1, logits = kv.verify(toks, want_logits=True)
        union = None
        if shape.get("n_experts"):
            u = np.zeros(d.n_layers, np.int32)
            check(lib().ih_model_moe_union(m.handle, u.ctypes.data))
            union = u.tolist()
        t0 = time.time()
        om = oracle.OracleModel(d, SEED, KV_SEED, P)
        t1 = time.time()
        ref_logits, ref_top1 = om.verify(toks)
        t2 = time.time()
        err = float(np.abs(logits - ref_logits).max())
        cos = cosine(logits, ref_logits)
        scale = float(np.abs(ref_logits).max())
        srt = np.sort(ref_logits, axis=1)
        margin = srt[:, -1] - srt[:, -2]
        sure = margin > 2 * err
        flips = int(np.sum(top1[sure] != ref_top1[sure]))
        near_ties = int(np.sum(~sure))
        near_tie_flips = int(np.sum(top1[~sure] != ref_top1[~sure]))
        # How far the oracle moves when its attention rounds p·vs to fp16, as the reference and the GPU do, reported next
        # to the error (configs 3 and 4: 0.020 and 0.115 against GPU errors of 0.021 and 0.13 at logit scales of 42 and
        # 44), and the GPU's distance from that variant (0.022 and 0.114: no closer — its own fp16 roundings are another
        # draw of the same size).
        with oracle.attn_p16():
            p16_logits, _ = om.verify(toks)
        p16_spread = float(np.abs(p16_logits - ref_logits).max())
        err_p16 = float(np.abs(logits - p16_logits).max())  # against the oracle at the reference's rounding point
        report(name, max_abs=err, rel=err / scale, cosine=cos, scale=scale, p16_spread=p16_spread, max_abs_p16=err_p16,
               near_tie_rows=near_ties,
               near_tie_flips=near_tie_flips, flips=flips, moe_union=union, oracle_build_s=round(t1 - t0, 2),
               oracle_step_s=round(t2 - t1, 2), top1=top1.tolist(), ref_top1=ref_top1.tolist())
        rel_tol, cos_tol = TOL["moe" if shape.get("n_experts") else "dense"]
        bound = rel_tol * scale
        if shape.get("n_experts"):
            sens = oracle_sensitivity(d, shape, P, toks, ref_logits)
            report(name + " conditioning", oracle_sensitivity=sens, rel_sensitivity=sens / scale)
            bound = max(bound, 1.5 * sens)
        assert err <= bound and cos >= cos_tol, (err, bound, scale, cos)
        if not shape.get("n_experts"):
            # The north star's example bound for the dense configurations: max-abs ≤ 2e-2 against the fp32 oracle
            # (measured 0.009–0.013 at logit scale ~70).
            assert err <= 2e-2, err
        assert flips == 0, (top1, ref_top1, margin, err)
        assert np.array_equal(top1, np.argmax(logits, axis=1).astype(np.uint32))

        # Greedy chain planted as drafts: iterate block[i + 1] = top1[i] until it is a fixed point (row i's top-1 depends
        # only on rows ≤ i, so B − 1 iterations suffice), then the oracle's top-1 on that block must give the same
        # accepted prefix, all B − 1 drafts; with a wrong draft planted at L, both accept exactly L. A row whose
        # oracle top-2 margin is inside twice the block's logit error may flip (a near tie): the accepted prefix must
        # then agree up to the first such row, and the case is reported.
        blk = toks.copy()
        for _ in range(B - 1):
            t = kv.verify(blk)
            blk[1:] = t[:-1]
        gt, gl = kv.verify(blk, want_logits=True)
        assert np.array_equal(blk[1:], gt[:-1])
        ol, ot = om.verify(blk)
        berr = float(np.abs(gl - ol).max())
        bs = np.sort(ol, axis=1)
        tie = (bs[:, -1] - bs[:, -2]) <= 2 * berr
        first_tie = int(np.argmax(tie)) if tie.any() else B
        assert np.array_equal(gt[~tie], ot[~tie])
        gm, om_m = accept(blk, gt).m, oracle.accept(blk, ot)[0]
        report(name + " chain", block_max_abs=berr, near_tie_rows=tie.nonzero()[0].tolist(), gpu_m=gm, oracle_m=om_m,
               distinct_tokens=len(set(blk.tolist())), chain=blk.tolist())
        assert gm == B - 1
        assert om_m == B - 1 or om_m >= first_tie
        L = B // 3
        bad = blk.copy()
        bad[L + 1] = (bad[L + 1] + 1) % d.vocab
        gb = kv.verify(bad)
        _, ob = om.verify(bad)
        r = accept(bad, gb)
        om_, oem = oracle.accept(bad, ob)
        assert r.m == L
        if first_tie >= L:
            assert om_ == L and r.emitted[:L] == list(oem[:L])
        om.free()
        assert kv.pos == P
    finally:
        kv.free()
        m.free()


def test_fullsize_drafter_block_matches_oracle(ctx):
    """The DFlash2 drafter of the bench's decode loop at its full shape (5 layers at config 1's hidden size, 32 q heads
    of 128, intermediate 12288, block 16, window 2048, rank 256, captures of target layers 1, 7, 13, 19, 25) on config
    1's target: the GPU's captures of a 17-row verify step at P = 8192 as context (three writes), then blocks at
    P = 51, against oracle.OracleDrafter on the same captures: drafts bit-exact (measured: equal, with confidences
    within 1e-3), confidences within 2e-2 (a confidence is softmax(score/1.5) over the 16 candidates; the scores carry
    the head's logit error, ~0.01 at config 1)."""
    print("[fullsize] drafter: building", flush=True)
    d = ModelDesc.make(**DENSE8B)
    m = Model(ctx, d, SEED)
    P = 8192
    kv = KVCache(m, P + 64)
    dd = DrafterDesc.make(targets=(1, 7, 13, 19, 25), n_layers=5, hidden=4096, n_q_heads=32, head_dim=128,
                          intermediate=12288, block=16, window=2048, rank=256, dyn_conv=1, mask_token=d.vocab - 1)
    dr = Drafter(m, dd, SEED + 1)
    od = oracle.OracleDrafter(dd, SEED + 1, d, SEED)
    try:
        kv.fill_synthetic(P, KV_SEED)
        dr.attach()
        toks = np.random.default_rng(5).integers(0, d.vocab, size=17).astype(np.uint32)
        kv.verify(toks)
        caps = dr.captures(17)
        for pos0 in (0, 17, 34):
            dr.context(17, 17, pos0)
            od.context(caps, 17, pos0)
        for anchor in (int(toks[3]), int(toks[11])):
            gd, gc = dr.block(anchor, 51)
            odr, oc = od.block(anchor, 51)
            report("drafter-fullsize", anchor=anchor, drafts=[int(x) for x in gd], oracle_drafts=[int(x) for x in odr],
                   conf_max_abs=float(np.abs(gc - oc).max()))
            assert list(gd) == list(odr), (anchor, gd, odr)
            assert np.abs(gc - oc).max() <= 2e-2, (gc, oc)
    finally:
        od.free()
        dr.free()
        kv.free()
        m.free()
