"""The whole verify step on the GPU against the CPU oracle, on small synthetic dense models.

Reference behaviour: HybridModel.encodeVerify (Sources/Ingot/ModelRound.swift:48-82) and the greedy acceptance /
commit of generateSpec (Sources/Ingot/Generate.swift:104-177). The reference's own checks of the same properties are
the attention round vs CPU (Tests/IngotTests/KernelCaseTests.swift:178-206, maxRel 5e-3), row invariance
(KernelCaseTests.swift:66-86) and rowscheck / gen --check (Sources/ingot-dev/Checks/RowsCheck.swift:6-50).
"""
import numpy as np
import pytest

import oracle
from ingot_amd._lib import Context, KVCache, Model, ModelDesc, accept, check, lib
from synth import cosine

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, vocab=1000)
GQA8 = dict(n_layers=2, hidden=512, n_q_heads=8, n_kv_heads=1, head_dim=64, intermediate=256, vocab=777)
# MoE like config 3 (int4 experts, softmax top-k, SiLU) and like config 4 (MXFP4 experts with router and expert biases,
# swiglu_oai, attention sinks, alternating sliding-window layers; hidden 192 and expert width 96 leave partial
# K-blocks).
MOE4 = dict(n_layers=1, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128, intermediate=0, vocab=1000,
            n_experts=8, top_k=2, expert_intermediate=128, expert_format=0)
SWA = dict(GQA8, sinks=1, sliding_window=16)
# Config 1's grouping (4 q heads per KV head): 17 rows make 68 query rows, five 16-row tiles, the fifth shared by
# four waves of the attention workgroup.
GQA4 = dict(n_layers=2, hidden=512, n_q_heads=8, n_kv_heads=2, head_dim=128, intermediate=256, vocab=1000)
MOEX = dict(n_layers=1, hidden=192, n_q_heads=8, n_kv_heads=2, head_dim=64, intermediate=0, vocab=777, n_experts=8,
            top_k=4, expert_intermediate=96, expert_format=1, router_bias=1, expert_bias=1, act=1, sinks=1,
            sliding_window=16)


def logits_close(got, ref):
    """(max-abs error, cosine) of GPU logits against the fp32 oracle."""
    err = np.abs(got - ref).max()
    return err, cosine(got, ref)


# Logits tolerance: max-abs ≤ 0.02 + 1% of max|ref|, cosine ≥ 0.9999. Both sides round the activations to bf16 at the
# same points (norm outputs, attention output, gated activation); the GPU also rounds each attention probability × V
# scale to fp16 before it weights V, as the reference does (verify_attn_pf.metal:273), where the oracle stays fp32. At
# these small shapes that rounding point dominates: switching it on in the oracle moves the logits by 0.03–0.06 at
# logit scale 8–10 (oracle.attn_rounding_spread), and the GPU's own draw of it differs from the oracle by 1.3–2.2 ×
# that; the occasional one-ulp flip of a bf16 or int8 KV level adds less (the oracle moves by ~0.01 when RoPE θ
# changes by one part in 10^7).
def within_tol(err, cos, scale):
    return err <= 0.02 + 0.01 * scale and cos >= 0.9999


# MoE models: max-abs ≤ 0.05 + 3% of max|ref|, cosine ≥ 0.999. The softmax router turns one-ulp rounding differences
# of its input into changed expert weights, and near a routing tie into a changed expert: the oracle against itself
# moves by 0.16 at logit scale 5 for one config-4-like token when RoPE θ changes by one part in 10^6, and by 0.08 for
# the two-layer config-3-like model at one part in 10^7 (test_oracle.py::test_moe_oracle_sensitivity_to_last_bit_changes).
# The routing itself (top-k, ties, weights, union) is checked bit-exactly in test_moe_gpu.py.
def within_moe_tol(err, cos, scale):
    return err <= 0.05 + 0.03 * scale and cos >= 0.999


def make(ctx, shape, seed=7, kv_seed=11, P=100, cap=512, chunk=0, **extra):
    d = ModelDesc.make(**shape, **extra)
    m = Model(ctx, d, seed)
    kv = KVCache(m, cap, chunk)
    kv.fill_synthetic(P, kv_seed)
    return d, m, kv


QWEN = dict(SMALL, qk_norm=1, qkv_bias=1)
QWEN64 = dict(GQA8, qk_norm=1, qkv_bias=1)
# Gated attention output with partial RoPE (Qwen3-Next: [q | gate] per head, × sigmoid(gate); AT_ROT < head_dim).
GATED = dict(SMALL, attn_gate=1, rotary_dims=32, qk_norm=1)
GATED64 = dict(GQA8, attn_gate=1, rotary_dims=16)
# gpt-oss-style attention: YaRN table (gpt-oss's parameters), q|k|v|o biases, sinks, alternating window.
YARN = dict(SWA, qkv_bias=1, o_bias=1, rope_type=2, rope_factor=32.0, rope_orig_max=4096.0, rope_no_truncate=1,
            rope_theta=150000.0)
# Proportional RoPE (a quarter of the pairs rotate, the rest angle 0) and linear scaling.
PROP = dict(SMALL, rope_type=3, rope_partial=0.25)
LINEAR = dict(GQA4, rope_type=1, rope_factor=4.0)
# The benchmark MoE configurations' synthetic i.i.d. routing.
MOEIID = dict(MOE4, iid_routing=1, n_experts=16, top_k=4)
MOEXIID = dict(MOEX, iid_routing=1)
# An int4 router in front of MXFP4 experts (gpt-oss packs): the router reads the experts' fp16 rows.
MOEXR4 = dict(MOEX, router_int4=1)


@pytest.mark.parametrize("shape", [SMALL, GQA8, SWA, MOE4, MOEX, QWEN, QWEN64, GATED, GATED64, YARN, PROP, LINEAR,
                                   MOEIID, MOEXIID, MOEXR4],
                         ids=["gqa2-hd128", "gqa8-hd64", "sinks-swa", "moe-int4", "moe-mxfp4", "qknorm-bias-hd128",
                              "qknorm-bias-hd64", "gated-rot32-hd128", "gated-rot16-hd64", "yarn-obias-sinks",
                              "proportional", "linear", "moe-int4-iid", "moe-mxfp4-iid", "moe-mxfp4-int4-router"])
@pytest.mark.parametrize("B", [1, 5, 9, 10, 17])
def test_verify_step_matches_oracle(ctx, shape, B):
    d, m, kv = make(ctx, shape)
    try:
        g = np.random.default_rng(B)
        toks = g.integers(0, d.vocab, size=B).astype(np.uint32)
        top1, logits = kv.verify(toks, want_logits=True)
        ref_logits, ref_top1 = oracle.verify_dense(d, 7, 11, 100, toks)
        err, cos = logits_close(logits, ref_logits)
        scale = np.abs(ref_logits).max()
        # Tolerance: bf16 activations and fp16 P·V on the GPU vs fp32 throughout in the oracle.
        tol = within_moe_tol if shape.get("n_experts") else within_tol
        assert tol(err, cos, scale), (err, cos, scale)
        # argmax: bit-exact unless the oracle's top-2 margin is inside the logit error.
        srt = np.sort(ref_logits, axis=1)
        margin = srt[:, -1] - srt[:, -2]
        for r in range(B):
            if margin[r] > 2 * err:
                assert top1[r] == ref_top1[r], (r, margin[r], err)
        assert np.array_equal(top1, np.argmax(logits, axis=1).astype(np.uint32))
        assert kv.pos == 100  # not advanced by the verify step
    finally:
        kv.free()
        m.free()


def test_moe_two_layers_within_routing_sensitivity(ctx):
    """Two MoE layers (configs 3 and 4 shapes, small): the MoE tolerance (within_moe_tol), argmax equal where the
    oracle's margin exceeds twice the error."""
    for shape in (MOE4, MOEX):
        d, m, kv = make(ctx, dict(shape, n_layers=2))
        try:
            toks = np.random.default_rng(17).integers(0, d.vocab, size=17).astype(np.uint32)
            top1, logits = kv.verify(toks, want_logits=True)
            ref_logits, ref_top1 = oracle.verify_dense(d, 7, 11, 100, toks)
            err, cos = logits_close(logits, ref_logits)
            scale = np.abs(ref_logits).max()
            assert within_moe_tol(err, cos, scale), (err, cos, scale)
            srt = np.sort(ref_logits, axis=1)
            margin = srt[:, -1] - srt[:, -2]
            for r in range(17):
                if margin[r] > 2 * err:
                    assert top1[r] == ref_top1[r], (r, margin[r], err)
        finally:
            kv.free()
            m.free()


@pytest.mark.parametrize("shape", [SMALL, GQA8, GQA4, SWA], ids=["gqa2-hd128", "gqa8-hd64", "gqa4-hd128", "swa16-sinks"])
@pytest.mark.parametrize("chunk", [32, 96, 1024, 0])
def test_verify_step_long_context_chunks(ctx, shape, chunk):
    """P = 1500 with key chunks of 32 (48 splits, half-filled 64-key pieces), 96 (16 splits, a partial last piece per
    split), 1024 (16 pieces per split through the ring) and automatic: the same oracle tolerance. In the sliding-window
    shape (window 16, sinks) the split holding the window starts at the window rounded down to 64 keys (1472 with
    the 1024-key chunk), not at the split's first key. A row whose oracle
    logits are themselves ill-conditioned (an int8 or bf16 rounding tie on the way: a one-part-in-10^7 change of RoPE θ
    moves them by more than 0.05) is held to the tolerance plus 5 × that measured movement instead; the GQA4 shape's
    token set at the automatic chunk has two such rows (0.11 and 0.07 under the perturbation)."""
    d, m, kv = make(ctx, shape, P=1500, cap=1600, chunk=chunk)
    try:
        if chunk:
            assert kv.chunk == chunk
        toks = np.random.default_rng(chunk + 1).integers(0, d.vocab, size=17).astype(np.uint32)
        top1, logits = kv.verify(toks, want_logits=True)
        ref_logits, ref_top1 = oracle.verify_dense(d, 7, 11, 1500, toks)
        err, cos = logits_close(logits, ref_logits)
        scale = np.abs(ref_logits).max()
        slack = np.zeros(17)
        if not within_tol(err, cos, scale):
            sens = np.zeros(17)
            for eps in (1e-7, -1e-7):
                alt = ModelDesc.make(**shape, rope_theta=d.rope_theta * (1 + eps))
                other, _ = oracle.verify_dense(alt, 7, 11, 1500, toks)
                sens = np.maximum(sens, np.abs(other - ref_logits).max(axis=1))
            slack = np.where(sens > 0.05, 5 * sens, 0.0)
            row_err = np.abs(logits - ref_logits).max(axis=1)
            assert np.all(row_err <= 0.02 + 0.01 * scale + slack), (row_err, sens)
            assert cos >= 0.9999, cos
        srt = np.sort(ref_logits, axis=1)
        margin = srt[:, -1] - srt[:, -2]
        for r in range(17):
            if margin[r] > 2 * err and slack[r] == 0:
                assert top1[r] == ref_top1[r], (r, margin[r], err)
    finally:
        kv.free()
        m.free()


def test_row_invariance_and_rollback(ctx):
    """Row r's logits are bit-identical whatever B and whatever the later rows hold (KernelCaseTests.swift:66-86);
    a rolled-back block leaves nothing behind (Generate.swift:515-540)."""
    d, m, kv = make(ctx, SMALL)
    try:
        g = np.random.default_rng(3)
        toks = g.integers(0, d.vocab, size=17).astype(np.uint32)
        _, full = kv.verify(toks, want_logits=True)
        for B in (1, 2, 9, 16):
            _, part = kv.verify(toks[:B], want_logits=True)
            assert np.array_equal(part.view(np.uint32), full[:B].view(np.uint32)), B
        other = toks.copy()
        other[6:] = g.integers(0, d.vocab, size=11)
        _, mixed = kv.verify(other, want_logits=True)
        assert np.array_equal(mixed[:6].view(np.uint32), full[:6].view(np.uint32))
        # Rollback: after verifying junk at P, verifying the original block again gives the original bits.
        _, again = kv.verify(toks, want_logits=True)
        assert np.array_equal(again.view(np.uint32), full.view(np.uint32))
    finally:
        kv.free()
        m.free()


@pytest.mark.parametrize("shape", [SMALL, GQA4, SWA, GATED, YARN], ids=["small", "gqa4", "swa-gqa8", "gated-rot32",
                                                                        "yarn-obias"])
def test_every_row_of_a_full_block_equals_its_row_decoded_alone(ctx, shape):
    """Row r of a 17-row block is bit-identical to the same token verified alone (and as the first row of a shorter
    block) once rows < r are in the cache: the speculative round's last row, which emits the bonus token, must give
    the bits plain decoding gives at that position (KernelCaseTests.swift:66-86; verify_attn_pf.metal:41-45)."""
    d, m, kv = make(ctx, shape)
    try:
        P = kv.pos
        toks = np.random.default_rng(5).integers(0, d.vocab, size=17).astype(np.uint32)
        _, full = kv.verify(toks, want_logits=True)
        for r in (16, 15, 8, 1):
            kv.set_pos(P + r)
            _, alone = kv.verify(toks[r:r + 1], want_logits=True)
            assert np.array_equal(alone[0].view(np.uint32), full[r].view(np.uint32)), r
            _, tail = kv.verify(toks[r:], want_logits=True)
            assert np.array_equal(tail.view(np.uint32), full[r:].view(np.uint32)), r
    finally:
        kv.free()
        m.free()


def test_commit_and_chained_rounds_match_plain_decode(ctx):
    """Speculative rounds give exactly the greedy tokens of plain one-token decoding (docs/adr/0002, 0005; gen
    --check): drafts that follow the greedy chain are all accepted, a wrong draft stops acceptance at its row."""
    d, m, kv = make(ctx, SMALL, P=50)
    try:
        # Plain decode: 8 tokens one at a time.
        tok = 17
        plain = []
        for _ in range(8):
            r = kv.verify_and_accept([tok])
            assert r.m == 0 and r.n_emitted == 1
            tok = r.tokens[0]
            plain.append(tok)
        assert kv.pos == 58
        # Speculative: roll back to 50 and verify the chain as drafts; plant a wrong draft after 5.
        kv.set_pos(50)
        drafts = [17] + plain[:7]
        bad = list(drafts)
        bad[6] = (bad[6] + 1) % d.vocab
        r = kv.verify_and_accept(bad)
        assert r.m == 5, r.m
        assert r.emitted == plain[:6]
        assert kv.pos == 56
        # Continue from the new anchor: the remaining plain tokens.
        r2 = kv.verify_and_accept([r.emitted[-1]] + plain[6:8])
        assert r2.m == 2 and r2.emitted[:2] == plain[6:8]
    finally:
        kv.free()
        m.free()


@pytest.mark.parametrize("chunk", [96, 64, 0])
def test_sliding_window_rows_are_block_invariant(ctx, chunk):
    """In a sliding-window layer with sinks, row i of a block verified at P has the same logit bits as the same token
    decoded alone at P + i after the block's first i rows were committed (the reference's 'same bits whatever the
    block', verify_attn_pf.metal:41-45): the window's split and its pieces do not depend on the block's P, and the sink
    merges after the splits."""
    d, m, kv = make(ctx, SWA, P=1500, cap=1600, chunk=chunk)
    try:
        toks = np.random.default_rng(chunk + 5).integers(0, d.vocab, size=17).astype(np.uint32)
        _, full = kv.verify(toks, want_logits=True)
        for i in (1, 5, 12, 16):
            kv.set_pos(1500)
            kv.verify(toks[:i])
            kv.commit(i)
            _, one = kv.verify(toks[i: i + 1], want_logits=True)
            assert np.array_equal(one[0].view(np.uint32), full[i].view(np.uint32)), i
        kv.set_pos(1500)
    finally:
        kv.free()
        m.free()


def test_cache_outliving_its_model_refuses_work(ctx):
    """Freeing the model first orphans its caches: a cache call that needs the model returns IH_EINVAL instead of
    touching freed memory, and the cache still frees."""
    from ingot_amd._lib import IngotError
    d = ModelDesc.make(**SMALL)
    m = Model(ctx, d, 7)
    kv = KVCache(m, 256)
    m.free()
    with pytest.raises(IngotError) as e:
        kv.fill_synthetic(10, 1)
    assert "freed" in str(e.value)
    kv.free()


@pytest.mark.parametrize("shape", [GQA4, MOEX], ids=["dense-gqa4", "moe-mxfp4"])
def test_recorded_step_replays_match_the_eager_step(shape):
    """A verify step with the same key on consecutive calls is recorded as a HIP graph on the second call and replayed
    afterwards. Every replay must give the bits of the first, eager step, also with other (eager) steps, host copies
    and synchronisations between the replays, and a step that changes the key must not replay a stale recording."""
    ctx = Context(0)
    d, m, kv = make(ctx, shape, P=300)
    toks = (np.arange(17, dtype=np.uint32) * 53 + 5) % d.vocab
    top_ref, log_ref = kv.verify(toks, want_logits=True)  # eager (first sight of the key)
    for i in range(4):  # recorded on the first of these, then replayed
        top, logits = kv.verify(toks, want_logits=True)
        assert np.array_equal(top, top_ref) and np.array_equal(logits, log_ref), f"replay {i} differs"
        other = kv.verify(toks[: 5 + i])  # a different key in between (eager)
        if not d.n_experts:  # dense rows do not depend on the block's other rows
            assert np.array_equal(other, top_ref[: 5 + i])
    # A new position is a new key: the first step there runs eagerly and its replays repeat it; none of them is a
    # replay of the recording at P = 300 (the rows' positions, hence their logits, differ).
    kv.set_pos(301)
    top_new, log_new = kv.verify(toks, want_logits=True)
    assert not np.array_equal(log_new, log_ref)
    for i in range(3):
        top, logits = kv.verify(toks, want_logits=True)
        assert np.array_equal(top, top_new) and np.array_equal(logits, log_new), f"replay {i} at P = 301 differs"
    kv.free()
    m.free()
    ctx.close()


def test_split_k_epilogues_match_the_whole_k_step():
    """K split over workgroups with the step's fused epilogues (RMSNorm-scaled projection, residual + next RMSNorm
    input, gated activation): each workgroup writes its partial sums with agent-coherent stores and the last of a row
    group to arrive adds them in split order and runs the epilogue. Forcing split shapes on every matrix of a model
    must reproduce the whole-K step up to the changed summation order, and the split step must be deterministic."""
    ctx = Context(0)
    toks = (np.arange(17, dtype=np.uint32) * 29 + 3) % GQA4["vocab"]
    d, m, kv = make(ctx, GQA4, P=200)
    top_ref, log_ref = kv.verify(toks, want_logits=True)
    kv.free()
    m.free()
    # qkv 1536×512, o 512×1024, gate|up 512×512, down 512×256: one-wave workgroups, one K-block each.
    shapes = ((1536, 512, 4, 1, 1), (512, 1024, 2, 1, 1), (512, 512, 2, 1, 1), (512, 256, 2, 1, 1))
    for n, k, r, kw, kpw in shapes:
        check(lib().ih_qmm_shape_override(ctx.handle, n, k, r, kw, kpw))
    runs = []
    for _ in range(2):
        d, m, kv = make(ctx, GQA4, P=200)
        runs.append(kv.verify(toks, want_logits=True))
        kv.free()
        m.free()
    for n, k, *_ in shapes:
        check(lib().ih_qmm_shape_override(ctx.handle, n, k, 0, 0, 0))
    (top, logits), (top2, logits2) = runs
    assert np.array_equal(logits, logits2) and np.array_equal(top, top2), "split-K step is not deterministic"
    err, cos = logits_close(logits, log_ref)
    scale = float(np.abs(log_ref).max())
    assert err <= 2e-3 * scale and cos >= 0.99999, (err, cos, scale)
    srt = np.sort(log_ref, axis=1)
    sure = (srt[:, -1] - srt[:, -2]) > 2 * err
    assert np.array_equal(top[sure], top_ref[sure])
    ctx.close()
