"""Copy-from-context drafting (CopyIndex, Sources/Ingot/CopySpec.swift:15-139): the library's host index and its
device scan against the brute-force rule of the reference's tests (CopySpecTests.naive,
Tests/IngotTests/CopySpecTests.swift:9-28), restated in the oracle and in plain Python."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from synth import zipf_context
from test_oracle import SplitMix, naive_py


def _reference_stream(seed: int = 3, trials: int = 20, steps: int = 1500):
    """The randomized histories of CopySpecTests.proposeMatchesNaive (CopySpecTests.swift:30-59): yields
    (trial, history so far, appended tokens, k) after every append."""
    g = SplitMix(seed)
    for trial in range(trials):
        h: list[int] = []
        vocab = 6 if trial % 2 == 0 else 40
        for _ in range(steps):
            if len(h) > 50 and g.next() % 4 == 0:
                s = g.next() % (len(h) - 20)
                ln = g.next() % 20 + 1
                new = h[s:s + ln]
            else:
                new = [g.next() % vocab]
            h += new
            k = g.next() % 16 + 1
            yield trial, h, new, k


def test_host_index_matches_naive_like_the_reference():
    """proposeMatchesNaive with the library's index (capacity 64, so its table grows many times), then the two sync
    cases of the same test: a history that extends the indexed one, and one that does not."""
    from ingot_amd._lib import CopyIndex

    ci = None
    last_trial = -1
    hist = None
    for trial, h, new, k in _reference_stream():
        if trial != last_trial:
            if ci is not None:
                _check_sync(ci, hist)
                ci.free()
            ci = CopyIndex(capacity=64)
            last_trial = trial
        ci.append(new)
        hist = h
        got = ci.propose(k)
        exp, m = oracle.copy_naive(np.array(h, np.uint32), k)
        assert got == list(exp) and ci.last_match == m, (trial, len(h), k)
    _check_sync(ci, hist)
    ci.free()


def _check_sync(ci, h):
    ext = list(h) + [1, 2, 3, 1, 2, 3]
    ci.sync(ext)
    assert len(ci) == len(ext)
    assert ci.propose(8) == list(oracle.copy_naive(np.array(ext, np.uint32), 8)[0])
    other = list(h[:700]) + [5, 5, 5, 5]
    ci.sync(other)
    assert len(ci) == len(other)
    exp = naive_py(other, 8)[0]
    assert ci.propose(8) == exp


def test_host_index_edge_cases():
    from ingot_amd._lib import CopyIndex

    ci = CopyIndex()
    assert ci.propose(16) == [] and ci.last_match == 0          # empty
    ci.append([7, 7, 7])
    assert ci.propose(16) == []                                  # n < 4
    ci.append([7])
    # 7 7 7 7: the trigram ending at 2 matches the current one (end 3); backward match len 3 (len ≤ p = 2 stops it).
    assert ci.propose(16) == [7] and ci.last_match == 3
    assert ci.propose(0) == [] and ci.last_match == 0
    ci.reset()
    assert len(ci) == 0 and ci.propose(4) == []
    # min_match 5: a trigram match of length 4 proposes nothing.
    c5 = CopyIndex(min_match=5)
    c5.append([1, 9, 2, 3, 4, 5, 8, 2, 3, 4])
    assert c5.propose(4) == [] and c5.last_match == 0
    c3 = CopyIndex()
    c3.append([1, 9, 2, 3, 4, 5, 8, 2, 3, 4])
    assert c3.propose(4) == [5, 8, 2, 3] and c3.last_match == 3
    # max_match caps the backward match.
    cm = CopyIndex(max_match=4)
    cm.append([1, 2, 3, 4, 5, 6, 1, 2, 3, 4, 5, 6])
    assert cm.propose(3) == [1, 2, 3] and cm.last_match == 4
    for c in (ci, c5, c3, cm):
        c.free()


def test_zipf_context_plants_the_tail():
    h, src = zipf_context(5, n=4096, spans=8)
    assert h.dtype == np.uint32 and h.size == 4096
    assert np.array_equal(h[-8:], h[src:src + 8])
    prop, m = oracle.copy_naive(h, 16)
    assert len(prop) == 16 and m >= 8


# ---- device scan --------------------------------------------------------------------------------------------------

@pytest.mark.gpu
def test_device_lookup_matches_naive_on_reference_stream(ctx):
    """Every 7th history of the reference's randomized stream (vocab 6 and 40: many trigram repeats), each uploaded and
    scanned on the device: proposal, match length and chosen end equal the naive rule."""
    from ingot_amd._lib import copy_lookup_dev

    checked = 0
    for i, (trial, h, _, k) in enumerate(_reference_stream(trials=4)):
        if i % 7 or len(h) < 4:
            continue
        d = ctx.to_device(np.array(h, np.uint32))
        got, m, _ = copy_lookup_dev(ctx, d, len(h), k)
        d.free()
        exp, em = oracle.copy_naive(np.array(h, np.uint32), k)
        assert got == list(exp) and m == em, (trial, len(h), k)
        checked += 1
    assert checked > 500


@pytest.mark.gpu
@pytest.mark.parametrize("min_match,max_match", [(3, 64), (5, 64), (3, 4), (3, 200)])
def test_device_lookup_options_and_edges(ctx, min_match, max_match):
    from ingot_amd._lib import copy_lookup_dev

    g = np.random.default_rng(min_match * 100 + max_match)
    cases = [np.array([7, 7, 7, 7], np.uint32), np.array([1, 2, 3, 4], np.uint32),
             np.array([1, 2, 3, 4, 5, 6] * 40, np.uint32)]
    for n in (5, 100, 1023, 1024, 1025, 4099):
        cases.append(g.integers(0, 3, size=n).astype(np.uint32))
    for h in cases:
        for k in (1, 16, 64):
            d = ctx.to_device(h)
            got, m, _ = copy_lookup_dev(ctx, d, len(h), k, min_match, max_match)
            d.free()
            exp, em = oracle.copy_naive(h, k, min_match, max(min_match, max_match))
            assert got == list(exp) and m == em, (len(h), k)


@pytest.mark.gpu
def test_device_lookup_config2_and_verify_block(ctx):
    """Config 2's context (131072 Zipf(1.1) ids, 64 planted spans of 32): the scan equals the naive rule and the verify
    block it writes is [anchor, 16 proposals]."""
    from ingot_amd._lib import copy_lookup_dev

    h, src = zipf_context(2026)
    d = ctx.to_device(h)
    vt = ctx.buffer(17 * 4).fill(0)
    got, m, end = copy_lookup_dev(ctx, d, len(h), 16, vtok_dev=vt, rows=17)
    exp, em = oracle.copy_naive(h, 16)
    assert got == list(exp) and m == em and len(got) == 16
    assert np.array_equal(h[end - m + 1:end + 1], h[len(h) - m:])
    block = vt.download(np.uint32, (17,))
    assert block[0] == h[-1] and list(block[1:]) == got
    d.free()
    vt.free()
