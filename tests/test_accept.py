"""Greedy acceptance (integer, host): the C ABI's ih_accept against the oracle and brute force.

spec_accept, Sources/Ingot/Shaders/yy_model.metal:616-642; Generate.swift:155-158.
"""
import numpy as np

import oracle
from ingot_amd._lib import accept


def brute(vtok, top1):
    B = len(vtok)
    best = 0
    for m in range(B):
        if all(vtok[i + 1] == top1[i] for i in range(m)):
            best = m
    return best


def test_host_accept_matches_oracle_and_brute_force():
    g = np.random.default_rng(5)
    for _ in range(500):
        B = int(g.integers(1, 18))
        top1 = g.integers(0, 3, size=B).astype(np.uint32)
        vtok = g.integers(0, 3, size=B).astype(np.uint32)
        r = accept(vtok, top1)
        m, em = oracle.accept(vtok, top1)
        assert r.m == m == brute(vtok, top1)
        assert r.emitted == list(em) == [int(x) for x in vtok[1 : m + 1]] + [int(top1[m])]


def test_accept_config0_forced_prefix():
    """Benchmark configuration 0: logits [8, 32000] ~ N(0,1), 7 drafts with the first 3 forced to the argmax → m ≥ 3."""
    g = np.random.default_rng(0)
    logits = g.normal(0, 1, size=(8, 32000)).astype(np.float32)
    top1 = oracle.argmax_rows(logits)
    assert np.array_equal(top1, np.argmax(logits, axis=1))
    vtok = np.concatenate([[g.integers(0, 32000)], g.integers(0, 32000, size=7)]).astype(np.uint32)
    vtok[1:4] = top1[0:3]
    r = accept(vtok, top1)
    assert r.m >= 3
    assert r.emitted[:3] == list(top1[:3])
