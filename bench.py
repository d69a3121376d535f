#!/usr/bin/env python3
"""Benchmark of the speculative-decoding verify step on one MI355X (BASELINE.json metric, configuration 1).

A step is one verify round of k = 16 drafts (B = 17 rows) of the 8B-class 4-bit dense model at 8192 positions of
int8 KV: the block runs through all 32 layers and the head (its K/V written at P…P+16), the device-side greedy
acceptance takes the longest draft prefix, and the block is rolled back (P restored) so every step sees the same
context. Drafts are planted to agree with the greedy chain for L = 0…16 tokens (cycling over the steps), and the bench
checks that the accepted length equals L.

Printed: one JSON line (the driver's contract) with `roofline` (the dominant kernel, the int4 qmm, from HIP events on
the library's stream) and `cpu_baseline` (the C++ oracle on the host, same workload, one full step).

Synthetic weights and KV (seeded, counter-based SplitMix64; the reference's checkpoints are not available).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "verify-step µs & tok/s at k=16, 4-bit; qmm/attn HBM GB/s vs 8 TB/s peak"

CONFIGS = {
    # hidden 4096, 32 q / 8 KV heads of 128, SwiGLU 14336, 32 layers, vocab 151936, RoPE θ 1e6,
    # RMSNorm eps 1e-6, MLX int4 g64 everywhere; k + 1 = 17 rows over 8192 int8 KV positions.
    "dense8b-8k": dict(
        desc=dict(n_layers=32, hidden=4096, n_q_heads=32, n_kv_heads=8, head_dim=128, intermediate=14336,
                  vocab=151936),
        P=8192, B=17),
    # The same model at 32K positions (the verify leg of config 2).
    "dense8b-32k": dict(
        desc=dict(n_layers=32, hidden=4096, n_q_heads=32, n_kv_heads=8, head_dim=128, intermediate=14336,
                  vocab=151936),
        P=32768, B=17),
}

SEED, KV_SEED, ANCHOR = 2026, 11, 1234


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=34)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--config", default="dense8b-8k", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-profile", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (the verify step shards "
              "across GPUs only by design, see DESIGN.md)", file=sys.stderr)
        return 2

    from ingot_amd._lib import (Context, HipEvents, KVCache, Model, ModelDesc, check, lib, ptr)

    cfg = CONFIGS[args.config]
    P, B = cfg["P"], cfg["B"]
    k = B - 1
    ctx = Context(0)
    desc = ModelDesc.make(**cfg["desc"])
    t0 = time.time()
    model = Model(ctx, desc, SEED)
    kv = KVCache(model, P + 2 * B)
    kv.fill_synthetic(P, KV_SEED)
    log(f"[bench] model {args.config} built in {time.time() - t0:.1f}s; weights {model.weight_bytes / 1e9:.3f} GB")

    # Greedy chain from the anchor (plain one-row steps), then back to P.
    chain = []
    tok = ANCHOR
    for _ in range(k + 1):
        r = kv.verify_and_accept([tok])
        tok = r.tokens[0]
        chain.append(tok)
    kv.set_pos(P)
    rng = np.random.default_rng(SEED)
    blocks = np.zeros((k + 1, B), np.uint32)
    for L in range(k + 1):
        blk = [ANCHOR] + chain[:L]
        if L < k:
            blk.append((chain[L] + 1) % desc.vocab)  # first wrong draft
            blk += list(rng.integers(0, desc.vocab, size=B - len(blk)))
        blocks[L] = blk
    d_blocks = ctx.to_device(blocks)
    d_vtok = ctx.buffer(B * 4)
    d_top1 = ctx.buffer(B * 4)
    d_st = ctx.to_device(np.zeros(8, np.uint32))
    RING = 64
    d_rec = ctx.buffer(RING * 24 * 4).fill(0)

    def step(i: int) -> None:
        L = i % (k + 1)
        check(lib().ih_memcpy_dtod(ctx.handle, d_vtok.ptr, d_blocks.ptr + L * B * 4, B * 4))
        check(lib().ih_verify_step_dev(model.handle, kv.handle, d_vtok.ptr, B, d_top1.ptr))
        check(lib().ih_spec_accept_dev(ctx.handle, d_st.ptr, d_vtok.ptr, d_top1.ptr, d_rec.ptr, RING, B))
        # Rollback: the verify step does not advance the host position, so the next step sees P again.

    for i in range(args.warmup):
        step(i)
    ctx.sync()
    d_st.upload(np.zeros(8, np.uint32))
    ev = HipEvents(ctx, 2)
    ctx.sync()
    ev.record(0)
    for i in range(args.steps):
        step(i)
    ev.record(1)
    ms_total = ev.elapsed_ms(0, 1)
    ctx.sync()
    ms = ms_total / args.steps
    rec = d_rec.download(np.uint32, (RING, 24))
    accepted = [int(rec[i % RING][0]) for i in range(min(args.steps, RING))]
    planted = [i % (k + 1) for i in range(min(args.steps, RING))]
    accept_ok = accepted == planted
    tok_per_L = {L: (L + 1) / (ms / 1e3) for L in range(k + 1)}
    tok_s = float(np.mean(list(tok_per_L.values())))

    # Per-kernel-class timing in a second, instrumented pass of the same steps.
    classes = {}
    if not args.no_kernel_profile:
        check(lib().ih_timing_enable(ctx.handle, 1))
        for i in range(args.steps):
            step(i)
        ctx.sync()
        names = ["qmm", "attention", "attn_prework", "attn_reduce", "rows", "argmax", "moe", "other"]
        for c, n in enumerate(names):
            t = C.c_double()
            cnt = C.c_int()
            by = C.c_double()
            check(lib().ih_timing_read(ctx.handle, c, C.byref(t), C.byref(cnt), C.byref(by)))
            if cnt.value:
                classes[n] = dict(ms_per_step=t.value / args.steps, launches_per_step=cnt.value / args.steps,
                                  gbs=by.value / (t.value * 1e6), bytes_per_step=by.value / args.steps)
        check(lib().ih_timing_enable(ctx.handle, 0))

    # Algorithmic bytes of one step: weights (MLX int4), KV of all layers, logits write + read.
    d = cfg["desc"]
    kv_bytes = d["n_layers"] * d["n_kv_heads"] * (P + B) * (2 * d["head_dim"] + 4)
    logit_bytes = 2 * B * d["vocab"] * 4
    step_bytes = model.weight_bytes + kv_bytes + logit_bytes
    roofline = None
    if "qmm" in classes:
        q = classes["qmm"]
        roofline = dict(bound="hbm", achieved=round(q["gbs"], 1), peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=round(q["gbs"] / HBM_PEAK_GBS, 4), traffic=None, kernel="qmm_int4",
                        avg_launch_us=round(q["ms_per_step"] / q["launches_per_step"] * 1e3, 2),
                        bytes_per_launch=round(q["bytes_per_step"] / q["launches_per_step"]))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(desc, P, blocks[k])

    model_name = f"synthetic 8B-class dense int4 g64 ({d['n_layers']}L h{d['hidden']} {d['n_q_heads']}q/" \
                 f"{d['n_kv_heads']}kv hd{d['head_dim']} I{d['intermediate']} V{d['vocab']})"
    out = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "us_per_step": round(ms * 1e3, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-g64 weights, bf16 activations, fp32 accumulate, int8 KV",
        "data": "synthetic (seeded SplitMix64 weights, N(0,1) int8 KV, planted drafts)",
        "config": {"workload": f"config 1: verify k=16 (B=17) at P={P}", "model": model_name, "k": k,
                   "context": P, "parallelism": "single GPU"},
        "tok_s_per_L": {str(L): round(v, 1) for L, v in tok_per_L.items()},
        "accepted_equals_planted": accept_ok,
        "accepted": accepted[: k + 1],
        "step_hbm_gbs": round(step_bytes / (ms * 1e6), 1),
        "step_roofline_frac": round(step_bytes / (ms * 1e6) / HBM_PEAK_GBS, 4),
        "step_algorithmic_bytes": step_bytes,
        "kernels": {n: {kk: round(vv, 3) for kk, vv in v.items()} for n, v in classes.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    kv.free()
    model.free()
    ctx.close()
    return 0


def cpu_baseline(desc, P: int, tokens) -> dict | None:
    """The C++ oracle (fp32 dequant + matmul) on the host: the full model with resident weights, one verify step of
    the same B = 17 block at the same P; tok/s as for the GPU (mean accepted + 1 over L = 0…16 → 9 tokens)."""
    try:
        import oracle
    except Exception as e:  # noqa: BLE001
        log(f"[bench] cpu baseline unavailable: {e}")
        return None
    t0 = time.time()
    m = oracle.OracleModel(desc, SEED, KV_SEED, P)
    t1 = time.time()
    m.verify(tokens)
    t2 = time.time()
    m.free()
    step_s = t2 - t1
    k = len(tokens) - 1
    mean_tokens = (k + 2) / 2.0
    log(f"[bench] cpu baseline: model built in {t1 - t0:.1f}s, one step {step_s:.2f}s")
    return {"value": round(mean_tokens / step_s, 3), "unit": "tok/s", "cores": oracle.num_threads(),
            "kind": "port", "sample": f"one full verify step (B={len(tokens)}, all {desc.n_layers} layers + head, "
                                      f"P={P}) of the C++ oracle with resident weights; {step_s:.2f} s/step",
            "s_per_step": round(step_s, 3)}


if __name__ == "__main__":
    sys.exit(main())
