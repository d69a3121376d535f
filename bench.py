#!/usr/bin/env python3
"""Benchmark of the speculative-decoding verify step on one MI355X (BASELINE.json metric).

Default (the headline line): configuration 1 — one verify round of k = 16 drafts (B = 17 rows) of the 8B-class 4-bit
dense model at 8192 positions of int8 KV: the block runs through all 32 layers and the head (its K/V written at
P…P+16), the device-side greedy acceptance takes the longest draft prefix, and the block is rolled back (P restored) so
every step sees the same context. Drafts are planted to agree with the greedy chain for L = 0…16 tokens (cycling over
the steps), and the bench checks that the accepted length equals L.

Other workloads (--config): configuration 2 (copy-from-context lookup over 131,072 Zipf ids writing the verify block,
then the config-1 model at 32K positions), 3 (48-layer MoE, 128 experts top-8, int4, 16K) and 4 (24-layer MXFP4 MoE,
32 experts top-4, sinks, alternating 128-token sliding window, B = 9, 64K).

Printed: one JSON line (the driver's contract) with `roofline` (the dominant kernel class, from HIP events on the
library's stream) and `cpu_baseline` (the C++ oracle on the host, same workload and block: median of 5 full steps after a
warm-up, with the GPU's top-1 and logits on that block compared against the oracle's; configuration 1 only by default).
With the default configuration the same line also carries side measurements: `config0_qmm_accept` (config 0's single
qmm and acceptance) and `other_configs` (configurations 2, 3 and 4, ten timed steps each).

Synthetic weights and KV (seeded, counter-based SplitMix64; the reference's checkpoints are not available).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "verify-step µs & tok/s at k=16, 4-bit; qmm/attn HBM GB/s vs 8 TB/s peak"

DENSE8B = dict(n_layers=32, hidden=4096, n_q_heads=32, n_kv_heads=8, head_dim=128, intermediate=14336, vocab=151936)
CONFIGS = {
    # Config 1: hidden 4096, 32 q / 8 KV heads of 128, SwiGLU 14336, 32 layers, vocab 151936, RoPE θ 1e6, RMSNorm eps
    # 1e-6, MLX int4 g64 everywhere; k + 1 = 17 rows over 8192 int8 KV positions.
    "dense8b-8k": dict(desc=DENSE8B, P=8192, B=17, label="config 1: verify k=16 (B=17) at P=8192"),
    # Config 2: copy-from-context lookup over 131,072 ids, proposing 16, then the config-1 model at 32K positions.
    "copy-dense8b-32k": dict(desc=DENSE8B, P=32768, B=17, copy=131072,
                             label="config 2: copy lookup over 131072 ids + verify k=16 at P=32768"),
    # Config 3: 48 layers, hidden 2048, 32 q / 4 KV heads of 128, 128 experts top-8 (softmax), expert SwiGLU 768, int4.
    "moe-e128-16k": dict(desc=dict(n_layers=48, hidden=2048, n_q_heads=32, n_kv_heads=4, head_dim=128, intermediate=0,
                                   vocab=151936, n_experts=128, top_k=8, expert_intermediate=768, expert_format=0,
                                   iid_routing=1),
                         P=16384, B=17, label="config 3: MoE E128 top-8 verify k=16 at P=16384"),
    # Config 4: 24 layers, hidden 2880, 64 q / 8 KV heads of 64, sinks, alternating 128-token sliding window / full,
    # 32 MXFP4 experts top-4 with intermediate 2880, router and expert biases, swiglu_oai, vocab 201088; B = 9.
    "mxfp4-moe-64k": dict(desc=dict(n_layers=24, hidden=2880, n_q_heads=64, n_kv_heads=8, head_dim=64, intermediate=0,
                                    vocab=201088, n_experts=32, top_k=4, expert_intermediate=2880, expert_format=1,
                                    router_bias=1, expert_bias=1, act=1, sinks=1, sliding_window=128,
                                    iid_routing=1),
                          P=65536, B=9, label="config 4: MXFP4 MoE E32 top-4 verify k=8 at P=65536"),
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
    ap.add_argument("--cpu-baseline", action="store_true", help="also for the non-default configurations")
    ap.add_argument("--no-kernel-profile", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the side measurements (config 0's qmm, the decode loop, the other configurations' step times)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only copy BYTES device-to-device 4 times (the reference kernel that scales the HBM counters)")
    ap.add_argument("--decode-loop-only", action="store_true",
                    help="only the decode-loop side measurement on config 1's model (for kernel traces of its rounds)")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.decode_loop_only:
        from ingot_amd._lib import Context, Model, ModelDesc

        ctx = Context(0)
        cfg = CONFIGS["dense8b-8k"]
        model = Model(ctx, ModelDesc.make(**cfg["desc"]), SEED)
        print(json.dumps({"decode_loop": decode_loop(model, cfg["P"], ANCHOR)}), flush=True)
        model.free()
        ctx.close()
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (sharding the verify step "
              "across GPUs is designed, not built)", file=sys.stderr)
        return 2

    from ingot_amd._lib import Context

    ctx = Context(0)
    want_cpu = not args.no_cpu_baseline and (args.config == "dense8b-8k" or args.cpu_baseline)
    out = run_config(ctx, args.config, args.steps, args.warmup, profile=not args.no_kernel_profile, cpu=want_cpu,
                     extra=not args.no_extra)
    if not args.no_extra and args.config == "dense8b-8k":
        # Side measurements in the same run (not the headline `value`): config 0's single qmm, and the step time of
        # every other configuration (fewer steps each).
        out["config0_qmm_accept"] = config0(ctx)
        others = {}
        for name in CONFIGS:
            if name == args.config:
                continue
            r = run_config(ctx, name, 10, 2, profile=True, cpu=False)
            keep = ("ms_per_step", "value", "step_hbm_gbs", "step_roofline_frac", "step_algorithmic_bytes",
                    "moe_distinct_experts_per_layer", "copy_lookup", "accepted_equals_planted", "roofline")
            others[name] = {k: r[k] for k in keep if k in r}
            others[name]["workload"] = r["config"]["workload"]
            others[name]["kernels_ms_per_step"] = {k: v["ms_per_step"] for k, v in r["kernels"].items()}
        out["other_configs"] = others
    print(json.dumps(out), flush=True)
    ctx.close()
    return 0


def decode_loop(model, P: int, anchor: int) -> dict:
    """Side measurement: the chained decode loop (ih_decode_greedy / ih_decode_sample, decodeSpec's hot loop) from
    position P with advancing positions (a cache of P + 1024 positions, the same synthetic history), two rounds in
    flight: copy-from-context drafts (rows = 17), plain one-row chained decoding (rows = 1), temperature sampling with
    copy drafts (rows = 17), and a synthetic DFlash2 drafter (rows = its block, 16; its drafts are noise against the synthetic
    target, so this times the round, not an acceptance rate). Host wall clock around each call (the call
    synchronises); the first call of each kind warms up the recorded steps and is not reported."""
    from ingot_amd._lib import Drafter, DrafterDesc, KVCache, SampleParams, check, lib

    kv = KVCache(model, P + 1024)
    kv.fill_synthetic(P, KV_SEED)
    out = {"cache_positions": P + 1024, "key_chunk": kv.chunk}
    hist = np.full(P, anchor, np.uint32)  # the context the copy drafter indexes (the greedy chain's token)
    # A drafter of the size class DFlash2 ships for 8B targets: 5 layers at the target's hidden size, 32 q heads of
    # 128, intermediate 12288, 5 target layers, 16-token blocks, a 2048-position window, a rank-256 selector.
    L_ = model.desc.n_layers
    ddesc = DrafterDesc.make(targets=tuple(range(1, L_, max(1, L_ // 5)))[:5], n_layers=5, hidden=model.desc.hidden,
                             n_q_heads=32, head_dim=128, intermediate=12288, block=16, window=2048, rank=256,
                             dyn_conv=1, mask_token=model.desc.vocab - 1)
    dr = Drafter(model, ddesc, SEED + 1)
    sp = SampleParams(temp=0.8, top_p=0.95, top_k=64, min_p=0.0)
    kinds = (("rows17", 17, 17 * 48, {"history": hist}, False),
             ("rows1", 1, 96, {"history": hist}, False),
             ("sample_rows17", 17, 17 * 48, {"history": hist}, True),
             ("drafter_rows16", 16, 16 * 24, {"drafter": dr}, False))
    for name, rows, ntok, extra, sample in kinds:
        if "drafter" in extra:
            dr.attach()  # the verify steps then capture the drafter's target layers

        def call():
            kv.set_pos(P)
            if sample:
                return kv.decode_sample(anchor, ntok, sp, 7, rows=rows, inflight=2, **extra)
            return kv.decode_greedy(anchor, ntok, rows=rows, inflight=2, **extra)
        call()
        t0 = time.perf_counter()
        toks, st = call()
        dt = time.perf_counter() - t0
        out[name] = {"tokens": len(toks), "rounds": st.rounds, "accepted": st.accepted, "finish": st.finish,
                     "ms": round(dt * 1e3, 2), "ms_per_round": round(dt * 1e3 / max(st.rounds, 1), 4),
                     "tok_s": round(len(toks) / dt, 1)}
    kv.set_pos(P)
    check(lib().ih_model_set_drafter(model.handle, None))
    out["drafter"] = {"n_layers": 5, "hidden": int(model.desc.hidden), "q_heads": 32, "intermediate": 12288,
                      "block": 16, "window": 2048, "rank": 256, "targets": list(ddesc.target_layers[:ddesc.n_targets])}
    dr.free()
    kv.free()
    return out


def run_config(ctx, config: str, steps: int, warmup: int, profile: bool, cpu: bool, extra: bool = False) -> dict:
    """Builds one configuration's model and cache, times `steps` verify rounds and returns the JSON line's fields."""
    from ingot_amd._lib import HipEvents, KVCache, Model, ModelDesc, check, lib

    cfg = CONFIGS[config]
    d = cfg["desc"]
    P, B = cfg["P"], cfg["B"]
    k = B - 1
    desc = ModelDesc.make(**d)
    t0 = time.time()
    model = Model(ctx, desc, SEED)
    kv = KVCache(model, P + 2 * B)
    kv.fill_synthetic(P, KV_SEED)
    log(f"[bench] model {config} built in {time.time() - t0:.1f}s; weights {model.weight_bytes / 1e9:.3f} GB, "
        f"key chunk {kv.chunk}")

    d_vtok = ctx.buffer(B * 4)
    d_top1 = ctx.buffer(B * 4)
    d_st = ctx.to_device(np.zeros(8, np.uint32))
    RING = 64
    d_rec = ctx.buffer(RING * 24 * 4).fill(0)
    copy_n = cfg.get("copy")
    bufs = [d_vtok, d_top1, d_st, d_rec]

    if copy_n:
        # Config 2: the copy drafter proposes from the context; the verify block is written on the device.
        sys.path.insert(0, str(ROOT / "tests"))
        from synth import zipf_context

        hist, _ = zipf_context(SEED, n=copy_n, vocab=d["vocab"])
        d_hist = ctx.to_device(hist)
        d_copy = ctx.buffer((4 + k) * 4)
        bufs += [d_hist, d_copy]
        blocks = None

        def step(i: int) -> None:
            check(lib().ih_copy_lookup_dev(ctx.handle, d_hist.ptr, copy_n, k, 3, 64, d_copy.ptr, d_vtok.ptr, B))
            check(lib().ih_verify_step_dev(model.handle, kv.handle, d_vtok.ptr, B, d_top1.ptr))
            check(lib().ih_spec_accept_dev(ctx.handle, d_st.ptr, d_vtok.ptr, d_top1.ptr, d_rec.ptr, RING, B))
    else:
        # Greedy chain from the anchor (plain one-row steps), then back to P; plant L = 0…k agreeing drafts.
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
                blk.append((chain[L] + 1) % d["vocab"])  # first wrong draft
                blk += list(rng.integers(0, d["vocab"], size=B - len(blk)))
            blocks[L] = blk
        d_blocks = ctx.to_device(blocks)
        bufs.append(d_blocks)
        log(f"[bench] greedy chain: {chain}")

        def one(src, L):
            check(lib().ih_memcpy_dtod(ctx.handle, d_vtok.ptr, src.ptr + L * B * 4, B * 4))
            check(lib().ih_verify_step_dev(model.handle, kv.handle, d_vtok.ptr, B, d_top1.ptr))
            check(lib().ih_spec_accept_dev(ctx.handle, d_st.ptr, d_vtok.ptr, d_top1.ptr, d_rec.ptr, RING, B))
            # Rollback: the verify step does not advance the host position, so the next step sees P again.

        def step(i: int) -> None:
            one(d_blocks, i % (k + 1))

    for i in range(warmup):
        step(i)
    ctx.sync()
    d_st.upload(np.zeros(8, np.uint32))
    ev = HipEvents(ctx, 2)
    ctx.sync()
    ev.record(0)
    for i in range(steps):
        step(i)
    ev.record(1)
    ms_total = ev.elapsed_ms(0, 1)
    ctx.sync()
    ev.close()
    ms = ms_total / steps
    # MoE: distinct experts per layer of the last timed step (the bytes actually streamed). The synthetic routing is
    # keyed by position, and every timed step runs at the same rolled-back position, so every step streams the same U.
    U = None
    if d.get("n_experts"):
        u = np.zeros(d["n_layers"], np.int32)
        check(lib().ih_model_moe_union(model.handle, u.ctypes.data))
        U = u.tolist()
    rec = d_rec.download(np.uint32, (RING, 24))
    nrec = min(steps, RING)
    accepted = [int(rec[i % RING][0]) for i in range(nrec)]
    if blocks is not None:
        planted = [i % (k + 1) for i in range(nrec)]
        accept_ok = accepted == planted
        tok_per_L = {L: (L + 1) / (ms / 1e3) for L in range(k + 1)}
        tok_s = float(np.mean(list(tok_per_L.values())))
    else:
        accept_ok = None
        tok_per_L = {}
        tok_s = float(np.mean([a + 1 for a in accepted])) / (ms / 1e3)

    # Per-kernel-class timing in a second, instrumented pass of the same steps.
    classes = {}
    if profile:
        check(lib().ih_timing_enable(ctx.handle, 1))
        for i in range(steps):
            step(i)
        ctx.sync()
        names = ["qmm", "attention", "attn_prework", "attn_reduce", "rows", "argmax", "moe", "other", "qmm_finish"]
        for c, n in enumerate(names):
            t = C.c_double()
            cnt = C.c_int()
            by = C.c_double()
            check(lib().ih_timing_read(ctx.handle, c, C.byref(t), C.byref(cnt), C.byref(by)))
            if cnt.value:
                classes[n] = dict(ms_per_step=t.value / steps, launches_per_step=cnt.value / steps,
                                  gbs=by.value / (t.value * 1e6), bytes_per_step=by.value / steps)
        check(lib().ih_timing_enable(ctx.handle, 0))

    # Algorithmic bytes of one step: weights actually read (MLX formats; MoE: the routed experts), the KV of every
    # layer (a sliding-window layer reads the window), logits written and read.
    L_, H, KVH, HD = d["n_layers"], d["hidden"], d["n_kv_heads"], d["head_dim"]
    per_expert = 0.0
    weight_bytes = float(model.weight_bytes)
    if d.get("n_experts"):
        IE, E = d["expert_intermediate"], d["n_experts"]
        bpw = 0.5625 if d.get("expert_format", 0) == 0 else 0.53125
        per_expert = 3 * IE * H * bpw
        dense_part = weight_bytes - L_ * E * per_expert
        weight_bytes = dense_part + sum(U) * per_expert
    kv_bytes = 0.0
    for l in range(L_):
        keys = P + B
        if d.get("sliding_window") and l % 2 == 0:
            keys = min(keys, d["sliding_window"] + B - 1)
        kv_bytes += KVH * keys * (2 * HD + 4)
    logit_bytes = 2 * B * d["vocab"] * 4
    step_bytes = weight_bytes + kv_bytes + logit_bytes

    roofline = None
    dom = max((n for n in ("qmm", "moe", "attention") if n in classes), key=lambda n: classes[n]["ms_per_step"],
              default=None)
    if dom:
        q = classes[dom]
        by = q["bytes_per_step"]
        if dom == "moe":
            # The gathered launches are sized for every expert slot; the bytes streamed are the routed experts'.
            by = sum(U) * per_expert
        gbs = by / (q["ms_per_step"] * 1e6)
        roofline = dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=round(gbs / HBM_PEAK_GBS, 4), traffic=None,
                        kernel={"qmm": "qmm_int4", "moe": "qmm_gather (MoE experts)", "attention": "attn"}[dom],
                        avg_launch_us=round(q["ms_per_step"] / q["launches_per_step"] * 1e3, 2),
                        bytes_per_launch=round(by / q["launches_per_step"]))
        traffic = _traffic(config, dom)
        if traffic is not None:
            roofline["traffic"] = traffic

    loop = None
    if config == "dense8b-8k" and profile and extra:
        loop = decode_loop(model, P, ANCHOR)

    cpu_res = None
    if cpu:
        cpu_res = cpu_baseline(desc, P, blocks[k] if blocks is not None else np.full(B, ANCHOR, np.uint32), kv)

    model_name = (f"synthetic {d['n_layers']}L h{d['hidden']} {d['n_q_heads']}q/{d['n_kv_heads']}kv hd{d['head_dim']} "
                  + (f"E{d['n_experts']} top-{d['top_k']} I{d['expert_intermediate']} "
                     f"{'mxfp4' if d.get('expert_format') else 'int4'} experts" if d.get("n_experts")
                     else f"I{d['intermediate']} int4 g64") + f" V{d['vocab']}")
    out = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 4),
        "us_per_step": round(ms * 1e3, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-g64/mxfp4 weights, bf16 (fp16 for mxfp4) activations, fp32 accumulate, int8 KV",
        "data": "synthetic (seeded SplitMix64 weights, N(0,1) int8 KV, planted drafts)",
        "config": {"workload": cfg["label"], "model": model_name, "k": k, "context": P, "parallelism": "single GPU"},
        "tok_s_per_L": {str(L): round(v, 1) for L, v in tok_per_L.items()},
        "accepted_equals_planted": accept_ok,
        "accepted": accepted[: k + 1],
        "step_hbm_gbs": round(step_bytes / (ms * 1e6), 1),
        "step_roofline_frac": round(step_bytes / (ms * 1e6) / HBM_PEAK_GBS, 4),
        "step_algorithmic_bytes": round(step_bytes),
        "kernels": {n: {kk: round(vv, 3) for kk, vv in v.items()} for n, v in classes.items()},
        "roofline": roofline,
        "cpu_baseline": cpu_res,
    }
    if loop is not None:
        out["decode_loop"] = loop
    if U is not None:
        out["moe_distinct_experts_per_layer"] = {"mean": round(float(np.mean(U)), 2), "min": min(U), "max": max(U)}
    if copy_n:
        out["copy_lookup"] = copy_lookup_timing(ctx, lib, check, d_hist, copy_n, k, d_copy, d_vtok, B)
    for b in bufs:
        b.free()
    kv.free()
    model.free()
    return out


def config0(ctx) -> dict:
    """Config 0: one verify-step qmm, X bf16 [8, 4096] · int4 g64 W [4096, 4096] (codes uniform, scale |N(0, 0.02)|,
    bias −8·scale), bf16 out, then argmax over logits [8, 32000] and the acceptance of 7 drafts. GB/s of the
    algorithmic 9,568,256 bytes, for a single launch (synchronised before and after) and for 64 back-to-back calls."""
    from ingot_amd._lib import HipEvents, QMat, check, lib

    def bf16(a):
        u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    g = np.random.default_rng(SEED)
    N = K = 4096
    M = 8
    q = g.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    sb = bf16(np.abs(g.normal(0, 0.02, size=(N, K // 64))))
    bb = bf16(-8 * (sb.astype(np.uint32) << 16).view(np.float32))
    W = QMat.int4(ctx, q, sb, bb)
    x = ctx.to_device(bf16(g.normal(0, 1, size=(M, K))))
    y = ctx.buffer(M * N * 2)
    algo = 9568256
    ev = HipEvents(ctx, 2)
    # A single call from an idle stream (events around the call only), then the kernel alone (per-dispatch events).
    single = []
    for _ in range(20):
        ctx.sync()
        ev.record(0)
        check(lib().ih_qmm_int4(ctx.handle, W.handle, x.ptr, K, M, y.ptr, N, 2))
        ev.record(1)
        single.append(ev.elapsed_ms(0, 1))
    check(lib().ih_timing_enable(ctx.handle, 1))
    for _ in range(20):
        check(lib().ih_qmm_int4(ctx.handle, W.handle, x.ptr, K, M, y.ptr, N, 2))
    ctx.sync()
    t = C.c_double()
    cnt = C.c_int()
    by = C.c_double()
    check(lib().ih_timing_read(ctx.handle, 0, C.byref(t), C.byref(cnt), C.byref(by)))
    kernel_us = t.value / cnt.value * 1e3
    check(lib().ih_timing_enable(ctx.handle, 0))
    ctx.sync()
    ev.record(0)
    for _ in range(64):
        check(lib().ih_qmm_int4(ctx.handle, W.handle, x.ptr, K, M, y.ptr, N, 2))
    ev.record(1)
    b2b_us = ev.elapsed_ms(0, 1) / 64 * 1e3
    # Acceptance over [8, 32000] N(0,1) logits, drafts 1..3 forced to the argmax of rows 0..2.
    logits = g.normal(0, 1, size=(8, 32000)).astype(np.float32)
    top = np.argmax(logits, axis=1).astype(np.uint32)
    vtok = g.integers(0, 32000, size=8).astype(np.uint32)
    vtok[1:4] = top[:3]
    dl, dt, dv = ctx.to_device(logits), ctx.buffer(8 * 4), ctx.to_device(vtok)
    d_st, d_rec = ctx.to_device(np.zeros(8, np.uint32)), ctx.buffer(24 * 4)
    ctx.sync()
    ev.record(0)
    reps = 50
    for _ in range(reps):
        check(lib().ih_argmax_rows(ctx.handle, dl.ptr, 8, 32000, dt.ptr))
        check(lib().ih_spec_accept_dev(ctx.handle, d_st.ptr, dv.ptr, dt.ptr, d_rec.ptr, 1, 8))
    ev.record(1)
    acc_us = ev.elapsed_ms(0, 1) / reps * 1e3
    m = int(d_rec.download(np.uint32, (24,))[0])
    gpu_top = dt.download(np.uint32, (8,))
    ev.close()
    for b in (x, y, dl, dt, dv, d_st, d_rec):
        b.free()
    W.free()
    return {"qmm_single_call_us": round(float(np.median(single)) * 1e3, 2),
            "qmm_kernel_us": round(kernel_us, 2), "qmm_kernel_gbs": round(algo / (kernel_us * 1e3), 1),
            "qmm_back_to_back_us": round(b2b_us, 2), "qmm_back_to_back_gbs": round(algo / (b2b_us * 1e3), 1),
            "qmm_algorithmic_bytes": algo,
            "note": "a call = bf16 rows to the activation layout + the qmm launch",
            "argmax_accept_us": round(acc_us, 2), "accepted_m": m,
            "argmax_equal": bool(np.array_equal(gpu_top, top))}


def _traffic(config: str, dom: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 counter runs (profiles/), if any."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        t = json.loads(f.read_text())
        return t.get(config, {}).get(dom)
    except (ValueError, OSError):
        return None


def copy_lookup_timing(ctx, lib, check, d_hist, n, k, d_copy, d_vtok, B) -> dict:
    """Device copy lookup alone over the config-2 context: µs per call and the context scan's GB/s."""
    from ingot_amd._lib import HipEvents

    for _ in range(5):
        check(lib().ih_copy_lookup_dev(ctx.handle, d_hist.ptr, n, k, 3, 64, d_copy.ptr, d_vtok.ptr, B))
    ev = HipEvents(ctx, 2)
    ctx.sync()
    reps = 50
    ev.record(0)
    for _ in range(reps):
        check(lib().ih_copy_lookup_dev(ctx.handle, d_hist.ptr, n, k, 3, 64, d_copy.ptr, d_vtok.ptr, B))
    ev.record(1)
    us = ev.elapsed_ms(0, 1) / reps * 1e3
    ctx.sync()
    out = d_copy.download(np.uint32, (4 + k,))
    return {"us": round(us, 2), "context_gbs": round(n * 4 / (us * 1e3), 1), "proposed": int(out[0]),
            "match": int(out[1])}


def copy_calibration(nbytes: int) -> int:
    """A plain device copy of known size (HIP's copy kernel through ih_memcpy_dtod), 4 times: rocprofv3's FETCH_SIZE
    and WRITE_SIZE per dispatch over it, against nbytes, give the scale factor for the counters of the other kernels."""
    from ingot_amd._lib import Context, check, lib

    ctx = Context(0)
    a, b = ctx.buffer(nbytes).fill(1), ctx.buffer(nbytes)
    ctx.sync()
    for _ in range(4):
        check(lib().ih_memcpy_dtod(ctx.handle, b.ptr, a.ptr, nbytes))
    ctx.sync()
    print(json.dumps({"copy_calibration_bytes": nbytes, "dispatches": 4}), flush=True)
    a.free()
    b.free()
    ctx.close()
    return 0


def cpu_model_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(desc, P: int, tokens, kv) -> dict | None:
    """The C++ oracle (fp32 dequant + matmul) on the host: the full model with resident weights, verify steps of the
    same block at the same P — one warm-up, then the median of 5 timed steps; tok/s as for the GPU (mean accepted + 1
    over L = 0…k → (k + 2) / 2 tokens). The same block on the GPU (ih_verify_step) is compared with the oracle's:
    top-1 equality, rows whose oracle top-2 margin is inside twice the logit error, max-abs and cosine of the logits."""
    try:
        import oracle
    except Exception as e:  # noqa: BLE001
        log(f"[bench] cpu baseline unavailable: {e}")
        return None
    t0 = time.time()
    m = oracle.OracleModel(desc, SEED, KV_SEED, P)
    t1 = time.time()
    ref_logits, ref_top1 = m.verify(tokens)  # warm-up
    times = []
    for _ in range(5):
        a = time.time()
        m.verify(tokens)
        times.append(time.time() - a)
    m.free()
    step_s = float(np.median(times))
    top1, logits = kv.verify(tokens, want_logits=True)
    err = float(np.abs(logits - ref_logits).max())
    a64, b64 = logits.astype(np.float64).ravel(), ref_logits.astype(np.float64).ravel()
    cos = float(a64 @ b64 / (np.linalg.norm(a64) * np.linalg.norm(b64)))
    srt = np.sort(ref_logits, axis=1)
    near = (srt[:, -1] - srt[:, -2]) <= 2 * err
    k = len(tokens) - 1
    mean_tokens = (k + 2) / 2.0
    log(f"[bench] cpu baseline: model built in {t1 - t0:.1f}s, steps {[round(t, 2) for t in times]}")
    return {"value": round(mean_tokens / step_s, 3), "unit": "tok/s", "cores": oracle.num_threads(),
            "cpu_model": cpu_model_name(), "kind": "port",
            "sample": f"full verify step (B={len(tokens)}, all {desc.n_layers} layers + head, P={P}) of the C++ oracle "
                      f"with resident weights: median of 5 after 1 warm-up, {step_s:.2f} s/step",
            "s_per_step": round(step_s, 3), "s_per_step_runs": [round(t, 3) for t in times],
            "oracle_top1_equal": bool(np.array_equal(top1, ref_top1)),
            "oracle_top1_equal_outside_near_ties": bool(np.array_equal(top1[~near], ref_top1[~near])),
            "near_tie_rows": int(near.sum()), "logits_max_abs": round(err, 4),
            "logits_rel": round(err / float(np.abs(ref_logits).max()), 5), "logits_cosine": round(cos, 7)}


if __name__ == "__main__":
    sys.exit(main())
