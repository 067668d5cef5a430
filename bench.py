#!/usr/bin/env python3
"""MoE layer benchmark on one MI355X (prints one JSON line on stdout).

Workload (the configuration the headline metric is quoted on): the
DeepSeek-V4-Flash-like decode MoE layer -- 256 routed experts + 1 shared
expert, hidden 4096, expert intermediate 2048, top-6 from sigmoid scores with
renormalised weights, W4A16 int4 group-128 weights with bf16 scales, bf16
activations ~ N(0,1), router logits ~ N(0,1), T = 64 tokens per step.

A step is one ``TP4MoE.forward_tensor`` call (router from the logits ->
alignment -> grouped w13 + SwiGLU -> grouped w2 x route weight -> combine with
the shared expert -> owning output clone) with inputs resident in HBM.  Inputs
rotate through a pool of seeded batches so every step routes differently.

Also reported (secondary, same line): the 8192-token prefill of the same
layer, and the CPU baseline (the oracle's restatement of the reference torch
path timed on this host's cores on a bounded sample).
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "MoE layer tokens/s; decode HBM GB/s and prefill MFMA TFLOP/s as % of peak"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--pool", type=int, default=16)
    ap.add_argument("--prefill-tokens", type=int, default=8192, help="0 skips the prefill line")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--cpu-baseline", type=int, default=1, help="0 skips the CPU baseline")
    ap.add_argument("--cpu-tokens", type=int, default=64)
    ap.add_argument("--seed", type=int, default=0)
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this build runs the whole MoE layer "
            "on one GPU (no collectives); run with --gpus 1",
            file=sys.stderr,
        )
        return 2
    import numpy as np
    import torch

    pkg = importlib.import_module("gaiban-lite_amd")
    S = pkg.synthetic
    ops = pkg.ops
    dev = torch.device("cuda:0")
    shape = S.FLASH
    E, H, I, K = shape.experts, shape.hidden, shape.inter, shape.topk
    T = args.tokens

    log(f"[bench] generating the layer (E={E}+1, H={H}, I={I}, k={K}) on {torch.cuda.get_device_name(0)}")
    w13, s13, w2, s2 = S.make_checkpoint_experts(shape, seed=args.seed, device=dev)
    resident = pkg.ResidentInt4MoEWeights.from_checkpoint_layout(
        w13, s13, w2, s2, experts=E, has_shared=True)
    cfg = pkg.TP4MoEConfig(hidden_size=H, intermediate_size=I, experts=E, topk=K,
                           route_scale=1.0, clamp_limit=0.0, score_func="sigmoid", shared_experts=1)
    gate_w = (torch.randn(E, H, device=dev) * 0.02).to(torch.bfloat16)
    gate = pkg.ResidentGateWeights(weight=gate_w)
    rows = [T] + ([args.prefill_tokens] if args.prefill_tokens else [])
    layer = pkg.TP4MoE(config=cfg, resident=resident, gate=gate, device=dev, global_row_shapes=rows)
    b_e = pkg.int4_g128_expert_bytes(H, I)
    b13 = 2 * I * H // 2 + 2 * I * (H // 128) * 2

    # ------------------------------------------------------------- decode
    xs = [S.make_hidden(T, H, seed=1000 + i, device=dev).view(1, T, H) for i in range(args.pool)]
    lgs = [S.make_logits(T, E, seed=2000 + i, device=dev) for i in range(args.pool)]
    distinct = []
    for lg in lgs:
        ids = pkg.route_from_logits(lg, topk=K, score_func="sigmoid").routing_ids
        distinct.append(int(torch.unique(ids).numel()))
    for i in range(args.warmup):
        layer.forward_tensor(xs[i % args.pool], router_logits=lgs[i % args.pool])
    torch.cuda.synchronize()

    def timed(nsteps, profile):
        if profile:
            ops.profile_begin(nsteps)
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        for i in range(nsteps):
            layer.forward_tensor(xs[i % args.pool], router_logits=lgs[i % args.pool])
        t1.record()
        torch.cuda.synchronize()
        prof = ops.profile_end() if profile else (None, 0)
        return t0.elapsed_time(t1) / nsteps, prof

    ms, (kern, ncalls) = timed(args.steps, True)
    ms_plain, _ = timed(args.steps, False)
    d_mean = float(np.mean([distinct[i % args.pool] for i in range(args.steps)]))
    layer_bytes = (d_mean + 1) * b_e + 2 * T * H * 2 + T * E * 4 + T * K * 8
    stage1_bytes = (d_mean + 1) * b13 + T * H * 2 + (T * K + T) * I * 2
    st1_ms = kern["stage1_w13"]
    achieved = stage1_bytes / (st1_ms * 1e-3) / 1e9
    log(f"[bench] decode T={T}: {ms:.4f} ms/step profiled, {ms_plain:.4f} ms/step plain; kernels {kern}")

    # ------------------------------------------------------------- prefill
    prefill = None
    if args.prefill_tokens:
        TP = args.prefill_tokens
        xp = S.make_hidden(TP, H, seed=3000, device=dev).view(1, TP, H)
        lp = S.make_logits(TP, E, seed=3001, device=dev)
        for _ in range(2):
            layer.forward_tensor(xp, router_logits=lp)
        torch.cuda.synchronize()
        ops.profile_begin(args.prefill_steps)
        p0 = torch.cuda.Event(enable_timing=True)
        p1 = torch.cuda.Event(enable_timing=True)
        p0.record()
        for _ in range(args.prefill_steps):
            layer.forward_tensor(xp, router_logits=lp)
        p1.record()
        torch.cuda.synchronize()
        pk, _ = ops.profile_end()
        pms = p0.elapsed_time(p1) / args.prefill_steps
        flops = 6.0 * TP * (K + 1) * H * I
        mm_ms = pk["stage1_w13"] + pk["stage2_w2"]
        prefill = {
            "tokens": TP,
            "ms_per_step": round(pms, 4),
            "tokens_per_s": round(TP / (pms * 1e-3), 1),
            "layer_tflops": round(flops / (pms * 1e-3) / 1e12, 2),
            "layer_frac_of_bf16_peak": round(flops / (pms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "grouped_gemm_tflops": round(flops / (mm_ms * 1e-3) / 1e12, 2),
            "kernel_ms": {k: round(v, 4) for k, v in pk.items()},
        }
        log(f"[bench] prefill T={TP}: {prefill}")

    # ------------------------------------------------------------ CPU baseline
    cpu = None
    if args.cpu_baseline:
        cpu = cpu_baseline(pkg, w13, s13, w2, s2, lgs[0], xs[0].view(T, H), args.cpu_tokens, E, K)

    line = {
        "metric": METRIC,
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations and logits, uniform int4, U(0.005,0.02) bf16 scales)",
        "config": {
            "workload": "decode MoE layer, 256 routed + 1 shared expert, H=4096, I=2048, top-6 sigmoid, "
                        f"W4A16 int4-g128 bf16 scales, T={T}, routing rotated over {args.pool} seeded batches",
            "tokens": T,
            "experts": E,
            "hidden": H,
            "intermediate": I,
            "topk": K,
            "distinct_experts_mean": round(d_mean, 2),
            "parallelism": "single GPU, whole layer resident",
        },
        "layer_hbm_gbs": round(layer_bytes / (ms * 1e-3) / 1e9, 1),
        "layer_frac_of_hbm_peak": round(layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "ms_per_step_unprofiled": round(ms_plain, 5),
        "kernel_ms": {k: round(v, 5) for k, v in kern.items()},
        "roofline": {
            "kernel": "expert_gemm_kernel stage 1 (w13 + SwiGLU), decode",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": int(stage1_bytes),
            "launch_ms": round(st1_ms, 5),
            "launches_timed": ncalls,
        },
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline(pkg, w13, s13, w2, s2, logits, x, tokens, E, K):
    """The oracle's restatement of the reference torch MoE path
    (dense_moe.py:289-354 op order, bf16 dequant-then-matmul, plus the shared
    expert and add), timed on the host over the first `tokens` rows of one
    decode batch: router, alignment and all touched experts."""

    import numpy as np
    import torch

    try:
        import oracle as O
    except Exception as exc:  # pragma: no cover
        log(f"[bench] cpu baseline unavailable: {exc}")
        return None
    from threadpoolctl import threadpool_limits

    cores = min(os.cpu_count() or 1, 16)
    lg = logits[:tokens].cpu().numpy()
    xn = x[:tokens].float().cpu().numpy()
    r = O.route_topk(lg, K, score_func=O.SCORE_SIGMOID)
    touched = sorted(set(np.unique(r.ids).tolist()) | {E})
    host = {}
    for e in touched:  # resident weights: copied before the timed region
        host[e] = (w13[e].cpu().numpy(), s13[e].contiguous().view(torch.int16).cpu().numpy().view(np.uint16),
                   w2[e].cpu().numpy(), s2[e].contiguous().view(torch.int16).cpu().numpy().view(np.uint16))

    class HostSource(O.ExpertSource):
        def __init__(self):
            super().__init__(None, None, None, None)

        def w13(self, e):
            return O.dequant_int4_g128(host[e][0], host[e][1])

        def w2(self, e):
            return O.dequant_int4_g128(host[e][2], host[e][3])

    src = HostSource()
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        rr = O.route_topk(lg, K, score_func=O.SCORE_SIGMOID)
        O.moe_align(rr.ids, 8, E)
        O.moe_bf16_mirror(xn, rr.ids, rr.weights, src, shared_index=E, workers=cores)
        dt = time.perf_counter() - t0
    log(f"[bench] cpu baseline: {tokens} tokens, {len(touched)} experts in {dt:.2f} s on {cores} threads")
    return {
        "value": round(tokens / dt, 2),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"one decode batch of {tokens} tokens of the same layer ({len(touched)} experts incl. shared), "
                  "router + alignment + bf16 dequant-then-matmul experts + combine, numpy, "
                  f"{dt:.2f} s wall",
    }


if __name__ == "__main__":
    sys.exit(main())
