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
rotate through a pool of seeded batches so every step routes differently (a
fixed-routing figure is reported beside it).

Order of the run: the prefill lines (T = 2048, 4096 and 8192 in ascending
order, each after its own untimed warm-up calls: TFLOP/s and fraction of the
bf16 peak, with a ``prefill_roofline`` block for the grouped w13 kernel at
T = 8192) come first, then the decode headline (W warm-up steps, K timed
steps with per-step times on stderr and in ``per_step_ms``), then the
secondary lines: decode at T in {1, 8, 256}, the layer from hidden states
(the gate GEMM in the call, T = 64 and 8192), decode as HIP-graph replays,
the W4A8 layer (uniform and Zipf routing, T = 64 and 8192), the layer with
MXFP4 experts (the reference checkpoint's E2M1 + E8M0 format), W4A8 over
those MXFP4 experts, the vendor's bf16 GEMM at the expert shapes, the
FP8-block shared expert, the W8A16 (int8 and FP8-block) and block-FP8 W8A8 dense linears at
K = 4096 (M <= 64 timed as 50 calls captured in a HIP graph, beside the
launch-bound Python-loop figure), and last the CPU baseline (the torch
restatement of the reference's dense path on this host's cores, the median
of three rounds per configuration, with its spread and the host's own bf16
GEMM rate).  ``env`` records versions, the device and the shader clock
read right after the headline region.

``--profile-run FMT:T:N[:graph|:hidden]`` only builds the layer and runs N
calls (the program for ``rocprofv3 --pmc`` passes and kernel traces);
``:graph`` adds N replays of the call captured as a HIP graph, ``:hidden``
routes from hidden states (the gate GEMM in every call).

``--copy-calibration`` instead runs a plain 512 MiB device copy (torch
``copy_``) 5 times: the reference kernel for scaling the FETCH_SIZE /
WRITE_SIZE counters of a ``rocprofv3 --pmc`` run to bytes.

``roofline.traffic`` (HBM bytes per stage-1 launch) is measured in the run:
after the timed work the bench starts two child processes, ``rocprofv3 --pmc
FETCH_SIZE`` and ``rocprofv3 --pmc WRITE_SIZE`` over ``bench.py
--traffic-run`` (the headline layer, one call per pooled batch, then two
512 MiB device copies), and scales each counter by what it reads for the
copy.  ``--traffic-pmc 0``, or passes that fail, fall back to the figure of
the committed counter summary, and ``traffic_source`` says which was used.
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "MoE layer tokens/s; decode HBM GB/s and prefill MFMA TFLOP/s as % of peak"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
TRAFFIC_PROFILE = ROOT / "profiles" / "expert_decode_w13_T64_hbm_traffic.md"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--pool", type=int, default=16)
    ap.add_argument("--prefill-tokens", type=int, default=8192, help="0 skips the prefill lines")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--prefill-warmup", type=int, default=10, help="untimed prefill calls before each prefill line")
    ap.add_argument("--secondary", type=int, default=1, help="0 skips the extra decode/prefill/W4A8/W8A16 lines")
    ap.add_argument("--cpu-baseline", type=int, default=1, help="0 skips the CPU baseline")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--traffic-pmc", type=int, default=1,
                    help="1 measures roofline.traffic with two rocprofv3 --pmc child passes; 0 uses the committed figure")
    ap.add_argument("--traffic-run", action="store_true",
                    help="child program of the traffic passes: one decode call per pooled batch, then two copies")
    ap.add_argument("--profile-run", default=None, metavar="FMT:T:N[:graph|:hidden]",
                    help="only run N layer calls (FMT int4|mxfp4|w4a8|w4a8-mxfp4, T tokens) for rocprofv3 counter passes; "
                         ":graph adds N replays of the captured call; FMT linear-w8a8|linear-w8a16: N calls of "
                         "the dense linear at M=T, K=4096, N in {1024, 4096, 16384} (tiled weights)")
    return ap.parse_args()


def copy_calibration() -> int:
    import torch

    copy_pair(torch, reps=5)
    print(json.dumps({"copy_calibration_bytes_per_launch": COPY_CAL_BYTES, "launches": 5}), flush=True)
    return 0


COPY_CAL_BYTES = 512 << 20


def copy_pair(torch, n=COPY_CAL_BYTES, reps=5):
    """``reps`` plain device copies of ``n`` bytes (one copy kernel each)."""

    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    a.fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def read_counter_csv(out_dir: Path):
    """Per-kernel lists of counter values (one entry per dispatch) from the
    ``*counter_collection.csv`` files a rocprofv3 --pmc pass wrote."""

    import csv

    per = {}
    for f in sorted(out_dir.rglob("*counter_collection.csv")):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                per.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return per


def measure_traffic(args, stage1_alg_bytes):
    """HBM bytes per stage-1 decode launch from two rocprofv3 --pmc child
    passes (FETCH_SIZE, then WRITE_SIZE) over ``bench.py --traffic-run``, each
    counter scaled by its reading for a plain 512 MiB device copy in the same
    pass.  Returns a dict, or None when rocprofv3 is absent or a pass fails.

    The child runs one decode call per pooled batch of the headline (the same
    seeds as the timed steps), so the counters cover the same routing mix;
    ``stage1_alg_bytes`` maps a distinct-expert count to that launch's
    algorithmic bytes, for the ratio of measured to algorithmic traffic."""

    import shutil
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if not exe or not shutil.which("timeout"):
        return None
    read = {}
    distinct = None
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        out = Path(tempfile.mkdtemp(prefix=f"bench_pmc_{ctr.lower()}_", dir="/tmp"))
        # a pass takes a few seconds; a stuck one costs at most ~1.5 minutes
        cmd = ["timeout", "-k", "10", "80", exe, "--pmc", ctr, "--output-format", "csv", "-d", str(out),
               "-o", "run", "--", sys.executable, str(Path(__file__).resolve()), "--traffic-run",
               "--tokens", str(args.tokens), "--pool", str(args.pool), "--seed", str(args.seed),
               "--prefill-tokens", "0", "--secondary", "0", "--cpu-baseline", "0"]
        log(f"[bench] traffic pass {ctr}: {' '.join(cmd)}")
        try:
            proc = subprocess.run(cmd, cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"}, stdout=subprocess.PIPE,
                                  text=True, timeout=100)
            info = None
            for ln in proc.stdout.splitlines():
                if ln.startswith('{"traffic_run"'):
                    info = json.loads(ln)
            per = read_counter_csv(out)
        except (OSError, subprocess.SubprocessError, ValueError, KeyError) as e:
            log(f"[bench] traffic pass {ctr} failed: {e!r}")
            return None
        finally:
            shutil.rmtree(out, ignore_errors=True)
        # rocprofv3 may end nonzero after the program finished and its files
        # are whole; the child's closing line and the dispatch counts decide
        st1 = [v for k, v in per.items() if "expert_decode_kernel<1" in k]
        # the 512 MiB copies are the largest copy dispatches (the layer's own
        # device copies are far smaller)
        cpy = sorted((x for k, v in per.items() if "copyBuffer" in k for x in v), reverse=True)
        if info is None or len(st1) != 1 or len(st1[0]) != info["stage1_launches"] or len(cpy) < info["copies"]:
            log(f"[bench] traffic pass {ctr}: rc={proc.returncode}, closing line {info is not None}, "
                f"stage-1 kernels {[len(v) for v in st1]}, copy dispatches {len(cpy)}: not used")
            return None
        distinct = info["distinct_per_launch"]
        read[ctr] = (sum(st1[0]) / len(st1[0]), sum(cpy[:info["copies"]]) / info["copies"])
        log(f"[bench] traffic pass {ctr}: rc={proc.returncode}, stage-1 mean {read[ctr][0]:.1f} KiB over "
            f"{len(st1[0])} launches, copy {read[ctr][1]:.1f} KiB")
    scale = {c: COPY_CAL_BYTES / (read[c][1] * 1024.0) for c in read}
    traffic = sum(read[c][0] * 1024.0 * scale[c] for c in read)
    alg = sum(stage1_alg_bytes(d) for d in distinct) / len(distinct)
    return {
        "bytes": int(round(traffic)),
        "fetch_kib": round(read["FETCH_SIZE"][0], 1),
        "write_kib": round(read["WRITE_SIZE"][0], 1),
        "fetch_scale": round(scale["FETCH_SIZE"], 4),
        "write_scale": round(scale["WRITE_SIZE"], 4),
        "launches": len(distinct),
        "algorithmic_bytes_same_launches": int(alg),
        "over_algorithmic": round(traffic / alg, 4),
    }


def traffic_from_profile():
    """HBM bytes per stage-1 decode launch measured by the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, calibrated), or None."""

    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch\s*=\s*([0-9]+)", text)
    return int(m.group(1)) if m else None


def read_sclk_sysfs():
    """The active shader-clock level of the GPU from the driver's sysfs table
    (``pp_dpm_sclk``; fast, no subprocess), or None when it is not readable."""

    import glob

    for path in sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk")):
        try:
            text = Path(path).read_text()
        except OSError:
            continue
        for line in text.splitlines():
            if line.strip().endswith("*"):
                m = re.search(r"(\d+)\s*M[Hh]z", line)
                if m:
                    return {"mhz": int(m.group(1)), "source": path}
    return None


def read_sclk():
    """The GPU shader clock as the system management tool reports it (MHz),
    or None when no tool answers within a few seconds."""

    import shutil
    import subprocess

    for cmd in (["amd-smi", "metric", "--clock", "--json"], ["rocm-smi", "--showclocks"]):
        if not shutil.which(cmd[0]):
            continue
        try:
            out = subprocess.run(cmd, capture_output=True, text=True, timeout=8).stdout
        except Exception:  # noqa: BLE001 - the witness is optional
            continue
        m = re.search(r"sclk[^0-9]*?(\d+)\s*M[Hh]z", out) or re.search(r'"GFX_0".*?"clk":\s*\{?[^0-9]*(\d+)', out, re.S)
        if m:
            return {"mhz": int(m.group(1)), "tool": cmd[0]}
    return None


def environment(torch, sclk_busy=None, sclk_end=None):
    """Versions and device of the run (a witness for the peak figures used)."""

    props = torch.cuda.get_device_properties(0)
    rocm = None
    for path in ("/opt/rocm/.info/version", "/opt/rocm/.info/version-dev"):
        try:
            rocm = Path(path).read_text().strip()
            break
        except OSError:
            pass
    return {
        "torch": torch.__version__,
        "hip": getattr(torch.version, "hip", None),
        "rocm": rocm,
        "device": torch.cuda.get_device_name(0),
        "arch": getattr(props, "gcnArchName", None),
        "compute_units": props.multi_processor_count,
        "hbm_bytes": props.total_memory,
        "sclk_during_decode": sclk_busy,
        "sclk_at_end": sclk_end,
        "host_cpus": os.cpu_count(),
    }


def cuda_timer(fn, n, per_step=None, sync_before=True):
    """Mean ms per call of `fn` over `n` calls, timed with events on the
    current stream.  With `per_step` (a list), an event is also recorded
    after every call and the per-call times are appended to it.  With
    `sync_before` False the timed calls queue right behind the work already
    on the stream (no idle gap before the first event)."""

    import torch

    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(n)] if per_step is not None else None
    if sync_before:
        torch.cuda.synchronize()
    t0.record()
    for i in range(n):
        fn(i)
        if marks is not None:
            marks[i].record()
    t1.record()
    torch.cuda.synchronize()
    if marks is not None:
        prev = t0
        for m in marks:
            per_step.append(prev.elapsed_time(m))
            prev = m
    return t0.elapsed_time(t1) / n


def graph_timer(fn, n, out):
    """Per-call GPU time of `fn` (kernels only, no host launch gaps): `n` calls
    captured into one HIP graph, replayed and timed with events.  The replay's
    output must equal an eager call's (`out` after each), else None."""

    import torch

    fn(0)
    torch.cuda.synchronize()
    want = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    ok = torch.equal(out, want)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(3):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ok = ok and torch.equal(out, want)
    del graph
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / (3 * n) if ok else None


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this build runs the whole MoE layer "
            "on one GPU (no collectives); run with --gpus 1",
            file=sys.stderr,
        )
        return 2
    if args.copy_calibration:
        return copy_calibration()
    if args.traffic_run:
        args.prefill_tokens, args.secondary = 0, 0
    import numpy as np
    import torch

    pkg = importlib.import_module("gaiban-lite_amd")
    if args.profile_run:
        return profile_run(pkg, args.profile_run, args.seed)
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
    decode_ts = [T] + ([1, 8, 256] if args.secondary else [])
    prefill_ts = []
    if args.prefill_tokens:
        prefill_ts = [args.prefill_tokens] + ([2048, 4096] if args.secondary else [])
    rows = sorted(set(decode_ts + prefill_ts))
    layer = pkg.TP4MoE(config=cfg, resident=resident, gate=gate, device=dev, global_row_shapes=rows)
    b_e = pkg.int4_g128_expert_bytes(H, I)
    b13 = 2 * I * H // 2 + 2 * I * (H // 128) * 2

    def layer_bytes(t, d):
        return (d + 1) * b_e + 2 * t * H * 2 + t * E * 4 + t * K * 8

    def pools(t, n, base):
        xs = [S.make_hidden(t, H, seed=base + i, device=dev).view(1, t, H) for i in range(n)]
        lgs = [S.make_logits(t, E, seed=base + 500 + i, device=dev) for i in range(n)]
        d = [int(torch.unique(pkg.route_from_logits(lg, topk=K, score_func="sigmoid").routing_ids).numel())
             for lg in lgs]
        return xs, lgs, d

    def stage1_alg_bytes(d):
        # stage-1 (w13 + SwiGLU) bytes of one decode launch with d distinct
        # routed experts: their w13 and scales plus the shared expert's, x
        # read, h written for the T k routed and T shared rows
        return (d + 1) * b13 + T * H * 2 + (T * K + T) * I * 2

    if args.traffic_run:
        # the program the traffic passes wrap: one warm-up call on batch 0,
        # one call per pooled batch (the headline's seeds), then the copies
        xs, lgs, distinct = pools(T, args.pool, 1000)
        order = [0] + list(range(args.pool))
        for i in order:
            layer.forward_tensor(xs[i], router_logits=lgs[i])
        torch.cuda.synchronize()
        copy_pair(torch, reps=2)
        print(json.dumps({"traffic_run": True, "stage1_launches": len(order), "copies": 2,
                          "distinct_per_launch": [distinct[i] for i in order]}), flush=True)
        return 0

    # ------------------------------------------------------------- prefill
    # Timed before the decode headline: a GPU that has just been idle (fresh
    # process, weights generated with host syncs between launches) runs its
    # first ~25 decode steps up to 30% slow while it ramps up (per-step times
    # fall from 0.59 to 0.46 ms); the prefill lines bring it to its steady
    # state, so the headline measures the sustained decode rate.
    prefill = None
    prefill_lines = {}
    if prefill_ts:
        # the smaller sizes first: the headline size is timed on a GPU that has
        # been running MFMA work for a while, and each line's timed calls queue
        # behind its own untimed warm-up calls (no idle gap, clocks settled)
        for tp in sorted(prefill_ts):
            xp = S.make_hidden(tp, H, seed=3000, device=dev).view(1, tp, H)
            lp = S.make_logits(tp, E, seed=3001, device=dev)
            for _ in range(args.prefill_warmup):
                layer.forward_tensor(xp, router_logits=lp)
            # ms_per_step without per-kernel events, then the same calls with
            # them for the per-stage times
            pms = cuda_timer(lambda i: layer.forward_tensor(xp, router_logits=lp), args.prefill_steps,
                             sync_before=False)
            ops.profile_begin(args.prefill_steps)
            pms_ev = cuda_timer(lambda i: layer.forward_tensor(xp, router_logits=lp), args.prefill_steps,
                                sync_before=False)
            pk, _ = ops.profile_end()
            flops = 6.0 * tp * (K + 1) * H * I
            mm_ms = pk["stage1_w13"] + pk["stage2_w2"]
            prefill_lines[tp] = {
                "tokens": tp,
                "ms_per_step": round(pms, 4),
                "ms_per_step_all_kernel_events": round(pms_ev, 4),
                "tokens_per_s": round(tp / (pms * 1e-3), 1),
                "tflops": round(flops / (pms * 1e-3) / 1e12, 2),
                "frac_of_bf16_peak": round(flops / (pms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                "grouped_gemm_tflops": round(flops / (mm_ms * 1e-3) / 1e12, 2),
                "stage1_ms": round(pk["stage1_w13"], 4),
                "stage2_ms": round(pk["stage2_w2"], 4),
                "combine_ms": round(pk["combine"], 4),
            }
            log(f"[bench] prefill T={tp}: {prefill_lines[tp]} kernels {pk}")
            del xp, lp
        tp = prefill_ts[0]
        prefill = prefill_lines[tp]
        # the dominant prefill kernel: grouped w13 + SwiGLU, 2 T (k+1) (2I) H flops per launch
        st1_flops = 2.0 * tp * (K + 1) * (2 * I) * H
        st1 = prefill["stage1_ms"]
        secondary_prefill_roofline = {
            "kernel": f"expert_prefill_kernel<1> (w13 + SwiGLU), prefill T={tp}",
            "bound": "mfma",
            "achieved": round(st1_flops / (st1 * 1e-3) / 1e12, 1),
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(st1_flops / (st1 * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "traffic": None,
            "algorithmic_flops_per_launch": int(st1_flops),
            "launch_ms": st1,
            "launches_timed": args.prefill_steps,
        }

    # ------------------------------------------------------------- decode
    # Inputs of every decode line are prepared first (host reads included).
    # The timed decode work then runs as one stream: the T=256 line (its
    # ms_per_step, timed with events), the headline's warm-up and the
    # headline's K timed steps, with no host synchronisation in between.  The
    # HBM-bound decode reaches its sustained rate only after ~10 ms of memory
    # traffic: the GPU's power management lowers clocks during idle or
    # compute-only stretches and raises them under load, so steps that start
    # after an idle gap run up to ~20% slow at first (per-step times falling
    # from ~0.53 to ~0.45 ms over 20 steps), while steps queued behind other
    # decode work run at the sustained rate from the first one.
    xs, lgs, distinct = pools(T, args.pool, 1000)
    other = {t: pools(t, 8, 4000 + t) for t in decode_ts[1:]} if args.secondary else {}
    lead_t = 256 if 256 in other else None
    torch.cuda.synchronize()
    if lead_t:
        xt, lt, _ = other[lead_t]
        lead_ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        lead_n = 100
        lead_ev[0].record()
        for i in range(lead_n):
            layer.forward_tensor(xt[i % 8], router_logits=lt[i % 8])
        lead_ev[1].record()
    for i in range(args.warmup):
        layer.forward_tensor(xs[i % args.pool], router_logits=lgs[i % args.pool])
    sclk_busy = read_sclk_sysfs()  # read while the queued decode work runs

    def step(i):
        layer.forward_tensor(xs[i % args.pool], router_logits=lgs[i % args.pool])

    # timed region: K steps with two HIP events per step around the roofline
    # kernel (stage 1), recorded by the library on the launch stream
    ops.profile_begin(args.steps, intervals=["stage1_w13"])
    step_ms: list[float] = []
    ms = cuda_timer(step, args.steps, per_step=step_ms, sync_before=False)
    roof, ncalls = ops.profile_end()
    lead_ms = lead_ev[0].elapsed_time(lead_ev[1]) / lead_n if lead_t else None
    log("[bench] headline per-step ms: " + " ".join(f"{v:.4f}" for v in step_ms))
    # the same steps with all seven stamps (per-kernel breakdown), and with none
    ops.profile_begin(args.steps)
    ms_all = cuda_timer(step, args.steps, sync_before=False)
    kern, _ = ops.profile_end()
    ms_plain = cuda_timer(step, args.steps, sync_before=False)
    ms_fixed = cuda_timer(lambda i: layer.forward_tensor(xs[0], router_logits=lgs[0]), args.steps,
                          sync_before=False)
    d_mean = float(np.mean([distinct[i % args.pool] for i in range(args.steps)]))
    stage1_bytes = stage1_alg_bytes(d_mean)
    st1_ms = roof["stage1_w13"]
    achieved = stage1_bytes / (st1_ms * 1e-3) / 1e9
    log(f"[bench] decode T={T}: {ms:.4f} ms/step (stage-1 events), {ms_all:.4f} with all kernel events, "
        f"{ms_plain:.4f} without events, {ms_fixed:.4f} fixed routing; kernels {kern}")

    secondary = {}
    if args.secondary:
        dec = {}
        for t in decode_ts[1:]:
            xt, lt, dt_ = other[t]
            n = 100
            if t == lead_t:
                ms_t = lead_ms
            else:
                for i in range(5):
                    layer.forward_tensor(xt[i % 8], router_logits=lt[i % 8])
                ms_t = cuda_timer(lambda i: layer.forward_tensor(xt[i % 8], router_logits=lt[i % 8]), n,
                                  sync_before=False)
            ops.profile_begin(n)
            cuda_timer(lambda i: layer.forward_tensor(xt[i % 8], router_logits=lt[i % 8]), n)
            kt, _ = ops.profile_end()
            dm = float(np.mean(dt_))
            gbs = layer_bytes(t, dm) / (ms_t * 1e-3) / 1e9
            dec[str(t)] = {"ms_per_step": round(ms_t, 4), "tokens_per_s": round(t / (ms_t * 1e-3), 1),
                           "distinct_experts_mean": round(dm, 1), "layer_hbm_gbs": round(gbs, 1),
                           "layer_frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                           "kernel_ms": {k: round(v, 4) for k, v in kt.items()}}
            log(f"[bench] decode T={t}: {dec[str(t)]}")
        secondary["decode_other_T"] = dec

    # -------------------------------------------------------- W4A8 and W8A16
    if args.secondary:
        secondary["layer_from_hidden_states"] = bench_from_hidden(
            pkg, layer, gate_w, dev, [T] + ([args.prefill_tokens] if args.prefill_tokens else []), args)
        secondary["decode_graph"] = bench_graph(layer, S, dev, [1, 8, T], H, E)
        secondary["w4a8"] = bench_w4a8(pkg, resident, gate, cfg, dev, T, args)
        secondary["mxfp4"] = bench_mxfp4(pkg, gate, cfg, dev, T, args)
        secondary["w4a8_mxfp4"] = bench_w4a8_mxfp4(pkg, gate, cfg, dev, T, args)
        secondary["vendor_bf16_gemm"] = bench_vendor_bf16_gemm(dev)
        secondary["fp8_shared"] = bench_shared_fp8(pkg, gate, cfg, dev, T, args)
        secondary["w8a16_linear"] = bench_w8a16(pkg, dev)
        secondary["w8a16_fp8_block_linear"] = bench_w8a16(pkg, dev, fmt="fp8")
        secondary["w8a8_block_fp8_linear"] = bench_block_fp8(pkg, dev)

    # ------------------------------------------------------------ CPU baseline
    cpu = None
    if args.cpu_baseline:
        cpu = cpu_baseline(pkg, w13, s13, w2, s2, args.seed)

    sclk_end = read_sclk()  # before the counter passes below
    traffic_pmc = measure_traffic(args, stage1_alg_bytes) if args.traffic_pmc else None
    if traffic_pmc is not None:
        traffic = traffic_pmc["bytes"]
        traffic_source = ("measured in this run: rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE child passes "
                          "over bench.py --traffic-run, each scaled by its reading for a 512 MiB device copy")
    else:
        traffic = traffic_from_profile()
        traffic_source = (f"committed counter summary {TRAFFIC_PROFILE.relative_to(ROOT)}"
                          + (" (the passes of this run failed)" if args.traffic_pmc else "")
                          if traffic is not None else None)
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
        "layer_hbm_gbs": round(layer_bytes(T, d_mean) / (ms * 1e-3) / 1e9, 1),
        "layer_frac_of_hbm_peak": round(layer_bytes(T, d_mean) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "ms_per_step_all_kernel_events": round(ms_all, 5),
        "ms_per_step_unprofiled": round(ms_plain, 5),
        "ms_per_step_fixed_routing": round(ms_fixed, 5),
        "kernel_ms": {k: round(v, 5) for k, v in kern.items()},
        "roofline": {
            "kernel": "expert_decode_kernel<1, 8, false> (w13 + SwiGLU), decode T=64",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "traffic_counters": traffic_pmc,
            "algorithmic_bytes_per_launch": int(stage1_bytes),
            "launch_ms": round(st1_ms, 5),
            "launches_timed": ncalls,
        },
        "prefill": prefill,
        "prefill_roofline": secondary_prefill_roofline if prefill_ts else None,
        "prefill_other_T": {str(t): v for t, v in prefill_lines.items() if prefill_ts and t != prefill_ts[0]},
        "per_step_ms": [round(v, 4) for v in step_ms],
        **secondary,
        "cpu_baseline": cpu,
        "env": environment(torch, sclk_busy=sclk_busy, sclk_end=sclk_end),
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_graph(layer, S, dev, ts, H, E):
    """The decode layer call captured once as a HIP graph (torch.cuda.graph,
    after resetting the slot's completion event, as the reference's stateful
    graphs do) and replayed, against the same call launched eagerly.

    Two pairs per T.  ``ms_per_step_graph`` / ``ms_per_step_eager``: the call
    on the captured input tensors with nothing between calls -- the layer as
    one node of a whole decode-stage graph sees it (its input written by the
    graph's previous node).  ``*_with_input_copies``: each step first copies a
    new activation and new logits into the captured inputs (two stream copies)
    and then replays or launches; the graph's first kernel then waits on the
    copy's completion signal, which costs about a microsecond more than the
    same wait between two eager launches."""

    import torch

    out = {}
    for t in ts:
        xs = [S.make_hidden(t, H, seed=7000 + t + i, device=dev).view(1, t, H) for i in range(8)]
        lgs = [S.make_logits(t, E, seed=7500 + t + i, device=dev) for i in range(8)]
        x_s, lg_s = xs[0].clone(), lgs[0].clone()
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(3):
                layer.forward_tensor(x_s, router_logits=lg_s)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        layer.reset_free_slot_completion_event(t, 0)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            layer.forward_tensor(x_s, router_logits=lg_s)
        torch.cuda.synchronize()

        def copy_in(i):
            x_s.copy_(xs[i % 8])
            lg_s.copy_(lgs[i % 8])

        def replay(i):
            graph.replay()

        def eager(i):
            layer.forward_tensor(x_s, router_logits=lg_s)

        def replay_copied(i):
            copy_in(i)
            graph.replay()

        def eager_copied(i):
            copy_in(i)
            layer.forward_tensor(x_s, router_logits=lg_s)

        n = 200
        for i in range(10):
            replay_copied(i)
        rec = {}
        # alternate the two modes twice so that neither always runs first
        for rnd in range(2):
            for name, fn in (("graph", replay), ("eager", eager), ("graph_with_input_copies", replay_copied),
                             ("eager_with_input_copies", eager_copied)):
                rec.setdefault(name, []).append(cuda_timer(fn, n))
        row = {f"ms_per_step_{k}": round(min(v), 4) for k, v in rec.items()}
        row["tokens_per_s_graph"] = round(t / (row["ms_per_step_graph"] * 1e-3), 1)
        out[str(t)] = row
        log(f"[bench] decode graph T={t}: {row}")
        del graph
        torch.cuda.synchronize()
        layer.reset_free_slot_completion_event(t, 0)
    return out


def bench_from_hidden(pkg, layer, gate_w, dev, ts, args):
    """The reference's timed unit (``a3_moe_bench.py:89-105``): the layer from
    hidden states, i.e. the fp32 gate GEMM x . Wg^T (``dsv4moe_gate_logits``)
    then route, align, experts and combine -- ``TP4MoE.forward_tensor``
    without router logits.  Also the gate GEMM alone and its share of the
    step, with its bytes (Wg + x + logits) and flops as rates."""

    import torch

    S, ops = pkg.synthetic, pkg.ops
    E, H = gate_w.shape
    out = {}
    for t in ts:
        xs = [S.make_hidden(t, H, seed=9000 + t + i, device=dev).view(1, t, H) for i in range(4)]
        lg = torch.empty((t, E), dtype=torch.float32, device=dev)
        n = 100 if t <= 256 else args.prefill_steps
        for i in range(3):
            layer.forward_tensor(xs[i % 4])
        ms = cuda_timer(lambda i: layer.forward_tensor(xs[i % 4]), n, sync_before=False)
        for i in range(3):
            ops.gate_logits_into(xs[0].view(t, H), gate_w, lg)
        gms = cuda_timer(lambda i: ops.gate_logits_into(xs[i % 4].view(t, H), gate_w, lg), n, sync_before=False)
        flops = 2.0 * t * E * H
        byts = E * H * 2 + t * H * 2 + t * E * 4
        out[f"T{t}"] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(t / (ms * 1e-3), 1),
                        "gate_gemm_us": round(gms * 1e3, 2), "gate_share_of_step": round(gms / ms, 4),
                        "gate_gemm_tflops": round(flops / (gms * 1e-3) / 1e12, 1),
                        "gate_gemm_gbs": round(byts / (gms * 1e-3) / 1e9, 1)}
        log(f"[bench] layer from hidden states T={t}: {out[f'T{t}']}")
        del xs, lg
    return out


def bench_vendor_bf16_gemm(dev):
    """The vendor library's dense bf16 GEMM (torch.bmm, hipBLASLt / rocBLAS)
    on plain bf16 operands at this layer's per-expert shapes -- 256 experts x
    192 tokens (the uniform T=8192 load) through w13 [4096 x 4096] and w2
    [4096 x 2048] -- and on a large square GEMM: what a tuned dense GEMM
    sustains on this GPU at its load-time clocks, with no dequantisation, as
    context for the prefill fractions of the nominal 2.5 PFLOP/s peak."""

    import torch

    out = {}
    for name, (batch, m, n, k, reps) in {"experts_w13_256x192x4096x4096": (256, 192, 4096, 4096, 10),
                                         "experts_w2_256x192x4096x2048": (256, 192, 4096, 2048, 10),
                                         "square_8192": (1, 8192, 8192, 8192, 5)}.items():
        a = torch.randn(batch, m, k, device=dev, dtype=torch.bfloat16)
        b = torch.randn(batch, k, n, device=dev, dtype=torch.bfloat16)  # contiguous right operand
        for _ in range(3):
            torch.bmm(a, b)
        ms = cuda_timer(lambda i: torch.bmm(a, b), reps)
        tf = 2.0 * batch * m * n * k / (ms * 1e-3) / 1e12
        out[name] = {"ms": round(ms, 4), "tflops": round(tf, 1), "frac_of_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
        log(f"[bench] vendor bf16 GEMM {name}: {out[name]}")
        del a, b
    torch.cuda.empty_cache()
    return out


def bench_w4a8_mxfp4(pkg, gate, cfg, dev, T, args):
    """W4A8 over the checkpoint's MXFP4 experts (E2M1 codes with E8M0 per-32
    scales against per-token e4m3 activations on the block-scaled fp8 x fp4
    MFMA): the lines of ``bench_w4a8`` with those weights."""

    import torch

    S = pkg.synthetic
    w13, s13, w2, s2 = S.make_checkpoint_experts_mxfp4(S.FLASH, seed=args.seed, device=dev)
    res = pkg.ResidentMXFP4MoEWeights.from_checkpoint_layout(w13, s13, w2, s2, experts=cfg.experts, has_shared=True,
                                                              marlin_input_dtype=torch.float8_e4m3fn)
    del w13, s13, w2, s2
    out = bench_w4a8(pkg, res, gate, cfg, dev, T, args, experts_into=pkg.ops.experts_w4a8_mxfp4_into,
                     label="w4a8 mxfp4", mxfp4=True)
    del res
    torch.cuda.empty_cache()
    return out


def bench_w4a8(pkg, resident, gate, cfg, dev, T, args, experts_into=None, label="w4a8", mxfp4=False):
    """W4A8 experts (fp8 activations, the same resident int4 weights) at the
    decode T and the prefill size, uniform routing (router from logits) and
    Zipf(1.1) routing (fixed ids).  A uniform step is the fused layer entry
    (route -> align with x quantised beside it -> experts -> combine); a Zipf
    step is the given ids' alignment + the experts entry (which quantises x
    itself) + combine; all stream-ordered launches."""

    import torch

    S, ops = pkg.synthetic, pkg.ops
    experts_into = experts_into or ops.experts_w4a8_into
    E, H, I, K = cfg.experts, cfg.hidden_size, cfg.intermediate_size, cfg.topk
    ts = [T] + ([args.prefill_tokens] if args.prefill_tokens else [])
    out = {}
    for t in ts:
        x = S.make_hidden(t, H, seed=5000 + t, device=dev)
        lg = S.make_logits(t, E, seed=5500 + t, device=dev)
        bs = ops.block_size_m(t, K, E, 1)
        cap = pkg.max_padded_tokens(t * K, E, bs)
        sorted_ids = torch.empty(cap, dtype=torch.int32, device=dev)
        expert_ids = torch.empty((cap + bs - 1) // bs, dtype=torch.int32, device=dev)
        ntpp = torch.empty(1, dtype=torch.int32, device=dev)
        ids = torch.empty((t, K), dtype=torch.int32, device=dev)
        w = torch.empty((t, K), dtype=torch.float32, device=dev)
        margin = torch.empty((t,), dtype=torch.float32, device=dev)
        o = torch.empty((t, H), dtype=torch.bfloat16, device=dev)
        ws = torch.empty(ops.experts_w4a8_workspace_bytes(t, K, H, I, True), dtype=torch.uint8, device=dev)
        zipf_ids = S.zipf_ids(t, E, K, seed=4, device=dev)
        counts = torch.bincount(zipf_ids.view(-1).long(), minlength=E).float()
        for routing in ("uniform", "zipf"):
            def step(i):
                if routing == "uniform":
                    ops.layer_w4a8_into(x, lg, None, topk=K, score_func="sigmoid", route_scale=1.0,
                                        w13q=resident.w13_q, w13s=resident.w13_s, w2q=resident.w2_q,
                                        w2s=resident.w2_s, experts=E, inter=I, has_shared=True, clamp_limit=0.0,
                                        block_size=bs, ids=ids, weights=w, margin=margin,
                                        sorted_token_ids=sorted_ids, expert_ids=expert_ids,
                                        num_tokens_post_padded=ntpp, out=o, workspace=ws, mxfp4=mxfp4)
                    return
                ids.copy_(zipf_ids)
                ops.align_into(ids, block_size=bs, num_experts=E, sorted_token_ids=sorted_ids,
                               expert_ids=expert_ids, num_tokens_post_padded=ntpp, workspace=ws)
                experts_into(x, w13q=resident.w13_q, w13s=resident.w13_s, w2q=resident.w2_q,
                             w2s=resident.w2_s, experts=E, inter=I, has_shared=True, route_weights=w,
                             sorted_token_ids=sorted_ids, expert_ids=expert_ids,
                             num_tokens_post_padded=ntpp, block_size=bs, clamp_limit=0.0, out=o,
                             workspace=ws)
            ops.route_topk_into(lg, None, topk=K, score_func="sigmoid", route_scale=1.0, ids=ids, weights=w)
            for i in range(10 if t > 256 else 3):
                step(i)
            n = 50 if t <= 256 else 10
            # ms_per_step without the library's per-kernel events (as the
            # headline's ms_per_step_unprofiled); kernel_ms from a second pass
            # with them, which adds a few us per step
            ms = cuda_timer(step, n, sync_before=False)
            ops.profile_begin(n)
            ms_ev = cuda_timer(step, n, sync_before=False)
            pk, _ = ops.profile_end()
            flops = 6.0 * t * (K + 1) * H * I
            entry = {"ms_per_step": round(ms, 4), "tokens_per_s": round(t / (ms * 1e-3), 1), "block_size": bs,
                     "ms_per_step_all_kernel_events": round(ms_ev, 4),
                     "kernel_ms": {k: round(v, 4) for k, v in pk.items() if k not in ("route", "align")}}
            if t > 256:
                entry["layer_tflops"] = round(flops / (ms * 1e-3) / 1e12, 2)
                entry["layer_frac_of_fp8_peak"] = round(flops / (ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4)
            if routing == "zipf":
                entry["hottest_over_mean_load"] = round(float(counts.max() / counts.mean()), 1)
            out[f"T{t}_{routing}"] = entry
            log(f"[bench] {label} T={t} {routing}: {entry}")
        del x, lg, o, ws
    return out


def bench_mxfp4(pkg, gate, cfg, dev, T, args):
    """The same layer with MXFP4 routed + shared experts (E2M1 codes, E8M0
    scale per 32 K: the reference checkpoint's routed-expert format) through
    the TP4MoE drop-in: decode at T (routing rotated over 8 batches) and
    prefill at the prefill size; stage-1 decode HBM rate and prefill TFLOP/s."""

    import numpy as np
    import torch

    S, ops = pkg.synthetic, pkg.ops
    E, H, I, K = cfg.experts, cfg.hidden_size, cfg.intermediate_size, cfg.topk
    w13, s13, w2, s2 = S.make_checkpoint_experts_mxfp4(S.FLASH, seed=args.seed, device=dev)
    res = pkg.ResidentMXFP4MoEWeights.from_checkpoint_layout(w13, s13, w2, s2, experts=E, has_shared=True)
    del w13, s13, w2, s2
    rows = [T] + ([args.prefill_tokens] if args.prefill_tokens else [])
    layer = pkg.TP4MoE(config=cfg, resident=res, gate=gate, device=dev, global_row_shapes=sorted(set(rows)))
    b13 = 2 * I * H // 2 + 2 * I * H // 32
    out = {"expert_bytes": pkg.mxfp4_g32_expert_bytes(H, I)}
    xs = [S.make_hidden(T, H, seed=7000 + i, device=dev).view(1, T, H) for i in range(8)]
    lgs = [S.make_logits(T, E, seed=7500 + i, device=dev) for i in range(8)]
    distinct = [int(torch.unique(pkg.route_from_logits(lg, topk=K, score_func="sigmoid").routing_ids).numel())
                for lg in lgs]
    for i in range(5):
        layer.forward_tensor(xs[i % 8], router_logits=lgs[i % 8])
    n = 100
    # ms_per_step without per-kernel events; kernel_ms (and the stage-1 rate)
    # from a second pass with them
    ms = cuda_timer(lambda i: layer.forward_tensor(xs[i % 8], router_logits=lgs[i % 8]), n, sync_before=False)
    ops.profile_begin(n)
    ms_ev = cuda_timer(lambda i: layer.forward_tensor(xs[i % 8], router_logits=lgs[i % 8]), n,
                       sync_before=False)
    pk, _ = ops.profile_end()
    d_mean = float(np.mean([distinct[i % 8] for i in range(n)]))
    st1 = (d_mean + 1) * b13 + T * H * 2 + (T * K + T) * I * 2
    layer_b = (d_mean + 1) * out["expert_bytes"] + 2 * T * H * 2 + T * E * 4 + T * K * 8
    out[f"decode_T{T}"] = {
        "ms_per_step": round(ms, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
        "ms_per_step_all_kernel_events": round(ms_ev, 4),
        "layer_hbm_gbs": round(layer_b / (ms * 1e-3) / 1e9, 1),
        "stage1_hbm_gbs": round(st1 / (pk["stage1_w13"] * 1e-3) / 1e9, 1),
        "stage1_frac_of_hbm_peak": round(st1 / (pk["stage1_w13"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "kernel_ms": {k: round(v, 4) for k, v in pk.items()},
    }
    log(f"[bench] mxfp4 decode T={T}: {out[f'decode_T{T}']}")
    if args.prefill_tokens:
        tp = args.prefill_tokens
        xp = S.make_hidden(tp, H, seed=3000, device=dev).view(1, tp, H)
        lp = S.make_logits(tp, E, seed=3001, device=dev)
        for _ in range(args.prefill_warmup):
            layer.forward_tensor(xp, router_logits=lp)
        pms = cuda_timer(lambda i: layer.forward_tensor(xp, router_logits=lp), args.prefill_steps,
                         sync_before=False)
        ops.profile_begin(args.prefill_steps)
        cuda_timer(lambda i: layer.forward_tensor(xp, router_logits=lp), args.prefill_steps, sync_before=False)
        pk, _ = ops.profile_end()
        flops = 6.0 * tp * (K + 1) * H * I
        mm_ms = pk["stage1_w13"] + pk["stage2_w2"]
        out[f"prefill_T{tp}"] = {
            "ms_per_step": round(pms, 4), "tokens_per_s": round(tp / (pms * 1e-3), 1),
            "layer_tflops": round(flops / (pms * 1e-3) / 1e12, 2),
            "layer_frac_of_bf16_peak": round(flops / (pms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "grouped_gemm_tflops": round(flops / (mm_ms * 1e-3) / 1e12, 2),
            "kernel_ms": {k: round(v, 4) for k, v in pk.items()},
        }
        log(f"[bench] mxfp4 prefill T={tp}: {out[f'prefill_T{tp}']}")
    del layer, res
    torch.cuda.empty_cache()
    return out


def bench_shared_fp8(pkg, gate, cfg, dev, T, args):
    """The FLASH layer with int4-g128 routed experts and the shared expert in
    the checkpoint's FP8 block format (dense W8A16 linears adding into the
    routed sum) at the decode T and the prefill size."""

    import dataclasses

    import torch

    S, ops = pkg.synthetic, pkg.ops
    E, H, I = cfg.experts, cfg.hidden_size, cfg.intermediate_size
    routed_shape = dataclasses.replace(S.FLASH, has_shared=False)
    w = S.make_checkpoint_experts(routed_shape, seed=args.seed, device=dev)
    sw = [S.make_fp8_block_linear(n, k, seed=args.seed + j, device=dev)
          for j, (n, k) in enumerate(((I, H), (I, H), (H, I)))]
    shared = pkg.ResidentFP8SharedExpert.from_checkpoint(sw[0][0], sw[0][1], sw[1][0], sw[1][1], sw[2][0], sw[2][1])
    res = pkg.ResidentInt4MoEWeights.from_checkpoint_layout(*w, experts=E, has_shared=False, shared_fp8=shared)
    del w, sw
    ts = [T] + ([args.prefill_tokens] if args.prefill_tokens else [])
    layer = pkg.TP4MoE(config=cfg, resident=res, gate=gate, device=dev, global_row_shapes=ts)
    out = {"shared_fp8_bytes": shared.resident_bytes}
    for t in ts:
        x = S.make_hidden(t, H, seed=8000 + t, device=dev).view(1, t, H)
        lg = S.make_logits(t, E, seed=8500 + t, device=dev)
        for _ in range(3):
            layer.forward_tensor(x, router_logits=lg)
        n = 100 if t == T else args.prefill_steps
        ms = cuda_timer(lambda i: layer.forward_tensor(x, router_logits=lg), n, sync_before=False)
        out[f"T{t}"] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(t / (ms * 1e-3), 1)}
        log(f"[bench] fp8 shared expert T={t}: {out[f'T{t}']}")
        del x, lg
    del layer, res, shared
    torch.cuda.synchronize()
    return out


def bench_w8a16(pkg, dev, fmt="int8"):
    """W8A16 dense linear, K = 4096, N in {4096, 1024, 16384}, M in {1, 64, 8192};
    fmt "int8" (per-channel bf16 scales, ``w8a16_int8_gemm_into``) or "fp8"
    (E4M3 with E8M0 128x128 block scales, the reference checkpoint's format:
    ``w8a16_gemm_into``), each on the weight as stored (row-major [N, K]) and
    on the load-time tiles (``w8a16_prepared_gemm_into``, reported as
    ``us_tiled``)."""

    import torch

    L = pkg.weight_only_linear
    S = pkg.synthetic
    out = {}
    k = 4096
    for n in (4096, 1024, 16384):
        if fmt == "fp8":
            q, s = S.make_fp8_block_linear(n, k, device=dev)
            prep = L.prepare_fp8_block_weight(q, s)
            w, ws_ = q.view(torch.float8_e4m3fn), s.view(torch.float8_e8m0fnu)
            gemm = L.w8a16_gemm_into
            scale_bytes = s.numel()
        else:
            q, s = S.make_int8_linear(n, k, device=dev)
            prep = L.prepare_int8_weight(q, s)
            w, ws_ = q, s
            gemm = L.w8a16_int8_gemm_into
            scale_bytes = 2 * n
        for m in (1, 64, 8192):
            a = S.make_hidden(m, k, seed=6000 + m, device=dev)
            plan = L.make_gemm_plan(m, n, k)
            o = torch.empty(plan.output_shape, dtype=torch.bfloat16, device=dev)
            wsp = L.allocate_workspace(plan, dev)
            calls = {"rowmajor": lambda i: gemm(a, w, ws_, o, wsp, plan=plan),
                     "tiled": lambda i: L.w8a16_prepared_gemm_into(a, prep, o, wsp, plan=plan)}
            times, eager = {}, {}
            for layout, fn in calls.items():
                for _ in range(3):
                    fn(0)
                it = 50 if m < 8192 else 10
                ms = cuda_timer(fn, it)
                if m <= 64:  # launch-bound from Python: time the kernels in a graph
                    g_ms = graph_timer(fn, 50, o)
                    eager[layout], ms = ms, (g_ms if g_ms is not None else ms)
                times[layout] = ms
            ms = times["rowmajor"]
            byts = n * k + scale_bytes + 2 * m * k + 2 * m * n
            fl = 2.0 * m * n * k
            entry = {"split_k": plan.split_k, "us": round(ms * 1e3, 2), "us_tiled": round(times["tiled"] * 1e3, 2),
                     "hbm_gbs": round(byts / (ms * 1e-3) / 1e9, 1), "tflops": round(fl / (ms * 1e-3) / 1e12, 2)}
            if m <= 64:
                entry["us_eager_python_loop"] = round(eager["rowmajor"] * 1e3, 2)
                entry["timing"] = "hip graph of 50 calls"
            entry["frac_of_peak"] = (round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if m <= 64
                                     else round(fl / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4))
            entry["bound"] = "hbm" if m <= 64 else "mfma"
            out[f"M{m}_N{n}"] = entry
            log(f"[bench] w8a16 {fmt} M={m} N={n}: {entry}")
            del a, o, wsp
        del prep, q, w
    return out


def bench_block_fp8(pkg, dev):
    """Block-FP8 W8A8 dense linear (fp8_linear.py): K = 4096, N in {4096, 1024,
    16384}, M in {1, 64, 8192}; the bf16 -> E4M3 activation quantiser and the
    GEMM timed separately (the reference launches them separately); the GEMM
    on the checkpoint weight as stored and on the load-time tiles
    (``us_tiled``)."""

    import torch

    F = pkg.fp8_linear
    L = pkg.weight_only_linear
    S = pkg.synthetic
    out = {}
    k = 4096
    for n in (4096, 1024, 16384):
        q, s = S.make_fp8_block_linear(n, k, device=dev)
        prep = L.prepare_fp8_block_weight(q, s)
        w, w_s = q.view(torch.float8_e4m3fn), s.view(torch.float8_e8m0fnu)
        for m in (1, 64, 8192):
            x = S.make_hidden(m, k, seed=7000 + m, device=dev)
            qp = F.make_quantization_plan(m, k)
            aq = torch.empty(qp.quantized_shape, dtype=F.FP8_DTYPE, device=dev)
            a_s = torch.empty(qp.scale_shape, dtype=F.E8M0_DTYPE, device=dev)
            plan = F.make_gemm_plan(m, n, k)
            o = torch.empty(plan.output_shape, dtype=torch.bfloat16, device=dev)
            ws = torch.empty(plan.workspace_shape, dtype=torch.float32, device=dev)
            it = 50 if m < 8192 else 10
            quant = lambda i: F.activation_quant_into(x, aq, a_s, plan=qp)
            gemms = {"rowmajor": lambda i: F.block_fp8_gemm_into(aq, a_s, w, w_s, o, ws, plan=plan),
                     "tiled": lambda i: F.block_fp8_gemm_into(aq, a_s, prep, None, o, ws, plan=plan)}
            quant(0)
            q_ms = cuda_timer(quant, it)
            if m <= 64:
                q_eager = q_ms
                g_q = graph_timer(quant, 50, aq.view(torch.uint8))
                q_ms = g_q if g_q is not None else q_ms
            times, eager = {}, {}
            for layout, fn in gemms.items():
                for _ in range(3):
                    fn(0)
                ms = cuda_timer(fn, it)
                if m <= 64:  # launch-bound from Python: time the kernels in a graph
                    g_ms = graph_timer(fn, 50, o)
                    eager[layout], ms = ms, (g_ms if g_ms is not None else ms)
                times[layout] = ms
            ms = times["rowmajor"]
            byts = n * k + prep.scale.numel() + m * k + m * (k // 128) + 2 * m * n
            fl = 2.0 * m * n * k
            entry = {"split_k": plan.split_k, "us": round(ms * 1e3, 2), "us_tiled": round(times["tiled"] * 1e3, 2),
                     "quant_us": round(q_ms * 1e3, 2),
                     "hbm_gbs": round(byts / (ms * 1e-3) / 1e9, 1), "tflops": round(fl / (ms * 1e-3) / 1e12, 2)}
            if m <= 64:
                entry["us_eager_python_loop"] = round(eager["rowmajor"] * 1e3, 2)
                entry["quant_us_eager_python_loop"] = round(q_eager * 1e3, 2)
                entry["timing"] = "hip graph of 50 calls"
            entry["frac_of_peak"] = (round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if m <= 64
                                     else round(fl / (ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4))
            entry["bound"] = "hbm" if m <= 64 else "mfma (fp8)"
            out[f"M{m}_N{n}"] = entry
            log(f"[bench] w8a8 block fp8 M={m} N={n}: {entry}")
            del x, aq, a_s, o, ws
        del prep, q, w
    return out


def cpu_baseline(pkg, w13, s13, w2, s2, seed):
    """The reference's torch path, restated in ``oracle/torch_path.py`` (the
    gate of ``moe_forward.py:80-87``, ``DenseRoutedExecutor``
    ``ops/dense_moe.py:289-354`` in bf16 with its chunk-of-8 dequantisation,
    ``shared_bf16_partial`` and the add), timed on this host's cores
    (``torch.set_num_threads(os.cpu_count())``): one batch each of C1 (the
    tiny layer, T=64), C2 at T in {1, 8, 64, 256} and C3 at T=2048, on the
    same weights as the GPU run (copied to the host before timing).
    ``value`` is C2 at T=64, the headline configuration."""

    import torch

    try:
        from oracle import torch_path as TP
    except Exception as exc:  # pragma: no cover
        log(f"[bench] cpu baseline unavailable: {exc}")
        return None
    S = pkg.synthetic
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    flash = TP.StackedExperts(w13.cpu(), s13.cpu(), w2.cpu(), s2.cpu())
    tiny = TP.StackedExperts(*S.make_checkpoint_experts(S.TINY, seed=seed, device="cpu"))
    cases = [("C1_T64", tiny, S.TINY, 64)] + [(f"C2_T{t}", flash, S.FLASH, t) for t in (1, 8, 64, 256)] + [
        ("C3_T2048", flash, S.FLASH, 2048)]
    # the host's own achievable bf16 GEMM rate (torch.matmul on the CPU, the
    # operation the restated path spends its time in): the CPU roofline the
    # per-config FLOP rates are compared with
    a = torch.randn(1024, 4096).to(torch.bfloat16)
    b = torch.randn(4096, 4096).to(torch.bfloat16)
    torch.matmul(a, b)
    t0 = time.perf_counter()
    for _ in range(3):
        torch.matmul(a, b)
    cpu_gemm_gflops = 3 * 2.0 * 1024 * 4096 * 4096 / (time.perf_counter() - t0) / 1e9
    rounds = 3
    per = {}
    total = 0.0
    for name, experts, shape, t in cases:
        x = S.make_hidden(t, shape.hidden, seed=9000 + t, device="cpu")
        logits = S.make_logits(t, shape.experts, seed=9500 + t, device="cpu")
        times = []
        for _ in range(rounds):
            t0 = time.perf_counter()
            ids, weights, _ = TP.gate_route(logits, topk=shape.topk, score_func="sigmoid")
            TP.dense_moe(x, ids, weights, experts, num_experts=shape.experts,
                         shared_index=shape.experts if shape.has_shared else None, dtype=torch.bfloat16)
            times.append(time.perf_counter() - t0)
        total += sum(times)
        med = sorted(times)[len(times) // 2]
        flops = 6.0 * t * (shape.topk + (1 if shape.has_shared else 0)) * shape.hidden * shape.inter
        per[name] = {"tokens": t, "seconds_median": round(med, 4), "seconds_min": round(min(times), 4),
                     "seconds_max": round(max(times), 4), "tokens_per_s": round(t / med, 2),
                     "gflops": round(flops / med / 1e9, 1),
                     "frac_of_cpu_gemm_rate": round(flops / med / 1e9 / cpu_gemm_gflops, 4)}
        log(f"[bench] cpu baseline {name}: {per[name]}")
    return {
        "value": per["C2_T64"]["tokens_per_s"],
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"median of {rounds} rounds per config (C1 T=64 tiny layer; C2 T=1/8/64/256 and C3 T=2048 on "
                   "the Flash layer) through the torch restatement of the reference's dense path in bf16, router "
                   f"included; {total:.1f} s of CPU time on {cores} threads; value = C2 T=64"),
        "cpu_bf16_gemm_gflops": round(cpu_gemm_gflops, 1),
        "configs": per,
    }


def profile_run_linear(pkg, fmt: str, m: int, n: int, dev) -> int:
    """The dense-linear programs of ``--profile-run``: N calls each at M=m,
    K=4096, N in {1024, 4096, 16384}, on the load-time tiled weights (W8A8:
    the block-FP8 GEMM after one activation quantisation; W8A16: int8
    weights)."""

    import torch

    F, L, S = pkg.fp8_linear, pkg.weight_only_linear, pkg.synthetic
    k = 4096
    for cols in (1024, 4096, 16384):
        if fmt == "linear-w8a8":
            q, s = S.make_fp8_block_linear(cols, k, device=dev)
            prep = L.prepare_fp8_block_weight(q, s)
            x = S.make_hidden(m, k, seed=7000 + m, device=dev)
            qp = F.make_quantization_plan(m, k)
            aq = torch.empty(qp.quantized_shape, dtype=F.FP8_DTYPE, device=dev)
            a_s = torch.empty(qp.scale_shape, dtype=F.E8M0_DTYPE, device=dev)
            F.activation_quant_into(x, aq, a_s, plan=qp)
            plan = F.make_gemm_plan(m, cols, k)
            o = torch.empty(plan.output_shape, dtype=torch.bfloat16, device=dev)
            ws = torch.empty(plan.workspace_shape, dtype=torch.float32, device=dev)
            for _ in range(n):
                F.block_fp8_gemm_into(aq, a_s, prep, None, o, ws, plan=plan)
        else:
            q, s = S.make_int8_linear(cols, k, device=dev)
            prep = L.prepare_int8_weight(q, s)
            a = S.make_hidden(m, k, seed=6000 + m, device=dev)
            plan = L.make_gemm_plan(m, cols, k)
            o = torch.empty(plan.output_shape, dtype=torch.bfloat16, device=dev)
            ws = L.allocate_workspace(plan, dev)
            for _ in range(n):
                L.w8a16_prepared_gemm_into(a, prep, o, ws, plan=plan)
        torch.cuda.synchronize()
    print(json.dumps({"profile_run": f"{fmt}:{m}:{n}", "calls_per_shape": n, "shapes": ["N=1024", "N=4096", "N=16384"]}),
          flush=True)
    return 0


def profile_run(pkg, spec: str, seed: int) -> int:
    """``--profile-run FMT:T:N[:graph|:hidden]``: build the Flash layer in
    format FMT (int4, mxfp4, w4a8 or w4a8-mxfp4), run one warm-up and N
    ``TP4MoE.forward_tensor`` calls at T tokens, and exit -- the program the
    rocprofv3 counter passes and kernel traces wrap.  With ``:graph`` the call
    is then captured once as a HIP graph and replayed N times (eager and
    replayed kernels in one trace); with ``:hidden`` every call routes from
    the hidden states (the gate GEMM included) instead of given logits."""

    import torch

    parts = spec.split(":")
    if len(parts) not in (3, 4) or (len(parts) == 4 and parts[3] not in ("graph", "hidden")):
        raise SystemExit(f"--profile-run: expected FMT:T:N, FMT:T:N:graph or FMT:T:N:hidden, got {spec!r}")
    fmt, t, n = parts[:3]
    t, n = int(t), int(n)
    graph_mode = len(parts) == 4 and parts[3] == "graph"
    from_hidden = len(parts) == 4 and parts[3] == "hidden"
    S = pkg.synthetic
    dev = torch.device("cuda:0")
    if fmt in ("linear-w8a8", "linear-w8a16"):
        if graph_mode:
            raise SystemExit("--profile-run: the dense linears run eager only")
        return profile_run_linear(pkg, fmt, t, n, dev)
    shape = S.FLASH
    E, H, I, K = shape.experts, shape.hidden, shape.inter, shape.topk
    fp8_act = fmt in ("w4a8", "w4a8-mxfp4")
    if fmt in ("mxfp4", "w4a8-mxfp4"):
        res = pkg.ResidentMXFP4MoEWeights.from_checkpoint_layout(
            *S.make_checkpoint_experts_mxfp4(shape, seed=seed, device=dev), experts=E, has_shared=True,
            marlin_input_dtype=torch.float8_e4m3fn if fp8_act else None)
    elif fmt in ("int4", "w4a8"):
        res = pkg.ResidentInt4MoEWeights.from_checkpoint_layout(
            *S.make_checkpoint_experts(shape, seed=seed, device=dev), experts=E, has_shared=True,
            marlin_input_dtype=torch.float8_e4m3fn if fmt == "w4a8" else None)
    else:
        raise SystemExit(f"--profile-run: unknown format {fmt!r} (int4, mxfp4, w4a8, w4a8-mxfp4)")
    cfg = pkg.TP4MoEConfig(hidden_size=H, intermediate_size=I, experts=E, topk=K, route_scale=1.0, clamp_limit=0.0,
                           score_func="sigmoid", shared_experts=1)
    gate_w = (torch.randn((E, H), device=dev, generator=torch.Generator(dev).manual_seed(seed + 7)) * 0.02)
    gate = pkg.ResidentGateWeights(weight=gate_w.to(torch.bfloat16))
    layer = pkg.TP4MoE(config=cfg, resident=res, gate=gate, device=dev, global_row_shapes=[t],
                       marlin_input_dtype=torch.float8_e4m3fn if fp8_act else None)
    x = S.make_hidden(t, H, seed=3000, device=dev).view(1, t, H)
    # ":hidden" routes from the hidden states (the gate GEMM runs in every call)
    logits = None if from_hidden else S.make_logits(t, E, seed=3001, device=dev)
    layer.forward_tensor(x, router_logits=logits)
    torch.cuda.synchronize()
    for _ in range(n):
        layer.forward_tensor(x, router_logits=logits)
    torch.cuda.synchronize()
    replays = 0
    if graph_mode:
        # then the same call captured once and replayed N times
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            layer.forward_tensor(x, router_logits=logits)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        layer.reset_free_slot_completion_event(t, 0)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            layer.forward_tensor(x, router_logits=logits)
        torch.cuda.synchronize()
        for _ in range(n):
            graph.replay()
        torch.cuda.synchronize()
        replays = n
        del graph
        torch.cuda.synchronize()
    print(json.dumps({"profile_run": spec, "calls": n + 2 if graph_mode else n + 1, "replays": replays}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
