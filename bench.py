"""Benchmark: trellis packed-linear decode-GEMV on MI355X, Qwen3-8B block at batch 1.

Workload: the seven linears of one Qwen3-8B decoder block,
q 4096->4096, k/v 4096->1024, o 4096->4096, gate/up 4096->12288, down 12288->4096, K=3,
MCG, packed bits uniform random from a seed, seeded +-1 signs, per-matrix scale, fp16
N(0,1) activations. One step = the seven packed linears of one block in forward order as four launches
(q/k/v grouped, o, gate/up grouped, down). Weights are
resident in HBM; to defeat the 256 MB Infinity Cache the steps rotate over `copies`
distinct blocks (>= 1 GB of packed bits by default).

value = packed-weight bytes of the block / seconds per step (GB/s, algorithmic bytes
n*k*K/8). The JSON line also carries us/layer, the dominant kernel's roofline from HIP
events on the launch stream, and a CPU baseline: this repo's torch-CPU restatement of
the reference decode+restore+matmul (oracle/torch_cpu.py) timed on a bounded sample.
"""
from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

LAYERS = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
          ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
# launches of one block in forward order: linears that share an input run as one group
# (trellis_packed_linear_group); o waits for attention and down for the MLP activation
GROUPS = [("qkv", ("q", "k", "v")), ("o", ("o",)), ("gate_up", ("gate", "up")),
          ("down", ("down",))]
DOMINANT = "gate_up"   # 2 x 18,874,368 packed bytes per launch
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "tmk_gate_up_b1_traffic.txt")


def traffic_from_profile(path=TRAFFIC_FILE):
    """HBM bytes per gate+up launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary, each counter scaled by what it reads for a device copy of known size.
    None when the summary is absent (counters cannot be read from inside this process)."""
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        parts = line.split()
        if len(parts) == 2 and not line.startswith("#"):
            vals[parts[0]] = float(parts[1])
    try:
        fetch = vals["fetch_kib"] * vals["copy_kib"] / vals["copy_fetch_kib"]
        write = vals["write_kib"] * vals["copy_kib"] / vals["copy_write_kib"]
    except KeyError:
        return None
    return int(round((fetch + write) * 1024))


def make_block(te, torch, dev, K, seed, codebook="mcg"):
    import numpy as np
    from_dev = te.PackedLinear.from_device
    g = torch.Generator(device=dev)
    block = {}
    for i, (name, n, k) in enumerate(LAYERS):
        g.manual_seed(seed * 100 + i)
        nt = (n // 16) * (k // 16)
        nw = 256 * K // 32
        bits = torch.randint(-2 ** 31, 2 ** 31 - 1, (nt, nw), generator=g, device=dev,
                             dtype=torch.int32)
        rng = np.random.default_rng(seed * 100 + i)
        su = torch.from_numpy((rng.integers(0, 2, k) * 2 - 1).astype(np.float32)).to(dev)
        sv = torch.from_numpy((rng.integers(0, 2, n) * 2 - 1).astype(np.float32)).to(dev)
        scale = float(np.float32(np.float16(0.02 / 1.2441)))
        isc = rng.uniform(0.5, 1.5, k)
        osc = rng.uniform(0.5, 1.5, n)
        isc = torch.from_numpy((isc / isc.mean()).astype(np.float16).astype(np.float32) *
                               np.float32(scale)).to(dev)
        osc = torch.from_numpy((osc / osc.mean()).astype(np.float16).astype(np.float32)).to(dev)
        block[name] = from_dev(n, k, K, bits, su, sv, isc, osc, scale=scale, codebook=codebook,
                               name=name)
    return block


def cpu_baseline(budget_s: float = 20.0):
    """torch-CPU decode+restore+matmul (oracle/torch_cpu.py) of the 8B q_proj, K=3 MCG,
    on all host cores; median over repeated runs within ~budget_s."""
    import numpy as np
    import torch
    from oracle import torch_cpu as tc
    from oracle import trellis_np as tn

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    n, k = 4096, 4096
    bits, rec = tn.synthetic_record(n, k, 3, seed=7)
    lut = tc.codebook_lut_torch("mcg")
    x = torch.from_numpy(np.random.default_rng(0).standard_normal(k).astype(np.float16)).float()
    tc.decode_matmul(bits, rec, x, lut)       # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        tc.decode_matmul(bits, rec, x, lut)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times) >= 3:
            break
    W = tc.w_hat(bits, rec, lut)
    mm = []
    for _ in range(5):
        t0 = time.perf_counter()
        _ = W @ x
        mm.append(time.perf_counter() - t0)
    med = statistics.median(times)
    packed = n * k * 3 // 8
    return {"value": round(packed / med / 1e9, 4), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"Qwen3-8B q_proj 4096x4096 K=3 MCG, torch-CPU decode+restore+matmul "
                      f"(oracle/torch_cpu.py), median of {len(times)} runs = {med * 1e3:.1f} ms; "
                      f"matmul alone on cached W_hat {statistics.median(mm) * 1e3:.2f} ms",
            "ms_per_layer": round(med * 1e3, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--K", type=int, default=3)
    ap.add_argument("--copies", type=int, default=0, help="distinct weight blocks (0: >= 1 GB)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the packed linear is "
                                   "measured on one MI355X; multi-GPU sharding is design-only"}))
        sys.exit(2)

    import torch
    te = importlib.import_module("trellis-everywhere_amd")
    te.library()
    dev = torch.device("cuda:0")
    block_bytes = sum(n * k * args.K // 8 for _, n, k in LAYERS)
    copies = args.copies or max(1, math.ceil(1.0e9 / block_bytes))
    blocks = [make_block(te, torch, dev, args.K, seed=c) for c in range(copies)]
    B = args.batch
    xs = {name: torch.randn((B, k), device=dev, dtype=torch.float16) for name, _, k in LAYERS}
    # group members that share an input read the same tensor
    xs["k"] = xs["v"] = xs["q"]
    xs["up"] = xs["gate"]
    ys = {name: torch.empty((B, n), device=dev, dtype=torch.float32) for name, n, _ in LAYERS}
    groups = [[(gname, te.PackedGroup([blk[m] for m in members]), members)
               for gname, members in GROUPS] for blk in blocks]
    for blk, grps in zip(blocks, groups):
        for lin in blk.values():
            lin._workspace(B)
        for _, grp, _ in grps:
            grp._workspace(B)

    def step(s, only=None):
        for gname, grp, members in groups[s % copies]:
            if only is None or gname == only:
                grp.forward([xs[m] for m in members], [ys[m] for m in members])

    def single(s, name):
        blocks[s % copies][name].forward(xs[name], out=ys[name])

    # warm up eagerly (allocates nothing later), then capture one HIP graph per weight
    # copy: the four launches of a block replay without per-call host overhead
    for s in range(max(args.warmup, copies)):
        step(s)
        for name, _, _ in LAYERS:
            single(s, name)
    torch.cuda.synchronize()

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(g):
            fn()
        return g

    graphs = [capture(lambda c=c: step(c)) for c in range(copies)]
    for s in range(args.warmup):
        graphs[s % copies].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        graphs[s % copies].replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    sec_per_step = (t1 - t0) / args.steps

    # launch durations from HIP events on the launch stream: one graph holding a
    # launch for every weight copy (distinct weights back to back), events around its
    # replays; average = elapsed / launches
    reps = max(1, args.steps // copies)

    def per_launch_us(fn_for_copy):
        g = capture(lambda: [fn_for_copy(c) for c in range(copies)])
        g.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * copies)

    us_layer = {name: round(per_launch_us(lambda c, name=name: single(c, name)), 3)
                for name, _, _ in LAYERS}
    us_group = {gname: round(per_launch_us(lambda c, gname=gname: step(c, gname)), 3)
                for gname, _ in GROUPS}
    dom_us = us_group[DOMINANT]
    dom_bytes = 2 * 12288 * 4096 * args.K // 8
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    gbs = block_bytes / sec_per_step / 1e9

    # known-size copy for the HBM-counter scale factor (FETCH_SIZE / WRITE_SIZE)
    src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()

    out = {
        "metric": "3-bit decode-GEMV HBM GB/s (% of peak) + us/layer, Qwen3-8B shapes, batch 1/64",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec_per_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32 packed K=3 trellis, fp16 activations, fp32 accumulate",
        "data": "synthetic: uniform random packed bits, seeded signs/scales, fp16 N(0,1) x",
        "config": {"workload": "Qwen3-8B decoder-block linears (q,k,v,o,gate,up,down), K=3, "
                               "MCG, batch %d" % B,
                   "batch": B, "K": args.K, "codebook": "mcg",
                   "block_packed_bytes": block_bytes, "weight_copies": copies,
                   "rotated_bytes": block_bytes * copies,
                   "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                   "us_per_block": round(sec_per_step * 1e6, 2),
                   "launches_per_block": [g for g, _ in GROUPS],
                   "us_per_group_launch": us_group,
                   "us_per_layer_single_launch": us_layer},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile() if args.batch == 1 and args.K == 3
                     else None,
                     "traffic_source": "profiles/tmk_gate_up_b1_traffic.txt (rocprofv3 "
                                       "FETCH_SIZE/WRITE_SIZE, copy-scaled)",
                     "kernel": "tmk_kernel<K=3,MCG,KS,XB=1> on the gate+up group "
                               "(2 x 12288x4096, one launch)",
                     "avg_launch_us": round(dom_us, 3),
                     "algorithmic_bytes_per_launch": dom_bytes},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_budget)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
