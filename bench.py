"""Benchmark: trellis packed-linear decode-matmul on MI355X, Qwen3-8B block linears.

Headline: the seven linears of one Qwen3-8B decoder block,
q 4096->4096, k/v 4096->1024, o 4096->4096, gate/up 4096->12288, down 12288->4096, K=3,
MCG, V=1, packed bits uniform random from a seed, seeded +-1 signs, per-matrix scale,
fp16 N(0,1) activations, batch 1. One step = the seven packed linears of one block in
forward order as four launches (q/k/v grouped, o, gate/up grouped, down: o waits for
attention and down for the MLP activation in a real forward pass). Weights are resident in
HBM; to defeat the 256 MB Infinity Cache the steps rotate over `copies` distinct blocks
(>= 1 GB of packed bits). One HIP graph holds a run of blocks, one per copy (a model's
forward pass is captured whole, so a graph launch is not charged to every block); the
timed region replays whole runs and then a graph of the remaining blocks, exactly `steps`
blocks. The same blocks with one graph per block (a graph launch each) are reported
beside it ("us_per_block_one_graph_per_block"). Every timed region follows at least W
untimed blocks and at least WARM_S = 50 ms of untimed replays: the GPU's clocks ramp up over
the first ~20-30 ms of load after idle.

value = packed-weight bytes of the block / seconds per step (GB/s, algorithmic bytes
n*k*K/8). The JSON line also carries us/layer, the dominant launch's HBM roofline (gate+up,
duration from HIP events on the launch stream), the same block at batch 16 and 64 and at a
512-token prefill with their fp16 MFMA rooflines (algorithmic 2*B*n*k flops), and a CPU baseline: this repo's torch-CPU
restatement of the reference decode+restore+matmul (oracle/torch_cpu.py) on a bounded
sample, per configuration and layer. The bit-rate sweep (configs[4]: K=2,3,4 x V=1,2 on
the 8B gate/up/down shapes, at batch 1 and at a 512-token prefill) runs by default
(--no-sweep skips it), each point with its own roofline.

The CPU-baseline leg also checks what the timed launches computed: after each timed run,
a graph of copy 0's block is replayed and sampled 128-row output blocks are copied to the
host (three per layer, one per layer at a sweep point); the oracle's float64 W_hat @ x
judges them at the reference's 1e-3 metric ("output_check"). A failed check prints the
JSON line and exits with status 3. --no-cpu-baseline skips both.
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
GROUPS = [("qkv", ("q", "k", "v")), ("o", ("o",)), ("gate_up", ("gate", "up")),
          ("down", ("down",))]
DOMINANT = "gate_up"   # 2 x 18,874,368 packed bytes per launch at K=3
MLP = [("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_gate_up_b1_traffic.txt")
# Untimed replays before every timed region last at least this long: the GPU's clocks ramp
# up over the first ~20-30 ms of load after idle (8B block at batch 1: 53.6 us in the first
# run of 14 blocks, 51.3 in the twelfth, 47.7 at steady state; batch 64: 119.6 -> 106.7; the
# ramp recurs after 0.5 s idle), and a timed region inside it reads the ramp, not the kernels.
WARM_S = 0.05


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def traffic_from_profile(path=TRAFFIC_FILE):
    """HBM bytes per gate+up launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary: the launch's FETCH_SIZE scaled by what that counter reads for the read-only
    calibration pass of known size (calibration_passes), its WRITE_SIZE by what that counter
    reads for the write-only pass. None when the summary is absent (counters cannot be read
    from inside this process)."""
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        parts = line.split()
        if len(parts) == 2 and not line.startswith("#"):
            vals[parts[0]] = float(parts[1])
    try:
        fetch = vals["fetch_kib"] * vals["cal_kib"] / vals["cal_read_fetch_kib"]
        write = vals["write_kib"] * vals["cal_kib"] / vals["cal_fill_write_kib"]
    except (KeyError, ZeroDivisionError):
        return None
    return int(round((fetch + write) * 1024))


def make_layers(te, torch, dev, layers, K, V, seed, codebook="mcg"):
    """Seeded synthetic packed linears on the device (uniform random bits, seeded signs/scales)."""
    import numpy as np
    from_dev = te.PackedLinear.from_device
    g = torch.Generator(device=dev)
    out = {}
    for i, (name, n, k) in enumerate(layers):
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
        out[name] = from_dev(n, k, K, bits, su, sv, isc, osc, scale=scale, codebook=codebook,
                             V=V, name=name)
    return out


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        fn()
    return g


def take_samples(blk, xs, ys, layers, label, per_layer):
    """Host copies for the output check of one timed run: per layer, the packed words of
    `per_layer` 128-row output blocks (first, middle, last) of one weight copy with its
    metadata, the input rows and the outputs that copy's timed launches wrote. A 128-row
    block of y depends only on its own 8 bands (the out-dim Hadamard block is 128)."""
    out = []
    for name, n, k in layers:
        lin = blk[name]
        tin, nb = k // 16, n // 128
        obs = sorted({0, nb // 2, nb - 1}) if per_layer >= 3 else [nb - 1]
        B = xs[name].shape[0]
        # every batch row up to 64; above, 32 rows spread over the batch (first and last)
        rows = list(range(B)) if B <= 64 else sorted({round(i * (B - 1) / 31) for i in range(32)})
        y = ys[name][rows]
        out.append({
            "run": label, "layer": name, "n": n, "k": k, "K": lin.K, "V": lin.V,
            "codebook": lin.codebook, "scale": lin.scale,
            "su": lin.su.cpu().numpy(), "sv": lin.sv.cpu().numpy(),
            "isc_scaled": lin.isc_scaled.cpu().numpy(), "osc": lin.osc.cpu().numpy(),
            "x": xs[name][rows].float().cpu().numpy(),
            "blocks": [(ob, lin.bits[ob * 8 * tin:(ob + 1) * 8 * tin].cpu().numpy().view("uint32"),
                        y[:, ob * 128:(ob + 1) * 128].cpu().numpy()) for ob in obs]})
    return out


def warm_up(torch, replay, at_least):
    """Untimed replays (replay(i) for i = 0, 1, ..) before a timed region: at least
    `at_least` of them and at least WARM_S seconds of them (synchronized every few, so the
    host clock follows the GPU's). Returns how many ran."""
    t0 = time.perf_counter()
    n = 0
    while n < at_least or time.perf_counter() - t0 < WARM_S:
        replay(n)
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def time_blocks(torch, step, copies, steps, warmup):
    """Seconds per block of `steps` blocks, block c of a run on weight copy c: one graph holds
    a run of `copies` blocks (a model's forward pass is captured whole, so a graph launch is
    not charged to every block), and the timed region replays whole runs and then a graph of
    the first `steps % copies` copies, exactly `steps` blocks between two synchronizations,
    after whole runs covering at least `warmup` blocks and WARM_S seconds (warm_up)."""
    run = capture(torch, lambda: [step(c) for c in range(copies)])
    tail_n = steps % copies
    tail = capture(torch, lambda: [step(c) for c in range(tail_n)]) if tail_n else None
    warm_up(torch, lambda i: run.replay(), max(1, math.ceil(warmup / copies)))
    t0 = time.perf_counter()
    for _ in range(steps // copies):
        run.replay()
    if tail is not None:
        tail.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def run_block(te, torch, dev, layers, groups, B, K, V, steps, warmup, min_bytes=1.0e9,
              per_launch=True, mma_f16=False, copies=None, singles=True, samples=None,
              label="", sample_blocks=3, graph_each=None):
    """Time `steps` blocks (each block's launches in order) over distinct weight copies
    (time_blocks: one graph per run of blocks, one block per copy). Returns (seconds per
    step, {group: us per launch}, {layer: us per launch}, copies); singles=False never launches the layers one by one (a counter run then sees
    only the group launches). With a `graph_each` dict, `steps` more blocks are timed with
    one graph per block (one graph launch per block) and their seconds per block stored
    under "sec". With a `samples` list, a graph of copy 0's block is replayed after the
    timed steps and what its launches wrote is appended for the output check
    (take_samples)."""
    block_bytes = sum(n * k * K // 8 for _, n, k in layers)
    if copies is None:
        copies = max(2, math.ceil(min_bytes / block_bytes))
    blocks = [make_layers(te, torch, dev, layers, K, V, seed=c) for c in range(copies)]
    kin = {name: k for name, _, k in layers}
    xs = {name: torch.randn((B, kin[name]), device=dev, dtype=torch.float16) for name, _, _ in layers}
    for gname, members in groups:            # members of a group share one input
        for m in members[1:]:
            xs[m] = xs[members[0]]
    ys = {name: torch.empty((B, n), device=dev, dtype=torch.float32) for name, n, _ in layers}
    grps = [[(gname, te.PackedGroup([blk[m] for m in members]), members)
             for gname, members in groups] for blk in blocks]

    def step(c, only=None):
        for gname, grp, members in grps[c % copies]:
            if only is None or gname == only:
                grp.forward([xs[m] for m in members], [ys[m] for m in members], mma_f16=mma_f16)

    def single(c, name):
        blocks[c % copies][name].forward(xs[name], out=ys[name], mma_f16=mma_f16)

    for c in range(copies):            # allocates every workspace once, before capture
        step(c)
        if singles:
            for name, _, _ in layers:
                single(c, name)
    torch.cuda.synchronize()
    sec = time_blocks(torch, step, copies, steps, warmup)
    if graph_each is not None:
        graphs = [capture(torch, lambda c=c: step(c)) for c in range(copies)]
        warm_up(torch, lambda i: graphs[i % copies].replay(), warmup)
        t0 = time.perf_counter()
        for s in range(steps):
            graphs[s % copies].replay()
        torch.cuda.synchronize()
        graph_each["sec"] = (time.perf_counter() - t0) / steps
        del graphs
    if samples is not None:
        g0 = capture(torch, lambda: step(0))
        g0.replay()
        torch.cuda.synchronize()
        samples.extend(take_samples(blocks[0], xs, ys, layers, label, sample_blocks))
        del g0

    us_group, us_layer = {}, {}
    if per_launch:
        # at least ~200 launches per figure, whatever the step count
        reps = max(math.ceil(200 / copies), steps // copies)

        def per_launch_us(fn_for_copy):
            # one graph holding the launch for every copy (distinct weights back to back),
            # HIP events on the launch stream around its replays
            g = capture(torch, lambda: [fn_for_copy(c) for c in range(copies)])
            warm_up(torch, lambda i: g.replay(), 1)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / (reps * copies)

        us_group = {gname: round(per_launch_us(lambda c, gname=gname: step(c, gname)), 3)
                    for gname, _ in groups}
        if singles:
            us_layer = {name: round(per_launch_us(lambda c, name=name: single(c, name)), 3)
                        for name, _, _ in layers}
    del grps, blocks
    torch.cuda.empty_cache()
    return sec, us_group, us_layer, copies


# CPU-baseline layers: (config, layer, n_out, k_in, K, codebook). Configurations 1 to 3 of
# the benchmark per layer (the 8B block's v, o and up have the shapes of k, q and gate) and
# one point of the bit-rate sweep.
CPU_LAYERS = [
    ("configs[0] SmolLM2-135M", "up_proj", 1536, 576, 3, "3inst"),
    ("configs[1] Qwen3-1.7B MLP", "gate/up", 6144, 2048, 3, "mcg"),
    ("configs[1] Qwen3-1.7B MLP", "down", 2048, 6144, 3, "mcg"),
    ("configs[2] Qwen3-8B block", "q/o", 4096, 4096, 3, "mcg"),
    ("configs[2] Qwen3-8B block", "k/v", 1024, 4096, 3, "mcg"),
    ("configs[2] Qwen3-8B block", "gate/up", 12288, 4096, 3, "mcg"),
    ("configs[2] Qwen3-8B block", "down", 4096, 12288, 3, "mcg"),
    ("configs[4] sweep K=4", "gate/up", 12288, 4096, 4, "mcg"),
]
# how many times each 8B shape occurs in the block (q, k, v, o, gate, up, down)
BLOCK_MULT = {"q/o": 2, "k/v": 2, "gate/up": 2, "down": 1}


def cpu_baseline(budget_s: float = 30.0):
    """The reference's decode-then-matmul restated in torch CPU ops (oracle/torch_cpu.py:
    decode + restore + matmul, qtip.py:82-110, 262-268) on every host core, per
    configuration and layer: (a) the whole call and (b) the matmul alone against a cached
    W_hat, medians of repeated runs after a warm-up. The headline value is the 8B block's
    packed bytes over the sum of its seven layers' (a) times."""
    import numpy as np
    import torch
    from oracle import torch_cpu as tc
    from oracle import trellis_np as tn

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    log(f"[bench] cpu baseline on {cores} threads")
    log(torch.__config__.parallel_info())
    t_start = time.perf_counter()
    per_layer = []
    block_s = 0.0
    runs = 3
    for cfg, layer, n, k, K, cb in CPU_LAYERS:
        bits, rec = tn.synthetic_record(n, k, K, seed=n + k + K, codebook=cb)
        lut = tc.codebook_lut_torch(cb)
        x = torch.from_numpy(np.random.default_rng(0).standard_normal(k).astype(np.float16)).float()
        tc.decode_matmul(bits, rec, x, lut)          # warm-up
        full = []
        for _ in range(runs):
            t0 = time.perf_counter()
            tc.decode_matmul(bits, rec, x, lut)
            full.append(time.perf_counter() - t0)
        W = tc.w_hat(bits, rec, lut)
        mm = []
        for _ in range(5):
            t0 = time.perf_counter()
            _ = W @ x
            mm.append(time.perf_counter() - t0)
        a, b = statistics.median(full), statistics.median(mm)
        pb = n * k * K // 8
        per_layer.append({"config": cfg, "layer": layer, "shape": f"{n}x{k}", "K": K,
                          "codebook": cb, "decode_restore_matmul_ms": round(a * 1e3, 2),
                          "matmul_only_ms": round(b * 1e3, 3),
                          "packed_GBps": round(pb / a / 1e9, 4)})
        log(f"[bench] cpu {cfg} {layer} {n}x{k} K={K}: {a * 1e3:.1f} ms (matmul {b * 1e3:.2f} ms)")
        if cfg.startswith("configs[2]"):
            block_s += BLOCK_MULT[layer] * a
    total_s = time.perf_counter() - t_start
    block_bytes = sum(n * k * 3 // 8 for _, n, k in LAYERS)
    # the encoder row: the C restatement of the tail-biting Viterbi (oracle/viterbi.c,
    # OpenMP over tiles) on 4 tiles per core, K=3 MCG
    from oracle import viterbi as ov
    wt = np.random.default_rng(1).standard_normal((4 * cores, 256)).astype(np.float32)
    lut_np = tn.codebook_lut("mcg")
    ov.viterbi_tb(wt[:cores], 3, lut_np)      # warm-up
    t0 = time.perf_counter()
    ov.viterbi_tb(wt, 3, lut_np)
    enc_s = time.perf_counter() - t0
    return {"value": round(block_bytes / block_s / 1e9, 4), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"torch-CPU decode+restore+matmul (oracle/torch_cpu.py) at batch 1, median "
                      f"of {runs} runs per layer after a warm-up, {len(CPU_LAYERS)} layers in "
                      f"{total_s:.1f} s; value = Qwen3-8B block packed bytes / sum of its seven "
                      f"layers' times ({block_s * 1e3:.0f} ms)",
            "us_per_block": round(block_s * 1e6, 1),
            "per_layer": per_layer,
            "encode_tiles_per_s": round(wt.shape[0] / enc_s, 1),
            "encode_sample": f"oracle/viterbi.c tail-biting encode, K=3 MCG, {wt.shape[0]} tiles "
                             f"on {cores} threads: {enc_s:.2f} s"}


OUTPUT_TOL = 1e-3   # validate_packed_linear.py:66-69: max|y - y_ref| / max|y_ref|


def check_outputs(samples, tol=OUTPUT_TOL):
    """Part of the CPU-baseline leg: every sampled 128-row output block of every timed run
    (take_samples) against the oracle's float64 W_hat @ x (oracle/trellis_np.py
    packed_linear_ref: decode, then the restore of qtip.py:262-268), by the metric of
    validate_packed_linear.py:66-69. The bench's layers fold an fp16 scale into fp16 input
    scales (isc_scaled = f32(isc) * scale, packed.js:51-52); that product is exact in f32,
    so isc is recovered exactly and the oracle sees the stored record."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    from oracle import trellis_np as tn

    def one(job):
        s, ob, bits, y = job
        scale = np.float32(s["scale"])
        isc = (s["isc_scaled"] / scale).astype(np.float16)
        if not np.array_equal(isc.astype(np.float32) * scale, s["isc_scaled"]):
            raise ValueError(f"{s['run']} {s['layer']}: isc_scaled is not f32(fp16 isc) * scale")
        sl = slice(ob * 128, ob * 128 + 128)
        rec = tn.IPRecord(128, s["k"], s["K"], s["su"], s["sv"][sl], isc, s["osc"][sl], scale,
                          codebook=s["codebook"], V=s["V"])
        return tn.rel_err(y, tn.packed_linear_ref(bits, rec, s["x"]))

    jobs = [(s, ob, bits, y) for s in samples for ob, bits, y in s["blocks"]]
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=min(8, len(os.sched_getaffinity(0)))) as ex:
        errs = list(ex.map(one, jobs))
    worst = max(range(len(jobs)), key=lambda i: errs[i]) if jobs else None
    bad = [f"{s['run']} {s['layer']} rows {ob * 128}+128: {e:.3g}"
           for (s, ob, _, _), e in zip(jobs, errs) if not e < tol]
    res = {"ok": not bad, "tol": tol, "metric": "max|y - y_oracle| / max|y_oracle| per block",
           "runs": len({s["run"] for s in samples}), "blocks_checked": len(jobs),
           "max_rel_err": float(f"{max(errs):.3g}") if errs else None,
           "worst": (f"{jobs[worst][0]['run']} {jobs[worst][0]['layer']} rows "
                     f"{jobs[worst][1] * 128}+128") if jobs else None,
           "failures": bad[:10], "seconds": round(time.perf_counter() - t0, 1)}
    log(f"[bench] output check: {res}")
    return res


def extras(te, torch, dev, steps, K=4, samples=None):
    """Next-row measurements on a Qwen3-8B vocab matrix (151936 x 4096, K=4, as the 8B export
    quantizes the LM head): the batch-1 LM-head GEMV, and embedding-row lookups
    (trellis_embed_rows) of 1 and 512 random token ids; 4 weight copies (1.2 GB) rotated.
    With a `samples` list, the LM head's output of its last timed launch (the last weight
    copy) is sampled for the output check (take_samples)."""
    n, k = 151936, 4096
    copies = 4
    mats = [make_layers(te, torch, dev, [("lm_head", n, k)], K, 1, seed=100 + c)["lm_head"]
            for c in range(copies)]
    x = torch.randn(k, device=dev, dtype=torch.float16)
    y = torch.empty(n, device=dev, dtype=torch.float32)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    toks = {nt: torch.randint(0, n, (copies, nt), generator=g, device=dev, dtype=torch.int32)
            for nt in (1, 512)}
    outs = {nt: torch.empty((nt, k), device=dev, dtype=torch.float32) for nt in (1, 512)}

    def timed(fn):
        for c in range(copies):
            fn(c)
        torch.cuda.synchronize()
        gr = capture(torch, lambda: [fn(c) for c in range(copies)])
        warm_up(torch, lambda i: gr.replay(), 1)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        reps = max(2, steps // copies)
        e0.record()
        for _ in range(reps):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * copies)

    us_head = timed(lambda c: mats[c].forward(x, out=y))
    if samples is not None:
        # every replay writes y from copy 0 to copy `copies - 1`, in that order
        samples.extend(take_samples({"lm_head": mats[-1]}, {"lm_head": x[None]}, {"lm_head": y[None]},
                                    [("lm_head", n, k)], "lm_head batch 1", 3))
    # the encoder row: trellis_encode_tiles on 4096 tiles (16 per workgroup), K=3 MCG
    wt = torch.randn((4096, 256), device=dev)
    te.encode_tiles(wt[:256], 3, "mcg", want_dq=False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    te.encode_tiles(wt, 3, "mcg", want_dq=False)
    torch.cuda.synchronize()
    enc_s = time.perf_counter() - t0
    us_emb = {nt: timed(lambda c, nt=nt: mats[c].embed_rows(toks[nt][c], out=outs[nt]))
              for nt in (1, 512)}
    del mats
    torch.cuda.empty_cache()
    pb = n * k * K // 8
    return {"matrix": f"{n}x{k} K={K} MCG (Qwen3-8B vocab)",
            "lm_head_b1_us": round(us_head, 2),
            "lm_head_b1_GBps": round(pb / (us_head * 1e-6) / 1e9, 1),
            "embed_rows_1_us": round(us_emb[1], 2),
            "embed_rows_512_us": round(us_emb[512], 2),
            "embed_rows_512_tokens_per_s": round(512 / (us_emb[512] * 1e-6), 0),
            "encode_tiles_per_s_K3": round(4096 / enc_s, 1),
            "encode_8b_block_s_K3": round(753664 / (4096 / enc_s), 2)}


def block_flops(layers, B):
    return sum(2 * B * n * k for _, n, k in layers)


def batched_figure(te, torch, dev, bs, K, V, args, samples=None):
    """The block at batch `bs` through the batched MFMA path (x fold, decode-to-MFMA GEMM,
    split-K fold), exact and in the fp16-weight mode, with the gate+up launch's fp16 MFMA
    roofline (algorithmic 2*bs*n*k flops over the launch, launch gap included)."""
    log(f"[bench] block batch {bs}")
    steps, warmup = max(20, args.steps // 10), max(3, args.warmup // 5)
    ge, geh = {}, {}
    sec, grp, _, copies = run_block(te, torch, dev, LAYERS, GROUPS, bs, K, V, steps, warmup,
                                    per_launch=True, samples=samples, label=f"block batch {bs}",
                                    graph_each=ge)
    fl = block_flops(LAYERS, bs)
    dom_fl = 2 * bs * 2 * 12288 * 4096
    dom_tf = dom_fl / (grp[DOMINANT] * 1e-6) / 1e12
    # the planner's width for gate+up (above 64 columns: 128 here, by its cost model)
    nc = 1 if bs <= 16 else 2 if bs <= 32 else 4 if bs <= 64 else 8
    out = {"us_per_block": round(sec * 1e6, 2),
           "us_per_block_one_graph_per_block": round(ge["sec"] * 1e6, 2),
           "blocks_per_graph": copies,
           "tflops": round(fl / sec / 1e12, 2),
           "mfma_frac_of_fp16_peak": round(fl / sec / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
           "us_per_group_launch": grp,
           "roofline": {"bound": "mfma", "achieved": round(dom_tf, 2),
                        "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(dom_tf / MFMA_FP16_PEAK_TFLOPS, 4),
                        "kernel": f"bgemm_kernel<K={K},MCG,V={V},NC={nc}> (+xfold, bfold) "
                                  f"on gate+up at batch {bs}",
                        "avg_launch_us": grp[DOMINANT],
                        "algorithmic_flops_per_launch": dom_fl}}
    log(f"[bench] batch {bs}: {out['us_per_block']} us/block, {out['tflops']} TFLOP/s")
    # the same block with the fp16-weight MFMA mode (each codebook value rounded once
    # to fp16, one MAC per weight; max rel err ~2-3e-4 against the exact default)
    sech, grph, _, _ = run_block(te, torch, dev, LAYERS, GROUPS, bs, K, V, steps, warmup,
                                 per_launch=True, mma_f16=True, samples=samples,
                                 label=f"block batch {bs} fp16-weight mode", graph_each=geh)
    out["mma_f16"] = {"us_per_block": round(sech * 1e6, 2),
                      "us_per_block_one_graph_per_block": round(geh["sec"] * 1e6, 2),
                      "tflops": round(fl / sech / 1e12, 2),
                      "mfma_frac_of_fp16_peak": round(fl / sech / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
                      "us_per_group_launch": grph,
                      "gate_up_tflops": round(dom_fl / (grph[DOMINANT] * 1e-6) / 1e12, 2)}
    log(f"[bench] batch {bs} mma_f16: {out['mma_f16']['us_per_block']} us/block, "
        f"{out['mma_f16']['tflops']} TFLOP/s")
    return out


def sweep_point(te, torch, dev, K, V, B, args, samples=None):
    """One point of the bit-rate sweep: gate, up and down of the 8B block, one launch each,
    at K bits, V weights per step and batch B (1, or a 512-token prefill), over >= 1 GB of
    distinct weight copies. Roofline of the whole point: HBM on the packed bytes at batch 1,
    fp16 MFMA on the algorithmic flops at 512."""
    log(f"[bench] sweep K={K} V={V} batch={B}")
    steps = max(20, args.steps) if B == 1 else 10
    sec, sg, _, copies = run_block(te, torch, dev, MLP, [(n, (n,)) for n, _, _ in MLP], B, K, V,
                                   steps, 3, per_launch=True, samples=samples,
                                   label=f"sweep K={K} V={V} batch {B}", sample_blocks=1)
    pb = sum(n * k * K // 8 for _, n, k in MLP)
    fl = block_flops(MLP, B)
    gbs, tfl = pb / sec / 1e9, fl / sec / 1e12
    if B == 1:
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(tfl, 2), "peak": MFMA_FP16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tfl / MFMA_FP16_PEAK_TFLOPS, 4)}
    return {"K": K, "V": V, "batch": B, "steps": steps, "weight_copies": copies,
            "us_gate_up_down": round(sec * 1e6, 2), "us_per_layer": sg,
            "packed_GBps": round(gbs, 1), "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
            "tflops": round(tfl, 2), "roofline": roof}


CAL_BYTES = 1 << 30


def calibration_passes(torch, dev):
    """Passes of known size for scaling the rocprofv3 HBM counters (run under --pmc, they
    appear as their own dispatches): a read-only sum over 1 GiB (FETCH_SIZE of exactly 1 GiB
    of reads, 4x the 256 MB MALL) and a fill of 1 GiB (WRITE_SIZE of 1 GiB of writes)."""
    a = torch.ones(CAL_BYTES // 4, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    for _ in range(3):
        s = a.sum()
    for _ in range(3):
        a.fill_(2.0)
    torch.cuda.synchronize()
    del a, s
    torch.cuda.empty_cache()


def ceilings(K):
    """What this decode allows on one MI355X, beside the targets: the batch-1 VALU floor of
    the block (13.4 VALU operations per 16x16 tile per wave at 4 cycles each, every one of
    the 1024 SIMDs issuing VALU every cycle at 2.4 GHz) and the batch-64 MFMA ceilings of
    the exact mode (the (hi, lo) pair is two MACs per weight). The measured figures are
    from microbenchmarks of this decode and of plain MFMA loops on the same GPU."""
    tiles = sum(n * k // 256 for _, n, k in LAYERS)
    floor_s = 13.4 * 4 * tiles / 1024 / 2.4e9
    block_bytes = sum(n * k * K // 8 for _, n, k in LAYERS)
    return {
        "batch1_valu_floor_us": round(floor_s * 1e6, 2),
        "batch1_valu_floor_pct_of_hbm_peak": round(100 * block_bytes / floor_s / 1e9
                                                   / HBM_PEAK_GBS, 1),
        "batch1_target_us": round(block_bytes / (0.6 * HBM_PEAK_GBS * 1e9) * 1e6, 2),
        "batch64_exact_mode_max_pct_of_fp16_peak": 50,
        "batch64_compute_only_loop_pct_of_fp16_peak": 35,
        "mfma_only_sustained_clock_ghz": [1.76, 1.90],
        "basis": "13.4 VALU ops/tile at 4 cycles on 1024 SIMDs at 2.4 GHz; exact mode = 2 "
                 "MACs per weight; decode + 4 MFMAs per band-tile at 4 waves/SIMD without "
                 "memory traffic: 91 cycles/band-tile, 70 % matrix busy"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=1, help="headline batch (default 1)")
    ap.add_argument("--K", type=int, default=3)
    ap.add_argument("--V", type=int, default=1)
    ap.add_argument("--no-batch64", action="store_true",
                    help="skip the batch-16, batch-64 and 512-prefill MFMA figures")
    ap.add_argument("--weight-copies", type=int, default=None,
                    help="distinct weight copies the steps rotate over (default: >= 1 GB of "
                         "packed bits, beyond the 256 MB MALL; 1 keeps a block resident in it)")
    ap.add_argument("--mma-f16", action="store_true",
                    help="the fp16-weight MFMA mode (TRELLIS_MMA_F16) for the block run (calls "
                         "on the batched path)")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the K x V bit-rate sweep on the gate/up/down shapes")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the LM-head GEMV and embedding-row lookup figures")
    ap.add_argument("--no-single", action="store_true",
                    help="skip the one-layer-per-launch figures (for counter runs: the group "
                         "launches are then the only ones of their grid sizes)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the packed linear is "
                                   "measured on one MI355X; multi-GPU sharding is design-only"}))
        sys.exit(2)

    import torch
    te = importlib.import_module("trellis-everywhere_amd")
    te.library()
    dev = torch.device("cuda:0")
    B, K, V = args.batch, args.K, args.V
    block_bytes = sum(n * k * K // 8 for _, n, k in LAYERS)

    # host copies of sampled output blocks of every timed run, checked against the oracle
    # in the CPU-baseline leg (check_outputs)
    samples = None if args.no_cpu_baseline else []
    log(f"[bench] block batch {B} K={K} V={V}")
    ge = {}
    sec, us_group, us_layer, copies = run_block(te, torch, dev, LAYERS, GROUPS, B, K, V,
                                                args.steps, args.warmup, mma_f16=args.mma_f16,
                                                copies=args.weight_copies,
                                                singles=not args.no_single, samples=samples,
                                                label=f"block batch {B}", graph_each=ge)
    gbs = block_bytes / sec / 1e9
    dom_us = us_group[DOMINANT]
    dom_bytes = 2 * 12288 * 4096 * K // 8
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    log(f"[bench] {sec * 1e6:.2f} us/block, {gbs:.1f} GB/s; groups {us_group}")

    batched = {}
    if not args.no_batch64 and B == 1:
        for bs in (16, 64, 512):
            batched[bs] = batched_figure(te, torch, dev, bs, K, V, args, samples)
    batch64 = batched.get(64)

    sweep = None
    if not args.no_sweep and B == 1:
        sweep = [sweep_point(te, torch, dev, Ks, Vs, Bs, args, samples)
                 for Ks in (2, 3, 4) for Vs in (1, 2) for Bs in (1, 512)]

    extra = None
    if not args.no_extras and B == 1:
        log("[bench] extras: LM head (K=4) and embedding rows")
        extra = extras(te, torch, dev, max(40, args.steps // 5), samples=samples)
        # small decode batches (the decode-GEMV carries the rows in its MFMA columns)
        small = {}
        for bs in (2, 4, 8):
            ssec_b, _, _, _ = run_block(te, torch, dev, LAYERS, GROUPS, bs, K, V,
                                        max(20, args.steps // 5), max(3, args.warmup // 5),
                                        per_launch=False, samples=samples,
                                        label=f"block batch {bs}")
            small[str(bs)] = round(ssec_b * 1e6, 2)
        extra["us_per_block_small_batch"] = small
        log(f"[bench] extras {extra}")

    calibration_passes(torch, dev)

    out = {
        "metric": "3-bit decode-GEMV HBM GB/s (% of peak) + us/layer, Qwen3-8B shapes, batch 1/64",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"u32 packed K={K} trellis (V={V}), fp16 activations, fp32 accumulate",
        "data": "synthetic: uniform random packed bits, seeded signs/scales, fp16 N(0,1) x",
        "config": {"workload": f"Qwen3-8B decoder-block linears (q,k,v,o,gate,up,down), K={K}, "
                               f"MCG, V={V}, batch {B}",
                   "batch": B, "K": K, "V": V, "codebook": "mcg",
                   "mma_f16": bool(args.mma_f16 and B > 4),
                   "block_packed_bytes": block_bytes, "weight_copies": copies,
                   "rotated_bytes": block_bytes * copies,
                   "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                   "us_per_block": round(sec * 1e6, 2),
                   "blocks_per_graph": copies,
                   "warmup_s_min": WARM_S,
                   "us_per_block_one_graph_per_block": round(ge["sec"] * 1e6, 2),
                   "launches_per_block": [g for g, _ in GROUPS],
                   "us_per_group_launch": us_group,
                   "us_per_layer_single_launch": us_layer,
                   "batch16": batched.get(16),
                   "batch64": batch64,
                   "prefill512": batched.get(512),
                   "sweep_configs4": sweep,
                   "next_rows": extra,
                   "ceilings": ceilings(K)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile() if B == 1 and K == 3 and V == 1 else None,
                     "traffic_source": "profiles/gemv_gate_up_b1_traffic.txt (rocprofv3 "
                                       "FETCH_SIZE / WRITE_SIZE of this launch, each scaled by "
                                       "what it reads for a read-only / write-only pass of "
                                       "known size)",
                     "kernel": f"gemv_kernel<K={K},MCG,V={V}> on the gate+up group "
                               "(2 x 12288x4096, one launch)" if B == 1 else
                               f"bgemm_kernel<K={K},MCG,V={V}> on the gate+up group",
                     "avg_launch_us": round(dom_us, 3),
                     "algorithmic_bytes_per_launch": dom_bytes},
    }
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline")
        out["cpu_baseline"] = cpu_baseline()
        out["output_check"] = check_outputs(samples)
    print(json.dumps(out), flush=True)
    if not out.get("output_check", {"ok": True})["ok"]:
        log("[bench] OUTPUT CHECK FAILED: the timed launches do not match the oracle")
        sys.exit(3)


if __name__ == "__main__":
    main()
