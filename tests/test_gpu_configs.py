"""GPU parity at the benchmark workloads themselves, through the launches bench.py times.

* Qwen3-8B block linears at decode batch 1 (the headline: the q/k/v group's split-K
  decode-GEMV over 240 items, gate+up as one launch of 192 whole blocks), 2, 4, 8, 16 and 64:
  q/k/v as one PackedGroup, o, gate/up as one PackedGroup, down, i.e. the exact plans of the
  bench (decode-GEMV up to 16 rows, the batched kernel for gate+up at 8 and 16 and for
  every launch at 64, with its split-K fold).
* Every point of the bit-rate sweep on the 8B gate/up/down shapes (4096 <-> 12288): K = 2,
  3, 4 x V = 1, 2 at batch 1 and at a 512-token prefill.

A dense float64 oracle of a whole 8B matrix (50M weights) would take minutes, so three
128-row output blocks (first, middle, last) of every member are checked against the oracle
for every batch row (an output block depends only on its own 8 bands of tiles), and the
whole output by linearity: f(a x1 + b x2) = a f(x1) + b f(x2). Metric and bar:
max|got - ref| / (max|ref| + 1e-6) <= 1e-3 (scripts/validate_packed_linear.py:66-69).
"""
import functools
import sys
import zlib

import numpy as np
import pytest
import torch

from oracle import trellis_np as tn

pytestmark = pytest.mark.gpu
TOL = 1e-3

SHAPES_8B = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
             "gate": (12288, 4096), "up": (12288, 4096), "down": (4096, 12288)}
GROUPS_8B = [("qkv", ("q", "k", "v")), ("o", ("o",)), ("gate_up", ("gate", "up")),
             ("down", ("down",))]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@functools.lru_cache(maxsize=8)
def _record(name, K, V):
    n, k = SHAPES_8B[name]
    return tn.synthetic_record(n, k, K, seed=zlib.crc32(f"{name}/{K}/{V}".encode()), V=V)


def _linear(te, name, K, V, device):
    bits, rec = _record(name, K, V)
    r = te.PackedRecord(rec.n, rec.k, rec.K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                        float(rec.scale), codebook=rec.codebook, V=rec.V)
    return te.PackedLinear(r, device=device)


def _oracle_block_rows(bits, rec, ob, x):
    """Oracle for output rows [128 ob, 128 ob + 128): those rows depend only on their own
    8 bands (the out-dim Hadamard block is 128)."""
    tin = rec.k // 16
    sub_bits = bits[ob * 8 * tin:(ob + 1) * 8 * tin]
    sl = slice(ob * 128, ob * 128 + 128)
    sub = tn.IPRecord(128, rec.k, rec.K, rec.su, rec.sv[sl], rec.isc, rec.osc[sl], rec.scale,
                      codebook=rec.codebook, V=rec.V)
    return tn.packed_linear_ref(sub_bits, sub, x)


def _check_members(te, names, K, V, batch, device, seed):
    lins = [_linear(te, nm, K, V, device) for nm in names]
    grp = te.PackedGroup(lins)
    k = lins[0].k_in
    x = np.random.default_rng(seed).standard_normal((batch, k)).astype(np.float16)
    xt = torch.from_numpy(x).to(device)
    ys = [y.cpu().numpy() for y in grp([xt] * len(lins))]
    for nm, y in zip(names, ys):
        bits, rec = _record(nm, K, V)
        nob = rec.n // 128
        for ob in (0, nob // 2, nob - 1):
            want = _oracle_block_rows(bits, rec, ob, x)
            got = y[:, ob * 128:(ob + 1) * 128]
            assert tn.rel_err(got, want) < TOL, (nm, ob)
            # every batch row on its own: rows must not mix
            for b in (0, batch // 2, batch - 1):
                assert tn.rel_err(got[b], want[b]) < TOL, (nm, ob, b)
    # linearity over the whole output, in fp32 inputs
    x1 = torch.randn((batch, k), device=device)
    x2 = torch.randn((batch, k), device=device)
    lhs = grp([0.75 * x1 - 1.5 * x2] * len(lins))
    r1, r2 = grp([x1] * len(lins)), grp([x2] * len(lins))
    for nm, a, p, q in zip(names, lhs, r1, r2):
        rhs = 0.75 * p - 1.5 * q
        assert (a - rhs).abs().max().item() / rhs.abs().max().item() < TOL, nm


@pytest.mark.parametrize("batch", [1, 2, 4, 8, 16, 64])
@pytest.mark.parametrize("gname,names", GROUPS_8B)
def test_qwen3_8b_block_batched(te, gpu_device, batch, gname, names):
    """The 8B block's four launches at decode batch 1 (the headline plans), 2, 4, 8 (the
    decode-GEMV with the rows in its MFMA columns; at 8, gate+up on the batched path), 16 and
    64, K=3 MCG V=1."""
    _say(f"[8B block] {gname} batch={batch}")
    _check_members(te, names, 3, 1, batch, gpu_device, seed=batch + len(gname))


@pytest.mark.parametrize("K,V", [(2, 1), (4, 1), (2, 2), (3, 2), (4, 2)])
@pytest.mark.parametrize("gname,names", [("gate_up", ("gate", "up")), ("down", ("down",))])
def test_sweep_batch1(te, gpu_device, K, V, gname, names):
    """The bit-rate sweep's batch-1 points on the 8B gate/up/down shapes (K=3 V=1 is the
    headline block's own gate+up and down, above)."""
    _say(f"[sweep] {gname} K={K} V={V} batch=1")
    _check_members(te, names, K, V, 1, gpu_device, seed=10 * K + V)


@pytest.mark.parametrize("K,V", [(3, 1), (2, 1), (3, 2), (2, 2), (4, 1), (4, 2)])
@pytest.mark.parametrize("gname,names", [("gate_up", ("gate", "up")), ("down", ("down",))])
def test_sweep_prefill512(te, gpu_device, K, V, gname, names):
    """The bit-rate sweep's 512-token prefill points on the 8B gate/up/down shapes."""
    _say(f"[sweep] {gname} K={K} V={V} batch=512")
    _check_members(te, names, K, V, 512, gpu_device, seed=100 + 10 * K + V)
