"""GPU parity of the batched path's fp16-weight mode (TRELLIS_MMA_F16), through the C ABI.

The mode rounds each decoded codebook value once to fp16 (hi + lo in one fp16 add) and
multiplies it by the fp16 activation once. Bars:
  * against the exact float64 oracle W_hat @ x: max|got-ref|/(max|ref|+1e-6) <= 1e-3
    (validate_packed_linear.py:66-69 metric and threshold), as for the default mode;
  * against an emulation of the mode on the CPU (codebook values rounded to fp16 with
    numpy's round-to-nearest-even cast, the folded activations rounded to fp16 as the
    kernels store them, float64 sums): <= 1e-4, far below the ~2e-4 the rounding itself
    moves the result, so a wrong pairing of tiles, halves or activations fails;
  * calls that run the exact decode-GEMV (batch 1 to 4, and 5 to 16 for narrow groups)
    ignore the flag (bit-identical to the default call).
"""
import functools
import sys

import numpy as np
import pytest
import torch

from oracle import trellis_np as tn

pytestmark = pytest.mark.gpu

TOL = 1e-3
TIGHT = 1e-4


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_linear(te, bits, rec, device):
    r = te.PackedRecord(rec.n, rec.k, rec.K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                        float(rec.scale), codebook=rec.codebook, V=rec.V)
    return te.PackedLinear(r, device=device)


@functools.lru_cache(maxsize=16)     # every case of CASES (pytest runs them batch by batch)
def _case(n, k, K, cb, V):
    bits, rec = tn.synthetic_record(n, k, K, seed=7 * n + k + 3 * K + V, codebook=cb, V=V)
    zt = tn.decode_packed_tiles(bits, K, cb, V)
    zq = tn.tiles_to_matrix(zt, n, k).astype(np.float64)
    return bits, rec, zq, tn.w_hat_from_record(bits, rec)


def _emulated(rec, zq, x):
    """The fp16-weight mode in float64: zq rounded to fp16 (1MAD's integer numerators are
    exact in fp16, so its values stay as they are), the fold xf = Hb_k(isc_s * su * x)
    rounded to fp16, t = xf @ zq16^T, y = sv * osc * Hb_n(t) (web/packed.js:163-181)."""
    zq16 = zq if rec.codebook == "1mad" else zq.astype(np.float16).astype(np.float64)
    isc_s = (rec.isc.astype(np.float32) * rec.scale).astype(np.float64)
    xf = tn.block_had(x.astype(np.float64) * rec.su.astype(np.float64) * isc_s, axis=1,
                      block=rec.block_in)
    xf = xf.astype(np.float16).astype(np.float64)
    y = tn.block_had(xf @ zq16.T, axis=1, block=rec.block_out)
    return y * rec.osc.astype(np.float64) * rec.sv.astype(np.float64)


CASES = [
    (256, 512, 3, "mcg", 1), (1536, 576, 3, "3inst", 1), (576, 1536, 3, "mcg", 1),
    (128, 4096, 2, "mcg", 1), (384, 1024, 4, "3inst", 1), (208, 336, 3, "1mad", 1),
    (208, 336, 3, "mcg", 1),     # 21 tile columns: an odd last tile pair
    (96, 48, 4, "3inst", 1),     # 3 tile columns, blocks of 16
    (256, 512, 3, "mcg", 2), (384, 1024, 2, "3inst", 2),
]


@pytest.mark.parametrize("n,k,K,cb,V", CASES)
@pytest.mark.parametrize("batch", [2, 17, 64, 130])
def test_mma_f16_vs_oracle(te, gpu_device, n, k, K, cb, V, batch):
    _say(f"[mma_f16] n={n} k={k} K={K} cb={cb} V={V} batch={batch}")
    bits, rec, zq, W = _case(n, k, K, cb, V)
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(batch + k).standard_normal((batch, k)).astype(np.float16)
    xt = torch.from_numpy(x).to(gpu_device)
    y = lin(xt, mma_f16=True).cpu().numpy()
    y0 = lin(xt).cpu().numpy()
    assert tn.rel_err(y, x.astype(np.float64) @ W.T) < TOL
    if batch <= 4:
        assert np.array_equal(y, y0)          # the exact decode-GEMV ignores the flag
        return
    assert tn.rel_err(y, _emulated(rec, zq, x)) < TIGHT
    if cb != "1mad":
        # the mode is in effect: the exact default differs by the fp16 rounding
        assert tn.rel_err(y, y0) > 1e-6


@pytest.mark.parametrize("batch", [300, 512])
def test_mma_f16_prefill(te, gpu_device, batch):
    _say(f"[mma_f16 prefill] batch={batch}")
    bits, rec, zq, W = _case(2048, 6144, 3, "mcg", 1)
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(batch).standard_normal((batch, 6144)).astype(np.float16)
    y = lin(torch.from_numpy(x).to(gpu_device), mma_f16=True).cpu().numpy()
    assert tn.rel_err(y, x.astype(np.float64) @ W.T) < TOL
    assert tn.rel_err(y, _emulated(rec, zq, x)) < TIGHT


def test_mma_f16_group_and_repeat(te, gpu_device):
    _say("[mma_f16 group]")
    shapes = [(512, 1024), (128, 1024), (384, 1024)]
    cases = [_case(n, k, 3, "mcg", 1) for n, k in shapes]
    lins = [make_linear(te, b, r, gpu_device) for b, r, _, _ in cases]
    grp = te.PackedGroup(lins)
    batch = 40
    x = np.random.default_rng(5).standard_normal((batch, 1024)).astype(np.float16)
    xt = torch.from_numpy(x).to(gpu_device)
    first = None
    for _ in range(3):
        ys = grp([xt] * 3, mma_f16=True)
        ys = [y.cpu().numpy() for y in ys]
        if first is None:
            first = ys
        for y, y1 in zip(ys, first):
            assert np.array_equal(y, y1)      # deterministic across calls
    for y, (b, rec, zq, W), lin in zip(first, cases, lins):
        assert tn.rel_err(y, x.astype(np.float64) @ W.T) < TOL
        assert tn.rel_err(y, _emulated(rec, zq, x)) < TIGHT
        assert np.array_equal(y, lin(xt, mma_f16=True).cpu().numpy())


def test_mma_f16_dtypes(te, gpu_device):
    bits, rec, zq, W = _case(256, 512, 3, "mcg", 1)
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(2).standard_normal((33, 512)).astype(np.float32)
    xt = torch.from_numpy(x).to(gpu_device)
    y16 = lin(xt, out_dtype=torch.float16, mma_f16=True).float().cpu().numpy()
    assert tn.rel_err(y16, x.astype(np.float64) @ W.T) < 2e-3


@pytest.mark.parametrize("batch", [1, 3, 8])
def test_mma_f16_ignored_by_the_gemv(te, gpu_device, batch):
    """Calls that run the exact decode-GEMV (batch 1 to 4; batch 8 of this narrow matrix,
    whose work items fit one round on the CUs) ignore the flag."""
    bits, rec, zq, W = _case(576, 1536, 3, "mcg", 1)
    lin = make_linear(te, bits, rec, gpu_device)
    x = torch.from_numpy(np.random.default_rng(1).standard_normal((batch, 1536)).astype(np.float16))
    x = x.to(gpu_device)
    assert torch.equal(lin(x, mma_f16=True), lin(x))
