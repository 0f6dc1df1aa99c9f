"""GPU parity of the embedding-row lookup (trellis_embed_rows, the DECODE_EMBED of
web/kernels.js:192-249 / PackedOps.embedRow of web/packed.js:137-146) against the CPU
oracle's restored matrix W_hat = restore(decode(bits)) (qtip.py:262-268).

Bar: max|got - W_hat[row]| / max|W_hat[row]| <= 1e-5 per call (fp32 sums of exact codebook
values against float64), bit-exact zeros for ids outside [0, n_out)."""
import sys

import numpy as np
import pytest
import torch

from oracle import trellis_np as tn

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_linear(te, bits, rec, device):
    r = te.PackedRecord(rec.n, rec.k, rec.K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                        float(rec.scale), codebook=rec.codebook, V=rec.V)
    return te.PackedLinear(r, device=device)


@pytest.mark.parametrize("n,k", [(256, 512), (384, 640), (96, 256), (1040, 272)])
@pytest.mark.parametrize("cb", ["mcg", "3inst", "1mad"])
@pytest.mark.parametrize("K,V", [(2, 1), (3, 1), (4, 1), (3, 2)])
def test_embed_rows_vs_oracle(te, gpu_device, n, k, cb, K, V):
    """Every row of small matrices, including Hadamard blocks below 128 (fit(1040,128) =
    16, fit(272,128) = 16, fit(640,128) = 128, fit(96,128) = 32)."""
    _say(f"[embed] n={n} k={k} cb={cb} K={K} V={V}")
    bits, rec = tn.synthetic_record(n, k, K, seed=n + k + K + 10 * V, codebook=cb, V=V)
    lin = make_linear(te, bits, rec, gpu_device)
    W = tn.w_hat_from_record(bits, rec)
    rows = np.arange(n, dtype=np.int32)
    got = lin.embed_rows(torch.from_numpy(rows)).cpu().numpy().astype(np.float64)
    assert got.shape == (n, k)
    err = np.abs(got - W).max(axis=1) / np.abs(W).max(axis=1)
    assert err.max() < TOL, err.max()


def test_embed_rows_out_of_range_and_f16(te, gpu_device):
    _say("[embed] ids out of range, f16 output, strided rows")
    bits, rec = tn.synthetic_record(256, 512, 3, seed=5)
    lin = make_linear(te, bits, rec, gpu_device)
    W = tn.w_hat_from_record(bits, rec)
    ids = torch.tensor([3, -1, 256, 255, 100000, 0], dtype=torch.int32)
    got = lin.embed_rows(ids).cpu().numpy()
    for i, r in enumerate(ids.tolist()):
        if 0 <= r < 256:
            assert tn.rel_err(got[i], W[r]) < TOL
        else:
            assert not got[i].any()
    h = lin.embed_rows(ids[:1], out_dtype=torch.float16).cpu().numpy().astype(np.float64)
    assert np.abs(h[0] - W[3]).max() <= 2.0 ** -10 * np.abs(W[3]).max()
    big = torch.zeros((4, 600), dtype=torch.float32, device=gpu_device)
    lin.embed_rows(torch.tensor([7, 8, 9, 10], dtype=torch.int32), out=big[:, :512])
    out = big.cpu().numpy()
    assert not out[:, 512:].any()
    assert tn.rel_err(out[1, :512], W[8]) < TOL
    ops = te.PackedOps()
    assert tn.rel_err(ops.embedRow(lin, 9).cpu().numpy(), W[9]) < TOL


def test_embed_row_dot_equals_linear(te, gpu_device):
    """At a Qwen3-8B-sized shape, where the float64 W_hat would be costly: the embedded
    row r dotted with x equals the packed linear's output r (two kernels, one matrix)."""
    _say("[embed] 4096x4096 row . x == linear(x)[row]")
    bits, rec = tn.synthetic_record(4096, 4096, 3, seed=11)
    lin = make_linear(te, bits, rec, gpu_device)
    rows = torch.tensor([0, 1, 127, 128, 2047, 4095], dtype=torch.int32)
    E = lin.embed_rows(rows).double()
    x = torch.randn(4096, device=gpu_device, dtype=torch.float32)
    y = lin(x).double()
    want = y[rows.long().to(gpu_device)]
    got = E @ x.double()
    assert (got - want).abs().max().item() <= 1e-3 * y.abs().max().item()
