"""Randomized launch plans against the float64 oracle: seeded draws of shape, K, codebook,
V, batch (1 to 257: across every decode-GEMV row count and batched column-block boundary,
ragged last column blocks, 64- and 128-column blocks, split-K or not) and MFMA mode, each
compared whole with W_hat @ x at the 1e-3 metric of validate_packed_linear.py:66-69, and
repeated once for bit-identical results (tickets and plans are deterministic)."""
import sys

import numpy as np
import pytest
import torch

from oracle import trellis_np as tn

pytestmark = pytest.mark.gpu
TOL = 1e-3

SHAPES = [(128, 256), (256, 512), (384, 768), (640, 1024), (1024, 1536), (1536, 2048),
          (2048, 1024), (512, 4096), (208, 336), (96, 48)]
BATCHES = [1, 2, 3, 4, 5, 7, 9, 15, 16, 17, 31, 33, 63, 64, 65, 100, 127, 128, 129, 200, 257]


def _cases(count=60, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n, k = SHAPES[rng.integers(len(SHAPES))]
        K = int(rng.integers(2, 5))
        cb = ["mcg", "3inst", "1mad"][rng.integers(3)]
        V = int(rng.integers(1, 3))
        batch = BATCHES[rng.integers(len(BATCHES))]
        f16 = bool(batch > 1 and rng.integers(4) == 0)
        out.append((i, n, k, K, cb, V, batch, f16))
    return out


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("i,n,k,K,cb,V,batch,f16", _cases())
def test_random_plan_vs_oracle(te, gpu_device, i, n, k, K, cb, V, batch, f16):
    _say(f"[plans] #{i} n={n} k={k} K={K} cb={cb} V={V} batch={batch} mma_f16={f16}")
    bits, rec = tn.synthetic_record(n, k, K, seed=1000 + i, codebook=cb, V=V)
    r = te.PackedRecord(rec.n, rec.k, rec.K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                        float(rec.scale), codebook=rec.codebook, V=rec.V)
    lin = te.PackedLinear(r, device=gpu_device)
    x = np.random.default_rng(i).standard_normal((batch, k)).astype(np.float16)
    xt = torch.from_numpy(x).to(gpu_device)
    y = lin(xt, mma_f16=f16).cpu().numpy()
    assert np.array_equal(y, lin(xt, mma_f16=f16).cpu().numpy())
    want = tn.packed_linear_ref(bits, rec, x)
    assert tn.rel_err(y, want) < TOL
    for b in (0, batch - 1):                 # rows are independent of each other
        assert tn.rel_err(y[b], want[b]) < TOL
