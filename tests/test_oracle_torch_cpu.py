"""The torch-CPU baseline restatement (oracle/torch_cpu.py) agrees with the numpy
oracle: decoded tiles bit-exact, W_hat @ x within fp32 rounding."""
import numpy as np
import pytest
import torch

from oracle import torch_cpu as tc
from oracle import trellis_np as tn


@pytest.mark.parametrize("K,cb", [(2, "mcg"), (3, "3inst"), (4, "1mad"), (3, "mcg")])
def test_decode_matches_numpy(K, cb):
    bits, rec = tn.synthetic_record(64, 192, K, seed=K, codebook=cb)
    lut = tc.codebook_lut_torch(cb)
    got = tc.decode_window_tb(tc.symbols_from_packed(bits, K), K, lut).numpy()
    assert np.array_equal(got.view(np.uint32), tn.decode_packed_tiles(bits, K, cb).view(np.uint32))


def test_matmul_matches_numpy():
    bits, rec = tn.synthetic_record(256, 576, 3, seed=9)
    x = np.random.default_rng(0).standard_normal((2, 576)).astype(np.float16)
    y = tc.decode_matmul(bits, rec, torch.from_numpy(x)).numpy()
    assert tn.rel_err(y, tn.packed_linear_ref(bits, rec, x)) < 1e-5
