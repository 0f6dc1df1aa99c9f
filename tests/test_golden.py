"""The committed fixtures (tests/golden/*.npz) against the oracle: guards the oracle
and the fixtures against drift (decoded-tile hashes and y_ref)."""
import glob
import hashlib
import os

import numpy as np
import pytest

from oracle import trellis_np as tn

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FILES = sorted(glob.glob(os.path.join(GOLD, "*.npz")))


def load_fixture(path):
    d = np.load(path)   # allow_pickle=False (default)
    K = int(d["K"])
    cb = str(d["codebook"])
    nt = d["bits"].shape[0]
    n = d["sv"].shape[0]
    k = d["su"].shape[0]
    assert nt == (n // 16) * (k // 16)
    rec = tn.IPRecord(n, k, K, d["su"], d["sv"], d["isc"], d["osc"], d["scale"], codebook=cb)
    return d, rec


@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f) for f in FILES])
def test_fixture_against_oracle(path):
    d, rec = load_fixture(path)
    zt = tn.decode_packed_tiles(d["bits"], rec.K, rec.codebook)
    assert hashlib.sha256(zt.astype(np.float32).tobytes()).hexdigest() == str(d["tiles_sha"])
    assert np.array_equal(zt[:8], d["tiles_head"])
    y = tn.packed_linear_ref(d["bits"], rec, d["x"])
    assert tn.rel_err(y, d["y_ref"]) < 1e-12


def test_config1_quality():
    d, rec = load_fixture(os.path.join(GOLD, "config1_smollm2_up.npz"))
    assert rec.codebook == "3inst" and rec.K == 3 and (rec.n, rec.k) == (1536, 576)
    assert rec.block_in == 64 and rec.block_out == 128
    # 3-bit TCQ of a Gaussian layer: relative MSE ~0.018
    assert float(d["w_rel_mse"]) < 0.03
