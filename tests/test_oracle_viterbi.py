"""Pins the C tail-biting encoder used for fixtures (oracle/viterbi.c; reference
qtip.py:124-196; tests/test_qtip.py:48-83; tests/test_trellis.py:15-36)."""
import itertools

import numpy as np
import pytest

from oracle import trellis_np as tn
from oracle import viterbi as vt


def _brute_force(w, L, K, lut):
    """min over all symbol streams of sum (w - lut[state])^2 with zero start state."""
    T = w.shape[0]
    best = np.inf
    for stream in itertools.product(range(1 << K), repeat=T):
        s, err = 0, 0.0
        for t, b in enumerate(stream):
            s = ((s << K) | b) & ((1 << L) - 1)
            err += (float(w[t]) - float(lut[s])) ** 2
        best = min(best, err)
    return best


def test_single_pass_is_optimal_tiny():
    """With a free start edge the DP optimum is the min over all start states as well;
    brute force enumerates the L-K initial edge bits too."""
    rng = np.random.default_rng(0)
    L, K, T = 6, 2, 5
    lut = rng.standard_normal(1 << L).astype(np.float32)
    for _ in range(4):
        w = rng.standard_normal((1, T)).astype(np.float32)
        st = vt.viterbi_pass(w, K, lut, L=L)
        got = float(((w[0] - lut[st[0]]) ** 2).sum())
        # brute force over (start edge, streams)
        best = np.inf
        for e0 in range(1 << (L - K)):
            for stream in itertools.product(range(1 << K), repeat=T):
                s, err = e0, 0.0
                for t, b in enumerate(stream):
                    s = ((s << K) | b) & ((1 << L) - 1)
                    err += (float(w[0, t]) - float(lut[s])) ** 2
                best = min(best, err)
        assert got == pytest.approx(best, abs=1e-4)
        # state path is a valid trellis path
        for t in range(1, T):
            assert (st[0, t] >> K) == (st[0, t - 1] & ((1 << (L - K)) - 1))


@pytest.mark.parametrize("K", [2, 3])
def test_tail_biting_wraps(K):
    """bits < 2^K and the packed wrapped stream alone reproduces the encoder's dq
    (tests/test_qtip.py:48-68)."""
    rng = np.random.default_rng(1)
    lut = tn.codebook_lut("mcg")
    w = rng.standard_normal((4, 256)).astype(np.float32)
    bits, dq, st = vt.viterbi_tb(w, K, lut)
    assert bits.max() < (1 << K) and bits.min() >= 0
    p = tn.pack_bits(bits, K)
    assert np.array_equal(tn.decode_packed_tiles(p, K, "mcg"), dq)


def test_k2_mse_bound():
    # tests/test_qtip.py:71-83: K=2 TCQ on N(0,1) reaches ~0.073 (bound 0.085)
    rng = np.random.default_rng(2)
    lut = tn.codebook_lut("mcg")
    w = rng.standard_normal((64, 256)).astype(np.float32)
    _, dq, _ = vt.viterbi_tb(w, 2, lut)
    assert ((w - dq) ** 2).mean() < 0.085


def test_encode_layer_roundtrip():
    """IP + encode + pack of a small layer: the packed record decodes to the encoder's
    zq and restore(zq) approximates w (3-bit TCQ rel-MSE well under scalar 3-bit)."""
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 128)) * 0.02).astype(np.float32)
    packed, rec, zq = vt.encode_layer(w, 3, "3inst", seed=0)
    zt = tn.decode_packed_tiles(packed, 3, "3inst")
    assert np.array_equal(tn.tiles_to_matrix(zt, 64, 128), zq)
    W = tn.w_hat_from_record(packed, rec)
    rel = ((W - w) ** 2).mean() / (w ** 2).mean()
    assert rel < 0.06
