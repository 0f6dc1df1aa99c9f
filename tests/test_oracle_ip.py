"""Pins the oracle's Hadamard / restore / fold (reference qtip.py:199-268,
web/packed.js:2-7, 163-181)."""
import numpy as np
import pytest
import scipy.linalg

from oracle import trellis_np as tn


@pytest.mark.parametrize("n", [1, 2, 16, 64, 128])
def test_hadamard_is_sylvester_and_involutive(n):
    H = tn.hadamard(n)
    assert np.allclose(H, scipy.linalg.hadamard(n) / np.sqrt(n))
    assert np.allclose(H @ H, np.eye(n))


@pytest.mark.parametrize("d,want", [(576, 64), (1536, 128), (4096, 128), (12288, 128),
                                    (48, 16), (16, 16), (96, 32)])
def test_fit_block(d, want):
    assert tn.fit_block(d, 128) == want


@pytest.mark.parametrize("d,block", [(576, 64), (1024, 128), (96, 32)])
def test_butterfly_equals_dense_block_had(d, block):
    rng = np.random.default_rng(d)
    x = rng.standard_normal((3, d))
    assert np.allclose(tn.fwht_blocks(x, block), tn.block_had(x, axis=1, block=128))


def test_block_had_is_kron():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((256,))
    Hbig = np.kron(np.eye(2), tn.hadamard(128))
    assert np.allclose(tn.block_had(x[None], axis=1)[0], Hbig @ x)


@pytest.mark.parametrize("shape", [(128, 256), (1536, 576), (64, 96)])
def test_restore_inverts_ip(shape):
    # tests/test_qtip.py:86-92 (restore(ip(w)) == w)
    rng = np.random.default_rng(7)
    w = rng.standard_normal(shape).astype(np.float32)
    z, su, sv, in_s, out_s, scale = tn.ip_encode(w, 1.0, np.random.default_rng(0))
    back = tn.restore(z, scale, su, sv, in_s, out_s)
    assert np.allclose(back, w, atol=1e-5)


def test_restore_matches_explicit_matrices():
    """restore == diag(sv)diag(out_s) Hn (scale Zq Hk) diag(in_s) diag(su) with the
    block Hadamards built as dense kron matrices."""
    rng = np.random.default_rng(2)
    n, k = 192, 96
    zq = rng.standard_normal((n, k))
    su, sv = rng.choice([-1.0, 1.0], k), rng.choice([-1.0, 1.0], n)
    in_s, out_s = rng.uniform(0.5, 1.5, k), rng.uniform(0.5, 1.5, n)
    Hn = np.kron(np.eye(n // 64), tn.hadamard(64))
    Hk = np.kron(np.eye(k // 32), tn.hadamard(32))
    want = np.diag(sv * out_s) @ Hn @ (0.3 * zq @ Hk) @ np.diag(in_s * su)
    assert np.allclose(tn.restore(zq, 0.3, su, sv, in_s, out_s), want)


@pytest.mark.parametrize("n,k,K,cb", [(256, 128, 3, "mcg"), (1536, 576, 3, "3inst"),
                                      (128, 256, 2, "1mad"), (64, 192, 4, "mcg")])
def test_fold_equals_dense(n, k, K, cb):
    """The reference's fold order (packed.js:163-181) computes W_hat @ x (packed.js:7
    reports 4.9e-7)."""
    bits, rec = tn.synthetic_record(n, k, K, seed=n + k + K, codebook=cb)
    x = np.random.default_rng(1).standard_normal((2, k)).astype(np.float16)
    dense = tn.packed_linear_ref(bits, rec, x)
    fold = tn.packed_linear_fold(bits, rec, x)
    assert tn.rel_err(fold, dense) < 1e-9


def test_planted_fold_mistake_is_caught():
    """Using the in-dim block for the out-dim Hadamard (the packed.js:173-175 bug) must
    break the fold identity when the blocks differ."""
    bits, rec = tn.synthetic_record(256, 576, 3, seed=1)
    x = np.random.default_rng(0).standard_normal(576)
    zq = tn.tiles_to_matrix(tn.decode_packed_tiles(bits, 3), 256, 576)
    isc = rec.isc.astype(np.float32) * rec.scale
    xf = tn.block_had((x * rec.su * isc)[None], 1, rec.block_in)
    t = xf @ zq.T
    wrong = tn.block_had(t, 1, rec.block_in)[0] * rec.osc * rec.sv   # block 64, not 128
    assert tn.rel_err(wrong, tn.packed_linear_ref(bits, rec, x)) > 1e-2
