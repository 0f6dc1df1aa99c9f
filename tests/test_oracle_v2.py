"""Pins the oracle's V=2 decode (two weights per trellis step; this build's definition, the
reference implements V=1 only: src/trellis/qtip.py:4, notes/qtip-exl3-spec.md:10, 21).

Definition under test: a tile's 256*K-bit stream is read as 128 steps of kV = 2K bits,
step u at stream bits (127-u)*2K (the V=1 reversed pack of export_packed.py:27-35 with
2K-bit symbols); the 16-bit state of step u is the wrapped window there (web/kernels.js:
115-122 with 2K in place of K) and the bitshift recursion s' = ((s << kV) | b) & 0xFFFF
(spec A); weight 2u is the codebook's first LCG iterate of the state (the V=1 value),
weight 2u+1 its second iterate of the same 32-bit map.
"""
import struct

import numpy as np
import pytest

from oracle import trellis_np as tn

MULADD = {"mcg": (0xCBAC1FED, 0), "3inst": (89226354, 64248484), "1mad": (34038481, 76625530)}


def _half(bits16):
    return struct.unpack("<e", struct.pack("<H", bits16))[0]


def _py_value(p, cb):
    """Output stage with Python ints and struct's IEEE half decoding (qtip.py:32-53)."""
    if cb == "1mad":
        y = (p & 255) + ((p >> 8) & 255) + ((p >> 16) & 255) + ((p >> 24) & 255)
        return float(np.float32(np.float32(y - 510) / np.float32(147.800537109375)))
    res = (p & 0x8FFF8FFF) ^ 0x3B603B60
    return _half(res >> 16) + _half(res & 0xFFFF)


def _py_pair(s, cb):
    m, a = MULADD[cb]
    p1 = (s * m + a) & 0xFFFFFFFF
    p2 = (p1 * m + a) & 0xFFFFFFFF
    return _py_value(p1, cb), _py_value(p2, cb)


@pytest.mark.parametrize("cb", ["mcg", "3inst", "1mad"])
def test_v2_all_states_vs_pure_python(cb):
    """Independent restatement over all 65536 states; the first value is exactly the V=1
    codebook (qtip.py:32-53)."""
    v0, v1 = tn.codebook_values_v2(np.arange(1 << 16), cb)
    assert np.array_equal(v0, tn.codebook_lut(cb))
    for s in range(0, 1 << 16, 7):
        a, b = _py_pair(s, cb)
        assert float(v0[s]) == a and float(v1[s]) == b, (cb, s)


def test_v2_hand_kats():
    """Derived by hand from the closed form: MCG state 0 -> P = 0 twice -> lop3 0x3B603B60
    -> 0.96875 + 0.875 = 1.84375 for both weights. MCG state 1 -> P1 = 0xCBAC1FED (the V=1
    KAT 0.134521484375), P2 = 0xCBAC1FED^2 mod 2^32 = 0xC8734169 -> lop3 0xB3133A09 ->
    fp16 0xB313 = -(1 + 787/1024)/8 = -0.2210693359375 and fp16 0x3A09 =
    (1 + 521/1024)/2 = 0.75439453125, sum 0.5333251953125."""
    v0, v1 = tn.codebook_values_v2(np.array([0, 1]), "mcg")
    assert float(v0[0]) == 1.84375 and float(v1[0]) == 1.84375
    assert float(v0[1]) == 0.134521484375
    assert float(v1[1]) == 0.5333251953125


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("cb", ["mcg", "1mad"])
def test_v2_packed_decode_is_tail_warmed_recursion(K, cb):
    """Packed V=2 decode equals the kV=2K bitshift recursion over 128 steps whose start
    state is filled from the stream's own tail (tail-biting), each state emitting its
    two codebook values."""
    rng = np.random.default_rng(30 + K)
    kv = 2 * K
    steps = rng.integers(0, 1 << kv, (5, 128))
    p = tn.pack_bits(steps, kv)
    assert p.shape == (5, 8 * K)
    got = tn.decode_packed_tiles(p, K, cb, V=2)
    v0, v1 = tn.codebook_values_v2(np.arange(1 << 16), cb)
    s = np.zeros(5, np.int64)
    for u in range(128 - (-(-16 // kv)), 128):
        s = ((s << kv) | steps[:, u]) & 0xFFFF
    want = np.empty((5, 256), np.float32)
    for u in range(128):
        s = ((s << kv) | steps[:, u]) & 0xFFFF
        want[:, 2 * u] = v0[s]
        want[:, 2 * u + 1] = v1[s]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("K", [2, 3, 4])
def test_v2_window_brute_force(K):
    """Every V=2 state equals the 16 bits read one by one from the circular stream at
    bit (127-u)*2K."""
    rng = np.random.default_rng(40 + K)
    p = rng.integers(0, 1 << 32, (2, 8 * K), dtype=np.uint64).astype(np.uint32)
    got = tn.decode_packed_tiles(p, K, "mcg", V=2)
    v0, v1 = tn.codebook_values_v2(np.arange(1 << 16), "mcg")
    total = 256 * K
    for i in range(2):
        stream = 0
        for w in range(8 * K):
            stream |= int(p[i, w]) << (32 * w)
        for u in range(0, 128, 5):
            bp = (127 - u) * 2 * K
            st = 0
            for j in range(16):
                st |= ((stream >> ((bp + j) % total)) & 1) << j
            assert got[i, 2 * u] == v0[st] and got[i, 2 * u + 1] == v1[st]


def test_v1_path_unchanged():
    bits, rec = tn.synthetic_record(32, 64, 3, seed=3)
    assert np.array_equal(tn.decode_packed_tiles(bits, 3, "mcg"),
                          tn.decode_packed_tiles(bits, 3, "mcg", V=1))


def test_v2_planted_mistake_is_caught():
    """Swapping the two values of a step (an easy slip in a kernel's lane layout) must
    fail the recursion check."""
    rng = np.random.default_rng(7)
    steps = rng.integers(0, 1 << 6, (2, 128))
    p = tn.pack_bits(steps, 6)
    got = tn.decode_packed_tiles(p, 3, "mcg", V=2)
    swapped = got.copy()
    swapped[:, 0::2], swapped[:, 1::2] = got[:, 1::2], got[:, 0::2]
    assert not np.array_equal(swapped, got)


def test_v2_fold_equals_dense():
    """The IP-folded evaluation order equals W_hat @ x for a V=2 record (packed.js:163-181)."""
    bits, rec = tn.synthetic_record(128, 256, 3, seed=9, V=2)
    x = np.random.default_rng(0).standard_normal((3, 256))
    assert tn.rel_err(tn.packed_linear_fold(bits, rec, x), tn.packed_linear_ref(bits, rec, x)) < 1e-12
