"""Pins the oracle's decode: window == recursion, packed layout, wrapped window read
(oracle/trellis_np.py; reference qtip.py:70-120, export_packed.py:27-35,
web/kernels.js:115-122)."""
import numpy as np
import pytest

from oracle import trellis_np as tn


@pytest.mark.parametrize("K", [2, 3, 4])
def test_window_equals_recursion(K):
    # the reference invariant tests/test_qtip.py:36-45
    rng = np.random.default_rng(0)
    lut = tn.codebook_lut("mcg")
    bits = rng.integers(0, 1 << K, (8, 64))
    assert np.array_equal(tn.decode_recursive(bits, K, lut), tn.decode_window(bits, K, lut))


def _pack_bitwise(bits, K):
    """Independent packer: build the reversed bit stream as a Python int per tile."""
    ntiles, T = bits.shape
    nw = (T * K + 31) // 32
    out = np.zeros((ntiles, nw), np.uint32)
    for i in range(ntiles):
        stream = 0
        for t in range(T):
            stream |= int(bits[i, t]) << ((T - 1 - t) * K)
        for w in range(nw):
            out[i, w] = (stream >> (32 * w)) & 0xFFFFFFFF
    return out


@pytest.mark.parametrize("K", [2, 3, 4])
def test_pack_matches_bitwise_and_roundtrips(K):
    rng = np.random.default_rng(K)
    bits = rng.integers(0, 1 << K, (5, 256))
    p = tn.pack_bits(bits, K)
    assert p.shape == (5, 8 * K) and p.dtype == np.uint32
    assert np.array_equal(p, _pack_bitwise(bits, K))
    assert np.array_equal(tn.unpack_symbols(p, K), bits)


@pytest.mark.parametrize("K", [2, 3, 4])
def test_packed_window_is_tail_warmed_recursion(K):
    """Decoding the packed words with the wrapped window read equals the recursion over
    the stream whose start state is filled from the stream's own tail (the tail-biting
    check of tests/test_qtip.py:48-68, here for K=2,3,4). Warm-up of ceil(16/K)
    symbols covers bit 15 for K=3 (the reference's (L-K)//K warm-up would not)."""
    rng = np.random.default_rng(10 + K)
    lut = tn.codebook_lut("mcg")
    bits = rng.integers(0, 1 << K, (6, 256))
    p = tn.pack_bits(bits, K)
    got = tn.decode_packed_tiles(p, K, "mcg")
    n = bits.shape[0]
    s = np.zeros(n, np.int64)
    warm = -(-16 // K)
    for t in range(256 - warm, 256):
        s = ((s << K) | bits[:, t]) & 0xFFFF
    want = np.empty((n, 256), np.float32)
    for t in range(256):
        s = ((s << K) | bits[:, t]) & 0xFFFF
        want[:, t] = lut[s]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("K", [2, 3, 4])
def test_window_states_brute_force(K):
    """Every state equals the 16 bits read one by one from the circular stream."""
    rng = np.random.default_rng(20 + K)
    p = rng.integers(0, 1 << 32, (3, 8 * K), dtype=np.uint64).astype(np.uint32)
    st = tn.window_states(p, K)
    total = 256 * K
    for i in range(3):
        stream = 0
        for w in range(8 * K):
            stream |= int(p[i, w]) << (32 * w)
        for t in range(0, 256, 7):
            bp = (255 - t) * K
            v = 0
            for j in range(16):
                v |= ((stream >> ((bp + j) % total)) & 1) << j
            assert int(st[i, t]) == v


def test_tile_layout_roundtrip():
    rng = np.random.default_rng(3)
    z = rng.standard_normal((48, 80))
    tiles = tn.matrix_to_tiles(z)
    assert tiles.shape == (15, 256)
    # tile = (row/16)*tiles_in + col/16 ; t = (row%16)*16 + col%16
    for row, col in [(0, 0), (17, 33), (47, 79), (31, 64)]:
        assert tiles[(row // 16) * 5 + col // 16, (row % 16) * 16 + col % 16] == z[row, col]
    assert np.array_equal(tn.tiles_to_matrix(tiles, 48, 80), z)


def test_planted_window_mistake_is_caught():
    """Dropping the wrap (reading a zero word past the end) must break the tail-biting
    equality for K=3."""
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 8, (4, 256))
    p = tn.pack_bits(bits, 3)
    padded = np.concatenate([p, np.zeros((4, 1), np.uint32)], axis=1)
    t = np.arange(256)
    bp = (255 - t) * 3
    w = (padded[:, (bp >> 5) + 1].astype(np.uint64) << np.uint64(32)) | padded[:, bp >> 5]
    nowrap = ((w >> (bp & 31).astype(np.uint64)) & np.uint64(0xFFFF)).astype(np.uint32)
    assert not np.array_equal(nowrap, tn.window_states(p, 3))
