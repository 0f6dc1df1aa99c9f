"""numpy restatement of the reference's trellis decode path (TEST INFRASTRUCTURE ONLY).

Every function cites the reference file:line it restates (paths relative to the
reference checkout). Integer work is done in uint32/uint64 numpy arithmetic; float
work follows the reference's fp32 steps where bit-exactness matters (codebook values,
decoded tiles) and uses float64 where only a tolerance is asked for (the dense
matmul reference).

Pins (see tests/test_oracle_*.py):
  codebooks      reference KAT cb_1mad(0) (tests/test_qtip.py:23-27), distribution
                 bounds (:28-32), an independent pure-Python-int + struct('<e')
                 restatement over all 65536 states, hand-derived KATs.
  window decode  reference invariant decode_window == decode_recursive
                 (tests/test_qtip.py:36-45), and packed-window decode == tail-warmed
                 recursion over the wrapped stream (tests/test_qtip.py:48-68 logic,
                 for K=2,3,4).
  pack_bits      round trip with unpack_symbols and a bit-by-bit pure-Python packer.
  hadamard       scipy.linalg.hadamard / sqrt(n); H @ H == I.
  restore / IP   reference invariant restore(ip(w)) == w (tests/test_qtip.py:86-92)
                 and an explicit dense-matrix restore (kron-built block Hadamards).
  fold           fold(x) == W_hat @ x (web/packed.js:2-7 claims 4.9e-7).
"""
from __future__ import annotations

import numpy as np

# qtip.py:20-23
MASK32 = 0xFFFFFFFF
L = 16
S = 1 << L
T_SEQ = 256
TILE = 16

CODEBOOK_IDS = {"mcg": 0, "3inst": 1, "1mad": 2}


# ----------------------------------------------------------------------------- codebooks
def _fp16_pair_sum(res: np.ndarray) -> np.ndarray:
    """fp16(res>>16) + fp16(res&0xFFFF), summed in fp32 (qtip.py:28-29, :45, :53)."""
    res = res.astype(np.uint32)
    hi = (res >> np.uint32(16)).astype(np.uint16).view(np.float16).astype(np.float32)
    lo = (res & np.uint32(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float32)
    return (hi + lo).astype(np.float32)


def lcg_raw(states: np.ndarray, codebook: str) -> np.ndarray:
    """The 32-bit integer stage of each computed codebook (qtip.py:35, :43, :51)."""
    x = np.asarray(states).astype(np.uint64) & np.uint64(0xFFFF)
    if codebook == "mcg":
        x = x * np.uint64(0xCBAC1FED)
    elif codebook == "3inst":
        x = x * np.uint64(89226354) + np.uint64(64248484)
    elif codebook == "1mad":
        x = x * np.uint64(34038481) + np.uint64(76625530)
    else:
        raise ValueError(f"unknown codebook {codebook!r}")
    return (x & np.uint64(MASK32)).astype(np.uint32)


def lop3_raw(p: np.ndarray) -> np.ndarray:
    """(x & 0x8FFF8FFF) ^ 0x3B603B60 (qtip.py:44, :52)."""
    return (p & np.uint32(0x8FFF8FFF)) ^ np.uint32(0x3B603B60)


def codebook_values(states: np.ndarray, codebook: str) -> np.ndarray:
    """state (u16) -> fp32 value for 'mcg' | '3inst' | '1mad' (qtip.py:32-53)."""
    p = lcg_raw(states, codebook)
    if codebook == "1mad":
        # qtip.py:36-37: byte sum, then (y - 510) / 147.800537109375 in fp32
        y = ((p & 255) + ((p >> 8) & 255) + ((p >> 16) & 255) + ((p >> 24) & 255))
        return ((y.astype(np.float32) - np.float32(510.0))
                / np.float32(147.800537109375)).astype(np.float32)
    return _fp16_pair_sum(lop3_raw(p))


# V=2 (two weights per trellis step). The reference implements V=1 only (qtip.py:4 and
# notes/qtip-exl3-spec.md:10, 21 name V=2 as QTIP's released setting, with a learned 2-D
# LUT this repository does not ship). This build defines V=2 on the reference's computed
# codebooks: the 16-bit state of step u yields weight 2u from the codebook's first LCG
# iterate (exactly the V=1 value) and weight 2u+1 from the second iterate of the same
# 32-bit map (MCG: s*C then s*C*C; 3INST/1MAD: x -> x*a + b applied twice), both through
# the codebook's usual output stage (lop3 + fp16-halves sum, or byte sum).
_LCG = {"mcg": (0xCBAC1FED, 0), "3inst": (89226354, 64248484), "1mad": (34038481, 76625530)}


def lcg_next(p: np.ndarray, codebook: str) -> np.ndarray:
    """One more iterate of the codebook's 32-bit affine map on a full 32-bit value."""
    mul, add = _LCG[codebook]
    x = np.asarray(p).astype(np.uint64) * np.uint64(mul) + np.uint64(add)
    return (x & np.uint64(MASK32)).astype(np.uint32)


def _output_stage(p: np.ndarray, codebook: str) -> np.ndarray:
    if codebook == "1mad":
        y = ((p & 255) + ((p >> 8) & 255) + ((p >> 16) & 255) + ((p >> 24) & 255))
        return ((y.astype(np.float32) - np.float32(510.0))
                / np.float32(147.800537109375)).astype(np.float32)
    return _fp16_pair_sum(lop3_raw(p))


def codebook_values_v2(states: np.ndarray, codebook: str):
    """state (u16) -> (first, second) fp32 values of the V=2 codebook defined above."""
    p1 = lcg_raw(states, codebook)
    return _output_stage(p1, codebook), _output_stage(lcg_next(p1, codebook), codebook)


def codebook_lut(codebook: str) -> np.ndarray:
    """All 2^16 states -> fp32 LUT (qtip.py:59-66)."""
    return codebook_values(np.arange(S, dtype=np.uint32), codebook)


def codebook_rms(codebook: str) -> float:
    """lut.square().mean().sqrt() (export_packed.py:53), computed in float64."""
    lut = codebook_lut(codebook).astype(np.float64)
    return float(np.sqrt(np.mean(lut * lut)))


# ----------------------------------------------------------------------------- decode
def decode_recursive(bits: np.ndarray, K: int, lut: np.ndarray, s0=None) -> np.ndarray:
    """Sequential state recursion s=((s<<K)|b)&0xFFFF (qtip.py:70-79)."""
    n, T = bits.shape
    s = np.zeros(n, np.int64) if s0 is None else np.asarray(s0, np.int64).copy()
    out = np.empty((n, T), np.float32)
    b = bits.astype(np.int64)
    for t in range(T):
        s = ((s << K) | b[:, t]) & (S - 1)
        out[:, t] = lut[s]
    return out


def decode_window(bits: np.ndarray, K: int, lut: np.ndarray) -> np.ndarray:
    """Random-access decode, s0 = 0: state_t = last 16 bits of the symbol stream
    ending at t, positions before t=0 read as zero (qtip.py:82-110)."""
    n, T = bits.shape
    steps = (L + K - 1) // K
    b = bits.astype(np.int64)
    state = np.zeros((n, T), np.int64)
    for j in range(steps):
        idx = np.arange(T) - (steps - 1 - j)
        sym = np.where(idx[None, :] >= 0, b[:, np.clip(idx, 0, None)], 0)
        state = ((state << K) | sym) & (S - 1)
    return lut[state]


def nwords_for(K: int, T: int = T_SEQ) -> int:
    """u32 words per tile (export_packed.py:28)."""
    return (T * K + 31) // 32


def pack_bits(bits: np.ndarray, K: int) -> np.ndarray:
    """[ntiles, T] K-bit symbols -> u32 [ntiles, nwords], reversed pack: symbol t bit kb
    at stream bit (T-1-t)*K + kb (export_packed.py:27-35; export_packed_8b.py:52-62)."""
    ntiles, T = bits.shape
    nw = nwords_for(K, T)
    out = np.zeros((ntiles, nw), np.uint32)
    b = bits.astype(np.int64)
    for t in range(T):
        for kb in range(K):
            pos = (T - 1 - t) * K + kb
            out[:, pos >> 5] |= (((b[:, t] >> kb) & 1).astype(np.uint32) << np.uint32(pos & 31))
    return out


def unpack_symbols(packed: np.ndarray, K: int, T: int = T_SEQ) -> np.ndarray:
    """Inverse of pack_bits: u32 [ntiles, nwords] -> [ntiles, T] symbols."""
    packed = np.asarray(packed, np.uint32)
    ntiles = packed.shape[0]
    out = np.zeros((ntiles, T), np.int64)
    for t in range(T):
        for kb in range(K):
            pos = (T - 1 - t) * K + kb
            bit = (packed[:, pos >> 5] >> np.uint32(pos & 31)) & np.uint32(1)
            out[:, t] |= bit.astype(np.int64) << kb
    return out


def window_states(packed: np.ndarray, K: int, T: int = T_SEQ) -> np.ndarray:
    """Wrapped 16-bit window read from the packed words (web/kernels.js:115-122):
    bp=((T-1-t)*K) % (T*K); w0=word[bp>>5]; w1=word[((bp>>5)+1) % nwords];
    state = funnel(w1:w0 >> (bp&31)) & 0xFFFF. Returns u32 [ntiles, T]."""
    packed = np.asarray(packed, np.uint32)
    nw = packed.shape[1]
    t = np.arange(T)
    bp = ((T - 1 - t) * K) % (T * K)
    i0 = bp >> 5
    i1 = (i0 + 1) % nw
    sh = (bp & 31).astype(np.uint64)
    w0 = packed[:, i0].astype(np.uint64)
    w1 = packed[:, i1].astype(np.uint64)
    win = ((w1 << np.uint64(32)) | w0) >> sh[None, :]
    return (win & np.uint64(0xFFFF)).astype(np.uint32)


def decode_packed_tiles(packed: np.ndarray, K: int, codebook: str = "mcg",
                        V: int = 1) -> np.ndarray:
    """Packed words -> fp32 z-space tiles [ntiles, 256] (the bit-exact decode).

    V=2: the stream is the same 256*K bits per tile, read as 128 steps of 2K bits (step u
    at stream bits (127-u)*2K, i.e. window_states with symbol width 2K over T=128); the
    state of step u gives weights 2u and 2u+1 (codebook_values_v2)."""
    if V == 1:
        return codebook_values(window_states(packed, K), codebook)
    if V != 2:
        raise ValueError("V must be 1 or 2")
    st = window_states(packed, 2 * K, T=T_SEQ // 2)
    v0, v1 = codebook_values_v2(st, codebook)
    out = np.empty((st.shape[0], T_SEQ), np.float32)
    out[:, 0::2] = v0
    out[:, 1::2] = v1
    return out


# ----------------------------------------------------------------------------- tile layout
def tiles_to_matrix(tiles: np.ndarray, n: int, k: int) -> np.ndarray:
    """[ntiles,256] -> [n,k]; tile=(row/16)*(k/16)+col/16, t=(row%16)*16+col%16
    (qtip.py:303; kernels.js:116-117)."""
    return (tiles.reshape(n // 16, k // 16, 16, 16).transpose(0, 2, 1, 3).reshape(n, k))


def matrix_to_tiles(z: np.ndarray) -> np.ndarray:
    """[n,k] -> [ntiles,256] (qtip.py:288; export_packed.py:55)."""
    n, k = z.shape
    return z.reshape(n // 16, 16, k // 16, 16).transpose(0, 2, 1, 3).reshape(-1, T_SEQ)


# ----------------------------------------------------------------------------- Hadamard / IP
def fit_block(d: int, block: int = 128) -> int:
    """Largest power-of-2 divisor of d, capped at block (qtip.py:208-213)."""
    b = 1
    while b < block and d % (b * 2) == 0:
        b *= 2
    return b


def hadamard(n: int, dtype=np.float64) -> np.ndarray:
    """Sylvester H_n / sqrt(n) (qtip.py:200-205)."""
    H = np.ones((1, 1), dtype)
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return (H / np.sqrt(n)).astype(dtype)


def block_had(x: np.ndarray, axis: int, block: int = 128) -> np.ndarray:
    """Block-diagonal normalized Hadamard along `axis`, block=fit_block(d, block)
    (qtip.py:216-223). Computed in x's dtype family (float64 unless x is float32)."""
    xm = np.moveaxis(x, axis, -1)
    d = xm.shape[-1]
    b = fit_block(d, block)
    H = hadamard(b, np.float64 if xm.dtype != np.float32 else np.float32)
    y = (xm.reshape(*xm.shape[:-1], d // b, b) @ H).reshape(xm.shape)
    return np.moveaxis(y, -1, axis)


def fwht_blocks(v: np.ndarray, block: int) -> np.ndarray:
    """Normalized block Hadamard of the last axis by explicit butterflies (the
    O(d log B) form; equal to block_had up to float rounding)."""
    v = np.array(v, dtype=np.float64, copy=True)
    d = v.shape[-1]
    assert d % block == 0
    h = 1
    while h < block:
        vv = v.reshape(*v.shape[:-1], d // (2 * h), 2, h)
        a = vv[..., 0, :].copy()
        b = vv[..., 1, :].copy()
        vv[..., 0, :] = a + b
        vv[..., 1, :] = a - b
        v = vv.reshape(v.shape)
        h *= 2
    return v / np.sqrt(block)


class IPRecord:
    """The per-matrix metadata of one packed linear, as stored by the exporter
    (export_packed.py:58-63): su, sv, isc, osc as f16, scale as f32."""

    def __init__(self, n, k, K, su, sv, isc, osc, scale, codebook="mcg", V=1):
        self.n, self.k, self.K, self.V = int(n), int(k), int(K), int(V)
        self.codebook = codebook
        self.su = np.asarray(su, np.float16)
        self.sv = np.asarray(sv, np.float16)
        self.isc = np.asarray(isc, np.float16)
        self.osc = np.asarray(osc, np.float16)
        self.scale = np.float32(scale)

    @property
    def block_in(self) -> int:
        return fit_block(self.k, 128)

    @property
    def block_out(self) -> int:
        # web/packed.js:173-176: out-dim block is fit(n,128), not the manifest's block
        return fit_block(self.n, 128)


def ip_encode(w: np.ndarray, cb_rms: float, rng: np.random.Generator, block: int = 128):
    """Encode-side incoherence processing (qtip.py:238-260): sv drawn before su, both
    ±1; per-out RMS (mean 1), block-Had(out); per-in RMS (mean 1), block-Had(in);
    global scale = rms(z)/cb_rms. Returns (z, su, sv, in_s, out_s, scale) in fp32.
    The sign draws use numpy's generator (the packed record stores the signs, so the
    generator does not affect decode parity)."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    sv = (rng.integers(0, 2, n).astype(np.float32) * 2 - 1)
    su = (rng.integers(0, 2, k).astype(np.float32) * 2 - 1)
    z = w * sv[:, None] * su[None, :]
    out_s = np.maximum(np.sqrt(np.mean(z * z, axis=1)), 1e-8).astype(np.float32)
    out_s = (out_s / out_s.mean()).astype(np.float32)
    z = z / out_s[:, None]
    z = block_had(z.astype(np.float32), axis=0, block=block)
    in_s = np.maximum(np.sqrt(np.mean(z * z, axis=0)), 1e-8).astype(np.float32)
    in_s = (in_s / in_s.mean()).astype(np.float32)
    z = z / in_s[None, :]
    z = block_had(z.astype(np.float32), axis=1, block=block)
    scale = float(np.sqrt(np.mean(z.astype(np.float64) ** 2)) / cb_rms)
    return (z / scale).astype(np.float32), su, sv, in_s, out_s, np.float32(scale)


def restore(zq: np.ndarray, scale, su, sv, in_s, out_s, block: int = 128) -> np.ndarray:
    """W_hat = restore(zq) (qtip.py:262-268): zq*scale -> block-Had(in) -> *in_s ->
    block-Had(out) -> *out_s -> *sv(rows) *su(cols). float64 throughout."""
    y = np.asarray(zq, np.float64) * float(scale)
    y = block_had(y, axis=1, block=block)
    y = y * np.asarray(in_s, np.float64)[None, :]
    y = block_had(y, axis=0, block=block)
    y = y * np.asarray(out_s, np.float64)[:, None]
    return y * np.asarray(sv, np.float64)[:, None] * np.asarray(su, np.float64)[None, :]


def w_hat_from_record(packed: np.ndarray, rec: IPRecord) -> np.ndarray:
    """restore(decode(bits)) from the packed words and stored f16/f32 metadata: the
    definition the packed-linear call must match (y = restore(decode(bits)) @ x;
    packed.js:51-52 folds scale into isc, which restore applies as zq*scale)."""
    zt = decode_packed_tiles(packed, rec.K, rec.codebook, rec.V)
    zq = tiles_to_matrix(zt, rec.n, rec.k)
    return restore(zq, rec.scale, rec.su.astype(np.float64), rec.sv.astype(np.float64),
                   rec.isc.astype(np.float64), rec.osc.astype(np.float64))


def packed_linear_ref(packed: np.ndarray, rec: IPRecord, x: np.ndarray) -> np.ndarray:
    """Dense reference y = W_hat @ x in float64. x: [k] or [B, k] (rows are tokens)
    -> [n] or [B, n]."""
    W = w_hat_from_record(packed, rec)
    x64 = np.asarray(x, np.float64)
    return x64 @ W.T if x64.ndim == 2 else W @ x64


def packed_linear_fold(packed: np.ndarray, rec: IPRecord, x: np.ndarray) -> np.ndarray:
    """The reference's IP-folded evaluation order (web/packed.js:163-181):
    xf = Hb_k((isc*scale) * (su*x)); t = zq @ xf; y = sv * (osc * Hb_n(t)).
    float64 arithmetic, fp32 fold of scale into isc as the loader does (:51-52)."""
    zt = decode_packed_tiles(packed, rec.K, rec.codebook, rec.V)
    zq = tiles_to_matrix(zt, rec.n, rec.k).astype(np.float64)
    isc_s = (rec.isc.astype(np.float32) * rec.scale).astype(np.float64)
    x64 = np.atleast_2d(np.asarray(x, np.float64))
    xf = block_had(x64 * rec.su.astype(np.float64) * isc_s, axis=1, block=rec.block_in)
    t = xf @ zq.T
    y = block_had(t, axis=1, block=rec.block_out)
    y = y * rec.osc.astype(np.float64) * rec.sv.astype(np.float64)
    return y if np.ndim(x) == 2 else y[0]


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got-ref| / (max|ref| + 1e-6) (validate_packed_linear.py:66)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / (np.abs(ref).max() + 1e-6))


# ----------------------------------------------------------------------------- synthetic records
def codebook_rms_v2(codebook: str) -> float:
    """RMS over both values of all 2^16 V=2 states, float64."""
    v0, v1 = codebook_values_v2(np.arange(S, dtype=np.uint32), codebook)
    both = np.concatenate([v0, v1]).astype(np.float64)
    return float(np.sqrt(np.mean(both * both)))


def synthetic_record(n: int, k: int, K: int, seed: int, codebook: str = "mcg",
                     mean1_scales: bool = True, V: int = 1):
    """Seeded synthetic packed linear as the benchmark configurations use: uniform random
    u32 bits (every stream is a valid tail-biting path), ±1 su/sv, per-matrix scale
    fp16(0.02 / RMS_codebook) stored as f32, isc/osc mean-1 (or ones)."""
    rng = np.random.default_rng(seed)
    ntiles = (n // 16) * (k // 16)
    nw = nwords_for(K)
    bits = rng.integers(0, 1 << 32, size=(ntiles, nw), dtype=np.uint64).astype(np.uint32)
    if (T_SEQ * K) % 32:
        # keep the unused tail bits of the last word zero, as pack_bits leaves them
        used = (T_SEQ * K) % 32
        bits[:, -1] &= np.uint32((1 << used) - 1)
    su = (rng.integers(0, 2, k) * 2 - 1).astype(np.float16)
    sv = (rng.integers(0, 2, n) * 2 - 1).astype(np.float16)
    if mean1_scales:
        isc = rng.uniform(0.5, 1.5, k)
        osc = rng.uniform(0.5, 1.5, n)
        isc = (isc / isc.mean()).astype(np.float16)
        osc = (osc / osc.mean()).astype(np.float16)
    else:
        isc = np.ones(k, np.float16)
        osc = np.ones(n, np.float16)
    rms = codebook_rms(codebook) if V == 1 else codebook_rms_v2(codebook)
    scale = np.float32(np.float16(0.02 / rms))
    rec = IPRecord(n, k, K, su, sv, isc, osc, scale, codebook=codebook, V=V)
    return bits, rec
