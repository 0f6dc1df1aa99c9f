"""Pins the oracle's codebooks (oracle/trellis_np.py; reference src/trellis/qtip.py:27-66)."""
import json
import os
import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import trellis_np as tn

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "codebook_kats.json")))
MULADD = {"mcg": (0xCBAC1FED, 0), "3inst": (89226354, 64248484), "1mad": (34038481, 76625530)}


def _py_raw(state, cb):
    m, a = MULADD[cb]
    return (state * m + a) & 0xFFFFFFFF


def _py_half(bits16):
    return struct.unpack("<e", struct.pack("<H", bits16))[0]


def test_reference_kat_1mad_zero():
    # tests/test_qtip.py:23-27
    v = tn.codebook_values(np.array([0]), "1mad")[0]
    assert abs(float(v) - (325 - 510) / 147.800537109375) < 1e-6


@pytest.mark.parametrize("cb", ["mcg", "3inst", "1mad"])
def test_hand_kats(cb):
    for s, want in KATS[cb].items():
        got = float(tn.codebook_values(np.array([int(s)]), cb)[0])
        assert got == pytest.approx(want, abs=1e-7), (cb, s, got, want)


def test_raw_lop3_kats():
    for key, want in KATS["raw_lop3"].items():
        cb, s = key.split(":")
        got = int(tn.lop3_raw(tn.lcg_raw(np.array([int(s)]), cb))[0])
        assert got == int(want, 16), (key, hex(got))


@pytest.mark.parametrize("cb", ["mcg", "3inst"])
def test_all_states_vs_pure_python(cb):
    """Independent restatement with Python ints and struct's IEEE half decoding over all
    65536 states; the float64 sum of the halves must equal the oracle's fp32 sum exactly
    (i.e. the fp32 sum of the two halves is exact, qtip.py:28-29)."""
    lut = tn.codebook_lut(cb)
    for s in range(1 << 16):
        res = (_py_raw(s, cb) & 0x8FFF8FFF) ^ 0x3B603B60
        v = _py_half(res >> 16) + _py_half(res & 0xFFFF)
        assert float(lut[s]) == v, (cb, s)


def test_1mad_all_states_correctly_rounded():
    """(y-510)/147.800537109375 must be the correctly rounded fp32 quotient for every
    byte sum y the LCG produces (qtip.py:36-37 divide in fp32)."""
    lut = tn.codebook_lut("1mad")
    c = Fraction(147.800537109375)
    seen = {}
    for s in range(1 << 16):
        x = _py_raw(s, "1mad")
        y = (x & 255) + ((x >> 8) & 255) + ((x >> 16) & 255) + ((x >> 24) & 255)
        seen.setdefault(y, float(lut[s]))
        assert float(lut[s]) == seen[y]
    for y, v in seen.items():
        exact = Fraction(y - 510) / c
        v32 = np.float32(v)
        up = np.nextafter(v32, np.float32(np.inf))
        dn = np.nextafter(v32, np.float32(-np.inf))
        err = abs(Fraction(float(v32)) - exact)
        assert err <= abs(Fraction(float(up)) - exact) and err <= abs(Fraction(float(dn)) - exact), y


@pytest.mark.parametrize("cb", ["1mad", "3inst", "mcg"])
def test_distribution_bounds(cb):
    # tests/test_qtip.py:28-32: every computed codebook ~N(0,1) over all states
    lut = tn.codebook_lut(cb).astype(np.float64)
    assert abs(lut.mean()) < 0.05 and 0.8 < lut.std(ddof=1) < 1.35


def test_mcg_rms_near_exl3_constant():
    # qtip.py:24 CODEBOOK_SCALE_EXL3 = 1.24371088; the LUT RMS is 1.24411
    assert tn.codebook_rms("mcg") == pytest.approx(KATS["mcg_rms_approx"], abs=2e-4)
    assert tn.codebook_rms("mcg") == pytest.approx(KATS["exl3_codebook_scale"], rel=1e-3)


def test_planted_mistake_is_caught():
    """A plausible slip (adding the fp16 halves in fp16 instead of fp32) must fail the
    pure-Python restatement: guards that the all-states check has teeth."""
    p = tn.lop3_raw(tn.lcg_raw(np.arange(1 << 16), "mcg"))
    hi = (p >> 16).astype(np.uint16).view(np.float16)
    lo = (p & 0xFFFF).astype(np.uint16).view(np.float16)
    wrong = (hi + lo).astype(np.float32)   # fp16 add
    assert not np.array_equal(wrong, tn.codebook_lut("mcg"))
