"""ctypes front end of oracle/viterbi.c (TEST INFRASTRUCTURE ONLY).

Restates the reference encoder src/trellis/qtip.py:124-196 (tail-biting Viterbi) and
the layer path of scripts/export_packed.py:52-61 (IP -> tiles -> encode -> pack), used
to build the config-1 fixture (the SmolLM2-135M up_proj configuration).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import trellis_np as tn

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libtrellis_viterbi.so")
_lib = None


def build() -> str:
    """Compile viterbi.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH) or (
                os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, "viterbi.c"))):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        f32p = ctypes.POINTER(ctypes.c_float)
        i32p = ctypes.POINTER(ctypes.c_int32)
        i64p = ctypes.POINTER(ctypes.c_int64)
        lib.trellis_oracle_viterbi_tb.argtypes = [f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                  ctypes.c_int, f32p, i32p, f32p, i32p,
                                                  ctypes.c_int]
        lib.trellis_oracle_viterbi_pass.argtypes = [f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                    ctypes.c_int, f32p, i64p, i32p, ctypes.c_int]
        _lib = lib
    return _lib


def _ptr(a, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def viterbi_tb(w: np.ndarray, K: int, lut: np.ndarray, L: int = tn.L, nthreads: int = 0):
    """Tail-biting encode of w [n, T] -> (bits [n,T] int32, dq [n,T] fp32, states [n,T])."""
    lib = _load()
    w = np.ascontiguousarray(w, np.float32)
    lut = np.ascontiguousarray(lut, np.float32)
    n, T = w.shape
    assert lut.shape[0] == 1 << L
    bits = np.empty((n, T), np.int32)
    dq = np.empty((n, T), np.float32)
    st = np.empty((n, T), np.int32)
    rc = lib.trellis_oracle_viterbi_tb(_ptr(w, ctypes.c_float), n, T, L, K,
                                       _ptr(lut, ctypes.c_float), _ptr(bits, ctypes.c_int32),
                                       _ptr(dq, ctypes.c_float), _ptr(st, ctypes.c_int32),
                                       nthreads)
    if rc:
        raise ValueError("viterbi_tb: bad parameters")
    return bits, dq, st


def viterbi_pass(w: np.ndarray, K: int, lut: np.ndarray, L: int = tn.L, overlap=None,
                 nthreads: int = 0) -> np.ndarray:
    """One DP pass (qtip.py:147-196) -> optimal state path [n, T]."""
    lib = _load()
    w = np.ascontiguousarray(w, np.float32)
    lut = np.ascontiguousarray(lut, np.float32)
    n, T = w.shape
    st = np.empty((n, T), np.int32)
    ov = None if overlap is None else np.ascontiguousarray(overlap, np.int64)
    rc = lib.trellis_oracle_viterbi_pass(_ptr(w, ctypes.c_float), n, T, L, K,
                                         _ptr(lut, ctypes.c_float),
                                         None if ov is None else _ptr(ov, ctypes.c_int64),
                                         _ptr(st, ctypes.c_int32), nthreads)
    if rc:
        raise ValueError("viterbi_pass: bad parameters")
    return st


def encode_layer(w: np.ndarray, K: int, codebook: str, seed: int):
    """IP + tiles + tail-biting encode + pack of one weight matrix, as
    export_packed.py:52-61 does. Returns (packed u32 [ntiles,nwords], IPRecord, zq fp32
    [n,k] from the encoder's dq)."""
    n, k = w.shape
    lut = tn.codebook_lut(codebook)
    cb_rms = tn.codebook_rms(codebook)
    rng = np.random.default_rng(seed)
    z, su, sv, in_s, out_s, scale = tn.ip_encode(w, cb_rms, rng)
    tiles = tn.matrix_to_tiles(z)
    bits, dq, _ = viterbi_tb(tiles, K, lut)
    packed = tn.pack_bits(bits, K)
    rec = tn.IPRecord(n, k, K, su.astype(np.float16), sv.astype(np.float16),
                      in_s.astype(np.float16), out_s.astype(np.float16), scale,
                      codebook=codebook)
    zq = tn.tiles_to_matrix(dq, n, k)
    return packed, rec, zq
