"""ctypes binding of include/trellis_amd.h (libtrellis_amd.so, built for gfx950).

The library is mandatory: importing the package works without it (so CPU-only tooling
can read manifests), but every compute call raises TrellisLibraryMissing when the .so
is absent. There is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# TRELLIS_AMD_LIB points the binding at another build of the same library
LIB_PATH = os.environ.get("TRELLIS_AMD_LIB") or os.path.join(HERE, "libtrellis_amd.so")

# enum trellis_codebook / trellis_dtype (include/trellis_amd.h)
CB_IDS = {"mcg": 0, "3inst": 1, "1mad": 2}
DT_F32, DT_F16 = 0, 1

STATUS_NAMES = {
    0: "TRELLIS_OK", 1: "TRELLIS_ERR_NULL", 2: "TRELLIS_ERR_SHAPE", 3: "TRELLIS_ERR_BLOCK",
    4: "TRELLIS_ERR_K", 5: "TRELLIS_ERR_V", 6: "TRELLIS_ERR_CODEBOOK", 7: "TRELLIS_ERR_NWORDS",
    8: "TRELLIS_ERR_ALIGN", 9: "TRELLIS_ERR_DTYPE", 10: "TRELLIS_ERR_WORKSPACE",
    11: "TRELLIS_ERR_BATCH", 12: "TRELLIS_ERR_RANGE", 13: "TRELLIS_ERR_LAUNCH",
    14: "TRELLIS_ERR_GROUP", 15: "TRELLIS_ERR_FLAGS", 16: "TRELLIS_ERR_SCRATCH",
    17: "TRELLIS_ERR_CAPTURE",
}

# TRELLIS_NOALLOC_SCRATCH_BYTES: the static workspace of trellis_packed_linear_group_noalloc
NOALLOC_SCRATCH_BYTES = 32 << 20

# enum trellis_flags
MMA_F16 = 1
ERR_WORKSPACE = 10   # TRELLIS_ERR_WORKSPACE: returned before anything is launched

# every symbol include/trellis_amd.h declares
EXPORTED = ("trellis_workspace_bytes", "trellis_packed_linear", "trellis_decode_tiles",
            "trellis_strerror", "trellis_version", "trellis_workspace_bytes_group",
            "trellis_packed_linear_group", "trellis_embed_rows",
            "trellis_encode_workspace_bytes", "trellis_encode_tiles",
            "trellis_packed_linear_ex", "trellis_packed_linear_group_ex",
            "trellis_packed_linear_group_noalloc")


class TrellisLibraryMissing(RuntimeError):
    pass


class TrellisError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


class TrellisDesc(ctypes.Structure):
    """struct trellis_desc (include/trellis_amd.h)."""
    _fields_ = [
        ("bits", ctypes.c_void_p),
        ("su", ctypes.c_void_p),
        ("sv", ctypes.c_void_p),
        ("isc_scaled", ctypes.c_void_p),
        ("osc", ctypes.c_void_p),
        ("n_out", ctypes.c_int32),
        ("k_in", ctypes.c_int32),
        ("K", ctypes.c_int32),
        ("V", ctypes.c_int32),
        ("codebook", ctypes.c_int32),
        ("block_in", ctypes.c_int32),
        ("block_out", ctypes.c_int32),
        ("nwords", ctypes.c_int32),
    ]


_lib = None


def load(path: str | None = None):
    """Load libtrellis_amd.so and declare the C signatures."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise TrellisLibraryMissing(
            f"{p} is missing: build it with `python trellis-everywhere_amd/build.py` "
            "(hipcc, gfx950). There is no CPU fallback.")
    lib = ctypes.CDLL(p)
    D = ctypes.POINTER(TrellisDesc)
    lib.trellis_workspace_bytes.argtypes = [D, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]
    lib.trellis_workspace_bytes.restype = ctypes.c_int
    lib.trellis_packed_linear.argtypes = [D, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                          ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_void_p]
    lib.trellis_packed_linear.restype = ctypes.c_int
    lib.trellis_packed_linear_ex.argtypes = [D, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                             ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                             ctypes.c_int, ctypes.c_void_p]
    lib.trellis_packed_linear_ex.restype = ctypes.c_int
    PP = ctypes.POINTER(ctypes.c_void_p)
    I64P = ctypes.POINTER(ctypes.c_int64)
    lib.trellis_workspace_bytes_group.argtypes = [ctypes.POINTER(D), ctypes.c_int, ctypes.c_int,
                                                  ctypes.POINTER(ctypes.c_size_t)]
    lib.trellis_workspace_bytes_group.restype = ctypes.c_int
    lib.trellis_packed_linear_group.argtypes = [ctypes.POINTER(D), ctypes.c_int, PP, I64P,
                                                ctypes.c_int, ctypes.c_int, PP, I64P, ctypes.c_int,
                                                ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.trellis_packed_linear_group.restype = ctypes.c_int
    lib.trellis_packed_linear_group_ex.argtypes = [ctypes.POINTER(D), ctypes.c_int, PP, I64P,
                                                   ctypes.c_int, ctypes.c_int, PP, I64P,
                                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                                   ctypes.c_int, ctypes.c_void_p]
    lib.trellis_packed_linear_group_ex.restype = ctypes.c_int
    lib.trellis_packed_linear_group_noalloc.argtypes = [ctypes.POINTER(D), ctypes.c_int, PP, I64P,
                                                        ctypes.c_int, ctypes.c_int, PP, I64P,
                                                        ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.trellis_packed_linear_group_noalloc.restype = ctypes.c_int
    lib.trellis_decode_tiles.argtypes = [D, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                         ctypes.c_void_p]
    lib.trellis_decode_tiles.restype = ctypes.c_int
    lib.trellis_embed_rows.argtypes = [D, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    lib.trellis_embed_rows.restype = ctypes.c_int
    lib.trellis_encode_workspace_bytes.argtypes = [ctypes.c_int, ctypes.c_uint32,
                                                   ctypes.POINTER(ctypes.c_size_t)]
    lib.trellis_encode_workspace_bytes.restype = ctypes.c_int
    lib.trellis_encode_tiles.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.trellis_encode_tiles.restype = ctypes.c_int
    lib.trellis_strerror.argtypes = [ctypes.c_int]
    lib.trellis_strerror.restype = ctypes.c_char_p
    lib.trellis_version.argtypes = []
    lib.trellis_version.restype = ctypes.c_char_p
    if path is None:
        _lib = lib
    return lib


def check(status: int) -> None:
    if status != 0:
        msg = load().trellis_strerror(status).decode()
        raise TrellisError(status, msg)
