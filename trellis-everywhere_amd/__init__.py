"""trellis-everywhere_amd: MI355X (gfx950) trellis packed-linear decode-matmul.

A drop-in for the reference's packed linear (web/packed.js PackedOps.linear, Python
mirror scripts/run_packed_headless.py:87-99): y = restore(decode(bits)) @ x over the
reference's packed K-bit trellis format (scripts/export_packed.py).

The directory name contains a hyphen, so import it with importlib:
    te = importlib.import_module("trellis-everywhere_amd")
"""
from . import _capi
from ._capi import TrellisError, TrellisLibraryMissing
from .format import PackedRecord, fit_block, read_packed, write_packed

__all__ = ["PackedRecord", "read_packed", "write_packed", "fit_block", "TrellisError",
           "TrellisLibraryMissing", "PackedLinear", "PackedGroup", "PackedOps", "load_packed",
           "encode_tiles", "library", "TrellisLinear", "TrellisGroupLinear", "swap_linears"]


def library():
    """The loaded libtrellis_amd.so (raises TrellisLibraryMissing when not built)."""
    return _capi.load()


def __getattr__(name):
    # torch-dependent pieces load lazily so the format tools import without torch
    if name in ("PackedLinear", "PackedGroup", "PackedOps", "load_packed", "encode_tiles"):
        from . import packed_linear
        return getattr(packed_linear, name)
    if name in ("TrellisLinear", "TrellisGroupLinear", "swap_linears"):
        from . import modules
        return getattr(modules, name)
    raise AttributeError(name)
