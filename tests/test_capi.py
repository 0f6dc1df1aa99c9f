"""The C-ABI library loads and exports every function include/trellis_amd.h declares;
host-side validation returns the documented status codes (no GPU compute here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "trellis_amd.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(trellis_[a-z_]+)\s*\(", src)))


def test_header_declares_the_binding_list(te):
    assert _declared() == sorted(te._capi.EXPORTED)


def test_library_exports_every_declared_symbol(te):
    lib = te.library()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.trellis_version().decode().startswith("trellis-amd")


def test_strerror_names_every_status(te):
    lib = te.library()
    for code in range(0, 18):
        assert lib.trellis_strerror(code).decode() not in ("", "unknown trellis status")
    assert lib.trellis_strerror(99).decode() == "unknown trellis status"


def _desc(te, **kw):
    d = dict(bits=16, su=16, sv=16, isc_scaled=16, osc=16, n_out=128, k_in=256, K=3, V=1,
             codebook=0, block_in=128, block_out=128, nwords=24)
    d.update(kw)
    return te._capi.TrellisDesc(**d)


@pytest.mark.parametrize("kw,status", [
    (dict(bits=None), 1), (dict(n_out=100), 2), (dict(k_in=0), 2), (dict(K=5, nwords=40), 4),
    (dict(V=3), 5), (dict(V=0), 5), (dict(codebook=3), 6), (dict(nwords=23), 7), (dict(block_in=64 + 32), 3),
    (dict(block_out=256), 3), (dict(bits=8), 8),
])
def test_validation_codes(te, kw, status):
    lib = te.library()
    n = ctypes.c_size_t(0)
    assert lib.trellis_workspace_bytes(ctypes.byref(_desc(te, **kw)), 1, ctypes.byref(n)) == status


def test_packed_linear_rejects_before_launch(te):
    lib = te.library()
    d = _desc(te)
    ok = ctypes.c_size_t(0)
    assert lib.trellis_workspace_bytes(ctypes.byref(d), 1, ctypes.byref(ok)) == 0
    # bad dtype, bad batch, missing workspace: all host-side checks
    assert lib.trellis_packed_linear(ctypes.byref(d), 16, 256, 1, 7, 16, 128, 0, None, 0, None) == 9
    assert lib.trellis_packed_linear(ctypes.byref(d), 16, 256, 0, 0, 16, 128, 0, None, 0, None) == 11
    if ok.value > 0:
        assert lib.trellis_packed_linear(ctypes.byref(d), 16, 256, 1, 0, 16, 128, 0, None, 0,
                                         None) == 10
    assert lib.trellis_decode_tiles(ctypes.byref(d), 100, 100, 16, None) == 12


def test_packed_linear_ex_flags(te):
    """Unknown flag bits are rejected on the host (TRELLIS_ERR_FLAGS); the workspace size
    covers every flag."""
    lib = te.library()
    d = _desc(te)
    assert lib.trellis_packed_linear_ex(ctypes.byref(d), 16, 256, 2, 0, 16, 128, 0, None, 0, 2,
                                        None) == 15
    assert lib.trellis_packed_linear_ex(ctypes.byref(d), 16, 256, 2, 0, 16, 128, 0, None, 0, 1,
                                        None) == 10
    arr = (ctypes.POINTER(te._capi.TrellisDesc) * 1)(ctypes.pointer(d))
    xp = (ctypes.c_void_p * 1)(16)
    ld = (ctypes.c_int64 * 1)(256)
    ldy = (ctypes.c_int64 * 1)(128)
    assert lib.trellis_packed_linear_group_ex(arr, 1, xp, ld, 2, 0, xp, ldy, 0, None, 0, -1,
                                              None) == 15
    assert te._capi.MMA_F16 == 1


def test_activation_range_limit(te):
    """A call whose activations span 2 GiB or more (batch x row stride x element size) is
    rejected on the host: the kernels address them through 32-bit byte ranges."""
    lib = te.library()
    d = _desc(te)
    arr = (ctypes.POINTER(te._capi.TrellisDesc) * 1)(ctypes.pointer(d))
    xp = (ctypes.c_void_p * 1)(16)
    ld = (ctypes.c_int64 * 1)(1 << 22)
    ldy = (ctypes.c_int64 * 1)(128)
    # 256 rows x 4M f32 elements = 4 GiB
    assert lib.trellis_packed_linear_group(arr, 1, xp, ld, 256, 0, xp, ldy, 0, None, 0, None) == 2


def test_embed_rows_rejects_before_launch(te):
    """trellis_embed_rows validates on the host: descriptor, token count, pointers, dtype
    and row stride (web/packed.js:137-146 has no error path)."""
    lib = te.library()
    d = _desc(te)
    assert lib.trellis_embed_rows(ctypes.byref(_desc(te, K=5, nwords=40)), 16, 1, 16, 256, 0,
                                  None) == 4
    assert lib.trellis_embed_rows(ctypes.byref(d), 16, -1, 16, 256, 0, None) == 11
    assert lib.trellis_embed_rows(ctypes.byref(d), 16, 0, None, 256, 0, None) == 0
    assert lib.trellis_embed_rows(ctypes.byref(d), None, 2, 16, 256, 0, None) == 1
    assert lib.trellis_embed_rows(ctypes.byref(d), 16, 2, None, 256, 0, None) == 1
    assert lib.trellis_embed_rows(ctypes.byref(d), 16, 2, 16, 256, 7, None) == 9
    assert lib.trellis_embed_rows(ctypes.byref(d), 16, 2, 16, 255, 0, None) == 8


def test_encode_tiles_rejects_before_launch(te):
    """trellis_encode_tiles validates K, codebook, pointers and workspace on the host."""
    lib = te.library()
    n = ctypes.c_size_t(0)
    assert lib.trellis_encode_workspace_bytes(5, 10, ctypes.byref(n)) == 4
    assert lib.trellis_encode_workspace_bytes(3, 10, None) == 1
    assert lib.trellis_encode_tiles(16, 10, 1, 0, 16, None, 256, 1 << 30, None) == 4
    assert lib.trellis_encode_tiles(16, 10, 3, 7, 16, None, 256, 1 << 30, None) == 6
    assert lib.trellis_encode_tiles(None, 10, 3, 0, 16, None, 256, 1 << 30, None) == 1
    assert lib.trellis_encode_tiles(16, 0, 3, 0, None, None, None, 0, None) == 0
    assert lib.trellis_encode_tiles(16, 10, 3, 0, 16, None, None, 0, None) == 10
    assert lib.trellis_encode_tiles(16, 10, 3, 0, 16, None, 256 + 8, 1 << 30, None) == 8


def test_workspace_plan_is_bounded(te):
    """Workspace for the largest benchmark shape stays small (partials of 128-row blocks)."""
    lib = te.library()
    d = _desc(te, n_out=12288, k_in=4096)
    n = ctypes.c_size_t(0)
    for b in (1, 2, 8, 64):
        assert lib.trellis_workspace_bytes(ctypes.byref(d), b, ctypes.byref(n)) == 0
        assert n.value < 64 << 20


def test_packed_linear_lives_on_a_gpu(te):
    """A packed linear on a host device is refused at construction: the kernels would
    dereference its pointers on the GPU."""
    from oracle import trellis_np as tn
    bits, rec = tn.synthetic_record(64, 128, 3, seed=1)
    r = te.PackedRecord(rec.n, rec.k, rec.K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                        float(rec.scale), codebook=rec.codebook, V=rec.V)
    with pytest.raises(ValueError):
        te.PackedLinear(r, device="cpu")


def test_noalloc_rejects_before_launch(te):
    """trellis_packed_linear_group_noalloc validates like the _ex entry point, and refuses
    a plan larger than its static scratch (TRELLIS_ERR_SCRATCH) before touching the GPU."""
    lib = te.library()
    d = _desc(te)
    arr = (ctypes.POINTER(te._capi.TrellisDesc) * 1)(ctypes.pointer(d))
    xp = (ctypes.c_void_p * 1)(16)
    ld = (ctypes.c_int64 * 1)(256)
    ldy = (ctypes.c_int64 * 1)(128)
    f = lib.trellis_packed_linear_group_noalloc
    assert f(arr, 1, xp, ld, 2, 0, xp, ldy, 0, 2, None) == 15          # unknown flag
    assert f(arr, 1, xp, ld, 0, 0, xp, ldy, 0, 0, None) == 11          # batch 0
    assert f(arr, 1, xp, ld, 2, 7, xp, ldy, 0, 0, None) == 9           # dtype
    assert f(arr, 0, xp, ld, 2, 0, xp, ldy, 0, 0, None) == 1           # empty group
    big = _desc(te, n_out=12288, k_in=4096)
    barr = (ctypes.POINTER(te._capi.TrellisDesc) * 1)(ctypes.pointer(big))
    bld = (ctypes.c_int64 * 1)(4096)
    bldy = (ctypes.c_int64 * 1)(12288)
    n = ctypes.c_size_t(0)
    assert lib.trellis_workspace_bytes(ctypes.byref(big), 4096, ctypes.byref(n)) == 0
    assert n.value > te._capi.NOALLOC_SCRATCH_BYTES
    assert f(barr, 1, xp, bld, 4096, 1, xp, bldy, 0, 0, None) == 16
    assert "scratch" in lib.trellis_strerror(16).decode()
