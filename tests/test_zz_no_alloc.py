"""The no-allocation entry point (trellis_packed_linear_group_noalloc) through the C ABI:
its outputs equal those of trellis_packed_linear_group_ex (the same plans and kernels, with
the workspace taken from the library's static scratch instead of the caller's), bit for bit,
on consecutive calls whose second input is smaller, and on a call after another group has
left its own data in the shared scratch (the split-K counters must be cleared). Also checked
against the float64 oracle at the 1e-3 metric of validate_packed_linear.py:66-69."""
import ctypes
import sys

import numpy as np
import pytest
import torch

from oracle import trellis_np as tn

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _group(te, shapes, seed, device):
    cases = []
    for i, (n, k) in enumerate(shapes):
        bits, rec = tn.synthetic_record(n, k, 3, seed=seed + i)
        r = te.PackedRecord(rec.n, rec.k, rec.K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                            float(rec.scale), codebook=rec.codebook, V=rec.V)
        cases.append((bits, rec, te.PackedLinear(r, device=device)))
    return cases, te.PackedGroup([c[2] for c in cases])


def _noalloc(te, grp, xs, ys):
    """One trellis_packed_linear_group_noalloc call on the current stream."""
    lib = te.library()
    n = len(xs)
    xp = (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs])
    yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    ldx = (ctypes.c_int64 * n)(*[x.stride(0) for x in xs])
    ldy = (ctypes.c_int64 * n)(*[y.stride(0) for y in ys])
    stream = torch.cuda.current_stream().cuda_stream
    st = lib.trellis_packed_linear_group_noalloc(
        grp._dptrs, n, xp, ldx, xs[0].shape[0], te._capi.DT_F16, yp, ldy, te._capi.DT_F32, 0,
        ctypes.c_void_p(stream))
    te._capi.check(st)


def _check(te, cases, grp, batch, rng, device):
    xs = [torch.from_numpy(rng.standard_normal((batch, rec.k)).astype(np.float16)).to(device)
          for _, rec, _ in cases]
    want = grp(xs)                                  # the existing entry point, own workspace
    got = [torch.full((batch, rec.n), float("nan"), device=device) for _, rec, _ in cases]
    _noalloc(te, grp, xs, got)
    torch.cuda.synchronize()
    for (bits, rec, _), x, w, g in zip(cases, xs, want, got):
        assert torch.equal(g, w), (rec.n, rec.k, batch)
        ref = tn.packed_linear_ref(bits, rec, x.cpu().numpy())
        assert tn.rel_err(g.cpu().numpy(), ref) < TOL


def test_noalloc_matches_group_ex(te, gpu_device):
    rng = np.random.default_rng(2024)
    # split-K at batch 1 (tickets in the scratch header), the batched path at 200 and 64
    cases, grp = _group(te, [(1024, 2048), (256, 2048), (384, 2048)], 500, gpu_device)
    for batch in (200, 64, 3, 1):
        _say(f"[noalloc] group A batch={batch}")
        _check(te, cases, grp, batch, rng, gpu_device)
    # another group's call after group A's batch-64 data filled the scratch: its ticket
    # header (laid out by its own shapes) is cleared before its launches
    cases_b, grp_b = _group(te, [(640, 1536), (128, 3072)], 600, gpu_device)
    for batch in (40, 2, 1):
        _say(f"[noalloc] group B batch={batch}")
        _check(te, cases_b, grp_b, batch, rng, gpu_device)
    _say("[noalloc] group A batch=1 again")
    _check(te, cases, grp, 1, rng, gpu_device)


def test_noalloc_refuses_a_plan_beyond_the_scratch(te, gpu_device):
    """A plan whose workspace exceeds the static scratch is refused with TRELLIS_ERR_SCRATCH
    before anything is launched, and the next call still works."""
    cases, grp = _group(te, [(512, 1024)], 700, gpu_device)
    big = 9000                       # folded activations alone: 9000 x 1024 x 4 B > 32 MiB
    x = torch.zeros((big, 1024), dtype=torch.float16, device=gpu_device)
    y = torch.zeros((big, 512), dtype=torch.float32, device=gpu_device)
    assert grp.workspace_bytes(big) > te._capi.NOALLOC_SCRATCH_BYTES
    with pytest.raises(te.TrellisError) as e:
        _noalloc(te, grp, [x], [y])
    assert e.value.status == 16
    assert torch.count_nonzero(y).item() == 0
    _check(te, cases, grp, 1, np.random.default_rng(5), gpu_device)


@pytest.mark.parametrize("batch", [1, 64])
def test_noalloc_inside_a_captured_graph(te, gpu_device, batch):
    """noalloc calls captured in a HIP graph (after an eager first call on the device, which
    looks up the scratch address outside the capture): at batch 1 the graph holds the
    ticket-clearing kernel and the split-K decode-GEMV, at 64 the x fold, the batched kernel
    and its split-K fold. Every replay, with new inputs copied in and eager noalloc calls on
    the same scratch between replays, equals the eager call bit for bit."""
    _say(f"[noalloc] graph capture batch={batch}")
    cases, grp = _group(te, [(1024, 2048), (256, 2048), (384, 2048)], 800, gpu_device)
    rng = np.random.default_rng(900 + batch)
    xs = [torch.from_numpy(rng.standard_normal((batch, rec.k)).astype(np.float16)).to(gpu_device)
          for _, rec, _ in cases]
    ys = [torch.empty((batch, rec.n), device=gpu_device) for _, rec, _ in cases]
    _noalloc(te, grp, xs, ys)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=gpu_device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _noalloc(te, grp, xs, ys)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        _noalloc(te, grp, xs, ys)
    torch.cuda.synchronize()
    for rep in range(4):
        xin = [torch.from_numpy(rng.standard_normal((batch, rec.k)).astype(np.float16)).to(gpu_device)
               for _, rec, _ in cases]
        for x, v in zip(xs, xin):
            x.copy_(v)
        g.replay()
        torch.cuda.synchronize()
        got = [y.clone() for y in ys]
        want = [torch.empty_like(y) for y in ys]
        _noalloc(te, grp, xin, want)
        torch.cuda.synchronize()
        for (bits, rec, _), a, b, v in zip(cases, got, want, xin):
            assert torch.equal(a, b), f"replay {rep}"
            assert tn.rel_err(a.cpu().numpy(), tn.packed_linear_ref(bits, rec, v.cpu().numpy())) < TOL
