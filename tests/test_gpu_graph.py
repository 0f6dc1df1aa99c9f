"""The packed linear inside captured HIP graphs (what bench.py times): every replay, with new
inputs copied in and eager calls of the same linears between the replays, must equal the
eager call on the same inputs bit for bit. Covers the batch-1 split-K tickets (reset by the
kernels, no memset in the graph), the decode-GEMV with 4 and 16 rows in its MFMA columns
(batch 3, 12; split k, one ticket per workgroup), the batched path with its x-fold and
split-K fold launches (at 64 and 200 columns, the latter also forced to 128-column blocks),
and the fp16-weight mode."""
import sys

import numpy as np
import pytest
import torch

from oracle import trellis_np as tn

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_linear(te, bits, rec, device):
    r = te.PackedRecord(rec.n, rec.k, rec.K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                        float(rec.scale), codebook=rec.codebook, V=rec.V)
    return te.PackedLinear(r, device=device)


@pytest.mark.parametrize("batch,mma_f16,nc", [(1, False, None), (3, False, None), (12, False, None),
                                              (64, False, None), (64, True, None),
                                              (200, False, None), (200, False, "8")])
def test_graph_replays_match_eager(te, gpu_device, monkeypatch, batch, mma_f16, nc):
    """nc forces the batched kernel's column-block width (8 chunks: the exact mode's
    two-wave 128-column kernel)."""
    _say(f"[graph] batch={batch} mma_f16={mma_f16} nc={nc}")
    if nc is not None:
        monkeypatch.setenv("TRELLIS_BGEMM_NC", nc)
    shapes = [(1024, 2048), (256, 2048), (512, 2048)]      # split-K plans at every batch
    lins = []
    for i, (n, k) in enumerate(shapes):
        bits, rec = tn.synthetic_record(n, k, 3, seed=40 + i)
        lins.append(make_linear(te, bits, rec, gpu_device))
    grp = te.PackedGroup(lins)
    single = lins[0]
    rng = np.random.default_rng(batch)
    x = torch.from_numpy(rng.standard_normal((batch, 2048)).astype(np.float16)).to(gpu_device)
    ys = [torch.empty((batch, n), device=gpu_device) for n, _ in shapes]
    y1 = torch.empty((batch, shapes[0][0]), device=gpu_device)

    def step():
        grp([x] * 3, ys, mma_f16=mma_f16)
        single.forward(x, out=y1, mma_f16=mma_f16)

    step()                                   # workspaces allocated before the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=gpu_device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for rep in range(4):
        xin = torch.from_numpy(rng.standard_normal((batch, 2048)).astype(np.float16)).to(gpu_device)
        x.copy_(xin)
        g.replay()
        torch.cuda.synchronize()
        got = [y.clone() for y in ys] + [y1.clone()]
        # eager calls on the same input (other outputs, same workspaces) between replays
        want = grp([xin] * 3, mma_f16=mma_f16) + [single(xin, mma_f16=mma_f16)]
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), f"replay {rep}"


def test_graph_survives_workspace_growth(te, gpu_device):
    """A graph captured at batch 1, then an eager call at a larger batch that needs a larger
    workspace: the linear swaps in a bigger workspace but keeps the one the graph holds
    alive, so every later replay still writes its split-K partials and counters into
    memory no other tensor owns, and still equals the eager batch-1 call."""
    _say("[graph] workspace growth after capture")
    bits, rec = tn.synthetic_record(1024, 2048, 3, seed=77)
    lin = make_linear(te, bits, rec, gpu_device)
    rng = np.random.default_rng(7)
    x = torch.from_numpy(rng.standard_normal((1, 2048)).astype(np.float16)).to(gpu_device)
    y = torch.empty((1, 1024), device=gpu_device)
    lin.forward(x, out=y)
    torch.cuda.synchronize()
    ws_captured = lin._ws
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=gpu_device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        lin.forward(x, out=y)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        lin.forward(x, out=y)
    torch.cuda.synchronize()
    xb = torch.from_numpy(rng.standard_normal((300, 2048)).astype(np.float16)).to(gpu_device)
    yb = lin(xb)                                   # grows the workspace
    assert lin._ws is not ws_captured and lin._ws.numel() > ws_captured.numel()
    assert any(w is ws_captured for w in lin._ws_retired)
    # churn the caching allocator: freed blocks would be handed out here
    junk = [torch.full((ws_captured.numel(),), 255, dtype=torch.uint8, device=gpu_device)
            for _ in range(4)]
    for rep in range(3):
        xin = torch.from_numpy(rng.standard_normal((1, 2048)).astype(np.float16)).to(gpu_device)
        x.copy_(xin)
        g.replay()
        torch.cuda.synchronize()
        got = y.clone()
        want = lin(xin)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}"
        assert tn.rel_err(got.cpu().numpy(), tn.packed_linear_ref(bits, rec, xin.cpu().numpy())) < 1e-3
    for j in junk:
        assert torch.all(j == 255)
    want_b = tn.packed_linear_ref(bits, rec, xb.cpu().numpy())
    assert tn.rel_err(yb.cpu().numpy(), want_b) < 1e-3
