"""torch.nn adapters (TrellisLinear, TrellisGroupLinear, swap_linears) on the GPU: a small
model whose nn.Linear weights are the oracle's W_hat of packed records, swapped for the
packed linears, against the same model in float64 on the CPU."""
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


def _record(n, k, seed, cb="mcg"):
    bits, rec = tn.synthetic_record(n, k, 3, seed=seed, codebook=cb)
    W = tn.w_hat_from_record(bits, rec)
    return bits, rec, W


def _packed_record(te, bits, rec):
    return te.PackedRecord(rec.n, rec.k, rec.K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                           float(rec.scale), codebook=rec.codebook, V=rec.V)


def _rel(got, want):
    return tn.rel_err(got.detach().float().cpu().numpy(), want)


@pytest.mark.parametrize("shape", [(1, 1), (1, 3), (2, 7), (4, 32)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_swap_linears_matches_dense(te, gpu_device, shape, dtype):
    _say(f"[modules] shape={shape} dtype={dtype}")
    b0, r0, W0 = _record(256, 512, 1)
    b1, r1, W1 = _record(384, 256, 2, "3inst")
    bias0 = np.random.default_rng(3).standard_normal(256).astype(np.float32) * 0.1
    model = torch.nn.Sequential(torch.nn.Linear(512, 256, bias=True), torch.nn.ReLU(),
                                torch.nn.Linear(256, 384, bias=False))
    with torch.no_grad():
        model[0].weight.copy_(torch.from_numpy(W0.astype(np.float32)))
        model[0].bias.copy_(torch.from_numpy(bias0))
        model[2].weight.copy_(torch.from_numpy(W1.astype(np.float32)))
    model = model.to(gpu_device)
    done = te.swap_linears(model, {"0.weight": _packed_record(te, b0, r0),
                                   "2.weight": _packed_record(te, b1, r1)},
                           device=gpu_device, strict=True)
    assert done == ["0", "2"]
    assert isinstance(model[0], te.TrellisLinear) and isinstance(model[2], te.TrellisLinear)
    x = np.random.default_rng(sum(shape)).standard_normal((*shape, 512)).astype(np.float32)
    xt = torch.from_numpy(x).to(gpu_device).to(dtype)
    with torch.no_grad():
        y = model(xt)
    assert y.shape == (*shape, 384) and y.dtype == dtype
    x64 = xt.float().cpu().numpy().astype(np.float64)
    h = np.maximum(x64 @ W0.T + bias0, 0.0)
    want = h @ W1.T
    tol = {torch.float32: TOL, torch.float16: 2e-3, torch.bfloat16: 1.5e-2}[dtype]
    assert _rel(y, want) < tol


def test_group_module_matches_singles(te, gpu_device):
    recs = [_record(n, 1024, 10 + i) for i, n in enumerate((512, 128, 128))]
    lins = [te.PackedLinear(_packed_record(te, b, r), device=gpu_device) for b, r, _ in recs]
    grp = te.TrellisGroupLinear(lins)
    singles = [te.TrellisLinear(l) for l in lins]
    for shape in ((1, 1), (3, 1), (2, 40)):
        x = torch.randn(*shape, 1024, device=gpu_device, dtype=torch.float16)
        with torch.no_grad():
            ys = grp(x)
            for y, s, (_, _, W) in zip(ys, singles, recs):
                assert y.shape == (*shape, W.shape[0])
                ref = s(x)
                # group and single launches may split k differently: fp32 order only
                assert (y.float() - ref.float()).abs().max().item() <= \
                    1e-3 * ref.float().abs().max().item()
                assert _rel(y, x.float().cpu().numpy().astype(np.float64) @ W.T) < 2e-3


def test_swap_linears_checks(te, gpu_device):
    b0, r0, _ = _record(256, 512, 1)
    model = torch.nn.Sequential(torch.nn.Linear(512, 256), torch.nn.Linear(256, 128))
    with pytest.raises(ValueError):
        te.swap_linears(model, {"1.weight": _packed_record(te, b0, r0)}, device=gpu_device)
    model = torch.nn.Sequential(torch.nn.Linear(512, 256))
    with pytest.raises(KeyError):
        te.swap_linears(model, {"0.weight": _packed_record(te, b0, r0),
                                "9.weight": _packed_record(te, b0, r0)},
                        device=gpu_device, strict=True)
    with pytest.raises(ValueError):
        te.PackedLinear(_packed_record(te, b0, r0), device="cpu")
