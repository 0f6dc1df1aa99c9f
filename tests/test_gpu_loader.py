"""End-to-end loader: an export directory as the 8B exporter lays it out (per-layer shard
files, `<module>.weight` names, one merged manifest, dense tensors beside the packed ones:
scripts/export_packed_8b.py:65-81, 134-143, 271-276) read by load_packed (loadPacked /
loadPackedSharded, web/packed.js:14-114) straight onto the GPU, and every loaded linear,
and a PackedGroup of a layer's q/k/v, checked against the float64 oracle built from the
records that were written (metric of scripts/validate_packed_linear.py:66-69)."""
import json
import os
import sys

import numpy as np
import pytest
import torch

from oracle import trellis_np as tn

pytestmark = pytest.mark.gpu
TOL = 1e-3

# a small decoder with the 8B model's proportions: hidden 256, GQA kv 64, MLP 768
HID, KV, MLP = 256, 64, 768
LAYER = {"self_attn.q_proj": (HID, HID), "self_attn.k_proj": (KV, HID),
         "self_attn.v_proj": (KV, HID), "self_attn.o_proj": (HID, HID),
         "mlp.gate_proj": (MLP, HID), "mlp.up_proj": (MLP, HID), "mlp.down_proj": (HID, MLP)}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _records(te, layer, K, cb):
    out, oracle = {}, {}
    for i, (mod, (n, k)) in enumerate(LAYER.items()):
        name = f"model.layers.{layer}.{mod}.weight"
        bits, rec = tn.synthetic_record(n, k, K, seed=1000 * layer + i, codebook=cb)
        out[name] = te.PackedRecord(n, k, K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                                    float(rec.scale), codebook=cb)
        oracle[name] = (bits, rec)
    return out, oracle


def test_sharded_export_loads_onto_gpu(te, gpu_device, tmp_path):
    d = str(tmp_path / "model")
    rec0, or0 = _records(te, 0, 3, "mcg")
    rec1, or1 = _records(te, 1, 2, "3inst")
    rng = np.random.default_rng(3)
    norm = rng.standard_normal(HID).astype(np.float16)
    emb = rng.standard_normal((32, HID)).astype(np.float16)
    cfg = {"hidden_size": HID, "num_hidden_layers": 2, "intermediate_size": MLP}
    te.write_packed(d, rec0, dense={"model.layers.0.input_layernorm.weight": norm},
                    config=cfg, shard="layer_00.bin")
    te.write_packed(d, rec1, shard="layer_01.bin", append=True)
    te.write_packed(d, {}, dense={"model.embed_tokens.weight": emb}, shard="emb.bin", append=True)
    man = json.load(open(os.path.join(d, "manifest.json")))
    assert {m.get("shard") for m in man.values()} == {"layer_00.bin", "layer_01.bin", "emb.bin"}
    assert not os.path.exists(os.path.join(d, "weights.bin"))

    _say("[loader] load_packed")
    loaded = te.load_packed(d, device=gpu_device)
    assert loaded["cfg"] == cfg
    T = loaded["tensors"]
    assert torch.equal(T["model.layers.0.input_layernorm.weight"].cpu(), torch.from_numpy(norm))
    assert torch.equal(T["model.embed_tokens.weight"].cpu(), torch.from_numpy(emb))
    oracle = {**or0, **or1}
    assert set(oracle) <= set(T)
    for name, (bits, rec) in oracle.items():
        lin = T[name]
        assert isinstance(lin, te.PackedLinear) and lin.device == gpu_device
        assert (lin.n_out, lin.k_in, lin.K, lin.codebook) == (rec.n, rec.k, rec.K, rec.codebook)
        # the uploaded words decode bit-exactly as the written ones
        got = lin.decode_tiles(0, 8).cpu().numpy()
        want = tn.decode_packed_tiles(bits[:8], rec.K, rec.codebook)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
        for batch in (1, 5):
            _say(f"[loader] {name} batch={batch}")
            x = rng.standard_normal((batch, rec.k)).astype(np.float16)
            y = lin(torch.from_numpy(x).to(gpu_device)).cpu().numpy()
            assert tn.rel_err(y, tn.packed_linear_ref(bits, rec, x)) < TOL, (name, batch)

    # the loaded q/k/v of each layer as one launch
    for layer in (0, 1):
        names = [f"model.layers.{layer}.self_attn.{p}_proj.weight" for p in "qkv"]
        grp = te.PackedGroup([T[n] for n in names])
        for batch in (1, 3, 20):
            _say(f"[loader] layer {layer} q/k/v group batch={batch}")
            x = rng.standard_normal((batch, HID)).astype(np.float16)
            xt = torch.from_numpy(x).to(gpu_device)
            ys = grp([xt] * 3)
            for n, y in zip(names, ys):
                bits, rec = oracle[n]
                assert tn.rel_err(y.cpu().numpy(), tn.packed_linear_ref(bits, rec, x)) < TOL
                single = T[n](xt)
                assert (single - y).abs().max().item() <= 1e-5 * y.abs().max().item()
