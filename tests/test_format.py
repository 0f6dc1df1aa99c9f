"""Packed format writer/reader (trellis-everywhere_amd/format.py; reference
scripts/export_packed.py:45-63, export_packed_8b.py:65-81, web/packed.js:14-114)."""
import json
import os

import numpy as np

from oracle import trellis_np as tn


def _rec(te, n, k, K, seed, cb="mcg"):
    bits, r = tn.synthetic_record(n, k, K, seed, codebook=cb)
    return te.PackedRecord(n, k, K, bits, r.su, r.sv, r.isc, r.osc, float(r.scale), codebook=cb)


def test_roundtrip_single_blob(te, tmp_path):
    recs = {"model.layers.0.mlp.up_proj": _rec(te, 64, 32, 3, 1),
            "model.layers.0.mlp.down_proj": _rec(te, 32, 64, 3, 2, cb="3inst")}
    dense = {"model.norm.weight": np.ones(32, np.float16)}
    te.write_packed(str(tmp_path), recs, dense, config={"K": 3})
    man = json.load(open(tmp_path / "manifest.json"))
    m = man["model.layers.0.mlp.up_proj"]
    # manifest keys of export_packed.py:62-63
    assert m == {"quant": True, "n_out": 64, "k_in": 32, "K": 3, "block": 32,
                 "tiles_out": 4, "tiles_in": 2}
    assert man["model.layers.0.mlp.up_proj.bits"]["dtype"] == "u32"
    assert man["model.layers.0.mlp.up_proj.bits"]["shape"] == [8, 24]
    assert man["model.layers.0.mlp.up_proj.scale"]["dtype"] == "f32"
    assert man["model.layers.0.mlp.down_proj"]["codebook"] == "3inst"
    got, gdense, cfg = te.read_packed(str(tmp_path))
    assert cfg == {"K": 3}
    for name, r in recs.items():
        g = got[name]
        assert np.array_equal(g.bits, r.bits) and g.codebook == r.codebook
        for f in ("su", "sv", "isc", "osc"):
            assert np.array_equal(getattr(g, f), getattr(r, f))
        assert np.float32(g.scale) == np.float32(r.scale)
    assert np.array_equal(gdense["model.norm.weight"], dense["model.norm.weight"])


def test_blob_bytes_match_reference_layout(te, tmp_path):
    """Offsets are consecutive in put() order: bits, su, sv, isc, osc, scale."""
    r = _rec(te, 32, 32, 3, 3)
    te.write_packed(str(tmp_path), {"l": r})
    man = json.load(open(tmp_path / "manifest.json"))
    blob = open(tmp_path / "weights.bin", "rb").read()
    off = 0
    for key, nbytes in (("bits", r.bits.nbytes), ("su", 64), ("sv", 64), ("isc", 64),
                        ("osc", 64), ("scale", 4)):
        assert man[f"l.{key}"]["offset"] == off
        off += nbytes
    assert len(blob) == off
    assert blob[:r.bits.nbytes] == r.bits.astype("<u4").tobytes()


def test_sharded_manifest(te, tmp_path):
    r = _rec(te, 32, 48, 2, 4)
    te.write_packed(str(tmp_path), {"model.layers.3.self_attn.q_proj.weight": r},
                    shard="layer_03.bin")
    man = json.load(open(tmp_path / "manifest.json"))
    assert all(m["shard"] == "layer_03.bin" for m in man.values())
    assert not os.path.exists(tmp_path / "weights.bin")
    got, _, _ = te.read_packed(str(tmp_path))
    assert np.array_equal(got["model.layers.3.self_attn.q_proj.weight"].bits, r.bits)


def test_v2_roundtrip_and_default(te, tmp_path):
    """The V extension key is written only for V != 1 and read back; absent means V=1."""
    bits, r = tn.synthetic_record(32, 64, 3, 5, V=2)
    rec2 = te.PackedRecord(32, 64, 3, bits, r.su, r.sv, r.isc, r.osc, float(r.scale), V=2)
    rec1 = _rec(te, 32, 64, 3, 6)
    te.write_packed(str(tmp_path), {"a": rec2, "b": rec1})
    man = json.load(open(tmp_path / "manifest.json"))
    assert man["a"]["V"] == 2 and "V" not in man["b"]
    got, _, _ = te.read_packed(str(tmp_path))
    assert got["a"].V == 2 and got["b"].V == 1
    assert np.array_equal(got["a"].bits, bits)


def test_validate_rejects_bad_v(te):
    import pytest
    bits, r = tn.synthetic_record(32, 64, 3, 5)
    rec = te.PackedRecord(32, 64, 3, bits, r.su, r.sv, r.isc, r.osc, float(r.scale), V=3)
    with pytest.raises(ValueError):
        rec.validate()


def test_manifest_block_other_than_fit_is_rejected(te, tmp_path):
    """The exporters write block = fit(k_in, 128) (export_packed.py:62) and this reader
    restores with that block; a manifest naming another in-dim block is refused rather
    than loaded into a linear that would restore its weights wrongly."""
    import pytest
    r = _rec(te, 32, 96, 3, 7)          # fit(96, 128) = 32
    te.write_packed(str(tmp_path), {"l": r})
    man = json.load(open(tmp_path / "manifest.json"))
    assert man["l"]["block"] == 32
    te.read_packed(str(tmp_path))        # the exporter's own value loads
    man["l"]["block"] = 16
    json.dump(man, open(tmp_path / "manifest.json", "w"))
    with pytest.raises(ValueError, match="block"):
        te.read_packed(str(tmp_path))
    del man["l"]["block"]                # absent: the exporter's value is implied
    json.dump(man, open(tmp_path / "manifest.json", "w"))
    got, _, _ = te.read_packed(str(tmp_path))
    assert np.array_equal(got["l"].bits, r.bits)


def test_append_merges_shards_into_one_manifest(te, tmp_path):
    """Shards written one call at a time join one manifest (export_packed_8b.py:271-276
    merges its per-shard fragments); every entry keeps its own shard's offsets; a shard
    name already in the manifest is refused."""
    import pytest
    a, b = _rec(te, 32, 48, 3, 21), _rec(te, 64, 32, 2, 22)
    te.write_packed(str(tmp_path), {"l0.q.weight": a}, shard="layer_00.bin")
    te.write_packed(str(tmp_path), {"l1.q.weight": b}, dense={"norm": np.ones(8, np.float16)},
                    shard="layer_01.bin", append=True)
    man = json.load(open(tmp_path / "manifest.json"))
    assert man["l0.q.weight.bits"]["shard"] == "layer_00.bin"
    assert man["l1.q.weight.bits"]["shard"] == "layer_01.bin"
    assert man["l1.q.weight.bits"]["offset"] == 0
    got, dense, _ = te.read_packed(str(tmp_path))
    assert np.array_equal(got["l0.q.weight"].bits, a.bits)
    assert np.array_equal(got["l1.q.weight"].bits, b.bits)
    assert got["l1.q.weight"].K == 2 and dense["norm"].shape == (8,)
    with pytest.raises(ValueError):
        te.write_packed(str(tmp_path), {"x": a}, shard="layer_01.bin", append=True)
