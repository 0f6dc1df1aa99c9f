"""Packed trellis weight format: manifest.json + weights.bin (or shards), byte-compatible
with the reference exporters.

Writer layout (scripts/export_packed.py:45-63): one flat blob; for every quantized
linear `name`:
    name.bits  u32 [ntiles, nwords]   reversed-pack K-bit symbols (export_packed.py:27-35)
    name.su    f16 [k_in]             input-dim signs
    name.sv    f16 [n_out]            output-dim signs
    name.isc   f16 [k_in]             per-in-channel scale (mean 1)
    name.osc   f16 [n_out]            per-out-channel scale (mean 1)
    name.scale f32 [1]                global scale
and manifest[name] = {"quant": true, "n_out", "k_in", "K", "block", "tiles_out",
"tiles_in"}; each sub-tensor entry is {"offset", "shape", "dtype"} with an optional
"shard" file name (export_packed_8b.py:65-81, 134-143). Readers group entries by shard,
defaulting to weights.bin (web/packed.js:14-33).

Extension (absent keys keep the reference meaning): "codebook" ("mcg" when absent,
export_packed.py:42 hard-codes it) and "V" (1 when absent).

Everything is read with numpy.frombuffer / json: nothing in a file is executed.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np

_DT = {"f16": np.float16, "u32": np.uint32, "f32": np.float32}
_DT_NAME = {np.dtype(np.float16): "f16", np.dtype(np.uint32): "u32", np.dtype(np.float32): "f32"}
SUBKEYS = ("bits", "su", "sv", "isc", "osc", "scale")


def fit_block(d: int, block: int = 128) -> int:
    """Largest power-of-2 divisor of d, capped at block (src/trellis/qtip.py:208-213)."""
    b = 1
    while b < block and d % (b * 2) == 0:
        b *= 2
    return b


@dataclass
class PackedRecord:
    """One quantized linear as stored on disk (host numpy arrays)."""
    n_out: int
    k_in: int
    K: int
    bits: np.ndarray            # u32 [ntiles, nwords]
    su: np.ndarray              # f16 [k_in]
    sv: np.ndarray              # f16 [n_out]
    isc: np.ndarray             # f16 [k_in]
    osc: np.ndarray             # f16 [n_out]
    scale: float                # f32
    codebook: str = "mcg"
    V: int = 1
    extra: dict = field(default_factory=dict)

    @property
    def tiles_out(self) -> int:
        return self.n_out // 16

    @property
    def tiles_in(self) -> int:
        return self.k_in // 16

    @property
    def nwords(self) -> int:
        return int(self.bits.shape[1])

    @property
    def block(self) -> int:
        """The manifest's in-dim Hadamard block (export_packed.py:62)."""
        return fit_block(self.k_in, 128)

    @property
    def block_out(self) -> int:
        """Out-dim block = fit(n_out, 128), not the manifest's block (web/packed.js:173-176)."""
        return fit_block(self.n_out, 128)

    def validate(self) -> None:
        if self.n_out % 16 or self.k_in % 16:
            raise ValueError(f"shape {self.n_out}x{self.k_in} not a multiple of 16")
        nt = self.tiles_out * self.tiles_in
        if self.bits.shape != (nt, (256 * self.K + 31) // 32):
            raise ValueError(f"bits shape {self.bits.shape} != ({nt}, {(256 * self.K + 31) // 32})")
        if self.V not in (1, 2):
            raise ValueError(f"V={self.V}: weights per trellis step must be 1 or 2")
        for nm, arr, ln in (("su", self.su, self.k_in), ("isc", self.isc, self.k_in),
                            ("sv", self.sv, self.n_out), ("osc", self.osc, self.n_out)):
            if arr.shape != (ln,):
                raise ValueError(f"{nm} shape {arr.shape} != ({ln},)")


class _Blob:
    def __init__(self):
        self.buf = bytearray()
        self.man = {}

    def put(self, name, arr, dtype, shard=None):
        a = np.ascontiguousarray(np.asarray(arr).astype(dtype))
        ent = {"offset": len(self.buf), "shape": list(a.shape), "dtype": _DT_NAME[a.dtype]}
        if shard:
            ent["shard"] = shard
        self.man[name] = ent
        self.buf.extend(a.tobytes())


def write_packed(out_dir: str, records: dict, dense: dict | None = None,
                 config: dict | None = None, shard: str | None = None,
                 append: bool = False) -> None:
    """Write records ({name: PackedRecord}) and optional dense f16 tensors in the
    reference layout. With `shard`, the blob is written as that file and every entry
    carries "shard" (export_packed_8b.py:65-81); otherwise weights.bin. With `append`,
    the entries join those of an existing manifest.json in out_dir (one shard per call,
    merged into one manifest as export_packed_8b.py:271-276 merges its shard fragments)."""
    os.makedirs(out_dir, exist_ok=True)
    blob = _Blob()
    mpath = os.path.join(out_dir, "manifest.json")
    if append and os.path.exists(mpath):
        with open(mpath) as f:
            old = json.load(f)
        target = shard or "weights.bin"
        if any(m.get("shard", "weights.bin") == target for m in old.values()):
            raise ValueError(f"{target} already holds entries of this manifest")
        blob.man.update(old)
    for name, r in records.items():
        r.validate()
        blob.put(f"{name}.bits", r.bits, np.uint32, shard)
        blob.put(f"{name}.su", r.su, np.float16, shard)
        blob.put(f"{name}.sv", r.sv, np.float16, shard)
        blob.put(f"{name}.isc", r.isc, np.float16, shard)
        blob.put(f"{name}.osc", r.osc, np.float16, shard)
        blob.put(f"{name}.scale", np.array([r.scale], np.float32), np.float32, shard)
        ent = {"quant": True, "n_out": r.n_out, "k_in": r.k_in, "K": r.K, "block": r.block,
               "tiles_out": r.tiles_out, "tiles_in": r.tiles_in}
        if r.codebook != "mcg":
            ent["codebook"] = r.codebook
        if r.V != 1:
            ent["V"] = r.V
        if shard:
            ent["shard"] = shard
        blob.man[name] = ent
    for name, t in (dense or {}).items():
        blob.put(name, t, np.float16, shard)
    with open(os.path.join(out_dir, shard or "weights.bin"), "wb") as f:
        f.write(bytes(blob.buf))
    with open(mpath, "w") as f:
        json.dump(blob.man, f)
    if config is not None:
        with open(os.path.join(out_dir, "config.json"), "w") as f:
            json.dump(config, f)


def _raw(blob: memoryview, m: dict) -> np.ndarray:
    dt = _DT[m["dtype"]]
    count = int(np.prod(m["shape"])) if m["shape"] else 1
    a = np.frombuffer(blob, dtype=dt, count=count, offset=int(m["offset"]))
    return a.reshape(m["shape"])


def read_packed(model_dir: str):
    """Read manifest + blob(s). Returns (records {name: PackedRecord},
    dense {name: np.ndarray}, config dict or None). Mirrors loadPacked /
    loadPackedSharded (web/packed.js:14-114) minus the device upload."""
    with open(os.path.join(model_dir, "manifest.json")) as f:
        man = json.load(f)
    cfg = None
    cp = os.path.join(model_dir, "config.json")
    if os.path.exists(cp):
        with open(cp) as f:
            cfg = json.load(f)
    by_shard: dict = {}
    for name, m in man.items():
        by_shard.setdefault(m.get("shard", "weights.bin"), {})[name] = m
    records, dense = {}, {}
    for shard in sorted(by_shard):
        entries = by_shard[shard]
        with open(os.path.join(model_dir, shard), "rb") as f:
            blob = memoryview(f.read())
        for name, m in entries.items():
            if m.get("quant"):
                # the in-dim Hadamard block this build applies is fit(k_in, 128), the
                # block every exporter writes (export_packed.py:62); the reference's loader
                # takes the manifest's value (web/packed.js:57, 166), so a manifest naming
                # another block describes weights this reader would restore wrongly
                want = fit_block(int(m["k_in"]), 128)
                if int(m.get("block", want)) != want:
                    raise ValueError(f"{name}: manifest block {m['block']} != fit(k_in={m['k_in']}, "
                                     f"128) = {want}; only the exporters' block is supported")
                sub = {k: man[f"{name}.{k}"] for k in SUBKEYS}
                bits = np.array(_raw(blob, sub["bits"]), np.uint32)
                rec = PackedRecord(
                    n_out=int(m["n_out"]), k_in=int(m["k_in"]), K=int(m["K"]), bits=bits,
                    su=np.array(_raw(blob, sub["su"]), np.float16),
                    sv=np.array(_raw(blob, sub["sv"]), np.float16),
                    isc=np.array(_raw(blob, sub["isc"]), np.float16),
                    osc=np.array(_raw(blob, sub["osc"]), np.float16),
                    scale=float(np.array(_raw(blob, sub["scale"]), np.float32).reshape(-1)[0]),
                    codebook=m.get("codebook", "mcg"), V=int(m.get("V", 1)))
                rec.validate()
                records[name] = rec
            elif name.rsplit(".", 1)[-1] in SUBKEYS and name.rsplit(".", 1)[0] in man \
                    and man[name.rsplit(".", 1)[0]].get("quant"):
                continue
            else:
                dense[name] = np.array(_raw(blob, m))
    return records, dense, cfg
