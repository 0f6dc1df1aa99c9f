"""bench.py's output check (check_outputs), on the CPU: outputs that equal the oracle's pass,
and a block whose output belongs to another row block, a single wrong value, or input
scales that are not f32(fp16 isc) * scale fail it."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from oracle import trellis_np as tn  # noqa: E402


def _sample(n=384, k=512, K=3, B=3, seed=7, obs=(0, 1, 2)):
    bits, rec = tn.synthetic_record(n, k, K, seed=seed)
    scale = np.float32(rec.scale)
    isc_scaled = rec.isc.astype(np.float32) * scale
    x = np.random.default_rng(seed).standard_normal((B, k)).astype(np.float16).astype(np.float32)
    y = tn.packed_linear_ref(bits, rec, x).astype(np.float32)       # the whole [B, n] output
    tin = k // 16
    return {"run": "unit", "layer": "w", "n": n, "k": k, "K": K, "V": 1, "codebook": "mcg",
            "scale": float(scale), "su": rec.su.astype(np.float32), "sv": rec.sv.astype(np.float32),
            "isc_scaled": isc_scaled, "osc": rec.osc.astype(np.float32), "x": x,
            "blocks": [(ob, bits[ob * 8 * tin:(ob + 1) * 8 * tin], y[:, ob * 128:(ob + 1) * 128])
                       for ob in obs]}


def test_check_passes_on_oracle_outputs():
    res = bench.check_outputs([_sample(), _sample(K=2, seed=3, obs=(2,))])
    assert res["ok"], res
    assert res["blocks_checked"] == 4 and res["max_rel_err"] < 1e-6


def test_check_fails_on_swapped_block_and_on_one_value():
    s = _sample()
    (o0, b0, y0), (o1, b1, y1) = s["blocks"][:2]
    s["blocks"][0] = (o0, b0, y1)                 # block 0 reports block 1's rows
    res = bench.check_outputs([s])
    assert not res["ok"] and len(res["failures"]) == 1 and "rows 0+128" in res["failures"][0]
    t = _sample()
    ob, bits, y = t["blocks"][2]
    y = y.copy()
    y[1, 77] += 0.01 * np.abs(y).max()            # 1 % of the block's max: 10x the tolerance
    t["blocks"][2] = (ob, bits, y)
    assert not bench.check_outputs([t])["ok"]


def test_check_rejects_inexact_scale_fold():
    s = _sample()
    s["isc_scaled"] = s["isc_scaled"] * np.float32(1.0 + 2.0 ** -20)
    try:
        bench.check_outputs([s])
    except ValueError as e:
        assert "isc_scaled" in str(e)
    else:
        raise AssertionError("an isc_scaled that is not f32(fp16) * scale was accepted")
