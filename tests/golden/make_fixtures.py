"""Generate the committed golden fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_fixtures.py``). Inputs and expected outputs only.

config1_smollm2_up.npz  the CPU-runnable configuration: SmolLM2-135M MLP up_proj shape (576 -> 1536,
    torch weight [1536, 576]), W ~ N(0, 0.02) fp32 from seed 0, IP with seeded +-1 signs
    (numpy generator, seed 1), tail-biting Viterbi (oracle/viterbi.c, L=16, K=3, V=1,
    16x16 tiles, 3INST codebook), packed as export_packed.py:27-35. x: fp16 N(0,1) [2, 576]
    (seed 2). y_ref = W_hat @ x in float64 (oracle), W_hat = restore(decode(bits)).
synth_K{K}_{cb}.npz  seeded synthetic records (uniform random bits, the benchmark
    configurations' recipe) at 64 x 128 for K in {2,3,4} x {mcg,3inst,1mad}: the first 8 decoded tiles,
    a sha256 of all decoded tiles, x [3, 128] fp16 and y_ref.
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import trellis_np as tn  # noqa: E402
from oracle import viterbi as vt  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def tiles_sha(tiles):
    return hashlib.sha256(np.ascontiguousarray(tiles, np.float32).tobytes()).hexdigest()


def save(name, **arrs):
    np.savez_compressed(os.path.join(OUT, name), **arrs)
    print("wrote", name, os.path.getsize(os.path.join(OUT, name + ".npz")), "bytes")


def config1():
    n, k = 1536, 576
    w = (np.random.default_rng(0).standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, rec, zq = vt.encode_layer(w, 3, "3inst", seed=1)
    x = np.random.default_rng(2).standard_normal((2, k)).astype(np.float16)
    y = tn.packed_linear_ref(packed, rec, x)
    W = tn.w_hat_from_record(packed, rec)
    zt = tn.decode_packed_tiles(packed, 3, "3inst")
    save("config1_smollm2_up", bits=packed, su=rec.su, sv=rec.sv, isc=rec.isc, osc=rec.osc,
         scale=np.float32(rec.scale), K=np.int32(3), codebook=np.array("3inst"),
         x=x, y_ref=y.astype(np.float64), tiles_sha=np.array(tiles_sha(zt)),
         tiles_head=zt[:8].astype(np.float32),
         w_rel_mse=np.float64(((W - w) ** 2).mean() / (w ** 2).mean()))


def synth():
    for K in (2, 3, 4):
        for cb in ("mcg", "3inst", "1mad"):
            bits, rec = tn.synthetic_record(64, 128, K, seed=100 * K + tn.CODEBOOK_IDS[cb],
                                            codebook=cb)
            x = np.random.default_rng(K).standard_normal((3, 128)).astype(np.float16)
            zt = tn.decode_packed_tiles(bits, K, cb)
            save(f"synth_K{K}_{cb}", bits=bits, su=rec.su, sv=rec.sv, isc=rec.isc,
                 osc=rec.osc, scale=np.float32(rec.scale), K=np.int32(K),
                 codebook=np.array(cb), x=x, y_ref=tn.packed_linear_ref(bits, rec, x),
                 tiles_sha=np.array(tiles_sha(zt)), tiles_head=zt[:8].astype(np.float32))


if __name__ == "__main__":
    synth()
    config1()
