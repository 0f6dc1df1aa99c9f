"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI.

Bars: decoded tiles bit-exact; matmul max|got-ref|/(max|ref|+1e-6) <= 1e-3 against the
float64 oracle W_hat @ x (validate_packed_linear.py:66-69 metric and threshold).
"""
import functools
import os
import sys
import zlib

import numpy as np
import pytest
import torch

from oracle import trellis_np as tn

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-3


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_linear(te, bits, rec, device):
    r = te.PackedRecord(rec.n, rec.k, rec.K, bits, rec.su, rec.sv, rec.isc, rec.osc,
                        float(rec.scale), codebook=rec.codebook, V=rec.V)
    return te.PackedLinear(r, device=device)


def fixture(name):
    d = np.load(os.path.join(GOLD, name + ".npz"))
    n, k = d["sv"].shape[0], d["su"].shape[0]
    rec = tn.IPRecord(n, k, int(d["K"]), d["su"], d["sv"], d["isc"], d["osc"], d["scale"],
                      codebook=str(d["codebook"]))
    return d, rec


# ------------------------------------------------------------------ decode bit-exactness
@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("cb", ["mcg", "3inst", "1mad"])
def test_decode_tiles_golden_bit_exact(te, gpu_device, K, cb):
    _say(f"[decode golden] K={K} cb={cb}")
    d, rec = fixture(f"synth_K{K}_{cb}")
    lin = make_linear(te, d["bits"], rec, gpu_device)
    got = lin.decode_tiles().cpu().numpy()
    want = tn.decode_packed_tiles(d["bits"], K, cb)
    assert got.view(np.uint32).tobytes() == want.view(np.uint32).tobytes()
    assert np.array_equal(got[:8], d["tiles_head"])


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("cb", ["mcg", "3inst", "1mad"])
def test_decode_tiles_all_states_bit_exact(te, gpu_device, K, cb):
    """A 4096x1024 random record (16384 tiles, 4.2M windows) covers every 16-bit state
    many times over; compare every decoded value bitwise, and a sub-range call."""
    _say(f"[decode large] K={K} cb={cb}")
    bits, rec = tn.synthetic_record(1024, 4096, K, seed=K * 7 + tn.CODEBOOK_IDS[cb], codebook=cb)
    lin = make_linear(te, bits, rec, gpu_device)
    got = lin.decode_tiles().cpu().numpy()
    want = tn.decode_packed_tiles(bits, K, cb)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    sub = lin.decode_tiles(1000, 77).cpu().numpy()
    assert np.array_equal(sub.view(np.uint32), want[1000:1077].view(np.uint32))


# ------------------------------------------------------------------ packed linear
def test_config1_golden(te, gpu_device):
    """The CPU-runnable configuration: SmolLM2 up_proj 576->1536, K=3, 3INST, real Viterbi encode."""
    _say("[linear] config1 golden")
    d, rec = fixture("config1_smollm2_up")
    lin = make_linear(te, d["bits"], rec, gpu_device)
    x = torch.from_numpy(d["x"]).to(gpu_device)
    for b in (1, 2):
        y = lin(x[:b]).cpu().numpy()
        assert tn.rel_err(y, d["y_ref"][:b]) < TOL
    y1 = lin(x[0]).cpu().numpy()
    assert y1.shape == (1536,)
    assert tn.rel_err(y1, d["y_ref"][0]) < TOL


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("cb", ["mcg", "3inst", "1mad"])
def test_linear_golden_synth(te, gpu_device, K, cb):
    _say(f"[linear golden] K={K} cb={cb}")
    d, rec = fixture(f"synth_K{K}_{cb}")
    lin = make_linear(te, d["bits"], rec, gpu_device)
    y = lin(torch.from_numpy(d["x"]).to(gpu_device)).cpu().numpy()
    assert tn.rel_err(y, d["y_ref"]) < TOL


# pytest runs the parametrized cases batch by batch across the shapes, so the cache holds
# every shape of a test (the largest W_hat, 2048 x 6144 float64, is 100 MB)
@functools.lru_cache(maxsize=16)
def _record_and_w_hat(n, k, K, cb):
    bits, rec = tn.synthetic_record(n, k, K, seed=n * 3 + k + K, codebook=cb)
    return bits, rec, tn.w_hat_from_record(bits, rec)


@pytest.mark.parametrize("n,k,K,cb", [
    (256, 512, 3, "mcg"), (1536, 576, 3, "3inst"), (576, 1536, 3, "mcg"), (2048, 6144, 3, "mcg"),
    (6144, 2048, 3, "mcg"), (128, 4096, 2, "mcg"), (384, 1024, 4, "3inst"), (208, 336, 3, "1mad"),
])
@pytest.mark.parametrize("batch", [1, 3, 8, 16, 37, 64])
def test_linear_vs_oracle(te, gpu_device, n, k, K, cb, batch):
    _say(f"[linear] n={n} k={k} K={K} cb={cb} batch={batch}")
    bits, rec, W = _record_and_w_hat(n, k, K, cb)
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(batch).standard_normal((batch, k)).astype(np.float16)
    want = x.astype(np.float64) @ W.T
    y = lin(torch.from_numpy(x).to(gpu_device)).cpu().numpy()
    assert tn.rel_err(y, want) < TOL


@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.float16, torch.float16),
                                     (torch.float32, torch.float16)])
@pytest.mark.parametrize("batch", [4, 40, 130])
def test_dtypes_and_strides(te, gpu_device, xdt, ydt, batch):
    """Strided rows (input stride k + 64, output stride n + 32) in every dtype pair, through
    the decode-GEMV (4 rows) and the batched path (40 rows: one ragged 64-column block; 130:
    several column blocks), whose x fold and output fold address rows by the strides."""
    _say(f"[linear dtypes] x={xdt} y={ydt} batch={batch}")
    n, k = 512, 1024
    bits, rec = tn.synthetic_record(n, k, 3, seed=11)
    lin = make_linear(te, bits, rec, gpu_device)
    xs = np.random.default_rng(batch).standard_normal((batch, k + 64)).astype(np.float32)
    xt = torch.from_numpy(xs).to(gpu_device).to(xdt)[:, :k]      # row stride k+64
    out = torch.zeros((batch, n + 32), dtype=ydt, device=gpu_device)[:, :n]
    lin.forward(xt, out=out)
    want = tn.packed_linear_ref(bits, rec, xt.float().cpu().numpy())
    assert tn.rel_err(out.float().cpu().numpy(), want) < (2e-3 if ydt == torch.float16 else TOL)
    # the padding columns of the output rows are never written
    assert torch.count_nonzero(out.as_strided((batch, 32), (n + 32, 1), n)).item() == 0


def test_repeat_calls_deterministic_and_ticket_reset(te, gpu_device):
    """Split-K tickets reset themselves: repeated calls give bit-identical results."""
    _say("[linear] determinism")
    bits, rec = tn.synthetic_record(1024, 4096, 3, seed=5)
    lin = make_linear(te, bits, rec, gpu_device)
    x = torch.randn(4096, device=gpu_device, dtype=torch.float16)
    ys = [lin(x).clone() for _ in range(5)]
    torch.cuda.synchronize()
    for y in ys[1:]:
        assert torch.equal(y, ys[0])
    want = tn.packed_linear_ref(bits, rec, x.cpu().numpy())
    assert tn.rel_err(ys[0].cpu().numpy(), want) < TOL


def _oracle_block_rows(bits, rec, ob, x):
    """Oracle for output rows [128*ob, 128*ob+128): those rows depend only on their own
    8 bands (the out-dim Hadamard block is 128)."""
    tin = rec.k // 16
    sub_bits = bits[ob * 8 * tin:(ob + 1) * 8 * tin]
    sl = slice(ob * 128, ob * 128 + 128)
    sub = tn.IPRecord(128, rec.k, rec.K, rec.su, rec.sv[sl], rec.isc, rec.osc[sl], rec.scale,
                      codebook=rec.codebook)
    return tn.packed_linear_ref(sub_bits, sub, x)


@pytest.mark.parametrize("name,n,k", [("q_proj", 4096, 4096), ("k_proj", 1024, 4096),
                                      ("gate_proj", 12288, 4096), ("down_proj", 4096, 12288)])
def test_qwen3_8b_shapes_sampled_blocks(te, gpu_device, name, n, k):
    """The Qwen3-8B block shapes at full size: every output row checked would need a 50M
    weight dense oracle, so three 128-row blocks (first, middle, last) are checked
    exactly and the rest by linearity: f(a*x1 + b*x2) = a f(x1) + b f(x2)."""
    _say(f"[8B] {name} {n}x{k}")
    bits, rec = tn.synthetic_record(n, k, 3, seed=zlib.crc32(name.encode()))
    lin = make_linear(te, bits, rec, gpu_device)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, k)).astype(np.float16)
    y = lin(torch.from_numpy(x).to(gpu_device)).cpu().numpy()[0]
    for ob in (0, (n // 128) // 2, n // 128 - 1):
        want = _oracle_block_rows(bits, rec, ob, x)[0]
        assert tn.rel_err(y[ob * 128:(ob + 1) * 128], want) < TOL
    x1 = torch.randn(k, device=gpu_device)
    x2 = torch.randn(k, device=gpu_device)
    lhs = lin(0.75 * x1 - 1.5 * x2)
    rhs = 0.75 * lin(x1) - 1.5 * lin(x2)
    assert (lhs - rhs).abs().max().item() / rhs.abs().max().item() < TOL


@pytest.mark.parametrize("batch", [1, 3])
def test_lm_head_shape_sampled_blocks(te, gpu_device, batch):
    """The Qwen3-8B vocab matrix at K=4 (151936 x 4096, the LM head the bench times): 1187
    output blocks, so the decode-GEMV's work items run in several rounds over the CUs.
    Blocks of the first, middle and last rounds against the oracle, every batch row."""
    _say(f"[lm head] 151936x4096 K=4 batch={batch}")
    n, k = 151936, 4096
    bits, rec = tn.synthetic_record(n, k, 4, seed=151936)
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(batch).standard_normal((batch, k)).astype(np.float16)
    y = lin(torch.from_numpy(x).to(gpu_device)).cpu().numpy()
    for ob in (0, 255, 256, (n // 128) // 2, n // 128 - 1):
        want = _oracle_block_rows(bits, rec, ob, x)
        assert tn.rel_err(y[:, ob * 128:(ob + 1) * 128], want) < TOL
        for b in range(batch):
            assert tn.rel_err(y[b, ob * 128:(ob + 1) * 128], want[b]) < TOL


@pytest.mark.parametrize("batch", [1, 2, 5, 40])
def test_group_matches_single_and_oracle(te, gpu_device, batch):
    """One grouped launch of q/k/v-like and odd-shaped members equals the oracle per
    member and the single-matrix calls."""
    _say(f"[group] batch={batch}")
    shapes = [(512, 1024), (128, 1024), (128, 1024), (1536, 576), (256, 336)]
    members = []
    for i, (n, k) in enumerate(shapes):
        bits, rec = tn.synthetic_record(n, k, 3, seed=40 + i)
        members.append((bits, rec, make_linear(te, bits, rec, gpu_device)))
    grp = te.PackedGroup([m[2] for m in members])
    rng = np.random.default_rng(batch)
    xs = [torch.from_numpy(rng.standard_normal((batch, rec.k)).astype(np.float16)).to(gpu_device)
          for _, rec, _ in members]
    ys = grp(xs)
    for (bits, rec, lin), x, y in zip(members, xs, ys):
        want = tn.packed_linear_ref(bits, rec, x.cpu().numpy())
        assert tn.rel_err(y.cpu().numpy(), want) < TOL
        # the k-slicing is planned per launch, so a member may be split differently in
        # the group than alone: equal up to fp32 summation order
        single = lin(x)
        assert (single - y).abs().max().item() <= 1e-5 * y.abs().max().item()


def test_group_rejects_mixed_k(te, gpu_device):
    b3, r3 = tn.synthetic_record(128, 256, 3, seed=1)
    b2, r2 = tn.synthetic_record(128, 256, 2, seed=2)
    with pytest.raises(ValueError):
        te.PackedGroup([make_linear(te, b3, r3, gpu_device), make_linear(te, b2, r2, gpu_device)])


@pytest.mark.parametrize("n,k,batch", [(2048, 6144, 512), (1024, 2048, 300), (256, 512, 129)])
def test_prefill_vs_oracle(te, gpu_device, n, k, batch):
    """The prefill shape class: the batched decode-once kernel over many
    column blocks (ragged last block), against the float64 oracle."""
    _say(f"[prefill] n={n} k={k} batch={batch}")
    bits, rec, W = _record_and_w_hat(n, k, 3, "mcg")
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(batch).standard_normal((batch, k)).astype(np.float16)
    want = x.astype(np.float64) @ W.T
    y = lin(torch.from_numpy(x).to(gpu_device)).cpu().numpy()
    assert tn.rel_err(y, want) < TOL
    # every batch row on its own (the metric is per linear call, rows must not mix)
    for b in (0, batch // 2, batch - 1):
        assert tn.rel_err(y[b], want[b]) < TOL


@pytest.mark.parametrize("n,k,batch", [(256, 2048, 4096), (384, 1024, 2500)])
def test_long_prefill_vs_oracle(te, gpu_device, n, k, batch):
    """Long prefills: thousands of x-fold jobs and tens of column blocks in one launch (a
    ragged last one at 2500), both MFMA modes, every row against the oracle."""
    _say(f"[long prefill] n={n} k={k} batch={batch}")
    bits, rec, W = _record_and_w_hat(n, k, 3, "mcg")
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(batch).standard_normal((batch, k)).astype(np.float16)
    want = x.astype(np.float64) @ W.T
    xt = torch.from_numpy(x).to(gpu_device)
    for f16 in (False, True):
        y = lin(xt, mma_f16=f16).cpu().numpy()
        assert tn.rel_err(y, want) < TOL, f16
        worst = max(tn.rel_err(y[b], want[b]) for b in range(batch))
        assert worst < TOL, (f16, worst)


@pytest.mark.parametrize("batch", [257, 258, 259, 262])
def test_prefill_ragged_fold_rows(te, gpu_device, batch):
    """From 256 rows up the x fold takes four batch rows per wave: a batch that is not a
    multiple of four leaves the last group 1, 2 or 3 rows, whose missing rows must be
    neither read into the result nor stored. Both MFMA modes, every row against the
    oracle, and its first 255 rows equal to a call on those rows alone (one row per wave in
    that call's fold; the plans may differ, so within 1e-5)."""
    _say(f"[prefill ragged fold] batch={batch}")
    n, k = 384, 1024
    bits, rec, W = _record_and_w_hat(n, k, 3, "mcg")
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(batch).standard_normal((batch, k)).astype(np.float16)
    want = x.astype(np.float64) @ W.T
    xt = torch.from_numpy(x).to(gpu_device)
    for f16 in (False, True):
        y = lin(xt, mma_f16=f16).cpu().numpy()
        worst = max(tn.rel_err(y[b], want[b]) for b in range(batch))
        assert worst < TOL, (f16, worst)
        head = lin(xt[:255], mma_f16=f16).cpu().numpy()
        assert tn.rel_err(y[:255], head) < 1e-5, f16


@pytest.mark.parametrize("K,cb,V", [(2, "mcg", 1), (3, "mcg", 1), (4, "mcg", 1), (3, "3inst", 2),
                                    (3, "1mad", 1), (4, "3inst", 1), (2, "1mad", 2)])
def test_prefill_column_block_width(te, gpu_device, monkeypatch, K, cb, V):
    """Above 64 columns the batched kernel runs 64-column blocks (16 waves) or, as the
    planner's cost model decides, 128-column blocks (8 waves in the exact mode, whose
    fragments and accumulators need two waves' worth of registers). Every width, forced
    with TRELLIS_BGEMM_NC in either mode, gives the oracle's result, and the exact mode's
    widths agree to fp32 summation order."""
    _say(f"[prefill width] K={K} cb={cb} V={V} batch=200")
    bits, rec = tn.synthetic_record(512, 1024, K, seed=200 + K, codebook=cb, V=V)
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(K).standard_normal((200, 1024)).astype(np.float16)
    xt = torch.from_numpy(x).to(gpu_device)
    want = tn.packed_linear_ref(bits, rec, x)
    planned = lin(xt).cpu().numpy()
    assert tn.rel_err(planned, want) < TOL
    for nc in ("8", "4"):
        monkeypatch.setenv("TRELLIS_BGEMM_NC", nc)
        forced = lin(xt).cpu().numpy()
        assert tn.rel_err(forced, want) < TOL, nc
        assert tn.rel_err(forced, planned) < 1e-5, nc
        assert np.array_equal(forced, lin(xt).cpu().numpy()), nc      # deterministic
        assert tn.rel_err(lin(xt, mma_f16=True).cpu().numpy(), want) < TOL, nc


@pytest.mark.parametrize("batch", [16, 64])
def test_batched_repeat_deterministic(te, gpu_device, batch):
    """Batched split-K: tickets reset themselves and repeated calls are bit-identical."""
    _say(f"[batched] determinism batch={batch}")
    bits, rec = tn.synthetic_record(1024, 4096, 3, seed=6)
    lin = make_linear(te, bits, rec, gpu_device)
    x = torch.randn(batch, 4096, device=gpu_device, dtype=torch.float16)
    ys = [lin(x).clone() for _ in range(4)]
    torch.cuda.synchronize()
    for y in ys[1:]:
        assert torch.equal(y, ys[0])
    want = tn.packed_linear_ref(bits, rec, x.cpu().numpy())
    assert tn.rel_err(ys[0].cpu().numpy(), want) < TOL


def test_group_many_column_blocks(te, gpu_device):
    """Regression: a group whose members each span several 128-column batch blocks (the
    grid holds blocks x column blocks x k-slices per member) must address every member's
    own items; checked per member against the oracle."""
    _say("[group] batch=160, two members")
    shapes = [(384, 1024), (256, 512)]
    members = []
    for i, (n, k) in enumerate(shapes):
        bits, rec = tn.synthetic_record(n, k, 3, seed=70 + i)
        members.append((bits, rec, make_linear(te, bits, rec, gpu_device)))
    grp = te.PackedGroup([m[2] for m in members])
    rng = np.random.default_rng(160)
    xs = [torch.from_numpy(rng.standard_normal((160, rec.k)).astype(np.float16)).to(gpu_device)
          for _, rec, _ in members]
    ys = grp(xs)
    for (bits, rec, _), x, y in zip(members, xs, ys):
        want = tn.packed_linear_ref(bits, rec, x.cpu().numpy())
        assert tn.rel_err(y.cpu().numpy(), want) < TOL


# ------------------------------------------------------------------ V=2 (this build's definition)
@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("cb", ["mcg", "3inst", "1mad"])
def test_v2_decode_tiles_bit_exact(te, gpu_device, K, cb):
    """V=2 decoded tiles bit-exact against the oracle over a 512x2048 random record
    (4096 tiles, 524k states), and a sub-range call."""
    _say(f"[v2 decode] K={K} cb={cb}")
    bits, rec = tn.synthetic_record(512, 2048, K, seed=K * 11 + tn.CODEBOOK_IDS[cb], codebook=cb,
                                    V=2)
    lin = make_linear(te, bits, rec, gpu_device)
    got = lin.decode_tiles().cpu().numpy()
    want = tn.decode_packed_tiles(bits, K, cb, V=2)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    sub = lin.decode_tiles(333, 41).cpu().numpy()
    assert np.array_equal(sub.view(np.uint32), want[333:374].view(np.uint32))


@functools.lru_cache(maxsize=4)
def _v2_record_and_w_hat(n, k, K, cb):
    bits, rec = tn.synthetic_record(n, k, K, seed=n + k + K, codebook=cb, V=2)
    return bits, rec, tn.w_hat_from_record(bits, rec)


@pytest.mark.parametrize("n,k,K,cb", [(256, 512, 3, "mcg"), (1536, 576, 2, "3inst"),
                                      (384, 2048, 4, "1mad"), (2048, 4096, 3, "mcg")])
@pytest.mark.parametrize("batch", [1, 2, 3, 5, 64])
def test_v2_linear_vs_oracle(te, gpu_device, n, k, K, cb, batch):
    _say(f"[v2 linear] n={n} k={k} K={K} cb={cb} batch={batch}")
    bits, rec, W = _v2_record_and_w_hat(n, k, K, cb)
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(batch).standard_normal((batch, k)).astype(np.float16)
    y = lin(torch.from_numpy(x).to(gpu_device)).cpu().numpy()
    assert tn.rel_err(y, x.astype(np.float64) @ W.T) < TOL


@pytest.mark.parametrize("n,k,K,cb", [(1536, 576, 3, "3inst"), (576, 1536, 3, "mcg"),
                                      (2048, 6144, 3, "mcg"), (384, 1024, 4, "3inst"),
                                      (208, 336, 3, "1mad")])
@pytest.mark.parametrize("batch", [2, 3, 4])
def test_small_batch_gemv_rows(te, gpu_device, n, k, K, cb, batch):
    """Batch 2 to 4 run the decode-GEMV with the batch rows in the MFMA's B columns (the
    same plan as batch 1): each output row is bit-identical to the batch-1 call on that
    input row, and within 1e-3 of the oracle."""
    _say(f"[small batch] n={n} k={k} K={K} cb={cb} batch={batch}")
    bits, rec, W = _record_and_w_hat(n, k, K, cb)
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(3 * batch + n).standard_normal((batch, k)).astype(np.float16)
    xt = torch.from_numpy(x).to(gpu_device)
    y = lin(xt).cpu().numpy()
    for b in range(batch):
        assert np.array_equal(y[b], lin(xt[b]).cpu().numpy())
    assert tn.rel_err(y, x.astype(np.float64) @ W.T) < TOL


def test_small_batch_group_strided(te, gpu_device):
    """A group at batch 3 with strided f32 inputs and f16 outputs through the decode-GEMV."""
    shapes = [(512, 1024), (128, 1024), (384, 1024)]
    cases = [_record_and_w_hat(nn, kk, 3, "mcg") for nn, kk in shapes]
    lins = [make_linear(te, b, r, gpu_device) for b, r, _ in cases]
    grp = te.PackedGroup(lins)
    xs = np.random.default_rng(9).standard_normal((3, 1024 + 96)).astype(np.float32)
    xt = torch.from_numpy(xs).to(gpu_device)[:, :1024]
    outs = [torch.zeros((3, nn + 64), dtype=torch.float16, device=gpu_device)[:, :nn]
            for nn, _ in shapes]
    grp([xt] * 3, outs)
    for o, (_, _, W) in zip(outs, cases):
        assert tn.rel_err(o.float().cpu().numpy(), xs[:, :1024].astype(np.float64) @ W.T) < 2e-3


@pytest.mark.parametrize("n,k,K,cb,V", [(1536, 576, 3, "3inst", 1), (576, 1536, 3, "mcg", 1),
                                        (2048, 6144, 3, "mcg", 1), (208, 336, 3, "1mad", 1),
                                        (384, 1024, 2, "3inst", 2), (96, 48, 4, "mcg", 1)])
@pytest.mark.parametrize("batch", [5, 8, 9, 16])
def test_batch_5_to_16_both_paths(te, gpu_device, monkeypatch, n, k, K, cb, V, batch):
    """Batch 5 to 16 run the decode-GEMV (8 or 16 rows in the MFMA's B columns, shorter
    k-ranges, one epilogue wave per row) or the batched path, as the planner decides
    (TRELLIS_SMALL_BATCH_GEMV forces either): both within 1e-3 of the oracle, and within
    fp32 summation order of each other."""
    _say(f"[batch 5-16] n={n} k={k} K={K} cb={cb} V={V} batch={batch}")
    bits, rec = tn.synthetic_record(n, k, K, seed=n + k + V, codebook=cb, V=V)
    W = tn.w_hat_from_record(bits, rec)
    lin = make_linear(te, bits, rec, gpu_device)
    x = np.random.default_rng(batch + n).standard_normal((batch, k)).astype(np.float16)
    xt = torch.from_numpy(x).to(gpu_device)
    ref = x.astype(np.float64) @ W.T
    ys = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("TRELLIS_SMALL_BATCH_GEMV", mode)
        ys[mode] = lin(xt).cpu().numpy()
        assert tn.rel_err(ys[mode], ref) < TOL, mode
        assert np.array_equal(ys[mode], lin(xt).cpu().numpy())     # deterministic
    assert tn.rel_err(ys["1"], ys["0"]) < 1e-5


def test_batch_5_to_16_group_strided(te, gpu_device, monkeypatch):
    """A q/k/v-like group at batch 12 through the decode-GEMV (16 rows in the B columns,
    split k) with strided f32 inputs and f16 outputs."""
    monkeypatch.setenv("TRELLIS_SMALL_BATCH_GEMV", "1")
    shapes = [(512, 2048), (128, 2048), (384, 2048)]
    cases = [_record_and_w_hat(nn, kk, 3, "mcg") for nn, kk in shapes]
    lins = [make_linear(te, b, r, gpu_device) for b, r, _ in cases]
    grp = te.PackedGroup(lins)
    xs = np.random.default_rng(12).standard_normal((12, 2048 + 64)).astype(np.float32)
    xt = torch.from_numpy(xs).to(gpu_device)[:, :2048]
    outs = [torch.zeros((12, nn + 32), dtype=torch.float16, device=gpu_device)[:, :nn]
            for nn, _ in shapes]
    grp([xt] * 3, outs)
    for o, (_, _, W) in zip(outs, cases):
        assert tn.rel_err(o.float().cpu().numpy(), xs[:, :2048].astype(np.float64) @ W.T) < 2e-3


def test_workspace_shared_across_batch_sizes(te, gpu_device):
    """One linear's workspace serves calls at every batch size: a large batched call fills
    it with partial sums and folded activations, and the split-K tickets of the calls after
    it (decode-GEMV at 1, 3, 8; batched at 64) sit in a header that no call's data reaches,
    so each result stays within 1e-3 of the oracle."""
    bits, rec, W = _record_and_w_hat(2048, 6144, 3, "mcg")
    lin = make_linear(te, bits, rec, gpu_device)
    rng = np.random.default_rng(77)
    for batch in (300, 1, 3, 8, 64, 1, 300, 2):
        _say(f"[workspace] batch={batch}")
        x = rng.standard_normal((batch, 6144)).astype(np.float16)
        y = lin(torch.from_numpy(x).to(gpu_device)).cpu().numpy()
        assert tn.rel_err(y, x.astype(np.float64) @ W.T) < TOL, batch
