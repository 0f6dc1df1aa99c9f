"""Host side of the packed trellis linear: device upload (the loader record of
web/packed.js:46-62, 88-103) and the packed-linear call (PackedOps.linear,
web/packed.js:163-182), dispatched to the gfx950 kernels through the C ABI.

PyTorch provides device memory and the current stream only; all compute runs in
libtrellis_amd.so. There is no CPU fallback: without the library every call raises.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _capi
from .format import PackedRecord, fit_block


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


# the current stream's handle on a device: torch's raw accessor (0.1 us) where it exists,
# else the public one (~2 us per call, a fifth of an eager call's host cost)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _ws_size(need: int) -> int:
    """Bytes of a new workspace for `need`: the next power of two (at least 256), so a run
    of growing batch sizes replaces the buffer O(log n) times and the retired buffers
    together stay smaller than the current one."""
    return 1 << max(8, (int(need) - 1).bit_length())


def _grow_workspace(owner, need: int) -> torch.Tensor:
    """The owner's workspace, replaced by a larger zero-filled one when `need` exceeds it
    (every call leaves its counters at zero again, so a workspace is zero-filled once).
    A replaced buffer is kept alive with its owner, never freed: a HIP graph captured
    earlier still holds its address, and its replays write split-K partials and counters
    there; released to the caching allocator, that memory could belong to another tensor
    by the next replay. Sizes grow geometrically (_ws_size), which bounds what is kept."""
    if owner._ws is None or owner._ws.numel() < need:
        if owner._ws is not None:
            owner._ws_retired.append(owner._ws)
        owner._ws = torch.zeros(_ws_size(need), dtype=torch.uint8, device=owner.device)
    return owner._ws


class PackedLinear:
    """One packed trellis linear resident on a GPU.

    Load-time fold (web/packed.js:51-52, 91-92): su, sv, osc are upcast f16 -> f32 and
    isc_scaled = f32(isc) * scale in fp32. The kernels then compute
    y = sv * osc * Hb_n(Zq @ Hb_k(isc_scaled * su * x)) = restore(decode(bits)) @ x.
    """

    def __init__(self, rec: PackedRecord, device="cuda", name: str = ""):
        rec.validate()
        bits = np.ascontiguousarray(rec.bits, np.uint32).view(np.int32)
        dev = torch.device(device)
        f32 = lambda a: torch.from_numpy(np.asarray(a, np.float16).astype(np.float32)).to(dev)
        isc_scaled = (np.asarray(rec.isc, np.float16).astype(np.float32) * np.float32(rec.scale))
        self._init(rec.n_out, rec.k_in, rec.K, rec.V, rec.codebook, float(np.float32(rec.scale)),
                   torch.from_numpy(bits.copy()).to(dev), f32(rec.su), f32(rec.sv),
                   torch.from_numpy(isc_scaled.astype(np.float32)).to(dev), f32(rec.osc), name)

    @classmethod
    def from_device(cls, n_out, k_in, K, bits, su, sv, isc_scaled, osc, scale=1.0,
                    codebook="mcg", V=1, name=""):
        """Wrap tensors already on the GPU: bits int32/uint32 [ntiles, nwords], f32
        su/sv/osc and the folded isc_scaled = f32(isc) * scale."""
        self = cls.__new__(cls)
        self._init(n_out, k_in, K, V, codebook, float(scale), bits, su, sv, isc_scaled, osc, name)
        return self

    def _init(self, n_out, k_in, K, V, codebook, scale, bits, su, sv, isc_scaled, osc, name):
        if codebook not in _capi.CB_IDS:
            raise ValueError(f"unknown codebook {codebook!r}")
        self.name = name
        self.n_out, self.k_in, self.K, self.V = int(n_out), int(k_in), int(K), int(V)
        self.codebook = codebook
        self.scale = scale
        self.block_in, self.block_out = fit_block(self.k_in), fit_block(self.n_out)
        self.nwords = (256 * self.K + 31) // 32
        self.device = bits.device
        if self.device.type != "cuda":
            # the kernels dereference these pointers on the GPU
            raise ValueError(f"a packed linear lives on a GPU device, not {self.device}")
        ntiles = (self.n_out // 16) * (self.k_in // 16)
        if tuple(bits.shape) != (ntiles, self.nwords) or not bits.is_contiguous():
            raise ValueError(f"bits must be contiguous [{ntiles}, {self.nwords}]")
        for nm, t, ln in (("su", su, self.k_in), ("isc_scaled", isc_scaled, self.k_in),
                          ("sv", sv, self.n_out), ("osc", osc, self.n_out)):
            if t.dtype != torch.float32 or t.numel() != ln or t.device != self.device:
                raise ValueError(f"{nm} must be a float32 [{ln}] tensor on {self.device}")
        self.bits, self.su, self.sv, self.isc_scaled, self.osc = (
            bits, su.contiguous(), sv.contiguous(), isc_scaled.contiguous(), osc.contiguous())
        self.desc = _capi.TrellisDesc(
            _ptr(self.bits), _ptr(self.su), _ptr(self.sv), _ptr(self.isc_scaled), _ptr(self.osc),
            self.n_out, self.k_in, self.K, self.V, _capi.CB_IDS[self.codebook],
            self.block_in, self.block_out, self.nwords)
        self._ws = None
        self._ws_retired = []

    @property
    def packed_bytes(self) -> int:
        return self.bits.numel() * 4

    # ------------------------------------------------------------------ workspace
    def workspace_bytes(self, batch: int) -> int:
        lib = _capi.load()
        n = ctypes.c_size_t(0)
        _capi.check(lib.trellis_workspace_bytes(ctypes.byref(self.desc), int(batch), ctypes.byref(n)))
        return int(n.value)

    def reserve(self, max_batch: int) -> torch.Tensor:
        """Size the workspace once for calls of up to `max_batch` rows. Call it before
        capturing calls in a HIP graph: a captured launch keeps the workspace's address,
        so a graph stays valid only while that buffer lives (see _workspace)."""
        return _grow_workspace(self, self.workspace_bytes(max_batch))

    def _workspace(self, batch: int) -> torch.Tensor:
        return _grow_workspace(self, self.workspace_bytes(batch))

    # ------------------------------------------------------------------ calls
    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None,
                out_dtype: torch.dtype = torch.float32,
                workspace: torch.Tensor | None = None, mma_f16: bool = False) -> torch.Tensor:
        """y = W_hat @ x for x [k_in] or [batch, k_in] (fp16 or fp32, on this device).

        mma_f16 (calls on the batched path only: batch > 16, or 5 to 16 for wide groups):
        round each codebook value once to fp16 and use one MAC per weight in the batched
        kernel (TRELLIS_MMA_F16: ~2-3e-4 max rel err against the
        exact default, about half the MFMA work and activation traffic)."""
        lib = _capi.load()
        squeeze = x.dim() == 1
        x2 = x.unsqueeze(0) if squeeze else x
        if x2.dim() != 2 or x2.shape[1] != self.k_in:
            raise ValueError(f"x shape {tuple(x.shape)} does not match k_in={self.k_in}")
        if x2.device != self.device:
            raise ValueError(f"x on {x2.device}, weights on {self.device}")
        if x2.dtype not in (torch.float16, torch.float32):
            raise ValueError(f"x dtype {x2.dtype} not supported")
        if x2.stride(1) != 1:
            x2 = x2.contiguous()
        B = x2.shape[0]
        if out is None:
            out = torch.empty((B, self.n_out), dtype=out_dtype, device=self.device)
        y2 = out.view(B, self.n_out) if out.dim() == 1 else out
        if y2.dtype not in (torch.float16, torch.float32) or y2.stride(1) != 1:
            raise ValueError("out must be fp16/fp32 with unit column stride")
        if B == 0:
            # no rows, nothing to launch (the C ABI rejects a batch of 0)
            return out
        stream = ctypes.c_void_p(_stream(self.device))
        xdt = _capi.DT_F16 if x2.dtype == torch.float16 else _capi.DT_F32
        ydt = _capi.DT_F16 if y2.dtype == torch.float16 else _capi.DT_F32
        flags = _capi.MMA_F16 if mma_f16 else 0

        def launch(ws):
            return lib.trellis_packed_linear_ex(
                ctypes.byref(self.desc), _ptr(x2), x2.stride(0), B, xdt, _ptr(y2), y2.stride(0),
                ydt, _ptr(ws), ws.numel(), flags, stream)

        if workspace is not None:
            st = launch(workspace)
        else:
            # the library checks the workspace size before it launches anything, so the
            # current buffer is tried first and sized (grown) only when it is too small
            st = launch(self._ws) if self._ws is not None else _capi.ERR_WORKSPACE
            if st == _capi.ERR_WORKSPACE:
                st = launch(self._workspace(B))
        _capi.check(st)
        return out[0] if (squeeze and out.dim() == 2) else out

    __call__ = forward

    def decode_tiles(self, tile_begin: int = 0, ntiles: int | None = None) -> torch.Tensor:
        """fp32 z-space tiles [ntiles, 256] (the bit-exact decode)."""
        lib = _capi.load()
        total = (self.n_out // 16) * (self.k_in // 16)
        nt = total - tile_begin if ntiles is None else ntiles
        out = torch.empty((nt, 256), dtype=torch.float32, device=self.device)
        stream = _stream(self.device)
        _capi.check(lib.trellis_decode_tiles(ctypes.byref(self.desc), tile_begin, nt, _ptr(out),
                                             ctypes.c_void_p(stream)))
        return out


    def embed_rows(self, tokens, out: torch.Tensor | None = None,
                   out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Rows of W_hat with the full restore: out[t] = W_hat[tokens[t]] ([ntok, k_in]);
        the embedding lookup of a quantized embedding matrix (PackedOps.embedRow,
        web/packed.js:137-146) for many tokens per call. An id outside [0, n_out) gives
        a row of zeros."""
        lib = _capi.load()
        tok = torch.as_tensor(tokens, dtype=torch.int32, device=self.device).reshape(-1)
        tok = tok.contiguous()
        nt = tok.numel()
        if out is None:
            out = torch.empty((nt, self.k_in), dtype=out_dtype, device=self.device)
        if out.dim() != 2 or out.shape != (nt, self.k_in) or out.stride(1) != 1:
            raise ValueError(f"out must be [{nt}, {self.k_in}] with unit column stride")
        if out.dtype not in (torch.float16, torch.float32):
            raise ValueError(f"out dtype {out.dtype} not supported")
        stream = _stream(self.device)
        _capi.check(lib.trellis_embed_rows(
            ctypes.byref(self.desc), _ptr(tok), nt, _ptr(out), out.stride(0),
            _capi.DT_F16 if out.dtype == torch.float16 else _capi.DT_F32,
            ctypes.c_void_p(stream)))
        return out


class PackedGroup:
    """Several packed linears evaluated in ONE launch (trellis_packed_linear_group): e.g.
    q/k/v or gate/up of a decoder block, which the reference dispatches one by one
    (web/model.js:80-100). All members share K, codebook and device."""

    def __init__(self, linears):
        linears = list(linears)
        if not 1 <= len(linears) <= 8:
            raise ValueError("a group holds 1..8 linears")
        dev = linears[0].device
        for lin in linears:
            if lin.device != dev or lin.K != linears[0].K or lin.codebook != linears[0].codebook:
                raise ValueError("group members must share device, K and codebook")
        self.linears = linears
        self.device = dev
        n = len(linears)
        self._descs = (_capi.TrellisDesc * n)(*[lin.desc for lin in linears])
        self._dptrs = (ctypes.POINTER(_capi.TrellisDesc) * n)(
            *[ctypes.pointer(self._descs[i]) for i in range(n)])
        self._ws = None
        self._ws_retired = []

    def workspace_bytes(self, batch: int) -> int:
        lib = _capi.load()
        nbytes = ctypes.c_size_t(0)
        _capi.check(lib.trellis_workspace_bytes_group(self._dptrs, len(self.linears), int(batch),
                                                      ctypes.byref(nbytes)))
        return int(nbytes.value)

    def reserve(self, max_batch: int) -> torch.Tensor:
        """As PackedLinear.reserve: size the group's workspace once, before capture."""
        return _grow_workspace(self, self.workspace_bytes(max_batch))

    def _workspace(self, batch: int) -> torch.Tensor:
        return _grow_workspace(self, self.workspace_bytes(batch))

    def forward(self, xs, outs=None, out_dtype: torch.dtype = torch.float32,
                mma_f16: bool = False):
        """xs: one activation per member ([k_i] or [batch, k_i], same batch and dtype);
        returns (or fills) one output per member. mma_f16 as PackedLinear.forward."""
        lib = _capi.load()
        n = len(self.linears)
        if len(xs) != n:
            raise ValueError(f"expected {n} inputs")
        squeeze = xs[0].dim() == 1
        x2 = [x.unsqueeze(0) if x.dim() == 1 else x for x in xs]
        x2 = [x if x.stride(1) == 1 else x.contiguous() for x in x2]
        B = x2[0].shape[0]
        dt = x2[0].dtype
        for lin, x in zip(self.linears, x2):
            if x.shape != (B, lin.k_in) or x.dtype != dt or x.device != self.device:
                raise ValueError("inputs must share batch, dtype and device and match k_in")
        if dt not in (torch.float16, torch.float32):
            raise ValueError(f"x dtype {dt} not supported")
        if outs is None:
            outs = [torch.empty((B, lin.n_out), dtype=out_dtype, device=self.device)
                    for lin in self.linears]
        y2 = [o.view(B, lin.n_out) if o.dim() == 1 else o for o, lin in zip(outs, self.linears)]
        ydt = y2[0].dtype
        if any(y.dtype != ydt or y.stride(1) != 1 for y in y2) or ydt not in (torch.float16,
                                                                               torch.float32):
            raise ValueError("outputs must share an fp16/fp32 dtype with unit column stride")
        if B == 0:
            # no rows: every member's output is [0, n_i], nothing to launch
            return outs
        xp = (ctypes.c_void_p * n)(*[x.data_ptr() for x in x2])
        yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in y2])
        ldx = (ctypes.c_int64 * n)(*[x.stride(0) for x in x2])
        ldy = (ctypes.c_int64 * n)(*[y.stride(0) for y in y2])
        stream = ctypes.c_void_p(_stream(self.device))

        def launch(ws):
            return lib.trellis_packed_linear_group_ex(
                self._dptrs, n, xp, ldx, B, _capi.DT_F16 if dt == torch.float16 else _capi.DT_F32,
                yp, ldy, _capi.DT_F16 if ydt == torch.float16 else _capi.DT_F32,
                _ptr(ws), ws.numel(), _capi.MMA_F16 if mma_f16 else 0, stream)

        # as PackedLinear.forward: the current workspace first, sized only when too small
        st = launch(self._ws) if self._ws is not None else _capi.ERR_WORKSPACE
        if st == _capi.ERR_WORKSPACE:
            st = launch(self._workspace(B))
        _capi.check(st)
        if squeeze:
            return [o[0] if o.dim() == 2 else o for o in outs]
        return outs

    __call__ = forward


class PackedOps:
    """Mirror of the reference's PackedOps (web/packed.js:130-184): linear(W, x)
    returns {"y": y, "scale": W.scale}."""

    def linear(self, W: PackedLinear, x: torch.Tensor, out_dtype=torch.float32) -> dict:
        return {"y": W.forward(x, out_dtype=out_dtype), "scale": W.scale}

    def embed_row(self, W: PackedLinear, token_id: int) -> torch.Tensor:
        """x[H] = W_hat[token_id] (PackedOps.embedRow, web/packed.js:137-146)."""
        return W.embed_rows([int(token_id)])[0]

    embedRow = embed_row


def encode_tiles(w: torch.Tensor, K: int, codebook: str = "mcg", want_dq: bool = True):
    """Tail-biting trellis encode of z-space tiles on the GPU (trellis_encode_tiles; the
    reference's viterbi_tb_triton / qtip.viterbi_tb, src/trellis/viterbi_triton.py:110-129).
    w: [ntiles, 256] float32 targets in tile order (row%16)*16 + col%16, on the GPU.
    Returns (bits int32 [ntiles, 8K] in the packed format, dq [ntiles, 256] or None)."""
    lib = _capi.load()
    if w.dim() != 2 or w.shape[1] != 256:
        raise ValueError("w must be [ntiles, 256]")
    w = w.to(torch.float32).contiguous()
    nt = w.shape[0]
    if codebook not in _capi.CB_IDS:
        raise ValueError(f"unknown codebook {codebook!r}")
    bits = torch.empty((nt, 8 * K), dtype=torch.int32, device=w.device)
    dq = torch.empty((nt, 256), dtype=torch.float32, device=w.device) if want_dq else None
    nbytes = ctypes.c_size_t(0)
    _capi.check(lib.trellis_encode_workspace_bytes(int(K), nt, ctypes.byref(nbytes)))
    ws = torch.empty(max(int(nbytes.value), 256), dtype=torch.uint8, device=w.device)
    stream = _stream(w.device)
    _capi.check(lib.trellis_encode_tiles(_ptr(w), nt, int(K), _capi.CB_IDS[codebook], _ptr(bits),
                                         _ptr(dq) if want_dq else None, _ptr(ws), ws.numel(),
                                         ctypes.c_void_p(stream)))
    return bits, dq


def load_packed(model_dir: str, device="cuda"):
    """Mirror of loadPacked / loadPackedSharded (web/packed.js:14-114): returns
    {"cfg": config, "tensors": {name: PackedLinear | torch.Tensor}}."""
    from .format import read_packed
    records, dense, cfg = read_packed(model_dir)
    tensors = {name: PackedLinear(r, device=device, name=name) for name, r in records.items()}
    for name, a in dense.items():
        tensors[name] = torch.from_numpy(np.ascontiguousarray(a)).to(device)
    return {"cfg": cfg, "tensors": tensors}
