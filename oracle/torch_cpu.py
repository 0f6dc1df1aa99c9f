"""torch-CPU restatement of the reference's decode-then-matmul (TEST INFRASTRUCTURE
ONLY: the timed CPU baseline of bench.py and a cross-check of trellis_np).

Follows the reference's own torch code path as it runs on CPU:
  symbols from the reversed pack  scripts/export_packed.py:27-35
  window decode                   src/trellis/qtip.py:82-110 (vectorized over all t; the
                                  start window is filled from the stream's own tail,
                                  which is the tail-biting wrap of web/kernels.js:119)
  codebook LUT                    qtip.py:59-66 (LUT built with the qtip.py:32-53 math)
  tile un-permute                 qtip.py:303
  restore                         qtip.py:262-268 (block Hadamard as a matmul, :216-223)
  y = W_hat @ x                   scripts/validate_packed_linear.py:23-25
"""
from __future__ import annotations

import numpy as np
import torch

from . import trellis_np as tn

L = 16
S = 1 << L


def codebook_lut_torch(codebook: str) -> torch.Tensor:
    return torch.from_numpy(tn.codebook_lut(codebook))


def symbols_from_packed(bits: np.ndarray, K: int) -> torch.Tensor:
    """u32 [ntiles, nwords] -> int64 symbols [ntiles, 256]."""
    w = torch.from_numpy(np.asarray(bits, np.uint32).astype(np.int64))
    nw = w.shape[1]
    t = torch.arange(256)
    p0 = (255 - t) * K
    word = p0 >> 5
    sh = p0 & 31
    w0 = w[:, word]
    w1 = w[:, torch.clamp(word + 1, max=nw - 1)]
    both = w0 | (w1 << 32)
    return (both >> sh) & ((1 << K) - 1)


def decode_window_tb(sym: torch.Tensor, K: int, lut: torch.Tensor) -> torch.Tensor:
    """qtip.py:82-110 with the window before t=0 taken from the end of the same stream."""
    steps = (L + K - 1) // K
    ext = torch.cat([sym[:, 256 - (steps - 1):], sym], dim=1)
    state = torch.zeros_like(sym)
    for j in range(steps):
        state = ((state << K) | ext[:, j:j + 256]) & (S - 1)
    return lut[state]


def block_had(x: torch.Tensor, dim: int, block: int = 128) -> torch.Tensor:
    """qtip.py:216-223."""
    x = x.movedim(dim, -1)
    d = x.shape[-1]
    b = tn.fit_block(d, block)
    H = torch.from_numpy(tn.hadamard(b, np.float32))
    y = (x.reshape(*x.shape[:-1], d // b, b) @ H).reshape(x.shape)
    return y.movedim(-1, dim)


def w_hat(bits: np.ndarray, rec: "tn.IPRecord", lut: torch.Tensor | None = None) -> torch.Tensor:
    """restore(decode(bits)) in fp32 torch CPU ops."""
    lut = codebook_lut_torch(rec.codebook) if lut is None else lut
    zt = decode_window_tb(symbols_from_packed(bits, rec.K), rec.K, lut)
    n, k = rec.n, rec.k
    zq = zt.view(n // 16, k // 16, 16, 16).permute(0, 2, 1, 3).reshape(n, k)
    y = zq * float(rec.scale)
    y = block_had(y, dim=1)
    y = y * torch.from_numpy(rec.isc.astype(np.float32)).view(1, -1)
    y = block_had(y, dim=0)
    y = y * torch.from_numpy(rec.osc.astype(np.float32)).view(-1, 1)
    return (y * torch.from_numpy(rec.sv.astype(np.float32)).view(-1, 1)
            * torch.from_numpy(rec.su.astype(np.float32)).view(1, -1))


def decode_matmul(bits: np.ndarray, rec: "tn.IPRecord", x: torch.Tensor,
                  lut: torch.Tensor | None = None) -> torch.Tensor:
    """y = W_hat @ x (x: [k] or [B, k] fp32) -> [n] or [B, n]."""
    W = w_hat(bits, rec, lut)
    return x.float() @ W.T if x.dim() == 2 else W @ x.float()
