"""torch.nn adapters of the packed linear, for PyTorch model code (the forward-pass call
site: the reference's TrellisModel._linearE, web/model.js:52-58, dispatching on W.quant).

TrellisLinear is a drop-in for an nn.Linear whose weight is a packed trellis record: any
leading shape, fp16 / fp32 / bf16 activations, optional bias. swap_linears replaces the
nn.Linear modules of a model whose weight names have packed records (the manifest names
`<module>.weight`, scripts/export_packed_8b.py:65-81). All compute runs in the gfx950
kernels (PackedLinear); there is no CPU path.
"""
from __future__ import annotations

import torch

from .packed_linear import PackedGroup, PackedLinear


def _as_kernel_input(x: torch.Tensor) -> torch.Tensor:
    # the kernels take f16 or f32 activations; bf16 widens to f32 exactly
    return x.float() if x.dtype == torch.bfloat16 else x


class TrellisLinear(torch.nn.Module):
    """y = x @ W_hat^T (+ bias) with W_hat = restore(decode(bits)) held packed on the GPU.

    x: [..., in_features] (f16, f32 or bf16) on the linear's device. The output has x's
    dtype (bf16 is computed in fp32 and rounded once). mma_f16 selects the batched
    kernel's fp16-weight mode (calls on the batched path only; see PackedLinear.forward)."""

    def __init__(self, packed: PackedLinear, bias: torch.Tensor | None = None,
                 mma_f16: bool = False):
        super().__init__()
        self.packed = packed
        self.in_features, self.out_features = packed.k_in, packed.n_out
        self.mma_f16 = mma_f16
        if bias is not None:
            self.register_buffer("bias", bias.detach().to(packed.device, torch.float32))
        else:
            self.bias = None

    @classmethod
    def from_record(cls, rec, device="cuda", bias=None, name: str = "", mma_f16=False):
        return cls(PackedLinear(rec, device=device, name=name), bias=bias, mma_f16=mma_f16)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.in_features:
            raise ValueError(f"last dim {x.shape[-1]} != in_features {self.in_features}")
        lead = x.shape[:-1]
        x2 = _as_kernel_input(x).reshape(-1, self.in_features)
        out_dtype = torch.float16 if x.dtype == torch.float16 else torch.float32
        if x2.shape[0] == 0:
            y = x2.new_zeros((0, self.out_features), dtype=out_dtype)
        else:
            y = self.packed.forward(x2, out_dtype=out_dtype, mma_f16=self.mma_f16)
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y.to(x.dtype).reshape(*lead, self.out_features)

    def extra_repr(self) -> str:
        p = self.packed
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"K={p.K}, V={p.V}, codebook={p.codebook}, bias={self.bias is not None}")


class TrellisGroupLinear(torch.nn.Module):
    """Several packed linears on one input in ONE launch (q/k/v, gate/up:
    trellis_packed_linear_group); forward returns one output per member, each
    [..., out_features_i] in x's dtype."""

    def __init__(self, members: list[PackedLinear], mma_f16: bool = False):
        super().__init__()
        self.group = PackedGroup(members)
        self.in_features = members[0].k_in
        if any(m.k_in != self.in_features for m in members):
            raise ValueError("grouped linears must share in_features")
        self.out_features = [m.n_out for m in members]
        self.mma_f16 = mma_f16

    def forward(self, x: torch.Tensor):
        lead = x.shape[:-1]
        x2 = _as_kernel_input(x).reshape(-1, self.in_features)
        out_dtype = torch.float16 if x.dtype == torch.float16 else torch.float32
        ys = self.group([x2] * len(self.out_features), out_dtype=out_dtype,
                        mma_f16=self.mma_f16)
        return [y.to(x.dtype).reshape(*lead, n) for y, n in zip(ys, self.out_features)]


def swap_linears(model: torch.nn.Module, records: dict, device="cuda", mma_f16=False,
                 strict: bool = False) -> list[str]:
    """Replace every nn.Linear `<name>` of model with a TrellisLinear when records holds
    `<name>.weight` (a PackedRecord, or a PackedLinear already on the GPU). The linear's
    bias, if any, is kept. Returns the replaced module names; strict=True raises when a
    record matches no nn.Linear or a shape disagrees."""
    replaced, used = [], set()
    for name, mod in list(model.named_modules()):
        if not isinstance(mod, torch.nn.Linear):
            continue
        key = f"{name}.weight"
        rec = records.get(key)
        if rec is None:
            continue
        packed = rec if isinstance(rec, PackedLinear) else PackedLinear(rec, device=device, name=key)
        if (packed.n_out, packed.k_in) != (mod.out_features, mod.in_features):
            raise ValueError(f"{key}: packed {packed.n_out}x{packed.k_in} vs nn.Linear "
                             f"{mod.out_features}x{mod.in_features}")
        new = TrellisLinear(packed, bias=mod.bias, mma_f16=mma_f16)
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, child, new)
        replaced.append(name)
        used.add(key)
    if strict:
        missing = [k for k in records if k not in used]
        if missing:
            raise KeyError(f"records without an nn.Linear: {missing}")
    return replaced
