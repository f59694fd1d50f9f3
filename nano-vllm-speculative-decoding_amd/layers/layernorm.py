"""RMSNorm of the decoder layer on one HIP launch, with the residual add of add_rms_forward fused in.
Replaces RMSNorm.forward (nanovllm/layers/layernorm.py:15-46) with the same call shape:
    norm(x)            -> rms_forward(x)
    norm(x, residual)  -> add_rms_forward(x, residual) = (normalised x + residual, x + residual)
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _lib


def _rows(x: torch.Tensor, hidden: int, name: str) -> tuple[torch.Tensor, int]:
    """x as [rows, hidden] with unit element stride; returns the 2-d view and its row stride."""
    if x.shape[-1] != hidden:
        raise ValueError(f"{name} has last dimension {x.shape[-1]}, expected {hidden}")
    x2 = x.view(-1, hidden) if x.dim() != 2 else x
    if x2.stride(-1) != 1:
        raise ValueError(f"{name} needs contiguous rows")
    return x2, x2.stride(0)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None,
             out: torch.Tensor | None = None) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """Without residual: dtype(dtype(x / sqrt(mean(x^2) + eps)) * weight) over the last dimension. With residual:
    s = x + residual in fp32, residual <- dtype(s) IN PLACE, and the norm of s; returns (out, residual) as
    add_rms_forward does. out may be x itself (not residual); a new tensor when None."""
    _lib.require_device(x, weight, residual, out)
    hidden = x.shape[-1]
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"rms_norm supports bf16 / fp16, got {x.dtype}")
    for name, t in (("weight", weight), ("residual", residual), ("out", out)):
        if t is not None and t.dtype != x.dtype:
            raise ValueError(f"{name} has dtype {t.dtype}, expected {x.dtype}")
    if weight.numel() != hidden or not weight.is_contiguous():
        raise ValueError(f"weight must be a contiguous [{hidden}] vector")
    x2, x_rs = _rows(x, hidden, "x")
    if out is None:
        out = torch.empty_like(x2)
    o2, o_rs = _rows(out, hidden, "out")
    r2, r_rs = (None, 0) if residual is None else _rows(residual, hidden, "residual")
    for name, t in (("out", o2), ("residual", r2)):
        if t is not None and t.shape[0] != x2.shape[0]:
            raise ValueError(f"{name} has {t.shape[0]} rows, x has {x2.shape[0]}")
    if r2 is not None and r2.data_ptr() == o2.data_ptr():
        raise ValueError("out must not alias residual")
    lib = _lib.load()
    _lib.check(lib.nvs_rms_norm(x2.data_ptr(), x_rs, _lib.ptr(r2), r_rs, weight.data_ptr(), float(eps),
                                o2.data_ptr(), o_rs, x2.shape[0], hidden, _lib.dtype_code(x.dtype),
                                _lib.stream_of(x)),
               "rms_norm")
    out = out.view(x.shape)
    return out if residual is None else (out, residual)


class RMSNorm(nn.Module):
    """Drop-in for nanovllm.layers.layernorm.RMSNorm: same constructor, weight parameter and forward."""

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if residual is None:
            return rms_norm(x, self.weight, self.eps)
        return rms_norm(x, self.weight, self.eps, residual=residual)
