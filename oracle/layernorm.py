"""Oracle of the decoder layer's elementwise ops: RMSNorm (with the residual add) and SiLU-and-mul, in eager torch
on the CPU, op by op as the reference writes them. TEST INFRASTRUCTURE: only tests/ use it, to compare the kernels
against.

Reference: RMSNorm.rms_forward / add_rms_forward (nanovllm/layers/layernorm.py:15-40), SiluAndMul.forward
(nanovllm/layers/activation.py:8-11). The reference runs both under torch.compile, which keeps the fp32
intermediates of an expression but honours the explicit .to(dtype) casts; the restatement follows that: the
norm rounds where the reference casts, silu(gate) * up is rounded once.
"""
from __future__ import annotations

import numpy as np
import torch


def rms_forward(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """layernorm.py:16-24: x fp32, var = mean(x^2), x * rsqrt(var + eps), cast to the input dtype, times weight."""
    dtype = x.dtype
    xf = x.to(torch.float32, copy=True)
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return xf.to(dtype) * weight


def add_rms_forward(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                    eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """layernorm.py:26-40: s = float(x) + float(residual); residual' = dtype(s); the norm of the fp32 s."""
    dtype = x.dtype
    s = x.float() + residual.float()
    new_residual = s.to(dtype)
    var = s.pow(2).mean(dim=-1, keepdim=True)
    s = s * torch.rsqrt(var + eps)
    return s.to(dtype) * weight, new_residual


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """activation.py:8-11: gate, up = x.chunk(2, -1); silu(gate) * up, fp32 inside, one rounding."""
    gate, up = x.float().chunk(2, -1)
    return (torch.nn.functional.silu(gate) * up).to(x.dtype)


def rms_norm_f64(x: np.ndarray, weight: np.ndarray, eps: float, residual: np.ndarray | None = None) -> np.ndarray:
    """The mathematics in fp64, no intermediate rounding: (x [+ residual]) / sqrt(mean((x [+ residual])^2) + eps)
    * weight."""
    s = x.astype(np.float64) + (0.0 if residual is None else residual.astype(np.float64))
    return s / np.sqrt((s * s).mean(axis=-1, keepdims=True) + eps) * weight.astype(np.float64)


def silu_and_mul_f64(x: np.ndarray) -> np.ndarray:
    w = x.shape[-1] // 2
    g, u = x[..., :w].astype(np.float64), x[..., w:].astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u
