"""SiLU-and-mul of the Qwen3 MLP on one HIP launch. Replaces SiluAndMul.forward (nanovllm/layers/activation.py:8-11):
x = [gate | up] along the last dimension, out = silu(gate) * up, computed in fp32 and rounded once."""
from __future__ import annotations

import torch
from torch import nn

from .. import _lib


def silu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """[..., 2 W] -> [..., W] in the input dtype (bf16 / fp16); rows need unit element stride."""
    _lib.require_device(x, out)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"silu_and_mul supports bf16 / fp16, got {x.dtype}")
    if x.shape[-1] % 2:
        raise ValueError("the last dimension must hold gate and up halves")
    width = x.shape[-1] // 2
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        raise ValueError("x needs contiguous rows")
    if out is None:
        out = torch.empty(*x.shape[:-1], width, dtype=x.dtype, device=x.device)
    o2 = out.view(-1, width)
    if out.dtype != x.dtype or o2.shape[0] != x2.shape[0] or o2.stride(-1) != 1:
        raise ValueError("out must be [..., W] in the input dtype with contiguous rows")
    lib = _lib.load()
    _lib.check(lib.nvs_silu_and_mul(x2.data_ptr(), x2.stride(0), o2.data_ptr(), o2.stride(0), x2.shape[0], width,
                                    _lib.dtype_code(x.dtype), _lib.stream_of(x)),
               "silu_and_mul")
    return out


class SiluAndMul(nn.Module):
    """Drop-in for nanovllm.layers.activation.SiluAndMul."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return silu_and_mul(x)
