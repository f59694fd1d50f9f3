"""CPU restatement of the q/k RMSNorm + rotary embedding + KV store sequence -- TEST INFRASTRUCTURE.

Eager torch, in the reference's op order and dtypes:
  rms_norm            nanovllm/layers/layernorm.py:15-24 (RMSNorm.rms_forward)
  apply_rotary_emb    nanovllm/layers/rotary_embedding.py:6-14
  rope                nanovllm/layers/rotary_embedding.py:37-47 (RotaryEmbedding.forward / apply_rotary_emb_k)
  rope_table          nanovllm/layers/rotary_embedding.py:25-33 (the cos_sin_cache buffer)
  qk_norm_rope_store  nanovllm/models/qwen3.py:82-85 followed by attention.py:63-64 (and dflash.py:88-96 with no q)
plus fp64 forms of the same mathematics (rms_norm_f64, rope_f64, rope_table_f64) that the checks compare against.
"""
from __future__ import annotations

import numpy as np
import torch

from . import attention as attn


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    orig_dtype = x.dtype
    xf = x.to(torch.float32, copy=True)
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    xf.mul_(torch.rsqrt(var + eps))
    return xf.to(orig_dtype).mul_(weight)


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return torch.cat((y1, y2), dim=-1).to(x.dtype)


def rope_table(head_size: int, max_position: int, base: float) -> torch.Tensor:
    """[max_position, head_size] fp32: cos of the head_size/2 frequencies, then their sin."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float) / head_size))
    t = torch.arange(max_position, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def rope(positions: torch.Tensor, x: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """x [T, H, D] rotated by the table rows of positions [T]."""
    cos_sin = table.reshape(table.shape[0], -1)[positions].unsqueeze(1)
    cos, sin = cos_sin.chunk(2, dim=-1)
    return apply_rotary_emb(x, cos, sin)


def qk_norm_rope_store(positions, q, k, v, q_norm_weight, k_norm_weight, eps, table, k_cache, v_cache,
                       slot_mapping):
    """Returns (q_rotated or None, k_rotated); writes k_rotated and v into the caches (slot -1 skipped)."""
    if q is not None:
        q = rms_norm(q, q_norm_weight, eps) if q_norm_weight is not None else q
        q = rope(positions, q, table)
    k = rms_norm(k, k_norm_weight, eps) if k_norm_weight is not None else k
    k = rope(positions, k, table)
    if slot_mapping is not None:
        attn.store_kvcache(k, v, k_cache, v_cache, slot_mapping)
    return q, k


# ---------------------------------------------------------------- fp64 mathematics

def rms_norm_f64(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(weight, dtype=np.float64)


def rope_table_f64(head_size: int, max_position: int, base: float) -> np.ndarray:
    inv_freq = base ** (-np.arange(0, head_size, 2, dtype=np.float64) / head_size)
    angles = np.arange(max_position, dtype=np.float64)[:, None] * inv_freq[None, :]
    return np.concatenate([np.cos(angles), np.sin(angles)], axis=-1)


def rope_f64(positions: np.ndarray, x: np.ndarray, table: np.ndarray) -> np.ndarray:
    """Rotation of each (x[i], x[i + D/2]) pair by the table's angle: the complex product (x1 + i x2) e^{i theta}."""
    x = np.asarray(x, dtype=np.float64)
    half = x.shape[-1] // 2
    cs = np.asarray(table, dtype=np.float64)[np.asarray(positions)][:, None, :]
    c, s = cs[..., :half], cs[..., half:]
    z = (x[..., :half] + 1j * x[..., half:]) * (c + 1j * s)
    return np.concatenate([z.real, z.imag], axis=-1)
