"""The per-head q/k RMSNorm, the rotary embedding and the paged KV store in one HIP launch.

Replaces, for layers whose qkv projection has no bias, the lines of Qwen3Attention.forward between the qkv split and
the attention kernel (nanovllm/models/qwen3.py:82-85) together with the store_kvcache call that opens
Attention.forward (nanovllm/layers/attention.py:63-64):

    q = self.q_norm(q); k = self.k_norm(k)                      RMSNorm.rms_forward, layernorm.py:15-24
    q, k = self.rotary_emb(positions, q, k)                     RotaryEmbedding.forward, rotary_embedding.py:37-47
    store_kvcache(k, v, k_cache, v_cache, slot_mapping)         attention.py:33-40

and, with q=None, the draft model's context-KV write (DFlashDraftModel.store_context_kv, dflash.py:88-96).
"""
from __future__ import annotations

import torch

from .. import _lib
from .attention import cache_geometry


def rope_cos_sin_cache(head_size: int, max_position: int, base: float, device: torch.device) -> torch.Tensor:
    """The reference's cos_sin_cache buffer (rotary_embedding.py:25-33): [max_position, head_size] fp32, cos of the
    head_size/2 frequencies then their sin, built with the same torch ops (a one-time table, not a per-step op)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float, device=device) / head_size))
    t = torch.arange(max_position, dtype=torch.float, device=device)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def _token_view(x: torch.Tensor, heads: int, head_dim: int, name: str) -> int:
    """Token stride of x [T, heads, head_dim] whose heads are contiguous (a view of the fused qkv output is fine)."""
    if x.dim() != 3 or x.shape[1] != heads or x.shape[2] != head_dim:
        raise ValueError(f"{name} must be [T, {heads}, {head_dim}], got {tuple(x.shape)}")
    if x.stride(2) != 1 or x.stride(1) != head_dim:
        raise ValueError(f"{name} needs contiguous heads (strides [*, {head_dim}, 1]), got {x.stride()}")
    return x.stride(0)


def qk_norm_rope_store(positions: torch.Tensor, q: torch.Tensor | None, k: torch.Tensor, v: torch.Tensor,
                       q_norm_weight: torch.Tensor | None, k_norm_weight: torch.Tensor | None, eps: float,
                       cos_sin_cache: torch.Tensor, k_cache: torch.Tensor | None, v_cache: torch.Tensor | None,
                       slot_mapping: torch.Tensor | None, q_out: torch.Tensor | None = None,
                       k_out: torch.Tensor | None = None) -> torch.Tensor | None:
    """Normalise and rotate q [T, Hq, D] and k [T, Hkv, D], write k and v [T, Hkv, D] into cache slot
    slot_mapping[t] (-1 = padding, skipped), and return the rotated q (written into q_out when given; q_out may be
    q itself). q=None runs the keys-only path and returns None. A None norm weight skips that norm (layers with a
    qkv bias). cos_sin_cache: the rotary table, [P, D] or the reference's [P, 1, D], fp32. k_out: optional
    [T, Hkv, D] buffer for the rotated keys (the paged attention reads them from the cache instead). The caches may
    be token-major or head-major [blocks, block_size, Hkv, D] views (attention.cache_geometry)."""
    T, hkv, head_dim = k.shape
    hq = 0 if q is None else q.shape[1]
    _lib.require_device(positions, q, k, v, q_norm_weight, k_norm_weight, cos_sin_cache, k_cache, v_cache,
                        slot_mapping, q_out, k_out)
    dtype = k.dtype
    if dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"qk_norm_rope_store supports bf16 / fp16 activations, got {dtype}")
    for name, t in (("q", q), ("v", v), ("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight),
                    ("k_cache", k_cache), ("v_cache", v_cache), ("q_out", q_out), ("k_out", k_out)):
        if t is not None and t.dtype != dtype:
            raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")
    k_ts = _token_view(k, hkv, head_dim, "k")
    v_ts = _token_view(v, hkv, head_dim, "v")
    q_ts = _token_view(q, hq, head_dim, "q") if q is not None else 0
    if q is not None and q_out is None:
        q_out = torch.empty(T, hq, head_dim, dtype=dtype, device=q.device)
    qo_ts = _token_view(q_out, hq, head_dim, "q_out") if q_out is not None else 0
    ko_ts = _token_view(k_out, hkv, head_dim, "k_out") if k_out is not None else 0
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if w is not None and (w.numel() != head_dim or not w.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous [{head_dim}] vector")
    cs = cos_sin_cache.reshape(cos_sin_cache.shape[0], -1)
    if cs.dtype != torch.float32 or cs.shape[1] != head_dim or not cs.is_contiguous():
        raise ValueError(f"cos_sin_cache must be contiguous fp32 [P, {head_dim}] (or [P, 1, {head_dim}])")
    if positions.dtype != torch.int64 or positions.numel() != T:
        raise ValueError("positions must be int64 with one entry per token")
    positions = positions.contiguous()
    geo = (0, 1, 0, 0, 0)
    if slot_mapping is not None:
        if k_cache is None or v_cache is None:
            raise ValueError("slot_mapping needs k_cache and v_cache")
        if slot_mapping.numel() != T:
            raise ValueError("slot_mapping needs one entry per token")
        geo = cache_geometry(k_cache, v_cache, hkv, head_dim)
        slot_mapping = slot_mapping.to(torch.int32).contiguous()
    lib = _lib.load()
    _lib.check(lib.nvs_qk_norm_rope_store(_lib.ptr(q), q_ts, k.data_ptr(), k_ts, v.data_ptr(), v_ts,
                                          positions.data_ptr(), _lib.ptr(q_norm_weight), _lib.ptr(k_norm_weight),
                                          float(eps), cs.data_ptr(), cs.shape[0], _lib.ptr(slot_mapping),
                                          _lib.ptr(k_cache), _lib.ptr(v_cache), *geo, _lib.ptr(q_out), qo_ts,
                                          _lib.ptr(k_out), ko_ts, T, hq, hkv, head_dim, _lib.dtype_code(dtype),
                                          _lib.stream_of(k)),
               "qk_norm_rope_store")
    return q_out
