"""Paged KV store and paged multi-query attention on MI355X, behind the reference's Attention interface.

Mirrors nanovllm/layers/attention.py:
  store_kvcache(key, value, k_cache, v_cache, slot_mapping)          attention.py:33-40
  Attention(num_heads, head_dim, scale, num_kv_heads).forward(q,k,v)  attention.py:43-77
and the two flash-attn entry points that forward calls, with the keyword arguments it passes:
  flash_attn_varlen_func(..., causal=True, block_table=...)  varlen_func: paged_attention_varlen when a block table
                                     is given (verify rows), otherwise the prefill function bound before the swap
  flash_attn_with_kvcache(q[B, Lq, H, D], ...)                paged_attention_with_kvcache (decode / draft block)
The paged calls run nvs_paged_attention (one HIP launch; when a row's keys are split, the last split of each unit
merges the partials inside it) and store_kvcache runs nvs_store_kvcache. bind(module) installs all three names on a
module written like the reference's.
"""
from __future__ import annotations

import ctypes

import torch
from torch import nn

from .. import _lib
from ..utils.context import get_context


def cache_geometry(k_cache: torch.Tensor, v_cache: torch.Tensor, num_kv_heads: int,
                   head_dim: int) -> tuple[int, int, int, int, int]:
    """(blocks, block_size, block_stride, token_stride, head_stride), in elements, of a K/V cache pair.

    A 4-D cache [blocks, block_size, Hkv, D] may have any strides with a contiguous head dimension: the
    token-major layout the reference allocates (model_runner.py:160), or a head-major view such as
    torch.empty(blocks, Hkv, block_size, D).transpose(1, 2), in which each (block, head) is one contiguous run.
    Other shapes must be contiguous [..., Hkv, D] and are one block of slots."""
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must have one shape and one set of strides")
    if tuple(k_cache.shape[-2:]) != (num_kv_heads, head_dim) or k_cache.stride(-1) != 1:
        raise ValueError(f"the caches must be [..., {num_kv_heads}, {head_dim}] with a contiguous last dimension")
    if k_cache.dim() == 4:
        blocks, block_size = k_cache.shape[:2]
        return blocks, block_size, k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    if not k_cache.is_contiguous():
        raise ValueError("a cache that is not [blocks, block_size, Hkv, D] must be contiguous")
    row = num_kv_heads * head_dim
    slots = k_cache.numel() // row
    return (1 if slots else 0), max(slots, 1), slots * row, row, head_dim


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    """Write token i's K/V rows into cache slot slot_mapping[i] (slot -1 = padding, skipped).

    key/value: [N, Hkv, D] with contiguous rows (value may be a strided view of the fused qkv output), the
    reference's preconditions (attention.py:36-39); k_cache/v_cache: [blocks, block_size, Hkv, D], token-major as
    the reference allocates them or head-major (cache_geometry); slot_mapping: [N] int32."""
    N, num_heads, head_dim = key.shape
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert slot_mapping.numel() == N
    _lib.require_device(key, value, k_cache, v_cache, slot_mapping)
    assert value.shape == key.shape and k_cache.dtype == key.dtype == value.dtype == v_cache.dtype
    geo = cache_geometry(k_cache, v_cache, num_heads, head_dim)
    if slot_mapping.dtype != torch.int32:
        slot_mapping = slot_mapping.to(torch.int32)
    if not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.contiguous()
    lib = _lib.load()
    _lib.check(lib.nvs_store_kvcache(key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
                                     k_cache.data_ptr(), v_cache.data_ptr(), *geo, slot_mapping.data_ptr(), N,
                                     num_heads, head_dim, _lib.dtype_code(key.dtype), _lib.stream_of(key)),
               "store_kvcache")


# The split merge's per-unit counters are kept in one zero-filled buffer per device, sized for at least this many
# (row, kv head, query tile) units so that graphs captured after smaller eager calls still fit in it.
_MIN_COUNTER_UNITS = 65536


def _paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                     cu_seqlens_q: torch.Tensor | None, cu_seqlens_k: torch.Tensor | None,
                     context_lens: torch.Tensor | None, query_len_per_seq: int, num_rows: int, max_seqlen_q: int,
                     max_seqlen_k: int, softmax_scale: float, causal: bool, out: torch.Tensor | None = None,
                     workspace: torch.Tensor | None = None) -> torch.Tensor:
    """q: [T, H, D] (last dim contiguous). Returns out [T, H, D] (written into `out` when given; `workspace`, a
    uint8 device buffer of at least the planned size, avoids an allocation per call)."""
    _lib.require_device(q, k_cache, v_cache, block_table, cu_seqlens_q, cu_seqlens_k, context_lens)
    T, H, D = q.shape
    assert k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride()
    _, block_size, Hkv, Dk = k_cache.shape
    assert Dk == D and H % Hkv == 0
    assert q.stride(-1) == 1 and k_cache.stride(-1) == 1
    assert q.dtype == k_cache.dtype == v_cache.dtype
    for name, t in (("block_table", block_table), ("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_k", cu_seqlens_k),
                    ("context_lens", context_lens)):
        if t is not None and t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32, got {t.dtype}")
    if block_table.stride(-1) != 1:
        block_table = block_table.contiguous()
    for t in (cu_seqlens_q, cu_seqlens_k, context_lens):
        if t is not None and not t.is_contiguous():
            raise ValueError("cu_seqlens / context_lens must be contiguous")
    if out is None:
        out = torch.empty((T, H, D), dtype=q.dtype, device=q.device)
    assert out.shape == (T, H, D) and out.dtype == q.dtype and out.stride(-1) == 1
    lib = _lib.load()
    nbytes = _lib.size_out()
    _lib.check(lib.nvs_paged_attention_workspace_size(num_rows, H, Hkv, D, max_seqlen_q, max_seqlen_k,
                                                      ctypes.byref(nbytes)),
               "paged_attention_workspace_size")
    ws = workspace if workspace is not None and workspace.numel() >= nbytes.value else \
        _lib.workspace(nbytes.value, q.device)
    # a plan that splits keys merges them in the launch: per-unit counters, zero between calls
    counters = None
    if nbytes.value > 0:
        q_tiles = ((H // Hkv) * max_seqlen_q + 31) // 32     # 32 packed query rows per tile
        units = num_rows * Hkv * q_tiles
        counters = _lib.persistent_workspace("attention_unit_counters", 4 * max(units, _MIN_COUNTER_UNITS), q.device)
    _lib.check(lib.nvs_paged_attention(
        q.data_ptr(), q.stride(0), q.stride(1), T, k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0],
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), block_table.data_ptr(), block_table.stride(0),
        block_table.shape[1], _lib.ptr(cu_seqlens_q), _lib.ptr(cu_seqlens_k), _lib.ptr(context_lens), query_len_per_seq,
        num_rows, max_seqlen_q, max_seqlen_k, H, Hkv, D, block_size, float(softmax_scale), int(bool(causal)),
        _lib.dtype_code(q.dtype), out.data_ptr(), out.stride(0), out.stride(1), _lib.ptr(counters), _lib.ptr(ws),
        nbytes.value, _lib.stream_of(q)),
        "paged_attention")
    return out


def paged_attention_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, max_seqlen_q: int,
                           cu_seqlens_q: torch.Tensor, max_seqlen_k: int, cu_seqlens_k: torch.Tensor,
                           softmax_scale: float, causal: bool = True,
                           block_table: torch.Tensor | None = None) -> torch.Tensor:
    """The call attention.py:67-70 makes with a block table: k, v are the paged caches [blocks, bs, Hkv, D];
    row r owns queries cu_seqlens_q[r]..cu_seqlens_q[r+1] and cu_seqlens_k[r+1]-cu_seqlens_k[r] keys.
    A call without a block table (k, v = the new rows of a prompt) is not paged attention: see varlen_func."""
    if block_table is None:
        raise NotImplementedError("paged_attention_varlen needs a block table; a prefill without a cached prefix "
                                  "goes to the prefill attention that varlen_func(prefill) forwards it to")
    return _paged_attention(q, k, v, block_table, cu_seqlens_q, cu_seqlens_k, None, 0, cu_seqlens_q.numel() - 1,
                            max_seqlen_q, max_seqlen_k, softmax_scale, causal)


def varlen_func(prefill=None):
    """A flash_attn_varlen_func for the module-level name Attention.forward calls (attention.py:67-70).

    The reference calls that one name for two different things:
      * block_table given (verify rows, prefill over a cached prefix): k, v are the paged caches. This runs
        nvs_paged_attention (paged_attention_varlen).
      * block_table None (prefill of prompts with no cached prefix, model_runner.py:176-185, and the runner's
        warm-up): k, v are the prompt's own new rows [N, Hkv, D], dense and unpaged. That is prompt attention, not
        the verify path, and it is handed unchanged to `prefill`: the function the name was bound to before the
        swap (flash-attn's, or any function with its signature).
    With prefill None such a call raises NotImplementedError."""

    def flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q, max_seqlen_k, cu_seqlens_k,
                               softmax_scale=None, causal=False, block_table=None, **kwargs):
        if block_table is None:
            if prefill is None:
                raise NotImplementedError("a prefill without a block table needs the prefill attention this name "
                                          "was bound to before the swap: bind(module) or varlen_func(prefill)")
            return prefill(q, k, v, max_seqlen_q=max_seqlen_q, cu_seqlens_q=cu_seqlens_q, max_seqlen_k=max_seqlen_k,
                           cu_seqlens_k=cu_seqlens_k, softmax_scale=softmax_scale, causal=causal,
                           block_table=None, **kwargs)
        if kwargs:
            raise TypeError(f"paged attention takes no further arguments, got {sorted(kwargs)}")
        if softmax_scale is None:
            softmax_scale = q.shape[-1] ** -0.5
        return paged_attention_varlen(q, k, v, max_seqlen_q, cu_seqlens_q, max_seqlen_k, cu_seqlens_k,
                                      softmax_scale, causal, block_table)

    flash_attn_varlen_func.prefill = prefill
    return flash_attn_varlen_func


def paged_attention_with_kvcache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                 cache_seqlens: torch.Tensor, block_table: torch.Tensor, softmax_scale: float,
                                 causal: bool = True, max_seqlen_k: int | None = None) -> torch.Tensor:
    """The call attention.py:72-75 makes: q [B, Lq, H, D] sequence-major, cache_seqlens [B] keys per row.
    Returns [B, Lq, H, D]. max_seqlen_k bounds every cache_seqlens entry; it defaults to the width of the block
    table (what the table can address), which keeps the launch independent of device values."""
    B, Lq, H, D = q.shape
    if max_seqlen_k is None:
        max_seqlen_k = block_table.shape[1] * k_cache.shape[1]
    out = _paged_attention(q.reshape(B * Lq, H, D), k_cache, v_cache, block_table, None, None, cache_seqlens, Lq,
                           B, Lq, max_seqlen_k, softmax_scale, causal)
    return out.view(B, Lq, H, D)


# The names Attention.forward calls in the reference. This module's own Attention looks them up here at call time,
# so they can be rebound (set_prefill_attention, or a test's monkeypatch) as the reference's module attributes can.
flash_attn_varlen_func = varlen_func(None)
flash_attn_with_kvcache = paged_attention_with_kvcache

_BOUND_NAMES = ("store_kvcache", "flash_attn_varlen_func", "flash_attn_with_kvcache")


def bind(module) -> dict:
    """Swap the attention names of a module written like nanovllm/layers/attention.py for this library's.

    module.store_kvcache          -> store_kvcache (nvs_store_kvcache); DFlashDraftModel.store_context_kv calls it
                                     through the module attribute too (dflash.py:95)
    module.flash_attn_with_kvcache -> paged_attention_with_kvcache (nvs_paged_attention, fixed-Lq mode)
    module.flash_attn_varlen_func  -> varlen_func(previous): paged calls run nvs_paged_attention, calls without a
                                     block table keep going to the function bound there before
    Binding twice keeps the first prefill function. Returns the previous bindings (for unbind)."""
    previous = {name: getattr(module, name, None) for name in _BOUND_NAMES}
    prefill = previous["flash_attn_varlen_func"]
    prefill = getattr(prefill, "prefill", prefill)    # already bound: keep the prefill it forwards to
    module.store_kvcache = store_kvcache
    module.flash_attn_varlen_func = varlen_func(prefill)
    module.flash_attn_with_kvcache = paged_attention_with_kvcache
    return previous


def unbind(module, previous: dict) -> None:
    """Restore the bindings bind() returned."""
    for name, value in previous.items():
        setattr(module, name, value)


def set_prefill_attention(prefill) -> None:
    """Where this module's own Attention sends prefill calls without a block table (None: they raise)."""
    global flash_attn_varlen_func
    flash_attn_varlen_func = varlen_func(prefill)


class Attention(nn.Module):
    """attention.py:43-77 on nvs_amd kernels: store the new K/V, then paged attention over the cache."""

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])

    def forward(self, q: torch.Tensor, k: torch.Tensor | None, v: torch.Tensor | None) -> torch.Tensor:
        """k = v = None: the new K/V rows are already in the cache (qk_norm_rope_store wrote them).
        The three kernels are the module-level names store_kvcache / flash_attn_varlen_func /
        flash_attn_with_kvcache, looked up at call time."""
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        if k is not None and k_cache.numel() and v_cache.numel():
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping)
        if context.is_prefill:
            paged = context.block_tables is not None      # a cached prefix: attend over the pages
            return flash_attn_varlen_func(q, k_cache if paged else k, v_cache if paged else v,
                                          max_seqlen_q=context.max_seqlen_q, cu_seqlens_q=context.cu_seqlens_q,
                                          max_seqlen_k=context.max_seqlen_k, cu_seqlens_k=context.cu_seqlens_k,
                                          softmax_scale=self.scale, causal=True, block_table=context.block_tables)
        # decode / draft block: query_len_per_seq queries per sequence, rows grouped by sequence
        o = flash_attn_with_kvcache(q.view(-1, context.query_len_per_seq, self.num_heads, self.head_dim),
                                    k_cache, v_cache, cache_seqlens=context.context_lens,
                                    block_table=context.block_tables, softmax_scale=self.scale,
                                    causal=context.causal)
        return o.view(-1, self.num_heads, self.head_dim)
