"""CPU oracle of the paged KV store and paged multi-query attention (test infrastructure; see oracle/__init__.py).

Semantics (nanovllm/layers/attention.py:10-77, restated by the reference in tests/fake_paged_attention.py:14-41):
  * store: for token i with slot_mapping[i] >= 0, cache.flat[slot] = row i (fake_paged_attention.py:14-17;
    attention.py:21-30 skips slot -1).
  * attention: row r owns Lq queries starting at q0 and Lk keys; key j is cache[block_tables[r, j // bs], j % bs]
    (fake_paged_attention.py:29-31); head h reads kv head h // (H / Hkv) (repeat_interleave by group, :32-33);
    with causal, query i sees keys j <= Lk - Lq + i (bottom-right alignment, :36-37); softmax(scale * q K^T) V.
Row descriptions come either from cu_seqlens (verify branch, attention.py:67-70) or from context_lens with a
fixed query length (decode branch, attention.py:72-76).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    """cache.view(-1, Hkv, D)[slot] = row for every slot >= 0 (fake_paged_attention.py:14-17)."""
    live = slot_mapping >= 0
    slots = slot_mapping[live].long()
    k_cache.view(-1, *key.shape[1:])[slots] = key[live]
    v_cache.view(-1, *value.shape[1:])[slots] = value[live]


def row_layout(cu_seqlens_q=None, cu_seqlens_k=None, context_lens=None, query_len_per_seq=None):
    """[(q0, Lq, Lk)] per row, from the varlen (cu_seqlens) or the fixed-length (context_lens) description."""
    if cu_seqlens_q is not None:
        cq = [int(x) for x in cu_seqlens_q]
        ck = [int(x) for x in cu_seqlens_k]
        return [(cq[r], cq[r + 1] - cq[r], ck[r + 1] - ck[r]) for r in range(len(cq) - 1)]
    lens = [int(x) for x in context_lens]
    return [(r * query_len_per_seq, query_len_per_seq, lens[r]) for r in range(len(lens))]


def gather_keys(cache: np.ndarray, table_row, n_keys: int) -> np.ndarray:
    """Keys 0..n_keys-1 of one row through its block table: [n_keys, Hkv, D]."""
    block_size = cache.shape[1]
    j = np.arange(n_keys)
    blocks = np.asarray(table_row, dtype=np.int64)[j // block_size]
    return cache[blocks, j % block_size]


def paged_attention_f64(q, k_cache, v_cache, block_tables, rows, scale: float, causal: bool,
                        out: np.ndarray | None = None) -> np.ndarray:
    """fp64 brute force. q [T, H, D], caches [blocks, bs, Hkv, D] (any float dtype, upcast to fp64 exactly),
    rows from row_layout. Returns [T, H, D] fp64; tokens of no row (or of rows with Lq = 0) stay 0 (or keep out's
    values). A query that sees no key gets zeros."""
    q = _f64(q)
    kc = _f64(k_cache)
    vc = _f64(v_cache)
    tables = np.asarray(block_tables.cpu() if isinstance(block_tables, torch.Tensor) else block_tables)
    T, H, D = q.shape
    Hkv = kc.shape[2]
    group = H // Hkv
    result = np.zeros((T, H, D)) if out is None else out
    for r, (q0, lq, lk) in enumerate(rows):
        if lq <= 0:
            continue
        keys = gather_keys(kc, tables[r], lk)          # [Lk, Hkv, D]
        vals = gather_keys(vc, tables[r], lk)
        heads = np.arange(H) // group                  # kv head of every query head
        kq = keys[:, heads]                            # [Lk, H, D]
        vq = vals[:, heads]
        qr = q[q0:q0 + lq]                             # [Lq, H, D]
        scores = np.einsum("ihd,jhd->hij", qr, kq, optimize=True) * scale   # [H, Lq, Lk]
        j = np.arange(lk)[None, :]
        i = np.arange(lq)[:, None]
        visible = (j <= lk - lq + i) if causal else np.ones((lq, lk), dtype=bool)
        scores = np.where(visible[None], scores, -np.inf)
        m = scores.max(axis=-1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        w = np.exp(scores - m)
        z = w.sum(axis=-1, keepdims=True)
        p = np.divide(w, z, out=np.zeros_like(w), where=z > 0)
        result[q0:q0 + lq] = np.einsum("hij,jhd->ihd", p, vq, optimize=True)
    return result


def paged_attention_t32(q, k_cache, v_cache, block_tables, rows, scale: float, causal: bool) -> torch.Tensor:
    """torch fp32 restatement of the reference's CPU stand-in (fake_paged_attention.py:20-41): per row, gather the
    keys through the block table, repeat kv heads over their query-head group, bottom-right causal mask, SDPA.
    This is the CPU baseline that bench.py times. Returns [T, H, D] fp32."""
    q = q.float()
    kc = k_cache.float()
    vc = v_cache.float()
    block_size, Hkv, D = kc.shape[1], kc.shape[2], kc.shape[3]
    all_keys = kc.reshape(-1, Hkv, D)
    all_values = vc.reshape(-1, Hkv, D)
    T, H, _ = q.shape
    group = H // Hkv
    out = torch.zeros(T, H, D, dtype=torch.float32)
    tables = block_tables.cpu()
    for r, (q0, lq, lk) in enumerate(rows):
        if lq <= 0:
            continue
        positions = torch.arange(lk)
        slots = tables[r, positions // block_size].long() * block_size + positions % block_size
        keys = all_keys[slots].repeat_interleave(group, dim=1)
        values = all_values[slots].repeat_interleave(group, dim=1)
        queries = q[q0:q0 + lq]
        mask = None
        if causal:
            mask = positions[None, :] <= (lk - lq + torch.arange(lq))[:, None]
        o = F.scaled_dot_product_attention(queries.transpose(0, 1), keys.transpose(0, 1), values.transpose(0, 1),
                                           attn_mask=mask, scale=scale)
        out[q0:q0 + lq] = o.transpose(0, 1)
    return out


def _f64(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().to(torch.float64).numpy()
    return np.asarray(t, dtype=np.float64)
