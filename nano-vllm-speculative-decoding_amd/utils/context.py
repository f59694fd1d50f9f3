"""Attention metadata handed from the runner to every Attention.forward through one module-level context.

Same fields, defaults and functions as nanovllm/utils/context.py:5-31, so code written against the reference's
set_context / get_context drives the nvs_amd Attention unchanged.
"""
from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    """The field order is the positional order of set_context, which the reference's runner and verify graphs
    call positionally. query_len_per_seq: how many query rows each sequence contributes on the decode branch (1
    for plain decoding, the block length when a drafter scores a whole draft block). causal: whether query i of a
    sequence is limited to keys up to its own position (bottom-right aligned); a draft block sees all its keys and
    sets it False."""
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    query_len_per_seq: int = 1
    causal: bool = True


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0, slot_mapping=None,
                context_lens=None, block_tables=None, query_len_per_seq=1, causal=True) -> None:
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, slot_mapping, context_lens,
                       block_tables, query_len_per_seq, causal)


def reset_context() -> None:
    global _CONTEXT
    _CONTEXT = Context()
