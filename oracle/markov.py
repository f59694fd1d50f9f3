"""Oracle of DSpark's Markov rows: TEST INFRASTRUCTURE (only tests/ use it, to compare the kernels against).

Restates DFlashDrafter._sample_markov / _markov_rows (nanovllm/engine/speculative.py:145-184) and num_candidates
(:46-50) on the CPU with the oracle's sampler functions. The Markov head is a function prev -> [B, V] bias, as the
reference's own tests pass it (tests/test_dspark_propose.py:24-33). The rows are drawn left to right: row j's logits
get the bias of the token drawn at row j-1 (the anchor for row 0).

Candidate order: torch.topk orders tied values in an unspecified way, and the race assigns noise by candidate rank,
so the restatement fixes the order as value descending, then index ascending (a stable sort). The kernel uses the
same order. Any fixed order draws from the same distribution, because the noise values are independent and
identically distributed.
"""
from __future__ import annotations

import torch

from . import spec_sampler as ss

TIE_MARGIN = 64


def num_candidates(max_top_k: int, all_top_k: bool, vocab: int) -> int:
    """speculative.py:46-50: the top max_top_k + 64 logits when every row truncates, else 0 (the whole vocabulary)."""
    return min(max_top_k + TIE_MARGIN, vocab) if all_top_k else 0


def topk_ordered(x: torch.Tensor, c: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The c largest values of each row and their indices, value descending, ties by index ascending."""
    values, ids = torch.sort(x, dim=-1, descending=True, stable=True)
    return values[..., :c], ids[..., :c]


def markov_rows(logits: torch.Tensor, anchors: torch.Tensor, bias_fn, temperatures: torch.Tensor | None,
                top_k: torch.Tensor, top_p: torch.Tensor, max_top_k: int, has_top_p: bool, all_top_k: bool,
                noise: torch.Tensor | None):
    """logits [B, k, V]; anchors [B] (the token before row 0); noise [B, k, C or V] (None when greedy).
    Returns drafts [B, k] int64, q [B, k, V] fp32 (None when greedy), and, for candidate rows, the candidate ids
    [B, k, C] and their probabilities [B, k, C] (else None, None)."""
    batch, k, vocab = logits.shape
    drafts = torch.empty(batch, k, dtype=torch.int64)
    greedy = temperatures is None
    cands = 0 if greedy else num_candidates(max_top_k, all_top_k, vocab)
    q = None if greedy else torch.zeros(batch, k, vocab, dtype=torch.float32)
    cand_ids = torch.zeros(batch, k, cands, dtype=torch.int64) if cands else None
    cand_probs = torch.zeros(batch, k, cands, dtype=torch.float32) if cands else None
    prev = anchors
    for row in range(k):
        row_logits = logits[:, row] + bias_fn(prev)
        if greedy:
            prev = row_logits.argmax(dim=-1)
        elif cands:
            values, ids = topk_ordered(row_logits, cands)
            probs = ss.probs_from_logits(values, temperatures, top_k, top_p, max_top_k, has_top_p)
            prev = ids.gather(-1, ss.race(probs, noise[:, row]).unsqueeze(-1)).squeeze(-1)
            q[:, row].scatter_(-1, ids, probs)
            cand_ids[:, row] = ids
            cand_probs[:, row] = probs
        else:
            q[:, row] = ss.probs_from_logits(row_logits, temperatures, top_k, top_p, max_top_k, has_top_p)
            prev = ss.race(q[:, row], noise[:, row])
        drafts[:, row] = prev
    return drafts, q, cand_ids, cand_probs
