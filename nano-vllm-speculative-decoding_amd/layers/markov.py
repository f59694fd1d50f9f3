"""DSpark's Markov rows on the MI355X path, with a sparse candidate format for q.

Replaces DFlashDrafter._sample_markov / _markov_rows (nanovllm/engine/speculative.py:145-184): the k draft rows
are drawn left to right, row j's logits biased by the Markov head on the token drawn at row j-1 (the anchor for
row 0), the noise of all k rows drawn before row 0 in one call. When every row truncates with top-k, a row is drawn
among its top num_candidates() logits by one nvs_markov_draw launch. The launch writes that row's q as candidate
rows, the kept token ids with their probabilities, instead of scattering them over a zeroed [B, k, V] tensor
(272 MB at batch 64). The candidates hold the row's kept tokens in value order, ties by index. Otherwise (some row
does not truncate) a row is drawn over the whole vocabulary with probs_from_logits and race, as the reference does.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable

import torch

from .. import _lib
from . import spec_sampler as ss

TIE_MARGIN = 64
# The widest top-k window nvs_markov_draw serves; wider batches draw their candidate rows with torch's topk and this
# library's probs_from_logits and race, as the reference composes them (speculative.py:178-181).
MARKOV_DRAW_MAX_TOP_K = 1024


def num_candidates(max_top_k: int, all_top_k: bool, vocab: int) -> int:
    """speculative.py:46-50: a candidate row holds the top max_top_k + 64 logits; 0 means the whole vocabulary."""
    return min(max_top_k + TIE_MARGIN, vocab) if all_top_k else 0


@dataclass
class CandidateRows:
    """Sparse q of a draft block: ids [B, k, C] int32 and probs [B, k, C] fp32. Each row holds its kept tokens in
    value order, then id -1 with probability 0. q[b, j, v] = probs[b, j, c] where ids[b, j, c] == v, else 0."""
    ids: torch.Tensor
    probs: torch.Tensor

    def to_dense(self, vocab: int) -> torch.Tensor:
        """The reference's [B, k, V] draft_probs (zero outside the candidates)."""
        q = torch.zeros(*self.ids.shape[:-1], vocab, dtype=torch.float32, device=self.ids.device)
        live = self.ids >= 0
        # padding entries add an exact 0 at index 0 (a plain scatter could overwrite token 0's probability)
        q.scatter_add_(-1, torch.where(live, self.ids, 0).long(), torch.where(live, self.probs, 0.0))
        return q


def markov_draw(row_logits: torch.Tensor, sampling: ss.SamplingTensors, candidates: int, noise: torch.Tensor,
                ids: torch.Tensor, probs: torch.Tensor, draws: torch.Tensor,
                bias: torch.Tensor | None = None) -> None:
    """One candidate row for every sequence: row_logits [B, V] (rows with unit element stride, any row stride),
    bias [B, V] the row's Markov bias or None, noise [B, >= C] fp32 by candidate rank. Writes ids [B, C] int32,
    probs [B, C] fp32 and draws [B] int64 (a column view of the drafts is fine). The kernel adds the bias with the
    reference's rounding when it has the logits' dtype; otherwise torch adds it first (the reference's promotion)."""
    _lib.require_device(row_logits, bias, noise, ids, probs, draws, sampling.temperatures, sampling.top_k)
    if sampling.temperatures is None:
        raise ValueError("greedy rows are drawn by argmax, not by markov_draw")
    if row_logits.dim() != 2 or row_logits.stride(-1) != 1:
        raise ValueError("row_logits must be [B, V] with contiguous rows")
    batch, vocab = row_logits.shape
    for name, t, dtype in (("noise", noise, torch.float32), ("ids", ids, torch.int32), ("probs", probs, torch.float32)):
        if t.dtype != dtype or t.dim() != 2 or t.shape[0] != batch or t.shape[1] < candidates or t.stride(-1) != 1:
            raise ValueError(f"{name} must be [B, >= {candidates}] {dtype} with contiguous rows")
    if ids.stride(0) != probs.stride(0):
        raise ValueError("ids and probs must share their row stride")
    if draws.dtype != torch.int64 or draws.shape != (batch,):
        raise ValueError("draws must be [B] int64")
    lib = _lib.load()
    nbytes = _lib.size_out()
    _lib.check(lib.nvs_markov_draw_workspace_size(batch, vocab, candidates, ctypes.byref(nbytes)),
               "markov_draw_workspace_size")
    if bias is not None and (bias.dtype != row_logits.dtype or bias.shape != row_logits.shape or nbytes.value == 0
                             or bias.stride(-1) != 1):
        row_logits, bias = row_logits + bias, None
    temps = ss._contig(sampling.temperatures, torch.float32)
    top_k = ss._contig(sampling.top_k, torch.int64)
    top_p = ss._contig(sampling.top_p, torch.float32)
    ws = _lib.workspace(nbytes.value, row_logits.device)
    # the split draw's per-row counters (the row's last segment merges), zero between calls
    counters = ss._row_counters("markov_row_counters", batch, row_logits.device)
    _lib.check(lib.nvs_markov_draw(row_logits.data_ptr(), _lib.dtype_code(row_logits.dtype), row_logits.stride(0),
                                   _lib.ptr(bias), 0 if bias is None else bias.stride(0), batch, vocab,
                                   temps.data_ptr(), top_k.data_ptr(), _lib.ptr(top_p), sampling.max_top_k,
                                   int(sampling.has_top_p), candidates, noise.data_ptr(), noise.stride(0),
                                   ids.data_ptr(), probs.data_ptr(), ids.stride(0), draws.data_ptr(), draws.stride(0),
                                   counters.data_ptr(), _lib.ptr(ws), nbytes.value, _lib.stream_of(row_logits)),
               "markov_draw")


def markov_rows(logits: torch.Tensor, prev: torch.Tensor, sampling: ss.SamplingTensors,
                markov_bias: Callable[[torch.Tensor], torch.Tensor], noise: torch.Tensor | None,
                drafts: torch.Tensor, candidates: int):
    """_markov_rows (speculative.py:163-184): draw the k rows into drafts [B, k] left to right, prev [B] holding the
    anchors. Returns CandidateRows with candidates, a dense [B, k, V] q without, None when greedy."""
    batch, k, vocab = logits.shape
    greedy = sampling.temperatures is None
    if candidates:
        rows = CandidateRows(torch.empty(batch, k, candidates, dtype=torch.int32, device=logits.device),
                             torch.empty(batch, k, candidates, dtype=torch.float32, device=logits.device))
    q = None if greedy or candidates else torch.empty(batch, k, vocab, dtype=torch.float32, device=logits.device)
    for row in range(k):
        if candidates and not greedy and sampling.max_top_k <= MARKOV_DRAW_MAX_TOP_K:
            # the kernel reads the row of the block's logits and the bias, and adds them itself
            markov_draw(logits[:, row], sampling, candidates, noise[:, row], rows.ids[:, row], rows.probs[:, row],
                        drafts[:, row], bias=markov_bias(prev))
        elif candidates and not greedy:
            # a window wider than the kernel's: the row's top `candidates` logits as the candidate row
            values, ids = (logits[:, row] + markov_bias(prev)).topk(candidates, dim=-1)
            probs = ss.probs_from_logits(values, sampling)
            drafts[:, row] = ids.gather(-1, ss.race(probs, noise[:, row]).unsqueeze(-1)).squeeze(-1)
            rows.ids[:, row] = ids.to(torch.int32)
            rows.probs[:, row] = probs
        else:
            row_logits = logits[:, row] + markov_bias(prev)
            if greedy:
                drafts[:, row] = row_logits.argmax(dim=-1)
            else:
                q[:, row] = ss.probs_from_logits(row_logits, sampling)
                drafts[:, row] = ss.race(q[:, row], noise[:, row])
        prev = drafts[:, row]
    if greedy:
        return None
    return rows if candidates else q


def sample_markov(logits: torch.Tensor, anchors: torch.Tensor, sampling: ss.SamplingTensors,
                  markov_bias: Callable[[torch.Tensor], torch.Tensor], generator: torch.Generator | None):
    """_sample_markov (speculative.py:145-161): logits [B, k, V] of the draft block, anchors [B] int64 (each
    sequence's last token). Draws the noise of all k rows first ([B, k, C], or [B, k, V] without candidates) from
    the generator, then the rows. Returns drafts [B, k] int64 and q: CandidateRows, a dense [B, k, V], or None."""
    batch, k, vocab = logits.shape
    drafts = torch.empty(batch, k, dtype=torch.int64, device=logits.device)
    candidates = num_candidates(sampling.max_top_k, sampling.all_top_k, vocab)
    noise = None
    if sampling.temperatures is not None:
        noise = ss.exponential_noise_(torch.empty(batch, k, candidates or vocab, dtype=torch.float32,
                                                  device=logits.device), generator)
    q = markov_rows(logits, anchors, sampling, markov_bias, noise, drafts, candidates)
    return drafts, q
