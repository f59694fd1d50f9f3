"""torch-CPU oracle of the speculative sampler (test infrastructure; see oracle/__init__.py).

A restatement of nanovllm/layers/spec_sampler.py with the random draws made explicit: the uniforms [B, k] and the
exponential noise [B, V] are arguments, so the HIP kernels and this oracle can be fed identical numbers. The
op sequence is the reference's, op for op, because bitwise agreement of the decisions depends on it:
  probs_from_logits      spec_sampler.py:65-69   fp32 upcast, IEEE division by the temperature, softmax
  truncate_logits        spec_sampler.py:72-96   topk(max_top_k) with multiplicity, ranks >= top_k -> -inf,
                                                 threshold = k-th candidate, top-p over the candidates' softmax
                                                 (mass_before = cumsum - nucleus < top_p), ties kept, top_k = 0 rows
                                                 untouched
  race                   spec_sampler.py:104-106 argmax(w / E), first index on ties
  verified_positions     spec_sampler.py:172-180
  accept_random_varlen   spec_sampler.py:123-150 accept iff u * q[d] < p[d] and verified, accepted prefix by
                                                 cumprod, residual max(p - q, 0) at the first rejection, p at the
                                                 bonus position
  accept_greedy_varlen   spec_sampler.py:161-169
Per-row parameters are [P] tensors broadcast over the middle dims of [P, n, V] logits (or per token for [T, V]).
"""
from __future__ import annotations

import torch

NOISE_FLOOR = 1e-10
NEG_INF = float("-inf")


def _rowwise(values: torch.Tensor, ndim: int) -> torch.Tensor:
    return values.reshape(values.shape[0], *([1] * (ndim - 1)))


def truncate_logits(scaled: torch.Tensor, top_k: torch.Tensor, top_p: torch.Tensor, max_top_k: int,
                    has_top_p: bool) -> torch.Tensor:
    if max_top_k == 0:
        return scaled
    nd = scaled.ndim
    k_row = _rowwise(top_k, nd)
    k_eff = k_row.clamp(min=1)
    width = min(max_top_k, scaled.shape[-1])
    cand = scaled.topk(width, dim=-1).values
    cand = cand.masked_fill(torch.arange(width) >= k_eff, NEG_INF)
    at = (k_eff - 1).clamp(max=width - 1).expand(*cand.shape[:-1], 1)
    cut = cand.gather(-1, at)
    if has_top_p:
        nucleus = torch.softmax(cand, dim=-1)
        before = nucleus.cumsum(dim=-1) - nucleus
        kept = (before < _rowwise(top_p, nd)).sum(dim=-1, keepdim=True)
        cut = torch.maximum(cut, cand.gather(-1, kept - 1))
    cut = torch.where(k_row > 0, cut, torch.full_like(cut, NEG_INF))
    return scaled.masked_fill(scaled < cut, NEG_INF)


def probs_from_logits(logits: torch.Tensor, temperatures: torch.Tensor, top_k: torch.Tensor, top_p: torch.Tensor,
                      max_top_k: int, has_top_p: bool) -> torch.Tensor:
    scaled = logits.float() / _rowwise(temperatures, logits.ndim)
    return torch.softmax(truncate_logits(scaled, top_k, top_p, max_top_k, has_top_p), dim=-1)


def exponential_noise(shape, generator: torch.Generator | None) -> torch.Tensor:
    return torch.empty(shape).exponential_(1.0, generator=generator).clamp_min_(NOISE_FLOOR)


def race(weights: torch.Tensor, noise: torch.Tensor) -> torch.Tensor:
    return (weights / noise).argmax(dim=-1)


def verified_positions(verified_lens: torch.Tensor, num_drafts: int):
    starts = verified_lens.cumsum(0) - verified_lens
    last = (verified_lens - 1).unsqueeze(1)
    steps = torch.arange(num_drafts)
    return starts, starts.unsqueeze(1) + torch.minimum(steps, last), steps < last


def accept_random_varlen(p: torch.Tensor, q: torch.Tensor, drafts: torch.Tensor, verified_lens: torch.Tensor,
                         uniforms: torch.Tensor, noise: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    batch, k = drafts.shape
    starts, positions, verified = verified_positions(verified_lens, k)
    p_at = p[positions, drafts]
    q_at = q.gather(-1, drafts.unsqueeze(-1)).squeeze(-1)
    accepted = (uniforms * q_at < p_at) & verified
    n_accept = accepted.long().cumprod(dim=-1).sum(dim=-1)
    p_next = p[starts + n_accept]
    q_next = q[torch.arange(batch), n_accept.clamp(max=k - 1)]
    residual = (p_next - q_next).clamp_(min=0)
    bonus = (n_accept == verified_lens - 1).unsqueeze(-1)
    return n_accept, race(torch.where(bonus, p_next, residual), noise)


def accept_random(p: torch.Tensor, q: torch.Tensor, drafts: torch.Tensor, uniforms: torch.Tensor,
                  noise: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Every row verifies all k drafts: p [B, k+1, V]."""
    batch, k = drafts.shape
    lens = torch.full((batch,), k + 1, dtype=torch.int64)
    return accept_random_varlen(p.flatten(0, 1), q, drafts, lens, uniforms, noise)


def draws(batch: int, num_drafts: int, vocab: int, generator: torch.Generator | None):
    """The uniforms, then the race noise: the order in which spec_sampler.py:141,149 consume the generator."""
    uniforms = torch.rand(batch, num_drafts, generator=generator)
    return uniforms, exponential_noise((batch, vocab), generator)


def accept_random_varlen_gen(p, q, drafts, verified_lens, generator):
    """accept_random_varlen drawing its own random numbers, as the reference does."""
    uniforms, noise = draws(drafts.shape[0], drafts.shape[1], p.shape[-1], generator)
    return accept_random_varlen(p, q, drafts, verified_lens, uniforms, noise)


def accept_random_gen(p, q, drafts, generator):
    uniforms, noise = draws(drafts.shape[0], drafts.shape[1], p.shape[-1], generator)
    return accept_random(p, q, drafts, uniforms, noise)


def sample(weights: torch.Tensor, generator: torch.Generator | None) -> torch.Tensor:
    return race(weights, exponential_noise(weights.shape, generator))


def accept_greedy_varlen(logits: torch.Tensor, drafts: torch.Tensor,
                         verified_lens: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    tokens = logits.argmax(dim=-1)
    starts, positions, verified = verified_positions(verified_lens, drafts.shape[1])
    accepted = (tokens[positions] == drafts) & verified
    n_accept = accepted.long().cumprod(dim=-1).sum(dim=-1)
    return n_accept, tokens[starts + n_accept]


def accept_greedy(logits: torch.Tensor, drafts: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    batch, k = drafts.shape
    lens = torch.full((batch,), k + 1, dtype=torch.int64)
    return accept_greedy_varlen(logits.flatten(0, 1), drafts, lens)


def accept_from_logits(logits: torch.Tensor, q: torch.Tensor, drafts: torch.Tensor, temperatures: torch.Tensor,
                       top_k: torch.Tensor, top_p: torch.Tensor, max_top_k: int, has_top_p: bool,
                       verified_lens: torch.Tensor | None, uniforms: torch.Tensor, noise: torch.Tensor):
    """SpeculativeDecoder._accept for a random batch (speculative.py:450-462) with explicit draws: per-row [B]
    parameters, repeated over each row's verified positions like sampling_per_token (spec_sampler.py:44-52)."""
    batch, k = drafts.shape
    if verified_lens is None:
        p = probs_from_logits(logits.reshape(batch, k + 1, -1), temperatures, top_k, top_p, max_top_k, has_top_p)
        return accept_random(p, q, drafts, uniforms, noise)
    n_pos = logits.shape[0]
    per_token = [x.repeat_interleave(verified_lens, output_size=n_pos) for x in (temperatures, top_k, top_p)]
    p = probs_from_logits(logits, *per_token, max_top_k, has_top_p)
    return accept_random_varlen(p, q, drafts, verified_lens, uniforms, noise)
