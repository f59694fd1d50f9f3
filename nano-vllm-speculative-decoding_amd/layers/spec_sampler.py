"""Sampling primitives of speculative verification on MI355X, with the reference's signatures.

Mirrors nanovllm/layers/spec_sampler.py: same dataclass, same functions, same argument meaning, same random
number consumption (torch.rand(B, k) first, then exponential_ over [B, V], from the caller's generator), so
SpeculativeDecoder._accept and the drafter call sites work unchanged. The arithmetic runs in libnvs_amd kernels:
  probs_from_logits / truncate_logits   one selection pass per row (top-k window with ties, top-p), then a write pass
  race / sample                         chunked argmax of w / E
  accept_random(_varlen)                accept test on gathered p, q; race over the vocabulary
  accept_greedy(_varlen)                argmax per position, prefix count
  accept_from_logits (no counterpart)   probs_from_logits + accept_random_varlen fused: the [T, V] probabilities
                                        are never materialised
Tensors must live on the ROCm device; nothing falls back to a CPU path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, replace

import torch

from .. import _lib

# The reference clamps the Exp(1) noise of the exponential race to avoid dividing by zero (spec_sampler.py:13).
EXPONENTIAL_NOISE_FLOOR = 1e-10
NEGATIVE_INFINITY = float("-inf")


@dataclass
class SamplingTensors:
    """One batch's per-row sampling parameters on the device, with the host-side summaries that size the kernels'
    launches (the reference's SamplingTensors, spec_sampler.py:17-24: same fields, same meaning).

    temperatures  fp32 [B]; None for a batch that decodes greedily throughout
    top_k         int64 [B]; a row with 0 keeps its whole vocabulary
    top_p         fp32 [B]; a row with 1.0 keeps its whole top-k window
    max_top_k     the batch's largest top_k, known on the host (0: no row truncates)
    has_top_p     True when at least one row's top_p is below 1
    all_top_k     True when every row truncates to a top-k window
    """
    temperatures: torch.Tensor | None
    top_k: torch.Tensor
    top_p: torch.Tensor
    max_top_k: int
    has_top_p: bool
    all_top_k: bool


def sampling_tensors(seqs, device: torch.device) -> SamplingTensors:
    """The parameters of a batch of sequences (spec_sampler.py:27-41). A batch is either all greedy (temperature 0)
    or all random; a mixture raises the reference's ValueError."""
    greedy = {seq.temperature == 0 for seq in seqs}
    if len(greedy) > 1:
        raise ValueError("mixed greedy and random sampling is not supported")
    top_k = [seq.top_k for seq in seqs]
    top_p = [seq.top_p for seq in seqs]
    all_greedy = seqs[0].temperature == 0
    return SamplingTensors(
        temperatures=None if all_greedy else _upload([seq.temperature for seq in seqs], torch.float32, device),
        top_k=_upload(top_k, torch.int64, device),
        top_p=_upload(top_p, torch.float32, device),
        max_top_k=max(top_k),
        has_top_p=min(top_p) < 1.0,
        all_top_k=min(top_k) > 0,
    )


def sampling_per_token(sampling: SamplingTensors, verified_lens: torch.Tensor, num_tokens: int) -> SamplingTensors:
    """The same parameters spread from rows to positions, [B] -> [num_tokens]: row r's values repeated
    verified_lens[r] times, for the flat [T, V] logits of a variable-length verification (spec_sampler.py:44-52).
    The host summaries do not change."""
    def spread(per_row: torch.Tensor) -> torch.Tensor:
        return per_row.repeat_interleave(verified_lens, output_size=num_tokens)

    return replace(sampling, top_k=spread(sampling.top_k), top_p=spread(sampling.top_p),
                   temperatures=None if sampling.temperatures is None else spread(sampling.temperatures))


def _upload(values: list, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """A host list as a device tensor, staged in pinned memory so the copy does not block the host."""
    staged = torch.tensor(values, dtype=dtype, pin_memory=(device.type == "cuda"))
    return staged.to(device, non_blocking=True)


def _rows_view(x: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    """x [..., V] as rows: (tensor with unit last stride and uniform row stride, n_rows, row_stride)."""
    vocab = x.shape[-1]
    rows = x.reshape(-1, vocab)
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    return rows, rows.shape[0], rows.stride(0)


def _param_rows(sampling: SamplingTensors, n_pos: int) -> int:
    n_param = sampling.top_k.shape[0]
    if n_param == 0 or n_pos % n_param:
        raise ValueError(f"{n_pos} logit rows do not broadcast over {n_param} parameter rows")
    return n_pos // n_param


def _contig(t: torch.Tensor | None, dtype: torch.dtype) -> torch.Tensor | None:
    if t is None:
        return None
    if t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def probs_from_logits(logits: torch.Tensor, sampling: SamplingTensors) -> torch.Tensor:
    """fp32 probabilities after temperature, top-k and top-p (spec_sampler.py:65-69); greedy batches have none.
    logits [..., V] (fp32 / bf16 / fp16); the [B] parameters broadcast over the middle dims (or are per token)."""
    assert sampling.temperatures is not None
    _lib.require_device(logits, sampling.temperatures, sampling.top_k, sampling.top_p)
    rows, n_pos, row_stride = _rows_view(logits)
    vocab = logits.shape[-1]
    probs = torch.empty(logits.shape, dtype=torch.float32, device=logits.device)
    if n_pos == 0:
        return probs
    per = _param_rows(sampling, n_pos)
    top_k = _contig(sampling.top_k, torch.int64)
    top_p = _contig(sampling.top_p, torch.float32)
    temps = _contig(sampling.temperatures, torch.float32)
    lib = _lib.load()
    _lib.check(lib.nvs_probs_from_logits(rows.data_ptr(), _lib.dtype_code(rows.dtype), row_stride, n_pos, vocab, per,
                                         temps.data_ptr(), top_k.data_ptr(), top_p.data_ptr(), sampling.max_top_k,
                                         int(sampling.has_top_p), probs.data_ptr(), None, 0, _lib.stream_of(logits)),
               "probs_from_logits")
    return probs


def truncate_logits(scaled: torch.Tensor, sampling: SamplingTensors) -> torch.Tensor:
    """-inf outside each row's top-k, then outside the top-p nucleus of those candidates (spec_sampler.py:72-96).
    Ties at the k-th value are kept; rows with top_k == 0 are returned unchanged."""
    if sampling.max_top_k == 0:
        return scaled
    _lib.require_device(scaled, sampling.top_k, sampling.top_p)
    if scaled.dtype != torch.float32:
        raise ValueError("truncate_logits expects the fp32 temperature-scaled logits")
    rows, n_pos, row_stride = _rows_view(scaled)
    vocab = scaled.shape[-1]
    out = torch.empty(scaled.shape, dtype=torch.float32, device=scaled.device)
    if n_pos == 0:
        return out
    per = _param_rows(sampling, n_pos)
    top_k = _contig(sampling.top_k, torch.int64)
    top_p = _contig(sampling.top_p, torch.float32)
    lib = _lib.load()
    _lib.check(lib.nvs_truncate_logits(rows.data_ptr(), row_stride, n_pos, vocab, per, top_k.data_ptr(),
                                       top_p.data_ptr(), sampling.max_top_k, int(sampling.has_top_p), out.data_ptr(),
                                       None, 0, _lib.stream_of(scaled)),
               "truncate_logits")
    return out


def exponential_noise_(out: torch.Tensor, generator: torch.Generator | None) -> torch.Tensor:
    """Fill out with the race's Exp(1) noise, in place; returns out (spec_sampler.py:99-101). The draws come from
    torch's generator so the stream of random numbers is the reference's."""
    return out.exponential_(1.0, generator=generator).clamp_min_(EXPONENTIAL_NOISE_FLOOR)


# Row counters of the one-launch races: int32 per row, zero between calls (each call leaves them zero). Sized for
# at least this many rows so that a graph captured after a smaller eager call still finds a large enough buffer.
_MIN_COUNTER_ROWS = 16384


def _row_counters(name: str, n_rows: int, device: torch.device) -> torch.Tensor:
    return _lib.persistent_workspace(name, 4 * max(n_rows, _MIN_COUNTER_ROWS), device)


def race(weights: torch.Tensor, noise: torch.Tensor) -> torch.Tensor:
    """argmax(w / E) over the last dim, first index on ties (spec_sampler.py:104-106)."""
    _lib.require_device(weights, noise)
    if weights.shape != noise.shape:
        raise ValueError(f"weights {tuple(weights.shape)} and noise {tuple(noise.shape)} differ")
    lead = weights.shape[:-1]
    vocab = weights.shape[-1]
    w, n_rows, w_stride = _rows_view(_contig(weights, torch.float32) if weights.dtype != torch.float32 else weights)
    e, _, e_stride = _rows_view(_contig(noise, torch.float32) if noise.dtype != torch.float32 else noise)
    out = torch.empty(n_rows, dtype=torch.int64, device=weights.device)
    if n_rows == 0:
        return out.view(lead)
    lib = _lib.load()
    nbytes = _lib.size_out()
    _lib.check(lib.nvs_race_workspace_size(n_rows, vocab, ctypes.byref(nbytes)), "race_workspace_size")
    ws = _lib.workspace(nbytes.value, weights.device)
    counters = _row_counters("race_row_counters", n_rows, weights.device)
    _lib.check(lib.nvs_race(w.data_ptr(), w_stride, e.data_ptr(), e_stride, n_rows, vocab, out.data_ptr(),
                            counters.data_ptr(), _lib.ptr(ws), nbytes.value, _lib.stream_of(weights)),
               "race")
    return out.view(lead)


def sample(weights: torch.Tensor, generator: torch.Generator | None) -> torch.Tensor:
    """Exponential race: argmax(w / E) with E ~ Exp(1) picks index i with probability w_i / sum(w)."""
    return race(weights, exponential_noise_(torch.empty_like(weights, dtype=torch.float32), generator))


def _draws(batch_size: int, num_drafts: int, vocab: int, device: torch.device,
           generator: torch.Generator | None) -> tuple[torch.Tensor, torch.Tensor]:
    """The uniforms and the race noise, drawn in the reference's order (spec_sampler.py:141 then :149)."""
    uniforms = torch.rand(batch_size, num_drafts, device=device, generator=generator)
    noise = exponential_noise_(torch.empty(batch_size, vocab, dtype=torch.float32, device=device), generator)
    return uniforms, noise


def accept_random(p: torch.Tensor, q: torch.Tensor, drafts: torch.Tensor,
                  generator: torch.Generator | None) -> tuple[torch.Tensor, torch.Tensor]:
    """Rejection sampling of k drafts per row, every row verifying all of them (spec_sampler.py:114-120).
    p: [B, k+1, V] at the k draft positions and the bonus position."""
    batch_size, num_drafts = drafts.shape
    return _accept_random(p.reshape(-1, p.shape[-1]), q, drafts, None, generator)


def accept_random_varlen(p: torch.Tensor, q: torch.Tensor, drafts: torch.Tensor, verified_lens: torch.Tensor,
                         generator: torch.Generator | None) -> tuple[torch.Tensor, torch.Tensor]:
    """Rejection sampling of each row's first verified_lens - 1 drafts (spec_sampler.py:123-150).
    p: [T, V] target probabilities at the verified positions, row after row; q: [B, k, V] draft probabilities;
    drafts: [B, k] int64; verified_lens: [B] int64 in 1..k+1 summing to T. Returns n_accept [B] and tail [B]."""
    return _accept_random(p, q, drafts, verified_lens, generator)


def _accept_random(p, q, drafts, verified_lens, generator):
    _lib.require_device(p, q, drafts, verified_lens)
    batch_size, num_drafts = drafts.shape
    vocab = p.shape[-1]
    uniforms, noise = _draws(batch_size, num_drafts, vocab, p.device, generator)
    p = _contig(p, torch.float32)
    q = _contig(q, torch.float32)
    drafts_c = _contig(drafts, torch.int64)
    lens = _contig(verified_lens, torch.int64)
    n_accept = torch.empty(batch_size, dtype=torch.int64, device=p.device)
    tail = torch.empty(batch_size, dtype=torch.int64, device=p.device)
    if batch_size == 0:
        return n_accept, tail
    assert q.shape == (batch_size, num_drafts, vocab), f"q {tuple(q.shape)} is not [B, k, V]"
    lib = _lib.load()
    nbytes = _lib.size_out()
    _lib.check(lib.nvs_accept_random_workspace_size(batch_size, vocab, ctypes.byref(nbytes)),
               "accept_random_workspace_size")
    ws = _lib.workspace(nbytes.value, p.device)
    counters = _row_counters("accept_random_row_counters", batch_size, p.device)
    _lib.check(lib.nvs_accept_random(p.data_ptr(), q.data_ptr(), drafts_c.data_ptr(), _lib.ptr(lens),
                                     uniforms.data_ptr(), noise.data_ptr(), batch_size, num_drafts, p.shape[0], vocab,
                                     n_accept.data_ptr(), tail.data_ptr(), counters.data_ptr(), _lib.ptr(ws),
                                     nbytes.value, _lib.stream_of(p)),
               "accept_random")
    return n_accept, tail


def accept_greedy(target_logits: torch.Tensor, drafts: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Greedy verification of all k drafts per row (spec_sampler.py:153-158). target_logits: [B, k+1, V]."""
    return _accept_greedy(target_logits.reshape(-1, target_logits.shape[-1]), drafts, None)


def accept_greedy_varlen(target_logits: torch.Tensor, drafts: torch.Tensor,
                         verified_lens: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Greedy verification of each row's first verified_lens - 1 drafts (spec_sampler.py:161-169): a draft is
    accepted iff it equals the target's argmax at its position. target_logits: [T, V]."""
    return _accept_greedy(target_logits, drafts, verified_lens)


def _accept_greedy(logits, drafts, verified_lens):
    _lib.require_device(logits, drafts, verified_lens)
    batch_size, num_drafts = drafts.shape
    rows, n_pos, row_stride = _rows_view(logits)
    vocab = logits.shape[-1]
    drafts_c = _contig(drafts, torch.int64)
    lens = _contig(verified_lens, torch.int64)
    n_accept = torch.empty(batch_size, dtype=torch.int64, device=logits.device)
    tail = torch.empty(batch_size, dtype=torch.int64, device=logits.device)
    if batch_size == 0:
        return n_accept, tail
    lib = _lib.load()
    nbytes = _lib.size_out()
    _lib.check(lib.nvs_accept_greedy_workspace_size(n_pos, vocab, ctypes.byref(nbytes)),
               "accept_greedy_workspace_size")
    ws = _lib.workspace(nbytes.value, logits.device)
    _lib.check(lib.nvs_accept_greedy(rows.data_ptr(), _lib.dtype_code(rows.dtype), row_stride, drafts_c.data_ptr(),
                                     _lib.ptr(lens), batch_size, num_drafts, n_pos, vocab, n_accept.data_ptr(),
                                     tail.data_ptr(), _lib.ptr(ws), nbytes.value, _lib.stream_of(logits)),
               "accept_greedy")
    return n_accept, tail


def _q_tensor(draft_probs):
    """The tensor to device-check for q: the dense q itself, or the ids of candidate rows."""
    return draft_probs.ids if hasattr(draft_probs, "ids") else draft_probs


def accept(target_logits: torch.Tensor, drafts: torch.Tensor, draft_probs, sampling: SamplingTensors,
           verified_lens: torch.Tensor | list[int] | None,
           generator: torch.Generator | None) -> tuple[torch.Tensor, torch.Tensor]:
    """The acceptance step of a speculative round, SpeculativeDecoder._accept (speculative.py:450-462), as one call.

    Which rule runs depends on the batch: greedy (sampling.temperatures is None) or random, and whether every row
    verifies all k drafts (verified_lens None, target_logits [B, k+1, V]) or row r only its first
    verified_lens[r] - 1 (target_logits [T, V], T = sum(verified_lens)):
        greedy, all drafts      accept_greedy(target_logits, drafts)
        greedy, variable        accept_greedy_varlen(target_logits, drafts, lens)
        random, all drafts      accept_from_logits(..., None, generator): accept_random(probs_from_logits(...))
        random, variable        accept_from_logits(..., lens, generator): accept_random_varlen(probs_from_logits(
                                  logits, sampling_per_token(...)), ...)
    The random rows run the fused one-launch accept, which reads the logits once and maps positions to rows
    itself (so the per-token parameters are never built), and draws rand(B, k) then exponential_([B, V]) from
    `generator`, as the reference does. Greedy rows draw nothing. verified_lens may be a host list (copied to the
    device as _accept copies it) or a [B] int64 device tensor. Returns (n_accept [B], tail [B]), int64."""
    if verified_lens is not None and not isinstance(verified_lens, torch.Tensor):
        verified_lens = _upload(list(verified_lens), torch.int64, target_logits.device)
    if sampling.temperatures is None:
        if verified_lens is None:
            return accept_greedy(target_logits, drafts)
        return accept_greedy_varlen(target_logits, drafts, verified_lens)
    return accept_from_logits(target_logits, draft_probs, drafts, sampling, verified_lens, generator)


def accept_from_logits(target_logits: torch.Tensor, draft_probs: torch.Tensor, drafts: torch.Tensor,
                       sampling: SamplingTensors, verified_lens: torch.Tensor | None,
                       generator: torch.Generator | None) -> tuple[torch.Tensor, torch.Tensor]:
    """What SpeculativeDecoder._accept computes for a random batch (speculative.py:450-462), fused:
        accept_random(probs_from_logits(logits, sampling), q, drafts, g)                       (verified_lens None)
        accept_random_varlen(probs_from_logits(logits, sampling_per_token(...)), q, drafts, lens, g)
    target_logits: [B, k+1, V] or [T, V]; sampling holds per-row [B] parameters. draft_probs: the dense
    [B, k, V] q, or DSpark's candidate rows (an object with ids [B, k, C] int32 and probs [B, k, C], as
    layers.markov.CandidateRows), which stand for the q they scatter to. Draws the same random numbers in the
    same order and returns the same (n_accept, tail)."""
    assert sampling.temperatures is not None, "greedy batches use accept_greedy(_varlen)"
    _lib.require_device(target_logits, _q_tensor(draft_probs), drafts, verified_lens, sampling.temperatures)
    batch_size, num_drafts = drafts.shape
    uniforms, noise = _draws(batch_size, num_drafts, target_logits.shape[-1], target_logits.device, generator)
    return spec_accept_with_draws(target_logits, draft_probs, drafts, sampling, verified_lens, uniforms, noise)


def spec_accept_with_draws(target_logits: torch.Tensor, draft_probs: torch.Tensor, drafts: torch.Tensor,
                           sampling: SamplingTensors, verified_lens: torch.Tensor | None, uniforms: torch.Tensor,
                           noise: torch.Tensor, workspace: torch.Tensor | None = None
                           ) -> tuple[torch.Tensor, torch.Tensor]:
    """accept_from_logits with the uniforms [B, k] and noise [B, V] supplied by the caller (tests, benchmarks,
    a caller that draws them elsewhere). workspace: optional uint8 scratch buffer for the per-position records.
    The per-row counters live in a persistent zero-filled buffer that every call leaves zero."""
    _lib.require_device(target_logits, _q_tensor(draft_probs), drafts, verified_lens, uniforms, noise)
    batch_size, num_drafts = drafts.shape
    rows, n_pos, row_stride = _rows_view(target_logits)
    vocab = target_logits.shape[-1]
    candidates = hasattr(draft_probs, "ids")
    if candidates:
        cand_ids = _contig(draft_probs.ids, torch.int32)
        cand_probs = _contig(draft_probs.probs, torch.float32)
        if cand_ids.shape[:2] != (batch_size, num_drafts) or cand_probs.shape != cand_ids.shape:
            raise ValueError(f"candidate rows {tuple(cand_ids.shape)} / {tuple(cand_probs.shape)} are not [B, k, C]")
        if not sampling.all_top_k or sampling.max_top_k <= 0:
            raise ValueError("candidate rows need every row to truncate with top-k (sampling.all_top_k)")
    else:
        q = _contig(draft_probs, torch.float32)
    drafts_c = _contig(drafts, torch.int64)
    lens = _contig(verified_lens, torch.int64)
    temps = _contig(sampling.temperatures, torch.float32)
    top_k = _contig(sampling.top_k, torch.int64)
    top_p = _contig(sampling.top_p, torch.float32)
    u = _contig(uniforms, torch.float32)
    e = _contig(noise, torch.float32)
    n_accept = torch.empty(batch_size, dtype=torch.int64, device=target_logits.device)
    tail = torch.empty(batch_size, dtype=torch.int64, device=target_logits.device)
    if batch_size == 0:
        return n_accept, tail
    lib = _lib.load()
    nbytes = _lib.size_out()
    _lib.check(lib.nvs_spec_accept_workspace_size(batch_size, num_drafts, n_pos, vocab, sampling.max_top_k,
                                                  ctypes.byref(nbytes)),
               "spec_accept_workspace_size")
    if workspace is None or workspace.numel() < nbytes.value:
        workspace = _lib.workspace(max(nbytes.value, 1), target_logits.device)
    counters = _row_counters("spec_accept_row_counters", batch_size, target_logits.device)
    if candidates:
        _lib.check(lib.nvs_spec_accept_candidates(
            rows.data_ptr(), _lib.dtype_code(rows.dtype), row_stride, temps.data_ptr(), top_k.data_ptr(),
            top_p.data_ptr(), sampling.max_top_k, int(sampling.has_top_p), cand_ids.data_ptr(), cand_probs.data_ptr(),
            cand_ids.shape[-1], cand_ids.shape[-1], drafts_c.data_ptr(), _lib.ptr(lens), u.data_ptr(), e.data_ptr(),
            batch_size, num_drafts, n_pos, vocab, n_accept.data_ptr(), tail.data_ptr(), counters.data_ptr(),
            workspace.data_ptr(), workspace.numel(), _lib.stream_of(target_logits)),
            "spec_accept_candidates")
        return n_accept, tail
    assert q.shape == (batch_size, num_drafts, vocab), f"draft_probs {tuple(q.shape)} is not [B, k, V]"
    _lib.check(lib.nvs_spec_accept(rows.data_ptr(), _lib.dtype_code(rows.dtype), row_stride, temps.data_ptr(),
                                   top_k.data_ptr(), top_p.data_ptr(), sampling.max_top_k, int(sampling.has_top_p),
                                   q.data_ptr(), drafts_c.data_ptr(), _lib.ptr(lens), u.data_ptr(), e.data_ptr(),
                                   batch_size, num_drafts, n_pos, vocab, n_accept.data_ptr(), tail.data_ptr(),
                                   counters.data_ptr(), workspace.data_ptr(), workspace.numel(),
                                   _lib.stream_of(target_logits)),
               "spec_accept")
    return n_accept, tail


def accept_random_with_draws(p: torch.Tensor, q: torch.Tensor, drafts: torch.Tensor,
                             verified_lens: torch.Tensor | None, uniforms: torch.Tensor,
                             noise: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """accept_random(_varlen) over dense p with the uniforms and noise supplied by the caller."""
    _lib.require_device(p, q, drafts, verified_lens, uniforms, noise)
    batch_size, num_drafts = drafts.shape
    vocab = p.shape[-1]
    p = _contig(p.reshape(-1, vocab), torch.float32)
    q = _contig(q, torch.float32)
    drafts_c = _contig(drafts, torch.int64)
    lens = _contig(verified_lens, torch.int64)
    u = _contig(uniforms, torch.float32)
    e = _contig(noise, torch.float32)
    n_accept = torch.empty(batch_size, dtype=torch.int64, device=p.device)
    tail = torch.empty(batch_size, dtype=torch.int64, device=p.device)
    if batch_size == 0:
        return n_accept, tail
    lib = _lib.load()
    nbytes = _lib.size_out()
    _lib.check(lib.nvs_accept_random_workspace_size(batch_size, vocab, ctypes.byref(nbytes)),
               "accept_random_workspace_size")
    ws = _lib.workspace(nbytes.value, p.device)
    counters = _row_counters("accept_random_row_counters", batch_size, p.device)
    _lib.check(lib.nvs_accept_random(p.data_ptr(), q.data_ptr(), drafts_c.data_ptr(), _lib.ptr(lens), u.data_ptr(),
                                     e.data_ptr(), batch_size, num_drafts, p.shape[0], vocab, n_accept.data_ptr(),
                                     tail.data_ptr(), counters.data_ptr(), _lib.ptr(ws), nbytes.value,
                                     _lib.stream_of(p)),
               "accept_random")
    return n_accept, tail
