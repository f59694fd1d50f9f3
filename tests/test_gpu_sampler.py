"""Parity of the HIP sampler kernels with the CPU oracle.

Accepted lengths and tails are compared bit for bit given the same logits, q, uniforms and noise; probabilities
within fp32 rounding (rtol 1e-5, atol 1e-7) with identical zero patterns; truncated logits exactly.
On a mismatch the decision margin is printed: a flip is only legitimate when u*q and p (or two race scores)
agree to a few ulps, because the kernel's exp and summation order differ from torch's CPU ones.
"""
import dataclasses
import json
import math
import pathlib

import numpy as np
import pytest
import torch

import known_answers as ka
import nvs_amd.workloads as wl
from conftest import log_case
from nvs_amd import _lib
from nvs_amd.layers import spec_sampler as ns
from oracle import spec_sampler as ref

pytestmark = pytest.mark.gpu
FROZEN = json.loads((pathlib.Path(__file__).parent / "golden" / "random_sampling_cases.json").read_text())


def sampling(rows, device):
    t = torch.tensor([r[0] for r in rows], dtype=torch.float32)
    k = torch.tensor([r[1] for r in rows], dtype=torch.int64)
    p = torch.tensor([r[2] for r in rows], dtype=torch.float32)
    st = ns.SamplingTensors(temperatures=t.to(device), top_k=k.to(device), top_p=p.to(device),
                            max_top_k=int(k.max()), has_top_p=bool((p < 1).any()), all_top_k=bool((k > 0).all()))
    return st, (t, k, p, int(k.max()), bool((p < 1).any()))


@pytest.mark.parametrize("case", ka.PROBS_CASES, ids=[c[0] for c in ka.PROBS_CASES])
def test_probs_known_answers(device, case):
    log_case(f"probs known answer {case[0]}")
    _, rows, logits, expected = case
    st, _ = sampling(rows, device)
    probs = ns.probs_from_logits(torch.tensor(logits, device=device), st)
    torch.testing.assert_close(probs.cpu(), torch.tensor(expected, dtype=torch.float32))


def test_truncation_broadcast_known_answer(device):
    log_case("truncate broadcast")
    rows, logits, expected = ka.BROADCAST_CASE
    st, _ = sampling(rows, device)
    assert ns.truncate_logits(torch.tensor(logits, device=device), st).cpu().tolist() == expected


def test_bonus_and_zero_mass_known_answers(device):
    log_case("accept_random bonus / zero mass")
    for make in (ka.bonus_case, ka.zero_mass_case):
        p, q, drafts, n_exp, tail_exp = make()
        g = torch.Generator(device=device).manual_seed(0)
        n, tail = ns.accept_random(p.to(device), q.to(device), drafts.to(device), g)
        assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)


def test_greedy_known_answers(device):
    log_case("greedy known answers")
    for _, logits, drafts, n_exp, tail_exp in ka.greedy_prefix_cases():
        n, tail = ns.accept_greedy(logits.to(device), drafts.to(device))
        assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)
    logits, drafts, n_exp, tail_exp = ka.greedy_per_row_case()
    n, tail = ns.accept_greedy(logits.to(device), drafts.to(device))
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)


def test_varlen_known_answers(device):
    log_case("varlen known answers")
    p, q, drafts, lens, n_exp, tail_exp = ka.varlen_case()
    g = torch.Generator(device=device).manual_seed(0)
    n, tail = ns.accept_random_varlen(p.to(device), q.to(device), drafts.to(device), lens.to(device), g)
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)
    n, tail = ns.accept_greedy_varlen(p.to(device), drafts.to(device), lens.to(device))
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)
    # the fused path on logits whose softmax is (numerically) the point masses
    st, _ = sampling([(1.0, 4, 1.0)] * 3, device)
    logits = torch.where(p > 0, 0.0, -1e4)
    g = torch.Generator(device=device).manual_seed(0)
    n, tail = ns.accept_from_logits(logits.to(device), q.to(device), drafts.to(device), st, lens.to(device), g)
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)


def test_race_ties_zero_weights_and_random_rows(device):
    log_case("race ties / zeros / random")
    w = torch.tensor([[0.0, 2.0, 2.0, 1.0], [0.0, 0.0, 0.0, 0.0]])
    assert ns.race(w.to(device), torch.ones(2, 4, device=device)).tolist() == [1, 0]
    gen = torch.Generator().manual_seed(7)
    w = torch.rand(33, 70000, generator=gen)
    w[w < 0.5] = 0
    e = torch.empty(33, 70000).exponential_(generator=gen).clamp_min_(1e-10)
    assert torch.equal(ns.race(w.to(device), e.to(device)).cpu(), ref.race(w, e))


def test_one_launch_races_leave_their_counters_at_zero(device):
    """race and accept_random pick each row's winner in the workgroup of the row's last chunk to finish, counting
    chunks on a zero-filled per-row counter that every call leaves at zero: calls of different sizes in a row and
    HIP-graph replays (with eager calls between them) all give the oracle's answer."""
    log_case("race / accept_random counters across calls and graph replays")
    gen = torch.Generator().manual_seed(11)
    cases = []
    for rows in (40, 7, 40):
        w = torch.rand(rows, 50000, generator=gen)
        w[w < 0.3] = 0
        e = torch.empty(rows, 50000).exponential_(generator=gen).clamp_min_(1e-10)
        cases.append((w.to(device), e.to(device), ref.race(w, e)))
    for w, e, want in cases:
        assert torch.equal(ns.race(w, e).cpu(), want)
    counters = _lib.persistent_workspace("race_row_counters", 4, torch.device(device))
    torch.cuda.synchronize()
    assert int(counters.view(torch.int32).abs().sum()) == 0
    w, e, want = cases[0]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ns.race(w, e)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = ns.race(w, e)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), want)
        assert torch.equal(ns.race(cases[1][0], cases[1][1]).cpu(), cases[1][2])   # eager work between replays
    case = wl.sampler_case(8, 7, 50000, verified_lens=[1, 8, 3, 5, 2, 7, 4, 6], draft_probs_fn=draft_probs)
    lens = case.verified_lens
    p = ref.probs_from_logits(case.logits, case.temperatures.repeat_interleave(lens),
                              case.top_k.repeat_interleave(lens), case.top_p.repeat_interleave(lens),
                              case.max_top_k, case.has_top_p)
    want = ref.accept_random_varlen(p, case.q, case.drafts, lens, case.uniforms, case.noise)
    for _ in range(3):
        got = ns.accept_random_with_draws(p.to(device), case.q.to(device), case.drafts.to(device), lens.to(device),
                                          case.uniforms.to(device), case.noise.to(device))
        assert torch.equal(got[0].cpu(), want[0]) and torch.equal(got[1].cpu(), want[1])
    counters = _lib.persistent_workspace("accept_random_row_counters", 4, torch.device(device))
    torch.cuda.synchronize()
    assert int(counters.view(torch.int32).abs().sum()) == 0


def test_sample_frequencies_follow_the_weights(device):
    log_case("sample frequencies")
    g = torch.Generator(device=device).manual_seed(0)
    weights = torch.tensor([0.1, 0.6, 0.3], device=device).expand(200_000, 3)
    counts = torch.bincount(ns.sample(weights, g), minlength=3).float().cpu() / 200_000
    torch.testing.assert_close(counts, torch.tensor([0.1, 0.6, 0.3]), atol=0.005, rtol=0)


def probs_params(n, vocab, top_k, top_p, temp, seed, dtype=torch.float32, sigma=3.0):
    gen = torch.Generator().manual_seed(seed)
    logits = (torch.randn(n, vocab, generator=gen) * sigma).to(dtype)
    rows = [(temp[i % len(temp)], top_k[i % len(top_k)], top_p[i % len(top_p)]) for i in range(n)]
    return logits, rows


@pytest.mark.parametrize("name, top_k, top_p, temp, dtype", [
    ("topk64", [64], [1.0], [1.0], torch.float32),
    ("topk_mixed_topp", [64, 5, 1, 20], [0.9, 1.0, 0.5, 0.3], [0.7, 1.0, 1.3], torch.float32),
    ("topk0_rows", [0, 64, 0, 3], [1.0], [1.0, 0.5], torch.float32),
    ("bf16_ties", [64, 50], [1.0, 0.8], [1.0], torch.bfloat16),
    ("fp16_mixed", [64, 20, 0, 5], [1.0, 0.9], [1.0, 0.8], torch.float16),
    ("topk1000", [1000, 700], [1.0, 0.95], [1.0], torch.float32),
])
@pytest.mark.parametrize("vocab", [4099, 5000, 151936])   # 4099: rows that are not 16-byte aligned
def test_probs_and_truncation_match_the_oracle(device, name, top_k, top_p, temp, dtype, vocab):
    log_case(f"probs_from_logits {name} V={vocab}")
    logits, rows = probs_params(16, vocab, top_k, top_p, temp, seed=len(name) + vocab)
    logits = logits.to(dtype)
    st, (t, k, p, mk, hp) = sampling(rows, device)
    want = ref.probs_from_logits(logits, t, k, p, mk, hp)
    got = ns.probs_from_logits(logits.to(device), st).cpu()
    assert torch.equal(got > 0, want > 0), "kept sets differ"
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-7)
    scaled = logits.float() / t[:, None]
    trunc_want = ref.truncate_logits(scaled, k, p, mk, hp)
    trunc_got = ns.truncate_logits(scaled.to(device), st).cpu()
    assert torch.equal(trunc_got, trunc_want)


def test_massive_ties_take_the_exact_path(device):
    log_case("probs constant rows (all tied)")
    vocab = 20000
    logits = torch.zeros(3, vocab)
    logits[1, ::7] = 1.0          # 2858 tied maxima
    logits[2, :5000] = 2.0
    st, (t, k, p, mk, hp) = sampling([(1.0, 10, 1.0), (1.0, 64, 0.5), (1.0, 3, 1.0)], device)
    want = ref.probs_from_logits(logits, t, k, p, mk, hp)
    got = ns.probs_from_logits(logits.to(device), st).cpu()
    assert torch.equal(got > 0, want > 0)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-7)


def fp32_ulps(a: float, b: float) -> float:
    """|a - b| in units in the last place (fp32) of the larger magnitude."""
    big = max(abs(a), abs(b))
    return 0.0 if big == 0.0 else abs(a - b) / float(np.spacing(np.float32(big)))


def margin_report(case, n_got, n_want, tail_got=None, tail_want=None):
    """For every batch row whose accepted length or tail differs from the oracle's, how close the oracle's own
    decisions were to a tie, in fp32 ulps: each verified draft's accept test u * q(d) < p(d) (spec_sampler.py:142),
    and the race at the row's tail position, the gap between its two best scores w / E (spec_sampler.py:106,
    w = p at the bonus position, else max(p - q, 0)). A legitimate flip (the kernel's exp and sums round apart from
    torch's CPU ones) shows a gap of a few ulps at the decision that differs; a bug shows a large one."""
    logits = case.logits.float()
    batch, k = case.drafts.shape
    lens = case.verified_lens if case.verified_lens is not None else torch.full((batch,), k + 1, dtype=torch.int64)
    starts = torch.cumsum(lens, 0) - lens
    t, tk, tp = (x.repeat_interleave(lens) for x in (case.temperatures, case.top_k, case.top_p))
    p = ref.probs_from_logits(logits, t, tk, tp, case.max_top_k, case.has_top_p)
    bad = n_got != n_want
    if tail_got is not None:
        bad |= tail_got != tail_want
    lines = []
    for b in torch.nonzero(bad).flatten().tolist():
        s, L = int(starts[b]), int(lens[b])
        head = f"row {b}: n_accept {int(n_got[b])} vs {int(n_want[b])}"
        if tail_got is not None:
            head += f", tail {int(tail_got[b])} vs {int(tail_want[b])}"
        lines.append(head)
        for j in range(min(L - 1, k)):
            d = int(case.drafts[b, j])
            uq = float(case.uniforms[b, j]) * float(case.q[b, j, d])
            pd = float(p[s + j, d])
            lines.append(f"  draft {j} (token {d}): u*q = {uq:.9g}, p = {pd:.9g}, accepted {uq < pd}, "
                         f"gap {fp32_ulps(uq, pd):.1f} ulps")
        n = int(n_want[b])
        w = p[s + n] if n == L - 1 else torch.clamp(p[s + n] - case.q[b, min(n, k - 1)], min=0.0)
        scores = w / case.noise[b]
        top = scores.topk(2)
        lines.append(f"  race at position {s + n}: best {int(top.indices[0])} ({float(top.values[0]):.9g}), "
                     f"second {int(top.indices[1])} ({float(top.values[1]):.9g}), "
                     f"gap {fp32_ulps(float(top.values[0]), float(top.values[1])):.1f} ulps")
    return "\n".join(lines)


def run_fused(case, device):
    g = case.to(device)
    st = ns.SamplingTensors(temperatures=g.temperatures, top_k=g.top_k, top_p=g.top_p, max_top_k=case.max_top_k,
                            has_top_p=case.has_top_p, all_top_k=bool((case.top_k > 0).all()))
    n, tail = ns.spec_accept_with_draws(g.logits, g.q, g.drafts, st, g.verified_lens, g.uniforms, g.noise)
    return n.cpu(), tail.cpu()


def run_oracle(case):
    return ref.accept_from_logits(case.logits.float() if case.logits.dtype != torch.float32 else case.logits,
                                  case.q, case.drafts, case.temperatures, case.top_k, case.top_p, case.max_top_k,
                                  case.has_top_p, case.verified_lens, case.uniforms, case.noise)


def draft_probs(draft_logits, temps, tk, tp):
    return ref.probs_from_logits(draft_logits, temps, tk, tp, int(tk.max()), bool((tp < 1).any()))


@pytest.mark.parametrize("name, kwargs", [
    ("c4_topk64", dict(batch=64, num_drafts=7, vocab=151936)),
    ("varlen", dict(batch=16, num_drafts=7, vocab=151936, verified_lens=[1, 8, 3, 5, 2, 7, 4, 6] * 2)),
    ("topp_temps", dict(batch=8, num_drafts=3, vocab=32000, top_k=[64, 20, 5, 64] * 2,
                        top_p=[0.9, 1.0, 0.6, 0.95] * 2, temperature=[0.7, 1.0, 1.5, 1.0] * 2)),
    ("dense_rows", dict(batch=4, num_drafts=3, vocab=32000, top_k=[0, 64, 0, 10])),
    # no row truncates (the reference's default sampling): the races run in the dense race kernels
    ("no_topk", dict(batch=16, num_drafts=7, vocab=151936, top_k=0)),
    ("no_topk_bf16_varlen_temps", dict(batch=8, num_drafts=7, vocab=151936, top_k=0, logits_dtype=torch.bfloat16,
                                       verified_lens=[1, 8, 3, 5, 2, 7, 4, 6], temperature=[0.7, 1.0, 1.3, 1.0] * 2)),
    ("no_topk_odd_vocab", dict(batch=4, num_drafts=3, vocab=32001, top_k=0, temperature=[0.7, 1.0] * 2)),
    ("bf16_logits", dict(batch=8, num_drafts=7, vocab=151936, logits_dtype=torch.bfloat16)),
    # an fp16 model's logits (model_runner.py:55-57 builds the model in hf_config.dtype)
    ("fp16_logits_topp_temps", dict(batch=8, num_drafts=7, vocab=151936, logits_dtype=torch.float16,
                                    top_k=[64, 20, 5, 64] * 2, top_p=[0.9, 1.0, 0.6, 0.95] * 2,
                                    temperature=[0.7, 1.0, 1.5, 1.0] * 2, verified_lens=[1, 8, 3, 5, 2, 7, 4, 6])),
    ("no_topk_fp16", dict(batch=8, num_drafts=7, vocab=32000, top_k=0, logits_dtype=torch.float16)),
    ("small_sigma", dict(batch=8, num_drafts=7, vocab=151936, sigma=0.5)),
])
def test_fused_accept_is_bit_exact(device, name, kwargs):
    log_case(f"fused accept {name}")
    case = wl.sampler_case(draft_probs_fn=draft_probs, **kwargs)
    n_got, tail_got = run_fused(case, device)
    n_want, tail_want = run_oracle(case)
    assert torch.equal(n_got, n_want), margin_report(case, n_got, n_want, tail_got, tail_want)
    assert torch.equal(tail_got, tail_want), margin_report(case, n_got, n_want, tail_got, tail_want)
    print(f"{name}: accepted {n_got.float().mean():.2f} of {case.drafts.shape[1]} on average")


def random_sampler_config(seed):
    """A seeded random verify batch: rows, drafts, vocabulary (aligned or not), fixed or variable lengths, logit
    scale and dtype, and per-row top-k (0 = off, mixed with truncating rows), top-p and temperature."""
    import random
    rng = random.Random(2000 + seed)
    batch = rng.randint(1, 24)
    k = rng.randint(1, 8)
    vocab = rng.choice([rng.randint(500, 70000), 4 * rng.randint(250, 40000)])
    varlen = rng.random() < 0.5
    all_dense = rng.random() < 0.2
    top_k = [0 if all_dense else rng.choice([0, 1, 5, 20, 64, 64, 200]) for _ in range(batch)]
    if not all_dense and max(top_k) == 0:
        top_k[0] = 64
    kwargs = dict(batch=batch, num_drafts=k, vocab=vocab, top_k=top_k,
                  top_p=[rng.choice([1.0, 1.0, 0.9, 0.5]) for _ in range(batch)],
                  temperature=[rng.choice([1.0, 1.0, 0.7, 1.3]) for _ in range(batch)],
                  sigma=rng.choice([1.0, 3.0, 8.0]),
                  logits_dtype=rng.choice([torch.float32, torch.bfloat16]))
    if varlen:
        kwargs["verified_lens"] = [rng.randint(1, k + 1) for _ in range(batch)]
    return kwargs


@pytest.mark.parametrize("seed", range(16))
def test_fused_accept_random_configs_are_bit_exact(device, seed):
    """Seeded random batches through the one-launch accept (and, when no row truncates, the dense race after it):
    accepted lengths and tail tokens bit for bit equal to the oracle's, given the same uniforms and noise."""
    kwargs = random_sampler_config(seed)
    log_case(f"fused accept random config seed={seed}: {kwargs}")
    case = wl.sampler_case(draft_probs_fn=draft_probs, **kwargs)
    n_got, tail_got = run_fused(case, device)
    n_want, tail_want = run_oracle(case)
    assert torch.equal(n_got, n_want), margin_report(case, n_got, n_want, tail_got, tail_want)
    assert torch.equal(tail_got, tail_want), margin_report(case, n_got, n_want, tail_got, tail_want)


def nucleus_margin(scaled_row, top_k, top_p, max_top_k, with_error=False):
    """How far the reference's nucleus test on one row is from a tie: the smallest |mass_before - top_p| over the
    row's top-k candidates and the total mass (spec_sampler.py:87-93). A kept set may legitimately differ from the
    oracle's only when this is a few ulps: the comparison then turns on the last bits of the fp32 softmax, which
    the GPU's exp and sum round differently from torch's CPU kernel.
    with_error: also the reference's own rounding there, the largest |mass_before(fp32) - mass_before(fp64)| over
    the window. Over a window of 10^5 values torch's fp32 softmax sum alone is off by ~1e-6, so a flip is also
    legitimate when the margin is within that error (the kernel's sums are kept in double on such windows)."""
    K = min(max_top_k, scaled_row.numel())
    cand = scaled_row.topk(K).values.clone()
    cand[max(top_k, 1):] = float("-inf")
    nucleus = torch.softmax(cand, dim=-1)
    cum = nucleus.cumsum(dim=-1)
    before = (cum - nucleus)[:max(top_k, 1)]
    margin = float(torch.cat([before, cum[-1:]]).sub(top_p).abs().min())
    if not with_error:
        return margin
    nucleus64 = torch.softmax(cand.double(), dim=-1)
    before64 = (nucleus64.cumsum(dim=-1) - nucleus64)[:max(top_k, 1)]
    return margin, float((before.double() - before64).abs().max())


@pytest.mark.parametrize("seed", range(8))
def test_unfused_rows_on_random_configs(device, seed):
    """The same seeded random batches through the unfused entry points, each against the oracle:
    probs_from_logits (per-token parameters, values within 1e-5 relative and the same kept set), truncate_logits
    (bit for bit), the race of sample() and accept_random over the oracle's own p (bit for bit).
    Kept sets are compared on probabilities at or above the smallest normal fp32 (1.18e-38): an untruncated row
    with a wide logit range has entries the CPU softmax keeps as denormals and the GPU's exp flushes to zero;
    every such disagreement must lie below that bound on both sides. A top-p row whose nucleus test is within
    4 ulps of a tie (nucleus_margin) may cut elsewhere; any other difference fails."""
    kwargs = random_sampler_config(seed)
    log_case(f"unfused sampler rows random config seed={seed}")
    case = wl.sampler_case(draft_probs_fn=draft_probs, **kwargs)
    logits = case.logits.float()
    B, k = case.drafts.shape
    lens = case.verified_lens if case.verified_lens is not None else torch.full((B,), k + 1, dtype=torch.int64)
    t, tk, tp = (x.repeat_interleave(lens) for x in (case.temperatures, case.top_k, case.top_p))
    st = ns.SamplingTensors(t.to(device), tk.to(device), tp.to(device), case.max_top_k, case.has_top_p,
                            bool((tk > 0).all()))
    want = ref.probs_from_logits(logits, t, tk, tp, case.max_top_k, case.has_top_p)
    got = ns.probs_from_logits(logits.to(device), st).cpu()
    scaled = logits / t[:, None]
    trunc_got = ns.truncate_logits(scaled.to(device), st).cpu()
    trunc_want = ref.truncate_logits(scaled, tk, tp, case.max_top_k, case.has_top_p)
    normal = torch.finfo(torch.float32).tiny
    ties = []
    for r in range(logits.shape[0]):
        same = (torch.equal(got[r] >= normal, want[r] >= normal) and
                torch.equal(torch.isfinite(trunc_got[r]), torch.isfinite(trunc_want[r])))
        if not same:
            margin = nucleus_margin(scaled[r], int(tk[r]), float(tp[r]), case.max_top_k)
            assert case.has_top_p and int(tk[r]) > 0 and margin <= 4 * 2.0 ** -23, \
                f"position {r}: kept sets differ with nucleus margin {margin:.3e}"
            ties.append((r, margin))
            continue
        differ = (got[r] > 0) != (want[r] > 0)
        assert bool((got[r][differ] < normal).all() and (want[r][differ] < normal).all())
        torch.testing.assert_close(got[r], want[r], rtol=1e-5, atol=1e-7)
        assert torch.equal(trunc_got[r], trunc_want[r])
    if ties:
        print(f"seed {seed}: nucleus ties (position, margin): {ties}")
    w = want[torch.cumsum(lens, 0) - 1]                      # each row's bonus position
    assert torch.equal(ns.race(w.to(device), case.noise.to(device)).cpu(), ref.race(w, case.noise))
    n_want, tail_want = ref.accept_random_varlen(want, case.q, case.drafts, lens, case.uniforms, case.noise)
    n_got, tail_got = ns.accept_random_with_draws(want.to(device), case.q.to(device), case.drafts.to(device),
                                                  lens.to(device), case.uniforms.to(device), case.noise.to(device))
    assert torch.equal(n_got.cpu(), n_want) and torch.equal(tail_got.cpu(), tail_want)


def ordered_logits(case, kind):
    """Target logits laid out against the streaming pass's first bound (taken from the first two 8192-element
    batches of a row): ascending rows put every large value after it (the lists fill and the row takes the exact
    path), descending rows put them all inside it, a rising trend makes the waves refine their bound mid-row, and
    quantised bf16 ramps add massive ties."""
    T, V = case.logits.shape
    ramp = torch.arange(V, dtype=torch.float32) / V
    rows = torch.arange(T, dtype=torch.float32)[:, None] * 1e-3
    g = torch.Generator().manual_seed(21)
    if kind == "ascending":
        return ramp[None, :] * 12.0 - 6.0 + rows
    if kind == "descending":
        return ramp.flip(0)[None, :] * 12.0 - 6.0 + rows
    if kind == "rising_trend":
        return torch.randn(T, V, generator=g) + 6.0 * ramp[None, :]
    if kind == "bf16_ramp_ties":
        return (torch.round((ramp[None, :] * 12.0 - 6.0 + rows) * 4) / 4).to(torch.bfloat16)
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["ascending", "descending", "rising_trend", "bf16_ramp_ties"])
def test_fused_accept_bound_refinement_and_exact_fallback(device, kind):
    log_case(f"fused accept ordered logits {kind}")
    base = wl.sampler_case(8, 7, 151936, draft_probs_fn=draft_probs)
    case = dataclasses.replace(base, logits=ordered_logits(base, kind))
    n_got, tail_got = run_fused(case, device)
    n_want, tail_want = run_oracle(case)
    assert torch.equal(n_got, n_want), margin_report(case, n_got, n_want, tail_got, tail_want)
    assert torch.equal(tail_got, tail_want), margin_report(case, n_got, n_want, tail_got, tail_want)


@pytest.mark.parametrize("top_k", [200, 700])
def test_fused_accept_large_top_k(device, top_k):
    """top-k 200 still fits the short threshold list; 700 exceeds the first bound's reach (ceil(K/8) > 64 lanes per
    wave) and every row takes the exact path."""
    log_case(f"fused accept top_k {top_k}")
    case = wl.sampler_case(8, 7, 151936, top_k=top_k, draft_probs_fn=draft_probs)
    n_got, tail_got = run_fused(case, device)
    n_want, tail_want = run_oracle(case)
    assert torch.equal(n_got, n_want), margin_report(case, n_got, n_want, tail_got, tail_want)
    assert torch.equal(tail_got, tail_want), margin_report(case, n_got, n_want, tail_got, tail_want)


@pytest.mark.parametrize("top_k, top_p", [(2000, [1.0]), (2000, [0.9, 1.0, 0.5, 0.97]), (151936, [0.95, 1.0]),
                                          (1 << 30, [1.0])])
def test_fused_accept_wide_top_k(device, top_k, top_p):
    """Windows wider than the 1024-value candidate lists (sampling_params.py:15-16 allows any top_k): the rank-th
    largest by a radix select over the row, top-p by the nucleus-mass radix descent, the race over the row."""
    log_case(f"fused accept wide top_k {top_k} top_p {top_p}")
    case = wl.sampler_case(8, 7, 151936, top_k=top_k, top_p=(top_p * 8)[:8], draft_probs_fn=draft_probs)
    n_got, tail_got = run_fused(case, device)
    n_want, tail_want = run_oracle(case)
    assert torch.equal(n_got, n_want), margin_report(case, n_got, n_want, tail_got, tail_want)
    assert torch.equal(tail_got, tail_want), margin_report(case, n_got, n_want, tail_got, tail_want)


@pytest.mark.parametrize("name, top_k, top_p, temp", [
    ("topk2000", [2000, 1500, 64, 3000], [1.0, 0.9, 1.0, 0.95], [1.0, 0.7]),
    ("topk_vocab", [1 << 30, 0, 5000, 1 << 30], [0.95, 1.0, 1.0, 1.0], [1.0, 1.3]),
    ("topk_vocab_no_topp", [1 << 30, 2000], [1.0], [1.0, 0.8]),
])
@pytest.mark.parametrize("vocab", [4099, 151936])
def test_wide_top_k_probs_and_truncation(device, name, top_k, top_p, temp, vocab):
    """probs_from_logits and truncate_logits with windows past 1024 values, up to the whole vocabulary, against the
    oracle: the same kept set (a top-p row may cut elsewhere only at a nucleus tie of <= 4 ulps, nucleus_margin),
    probabilities within 1e-5 relative, truncated logits bit for bit."""
    log_case(f"wide top-k probs {name} V={vocab}")
    logits, rows = probs_params(16, vocab, top_k, top_p, temp, seed=len(name) + vocab)
    st, (t, k, p, mk, hp) = sampling(rows, device)
    want = ref.probs_from_logits(logits, t, k, p, mk, hp)
    got = ns.probs_from_logits(logits.to(device), st).cpu()
    scaled = logits / t[:, None]
    trunc_want = ref.truncate_logits(scaled, k, p, mk, hp)
    trunc_got = ns.truncate_logits(scaled.to(device), st).cpu()
    normal = torch.finfo(torch.float32).tiny
    for r in range(logits.shape[0]):
        if not torch.equal(torch.isfinite(trunc_got[r]), torch.isfinite(trunc_want[r])):
            margin, err = nucleus_margin(scaled[r], int(k[r]), float(p[r]), mk, with_error=True)
            assert hp and margin <= 4 * 2.0 ** -23 + 2 * err, \
                f"position {r}: kept sets differ with nucleus margin {margin:.3e} (reference rounding {err:.3e})"
            print(f"position {r}: nucleus tie, margin {margin:.3e}, reference rounding {err:.3e}")
            continue
        assert torch.equal(trunc_got[r], trunc_want[r])
        differ = (got[r] > 0) != (want[r] > 0)
        assert bool((got[r][differ] < normal).all() and (want[r][differ] < normal).all())
        # the probabilities against the fp64 softmax of the same kept set (the kernel sums in double here), and
        # against the oracle within the oracle's own error against that fp64 softmax
        kept = torch.isfinite(trunc_want[r])
        p64 = torch.softmax(scaled[r].double().masked_fill(~kept, float("-inf")), dim=0)
        live = p64 > 1e-30
        ref_rel = float(((want[r].double() - p64).abs() / p64.clamp_min(1e-300))[live].max())
        if int(k[r]) > 0:   # the truncating rows' sums are exact to fp32 (double on wide windows)
            torch.testing.assert_close(got[r].double()[live], p64[live], rtol=1e-5, atol=0.0)
        torch.testing.assert_close(got[r], want[r], rtol=max(1e-5, 2 * ref_rel), atol=1e-7)


@pytest.mark.parametrize("kind", ["ascending", "rising_trend"])
def test_probs_on_ordered_logits(device, kind):
    log_case(f"probs ordered logits {kind}")
    base = wl.sampler_case(4, 1, 151936, draft_probs_fn=draft_probs)   # 8 rows: 2 positions x 4 parameter rows
    logits = ordered_logits(base, kind).reshape(4, 2, -1)
    st, (t, k, p, mk, hp) = sampling([(1.0, 64, 1.0), (0.8, 5, 1.0), (1.0, 200, 1.0), (1.3, 64, 0.8)], device)
    want = ref.probs_from_logits(logits, t, k, p, mk, hp)
    got = ns.probs_from_logits(logits.to(device), st).cpu()
    assert torch.equal(got > 0, want > 0)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("top_k", [64, 0])   # 0: the dense race kernels run in the graph too
def test_fused_accept_repeats_and_replays_in_a_graph(device, top_k):
    """The per-row counters the fused accept keeps in its workspace return to zero after every call: repeated eager
    calls and HIP-graph replays give the same (bit-exact) answer."""
    log_case(f"fused accept repeated calls and graph replays top_k={top_k}")
    case = wl.sampler_case(16, 7, 32000, top_k=top_k, verified_lens=[1, 8, 3, 5, 2, 7, 4, 6] * 2,
                           draft_probs_fn=draft_probs)
    n_want, tail_want = run_oracle(case)
    g = case.to(device)
    st = ns.SamplingTensors(g.temperatures, g.top_k, g.top_p, case.max_top_k, case.has_top_p, top_k > 0)

    def call():
        return ns.spec_accept_with_draws(g.logits, g.q, g.drafts, st, g.verified_lens, g.uniforms, g.noise)

    for _ in range(3):
        n, tail = call()
        assert torch.equal(n.cpu(), n_want) and torch.equal(tail.cpu(), tail_want)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        n_g, tail_g = call()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(n_g.cpu(), n_want) and torch.equal(tail_g.cpu(), tail_want)
        n, tail = call()  # eager work between replays
        assert torch.equal(n.cpu(), n_want)


def test_graph_captured_before_the_counters_grow(device):
    """A graph of the fused accept captured while its row counters were small replays correctly after a larger
    eager call replaced them: a replaced counter buffer stays allocated, and every call leaves it zero."""
    log_case("fused accept: graph replays after the row counters grew")
    small = wl.sampler_case(8, 3, 4096, draft_probs_fn=draft_probs)
    n_want, tail_want = run_oracle(small)
    g = small.to(device)
    st = ns.SamplingTensors(g.temperatures, g.top_k, g.top_p, small.max_top_k, small.has_top_p, True)

    def call():
        return ns.spec_accept_with_draws(g.logits, g.q, g.drafts, st, None, g.uniforms, g.noise)

    call()
    before = _lib.persistent_workspace("spec_accept_row_counters", 4, torch.device(device))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        n_g, tail_g = call()
    big = wl.sampler_case(20000, 1, 64, top_k=8, draft_probs_fn=draft_probs)   # past the counters' minimum size
    n_big, tail_big = run_fused(big, device)
    n_big_want, tail_big_want = run_oracle(big)
    assert torch.equal(n_big, n_big_want) and torch.equal(tail_big, tail_big_want)
    after = _lib.persistent_workspace("spec_accept_row_counters", 4, torch.device(device))
    assert after.data_ptr() != before.data_ptr() and after.numel() >= 4 * 20000
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(n_g.cpu(), n_want) and torch.equal(tail_g.cpu(), tail_want)
        assert int(before.view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("greedy", [False, True], ids=["random", "greedy"])
@pytest.mark.parametrize("varlen", [False, True], ids=["all_drafts", "varlen"])
def test_accept_dispatch_follows_the_reference_branches(device, greedy, varlen):
    """accept() is SpeculativeDecoder._accept (speculative.py:450-462): greedy or random rows, every row verifying
    all k drafts ([B, k+1, V] logits) or verified_lens[r] - 1 of them ([T, V], lens handed over as the host list
    _accept receives). Each branch against the oracle's, bit for bit, and the generator left exactly where the
    reference leaves it: rand(B, k) then exponential_([B, V]) for random rows, untouched for greedy ones."""
    log_case(f"accept dispatch greedy={greedy} varlen={varlen}")
    lens = [1, 8, 3, 5, 2, 7, 4, 6] if varlen else None
    case = wl.sampler_case(8, 7, 32000, top_k=[64, 20, 5, 64] * 2, top_p=[0.9, 1.0, 0.6, 0.95] * 2,
                           temperature=[0.7, 1.0, 1.5, 1.0] * 2, verified_lens=lens, draft_probs_fn=draft_probs)
    g = case.to(device)
    batch, k = case.drafts.shape
    logits = g.logits if varlen else g.logits.view(batch, k + 1, -1)
    st = ns.SamplingTensors(None if greedy else g.temperatures, g.top_k, g.top_p, case.max_top_k, case.has_top_p,
                            True)
    ours = torch.Generator(device=device).manual_seed(77)
    n, tail = ns.accept(logits, g.drafts, None if greedy else g.q, st, lens, ours)
    theirs = torch.Generator(device=device).manual_seed(77)
    if greedy:
        want = ref.accept_greedy_varlen(case.logits, case.drafts, case.verified_lens) if varlen else \
            ref.accept_greedy(case.logits.view(batch, k + 1, -1), case.drafts)
    else:
        uniforms = torch.rand(batch, k, device=device, generator=theirs)
        noise = torch.empty(batch, 32000, device=device).exponential_(1.0, generator=theirs).clamp_min_(1e-10)
        want = ref.accept_from_logits(case.logits, case.q, case.drafts, case.temperatures, case.top_k, case.top_p,
                                      case.max_top_k, case.has_top_p, case.verified_lens, uniforms.cpu(),
                                      noise.cpu())
    assert torch.equal(ours.get_state(), theirs.get_state())
    assert torch.equal(n.cpu(), want[0]) and torch.equal(tail.cpu(), want[1])


@pytest.mark.parametrize("vocab", [50000, 50001])   # 16-byte pieces / element loads
@pytest.mark.parametrize("varlen", [False, True])
def test_dense_accept_random_is_bit_exact(device, varlen, vocab):
    log_case(f"accept_random dense varlen={varlen} V={vocab}")
    lens = [1, 8, 3, 5, 2, 7, 4, 6] if varlen else None
    case = wl.sampler_case(8, 7, vocab, verified_lens=lens, draft_probs_fn=draft_probs)
    p = ref.probs_from_logits(case.logits, case.temperatures.repeat_interleave(case.verified_lens)
                              if varlen else case.temperatures.repeat_interleave(8),
                              case.top_k.repeat_interleave(case.verified_lens) if varlen
                              else case.top_k.repeat_interleave(8),
                              case.top_p.repeat_interleave(case.verified_lens) if varlen
                              else case.top_p.repeat_interleave(8), case.max_top_k, case.has_top_p)
    want = ref.accept_random_varlen(p, case.q, case.drafts, case.verified_lens if varlen else
                                    torch.full((8,), 8, dtype=torch.int64), case.uniforms, case.noise)
    got = ns.accept_random_with_draws(p.to(device), case.q.to(device), case.drafts.to(device),
                                      None if lens is None else case.verified_lens.to(device),
                                      case.uniforms.to(device), case.noise.to(device))
    assert torch.equal(got[0].cpu(), want[0]) and torch.equal(got[1].cpu(), want[1])


def test_greedy_matches_the_oracle_on_random_logits(device):
    log_case("greedy random")
    gen = torch.Generator().manual_seed(4)
    logits = (torch.randn(40, 151936, generator=gen) * 3).to(torch.bfloat16)
    lens = torch.tensor([8, 1, 5, 8, 3, 7, 8])
    drafts = torch.randint(151936, (7, 7), generator=gen)
    tokens = logits.float().argmax(-1)
    starts = lens.cumsum(0) - lens
    for b in range(7):   # make some drafts right
        for j in range(int(lens[b]) - 1):
            if (b + j) % 3:
                drafts[b, j] = tokens[starts[b] + j]
    want = ref.accept_greedy_varlen(logits.float(), drafts, lens)
    got = ns.accept_greedy_varlen(logits.to(device), drafts.to(device), lens.to(device))
    assert torch.equal(got[0].cpu(), want[0]) and torch.equal(got[1].cpu(), want[1])


def test_generator_consumption_matches_the_reference_order(device):
    """accept_random_varlen draws rand(B, k) then exponential_([B, V]) from the generator, nothing else."""
    log_case("generator order")
    p, q, drafts, lens, _, _ = ka.varlen_case()
    ours = torch.Generator(device=device).manual_seed(42)
    theirs = torch.Generator(device=device).manual_seed(42)
    ns.accept_random_varlen(p.to(device), q.to(device), drafts.to(device), lens.to(device), ours)
    torch.rand(3, 3, device=device, generator=theirs)
    torch.empty(3, 4, device=device).exponential_(1.0, generator=theirs)
    assert torch.equal(ours.get_state(), theirs.get_state())


MULTI = [c for c in FROZEN["cases"] if "p_rows" in c]


@pytest.mark.parametrize("case, k", [(c, 3) for c in MULTI] + [(FROZEN["k7_case"], 7)],
                         ids=lambda v: v["name"] if isinstance(v, dict) else f"k{v}")
def test_gpu_rounds_follow_the_target(device, case, k):
    """test_accept_random_multistep.py's gate through the HIP accept_random on the device: whole speculative rounds
    of the frozen Markov cases, 100k rows, every output sequence within the Hoeffding bound (delta = 0.001)."""
    log_case(f"multistep gate {case['name']}")
    from collections import Counter

    from test_oracle_sampler import hoeffding, target_outputs
    g = torch.Generator(device=device).manual_seed(17011)
    p_rows = torch.tensor(case["p_rows"], dtype=torch.float32, device=device)
    q_rows = torch.tensor(case["q_rows"], dtype=torch.float32, device=device)
    eos, cap = case["eos_token_id"], case["max_tokens"]
    trials = 100_000
    outputs = [[] for _ in range(trials)]
    state = torch.zeros(trials, dtype=torch.long)   # host copy; per-row updates stay off the device
    active = list(range(trials))
    while active:
        idx = torch.tensor(active)
        states, drafts = [state[idx].to(device)], []
        for _ in range(k):
            drafts.append(ns.sample(q_rows[states[-1]], g))
            states.append(drafts[-1] + 1)
        p = torch.stack([p_rows[s] for s in states], dim=1)
        q = torch.stack([q_rows[s] for s in states[:-1]], dim=1)
        drafts = torch.stack(drafts, dim=1)
        n_acc, tail = ns.accept_random(p, q, drafts, g)
        rounds = torch.cat([drafts, tail[:, None]], dim=1).tolist()
        keep = []
        for row, toks, cnt in zip(active, rounds, n_acc.tolist()):
            for tok in toks[:cnt] + [toks[k]]:
                outputs[row].append(tok)
                if tok == eos or len(outputs[row]) == cap:
                    break
            if outputs[row][-1] != eos and len(outputs[row]) < cap:
                keep.append(row)
                state[row] = outputs[row][-1] + 1
        active = keep
    expected = {s: float(v) for s, v in target_outputs(case).items()}
    counts = Counter(tuple(o) for o in outputs)
    assert set(counts) <= set(expected)
    bound = hoeffding(len(expected), trials)
    worst = max(abs(counts[s] / trials - v) for s, v in expected.items())
    assert worst <= bound, (worst, bound)
    assert math.isfinite(worst)
