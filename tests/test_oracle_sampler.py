"""Pins the CPU sampler oracle (oracle/spec_sampler.py) against the reference's known answers, its frozen
distribution cases and the mathematics of rejection sampling. CPU only."""
import hashlib
import json
import math
import pathlib
from collections import Counter
from fractions import Fraction

import pytest
import torch

import known_answers as ka
from oracle import spec_sampler as ref

GOLDEN = pathlib.Path(__file__).parent / "golden" / "random_sampling_cases.json"
FROZEN = json.loads(GOLDEN.read_text())
CASES = FROZEN["cases"]
K7_CASE = FROZEN["k7_case"]


def params(rows):
    t = torch.tensor([r[0] for r in rows], dtype=torch.float32)
    k = torch.tensor([r[1] for r in rows], dtype=torch.int64)
    p = torch.tensor([r[2] for r in rows], dtype=torch.float32)
    return t, k, p, int(k.max()), bool((p < 1.0).any())


@pytest.mark.parametrize("case", ka.PROBS_CASES, ids=[c[0] for c in ka.PROBS_CASES])
def test_probs_known_answers(case):
    _, rows, logits, expected = case
    t, k, p, max_k, has_p = params(rows)
    probs = ref.probs_from_logits(torch.tensor(logits), t, k, p, max_k, has_p)
    torch.testing.assert_close(probs, torch.tensor(expected, dtype=torch.float32))


def test_truncation_broadcasts_over_positions():
    rows, logits, expected = ka.BROADCAST_CASE
    t, k, p, max_k, has_p = params(rows)
    out = ref.truncate_logits(torch.tensor(logits), k, p, max_k, has_p)
    assert out.tolist() == expected


def test_race_frequencies_follow_the_weights():
    g = torch.Generator().manual_seed(0)
    weights = torch.tensor([0.1, 0.6, 0.3]).expand(200_000, 3)
    counts = torch.bincount(ref.sample(weights, g), minlength=3).float() / 200_000
    torch.testing.assert_close(counts, torch.tensor([0.1, 0.6, 0.3]), atol=0.005, rtol=0)


def test_race_never_picks_zero_weight():
    g = torch.Generator().manual_seed(1)
    weights = torch.tensor([0.0, 1.0, 0.0]).expand(10_000, 3)
    assert (ref.sample(weights, g) == 1).all()


def test_race_first_index_wins_ties_and_zero_weights_give_index_zero():
    w = torch.tensor([[0.0, 2.0, 2.0, 1.0], [0.0, 0.0, 0.0, 0.0]])
    e = torch.ones(2, 4)
    assert ref.race(w, e).tolist() == [1, 0]


SINGLE = [c for c in CASES if "p" in c]


@pytest.mark.parametrize("case", SINGLE, ids=[c["name"] for c in SINGLE])
def test_accept_random_emits_the_target_distribution(case):
    # test_spec_sampler.py:113-126: drafts ~ q, one verified position + bonus; output frequencies within TV 0.01
    n = 200_000
    g = torch.Generator().manual_seed(1234)
    p_row = torch.tensor(case["p"])
    q_row = torch.tensor(case["q"])
    vocab = p_row.numel()
    drafts = ref.sample(q_row.expand(n, vocab), g).unsqueeze(1)
    n_accept, tail = ref.accept_random_gen(p_row.expand(n, 2, vocab), q_row.expand(n, 1, vocab), drafts, g)
    emitted = torch.where(n_accept == 1, drafts[:, 0], tail)
    freq = torch.bincount(emitted, minlength=vocab).float() / n
    assert 0.5 * (freq - p_row).abs().sum().item() < 0.01


def test_bonus_row_when_all_accepted():
    p, q, drafts, n_exp, tail_exp = ka.bonus_case()
    n, tail = ref.accept_random_gen(p, q, drafts, torch.Generator().manual_seed(0))
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)


def test_rejects_where_target_has_zero_mass():
    p, q, drafts, n_exp, tail_exp = ka.zero_mass_case()
    n, tail = ref.accept_random_gen(p, q, drafts, torch.Generator().manual_seed(0))
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)


@pytest.mark.parametrize("case", ka.greedy_prefix_cases(), ids=lambda c: c[0])
def test_greedy_counts_the_matching_prefix(case):
    _, logits, drafts, n_exp, tail_exp = case
    n, tail = ref.accept_greedy(logits, drafts)
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)


def test_greedy_is_per_row():
    logits, drafts, n_exp, tail_exp = ka.greedy_per_row_case()
    n, tail = ref.accept_greedy(logits, drafts)
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)


def test_varlen_accepts_at_most_the_verified_drafts():
    p, q, drafts, lens, n_exp, tail_exp = ka.varlen_case()
    n, tail = ref.accept_random_varlen_gen(p, q, drafts, lens, torch.Generator().manual_seed(0))
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)
    n, tail = ref.accept_greedy_varlen(p, drafts, lens)
    assert (n.tolist(), tail.tolist()) == (n_exp, tail_exp)


def fixed_length_rule(p, q, drafts, generator):
    """The fixed-length acceptance the variable-length rule must reproduce when every row verifies all drafts
    (test_spec_sampler.py:180-195): gathers on [B, k+1, V] directly, bonus when all k are accepted."""
    batch, k = drafts.shape
    index = drafts.unsqueeze(-1)
    p_d = p[:, :k].gather(-1, index).squeeze(-1)
    q_d = q.gather(-1, index).squeeze(-1)
    u = torch.rand(batch, k, generator=generator)
    n = (u * q_d < p_d).long().cumprod(dim=-1).sum(dim=-1)
    rows = torch.arange(batch)
    p_next = p[rows, n]
    q_next = q[rows, n.clamp(max=k - 1)]
    w = torch.where((n == k).unsqueeze(-1), p_next, (p_next - q_next).clamp(min=0))
    return n, ref.sample(w, generator)


@pytest.mark.parametrize("seed", range(5))
def test_varlen_rule_reproduces_the_fixed_length_rule(seed):
    torch.manual_seed(seed)
    p = torch.softmax(torch.randn(6, 8, 5), dim=-1)
    q = torch.softmax(torch.randn(6, 7, 5), dim=-1)
    drafts = torch.randint(5, (6, 7))
    ours, theirs = torch.Generator().manual_seed(seed), torch.Generator().manual_seed(seed)
    for got, want in zip(ref.accept_random_gen(p, q, drafts, ours), fixed_length_rule(p, q, drafts, theirs)):
        assert torch.equal(got, want)
    assert torch.equal(ours.get_state(), theirs.get_state())


def test_per_token_parameters_equal_per_row_broadcast():
    # test_spec_sampler.py:247-253
    t, k, p, max_k, has_p = params([(0.7, 3, 0.9), (1.0, 0, 1.0)])
    logits = torch.randn(2, 4, 6, generator=torch.Generator().manual_seed(3))
    lens = torch.tensor([4, 4])
    per_tok = [x.repeat_interleave(lens, output_size=8) for x in (t, k, p)]
    flat = ref.probs_from_logits(logits.flatten(0, 1), *per_tok, max_k, has_p)
    assert torch.equal(flat, ref.probs_from_logits(logits, t, k, p, max_k, has_p).flatten(0, 1))


def test_top_k_zero_rows_keep_every_token_and_top_p_one_keeps_all_candidates():
    logits = torch.randn(3, 50, generator=torch.Generator().manual_seed(4))
    t, k, p, max_k, has_p = params([(1.0, 0, 1.0), (1.0, 50, 1.0), (1.0, 5, 1.0)])
    probs = ref.probs_from_logits(logits, t, k, p, max_k, has_p)
    torch.testing.assert_close(probs[0], torch.softmax(logits[0], -1))
    torch.testing.assert_close(probs[1], torch.softmax(logits[1], -1))
    assert int((probs[2] > 0).sum()) == 5


# ---------------------------------------------------------------- exact distributions of the frozen cases
def test_frozen_cases_identity():
    # tests/test_random_reference.py:20,132-136
    assert len(CASES) == 12 and len({c["name"] for c in CASES}) == 12
    encoded = json.dumps(CASES, sort_keys=True, separators=(",", ":")).encode()
    assert hashlib.sha256(encoded).hexdigest() == "e918671a27e2d6688448e8e85ac8f5f1587b8ace3135a901971204229eaa8b4a"


def exact(row):
    return tuple(Fraction(str(v)) for v in row)


def target_outputs(case):
    """Exact output distribution of the target alone: a Markov chain stopping at EOS or max_tokens."""
    if "p" in case:
        return {(i,): Fraction(str(v)) for i, v in enumerate(case["p"])}
    rows = [exact(r) for r in case["p_rows"]]
    out = {}

    def visit(prefix, mass):
        if len(prefix) == case["max_tokens"] or (prefix and prefix[-1] == case["eos_token_id"]):
            out[prefix] = mass
            return
        for tok, v in enumerate(rows[0 if not prefix else prefix[-1] + 1]):
            visit(prefix + (tok,), mass * v)

    visit((), Fraction(1))
    return out


def speculative_outputs(case, draft_len):
    """Exact output distribution of whole speculative rounds (draft, accept min(1, p/q), residual or bonus),
    enumerated with Fractions; it must equal the target's."""
    p_rows = [exact(r) for r in case["p_rows"]]
    q_rows = [exact(r) for r in case["q_rows"]]
    cap, eos = case["max_tokens"], case["eos_token_id"]

    def stopped(x):
        return len(x) == cap or bool(x and x[-1] == eos)

    def row(rows, x):
        return rows[0 if not x else x[-1] + 1]

    memo = {}

    def rounds(prefix):
        if stopped(prefix):
            return {prefix: Fraction(1)}
        if prefix in memo:
            return memo[prefix]
        result = {}

        def add(history, mass):
            if mass:
                for seq, cond in rounds(history).items():
                    result[seq] = result.get(seq, 0) + mass * cond

        def proposals(draft=(), mass=Fraction(1)):
            if len(draft) == draft_len or stopped(prefix + draft):
                yield draft, mass
                return
            for tok, qm in enumerate(row(q_rows, prefix + draft)):
                if qm:
                    yield from proposals(draft + (tok,), mass * qm)

        def verify(history, draft, i, mass):
            if stopped(history):
                result[history] = result.get(history, 0) + mass
                return
            p = row(p_rows, history)
            if i == len(draft):
                for tok, v in enumerate(p):
                    add(history + (tok,), mass * v)
                return
            q = row(q_rows, history)
            d = draft[i]
            a = min(Fraction(1), p[d] / q[d])
            if a:
                verify(history + (d,), draft, i + 1, mass * a)
            if a < 1:
                pos = [max(Fraction(0), px - qx) for px, qx in zip(p, q)]
                tot = sum(pos)
                for tok, v in enumerate(pos):
                    add(history + (tok,), mass * (1 - a) * v / tot)

        for draft, mass in proposals():
            verify(prefix, draft, 0, mass)
        memo[prefix] = result
        return result

    return rounds(())


MULTI = [c for c in CASES if "p_rows" in c]


@pytest.mark.parametrize("case", MULTI + [K7_CASE], ids=lambda c: c["name"])
@pytest.mark.parametrize("draft_len", [1, 2, 3])
def test_speculative_rounds_reproduce_the_target_exactly(case, draft_len):
    def nonzero(d):
        return {seq: v for seq, v in d.items() if v}
    assert nonzero(speculative_outputs(case, draft_len)) == nonzero(target_outputs(case))


def hoeffding(categories, trials, delta=0.001):
    return math.sqrt(math.log(2 * categories / delta) / (2 * trials))


def test_hoeffding_bound_matches_the_reference_value():
    # test_accept_random_multistep.py:117-118
    assert hoeffding(13, 100_000) == pytest.approx(0.0071295, abs=1e-6)


def simulate(case, k, trials, accept_fn, generator, lengths=None):
    """Rows run speculative rounds until they stop (test_accept_random_multistep.py:30-84). accept_fn(p, q, drafts,
    lens) -> (n_accept, tail); p is [n, k+1, V] flattened to the verified positions when lens is given."""
    p_rows = torch.tensor(case["p_rows"], dtype=torch.float32)
    q_rows = torch.tensor(case["q_rows"], dtype=torch.float32)
    eos, cap = case["eos_token_id"], case["max_tokens"]
    outputs = [[] for _ in range(trials)]
    state = torch.zeros(trials, dtype=torch.long)
    active = list(range(trials))
    while active:
        idx = torch.tensor(active)
        states, drafts = [state[idx]], []
        for _ in range(k):
            drafts.append(ref.sample(q_rows[states[-1]], generator))
            states.append(drafts[-1] + 1)
        p = torch.stack([p_rows[s] for s in states], dim=1)
        q = torch.stack([q_rows[s] for s in states[:-1]], dim=1)
        drafts = torch.stack(drafts, dim=1)
        if lengths is None:
            n_acc, tail = accept_fn(p, q, drafts, None)
        else:
            lens = lengths(len(active))
            verified = torch.arange(k + 1) < lens.unsqueeze(1)
            n_acc, tail = accept_fn(p[verified], q, drafts, lens)
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
    return [tuple(o) for o in outputs]


def assert_target(case, outputs):
    expected = {seq: float(v) for seq, v in target_outputs(case).items()}
    counts = Counter(outputs)
    assert set(counts) <= set(expected)
    bound = hoeffding(len(expected), len(outputs))
    worst = max(abs(counts[s] / len(outputs) - v) for s, v in expected.items())
    assert worst <= bound, (case["name"], worst, bound)


@pytest.mark.parametrize("case, k", [(c, 3) for c in MULTI] + [(K7_CASE, 7)], ids=lambda v: v["name"] if isinstance(v, dict) else f"k{v}")
@pytest.mark.parametrize("varlen", [False, True], ids=["fixed", "varlen"])
def test_oracle_rounds_follow_the_target(case, k, varlen):
    # test_accept_random_multistep.py:126-163 with 40k trials
    g = torch.Generator().manual_seed(17011)
    lg = torch.Generator().manual_seed(110017)

    def accept(p, q, drafts, lens):
        if lens is None:
            return ref.accept_random_gen(p, q, drafts, g)
        return ref.accept_random_varlen_gen(p, q, drafts, lens, g)

    lengths = (lambda n: torch.randint(1, k + 2, (n,), generator=lg)) if varlen else None
    assert_target(case, simulate(case, k, 40_000, accept, g, lengths))


def test_a_planted_mistake_fails_the_gate():
    """The distribution gate has power: accepting with u * q < p + 0.2 (a wrong acceptance rule) is caught."""
    case = MULTI[0]
    g = torch.Generator().manual_seed(5)

    def wrong(p, q, drafts, lens):
        uniforms, noise = ref.draws(drafts.shape[0], drafts.shape[1], p.shape[-1], g)
        return ref.accept_random(p + 0.2 * (p > 0), q, drafts, uniforms, noise)

    with pytest.raises(AssertionError):
        assert_target(case, simulate(case, 3, 40_000, wrong, g))
