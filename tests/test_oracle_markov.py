"""Pinning of oracle.markov against the known answers of the reference's tests/test_dspark_propose.py and against
what the mathematics fixes: the greedy Markov chain, q equal to each row's distribution after its bias, candidate
rows equal to the whole-vocabulary distribution (ties at the cut included), the bias of the token drawn before
(never of the row's own draft), and a single kept token that wins whatever the noise."""
import torch

from oracle import markov as om
from oracle import spec_sampler as ss

# The reference tests' Markov bias by previous token: token 0 adds 2 to token 1's logit (test_dspark_propose.py:18-21).
BIAS = torch.tensor([[0.0, 2.0, 0.0],
                     [0.0, 0.0, 0.0],
                     [0.0, 0.0, 0.0]])


def params(temps, top_k, top_p):
    t = None if temps is None else torch.tensor(temps, dtype=torch.float32)
    k = torch.tensor(top_k, dtype=torch.int64)
    p = torch.tensor(top_p, dtype=torch.float32)
    return t, k, p, int(k.max()), bool((p < 1).any()), bool((k > 0).all())


def test_greedy_drafts_follow_the_markov_chain():
    # test_dspark_propose.py:36-42: base logits [2, 1, 0] at every row; anchors 0 and 1 give 1,0,1 and 0,1,0
    logits = torch.tensor([2.0, 1.0, 0.0]).expand(2, 3, 3)
    t, k, p, mk, hp, ak = params(None, [0, 0], [1.0, 1.0])
    drafts, q, ids, probs = om.markov_rows(logits, torch.tensor([0, 1]), lambda prev: BIAS[prev], t, k, p, mk, hp,
                                           ak, None)
    assert drafts.tolist() == [[1, 0, 1], [0, 1, 0]] and q is None and ids is None


def test_q_is_each_row_distribution_after_its_bias():
    # test_dspark_propose.py:45-53: rows (T 1) and (T 0.7, top-k 2); one row does not truncate -> dense rows
    t, k, p, mk, hp, ak = params([1.0, 0.7], [0, 2], [1.0, 1.0])
    logits = torch.randn(2, 4, 3, generator=torch.Generator().manual_seed(1))
    noise = ss.exponential_noise((2, 4, 3), torch.Generator().manual_seed(0))
    drafts, q, ids, _ = om.markov_rows(logits, torch.tensor([0, 1]), lambda prev: BIAS[prev], t, k, p, mk, hp, ak,
                                       noise)
    assert ids is None
    prev = torch.tensor([0, 1])
    for row in range(4):
        assert torch.equal(q[:, row], ss.probs_from_logits(logits[:, row] + BIAS[prev], t, k, p, mk, hp))
        prev = drafts[:, row]


def test_without_a_bias_the_rows_draw_what_dflash_draws():
    # test_dspark_propose.py:56-71: zero bias, dense rows -> DFlash's q and drafts from the same noise
    t, k, p, mk, hp, ak = params([1.0, 0.7], [0, 3], [1.0, 0.9])
    logits = torch.randn(2, 4, 6, generator=torch.Generator().manual_seed(2))
    noise = ss.exponential_noise((2, 4, 6), torch.Generator().manual_seed(0))
    drafts, q, _, _ = om.markov_rows(logits, torch.tensor([2, 0]), lambda prev: torch.zeros(len(prev), 6), t, k, p,
                                     mk, hp, ak, noise)
    dflash = ss.probs_from_logits(logits, t, k, p, mk, hp)
    assert torch.equal(q, dflash)
    assert torch.equal(drafts, ss.race(dflash, noise))


def test_candidate_rows_give_the_whole_vocabulary_distribution():
    # test_dspark_propose.py:74-88: every row truncates, so rows are drawn among the top 20 + 64 = 84 logits; in
    # the top-3 row thirty tokens tie with the cut value 3, out to rank 31, and the candidates keep them all
    vocab, k = 200, 4
    t, kk, p, mk, hp, ak = params([0.7, 1.0], [3, 20], [1.0, 0.8])
    assert om.num_candidates(mk, ak, vocab) == 84
    logits = torch.randn(2, k, vocab, generator=torch.Generator().manual_seed(5))
    logits[0] = logits[0].clamp(max=2.5)
    logits[0, :, :32] = torch.tensor([5.0, 4.0] + [3.0] * 30)
    noise = ss.exponential_noise((2, k, 84), torch.Generator().manual_seed(0))
    drafts, q, ids, probs = om.markov_rows(logits, torch.tensor([2, 0]), lambda prev: torch.zeros(len(prev), vocab),
                                           t, kk, p, mk, hp, ak, noise)
    whole = ss.probs_from_logits(logits, t, kk, p, mk, hp)
    assert torch.equal(q > 0, whole > 0)
    assert torch.allclose(q, whole, rtol=0, atol=1e-6)
    assert bool((q.gather(-1, drafts.unsqueeze(-1)) > 0).all())
    # the candidate rows are the scattered q, in value order with ties by index
    assert torch.equal(q.gather(-1, ids), probs)
    assert ids[0, 0, :32].tolist() == list(range(32))


def test_the_bias_comes_from_the_token_drawn_before():
    # with a bias that forces token (prev + 1) % V, the chain from anchor a is a+1, a+2, ... whatever the logits;
    # a bias keyed on the row's own draft would be circular and could not produce it
    vocab = 16
    forced = torch.full((vocab, vocab), -1e4)
    forced[torch.arange(vocab), (torch.arange(vocab) + 1) % vocab] = 0.0
    t, k, p, mk, hp, ak = params([1.0, 1.0], [5, 5], [1.0, 1.0])
    logits = torch.randn(2, 6, vocab, generator=torch.Generator().manual_seed(3))
    noise = ss.exponential_noise((2, 6, om.num_candidates(mk, ak, vocab)), torch.Generator().manual_seed(4))
    drafts, _, _, _ = om.markov_rows(logits, torch.tensor([3, 15]), lambda prev: forced[prev], t, k, p, mk, hp, ak,
                                     noise)
    assert drafts.tolist() == [[4, 5, 6, 7, 8, 9], [0, 1, 2, 3, 4, 5]]


def test_one_kept_token_wins_whatever_the_noise():
    t, k, p, mk, hp, ak = params([1.0], [1], [1.0])
    logits = torch.randn(1, 3, 50, generator=torch.Generator().manual_seed(6))
    for seed in range(5):
        noise = ss.exponential_noise((1, 3, 50), torch.Generator().manual_seed(seed))
        drafts, _, ids, probs = om.markov_rows(logits, torch.tensor([0]), lambda prev: torch.zeros(1, 50), t, k, p,
                                               mk, hp, ak, noise)
        assert drafts[0].tolist() == logits[0].argmax(-1).tolist()
        assert torch.equal(probs[..., 0], torch.ones(1, 3)) and bool((probs[..., 1:] == 0).all())
