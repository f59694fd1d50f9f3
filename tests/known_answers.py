"""Known answers of the reference's sampler tests (tests/test_spec_sampler.py), as data.

Each case gives inputs and expected outputs; tests/test_oracle_sampler.py checks the CPU oracle against them and
tests/test_gpu_sampler.py the HIP kernels. Line numbers cite the reference test each case comes from.
"""
import math

import torch

INF = math.inf


def softmax(values):
    return torch.softmax(torch.tensor(values, dtype=torch.float32), dim=-1).tolist()


# (name, rows of (temperature, top_k, top_p), logits, expected probabilities)   test_spec_sampler.py:47-89
PROBS_CASES = [
    ("temperature_scales_logits", [(0.5, 0, 1.0)], [[1.0, 0.0]], [softmax([2.0, 0.0])]),          # :47-52
    ("top_k_keeps_k_largest", [(1.0, 2, 1.0)], [[1.0, 3.0, 2.0, 0.0]],
     [[0.0] + softmax([3.0, 2.0]) + [0.0]]),                                                      # :55-60
    ("top_k_keeps_ties", [(1.0, 1, 1.0)], [[2.0, 2.0, 1.0, 0.0]], [[0.5, 0.5, 0.0, 0.0]]),        # :63-67
    ("top_p_smallest_prefix", [(1.0, 4, 0.5)], [[math.log(w) for w in (0.4, 0.3, 0.2, 0.1)]],
     [[4 / 7, 3 / 7, 0.0, 0.0]]),                                                                 # :70-74
    ("top_p_within_top_k", [(1.0, 2, 0.99)], [[math.log(w) for w in (0.4, 0.3, 0.2, 0.1)]],
     [[4 / 7, 3 / 7, 0.0, 0.0]]),                                                                 # :77-81
    ("mixed_rows", [(1.0, 0, 1.0), (1.0, 1, 1.0)], [[1.0, 2.0, 3.0], [1.0, 2.0, 3.0]],
     [softmax([1.0, 2.0, 3.0]), [0.0, 0.0, 1.0]]),                                                # :84-89
]

# truncation broadcast over a middle positions dimension, test_spec_sampler.py:92-97
BROADCAST_CASE = ([(1.0, 1, 1.0)], [[[1.0, 5.0, 2.0], [9.0, 5.0, 2.0]]],
                  [[[-INF, 5.0, -INF], [9.0, -INF, -INF]]])


def bonus_case():
    """All drafts accepted -> tail drawn from the bonus position (test_spec_sampler.py:129-139)."""
    p = torch.zeros(1, 3, 4)
    p[0, :2] = torch.tensor([0.25, 0.25, 0.25, 0.25])
    p[0, 2, 3] = 1.0
    q = p[:, :2].clone()
    return p, q, torch.tensor([[0, 1]]), [2], [3]


def zero_mass_case():
    """The target never emits the draft -> rejected, residual is a point mass on token 0 (:142-149)."""
    p = torch.tensor([[[1.0, 0.0], [0.5, 0.5]]])
    q = torch.tensor([[[0.0, 1.0]]])
    return p, q, torch.tensor([[1]]), [0], [0]


def greedy_prefix_cases():
    """(num_drafts, first_mismatch) grid of test_spec_sampler.py:152-167."""
    out = []
    for num_drafts in (1, 2, 4):
        for first_mismatch in range(5):
            if first_mismatch > num_drafts:
                continue
            vocab = 16
            drafts = torch.arange(1, num_drafts + 1).unsqueeze(0)
            target_tokens = list(range(1, num_drafts + 2))
            if first_mismatch < num_drafts:
                target_tokens[first_mismatch] = 9
            logits = torch.full((1, num_drafts + 1, vocab), -10.0)
            logits[0, torch.arange(num_drafts + 1), torch.tensor(target_tokens)] = 10.0
            count = min(first_mismatch, num_drafts)
            out.append((f"k{num_drafts}_mismatch{first_mismatch}", logits, drafts, [count], [target_tokens[count]]))
    return out


def greedy_per_row_case():
    """test_spec_sampler.py:170-176."""
    logits = torch.full((2, 2, 4), -10.0)
    logits[0, 0, 1] = logits[0, 1, 2] = 10.0
    logits[1, 0, 3] = logits[1, 1, 2] = 10.0
    return logits, torch.tensor([[1], [1]]), [1, 0], [2, 3]


def varlen_case():
    """Rows verifying 1, 2 and 4 positions over point masses (test_spec_sampler.py:224-244): n_accept [0, 1, 3],
    tail [3, 2, 0] for both the random and the greedy rule."""
    point = torch.eye(4)
    p = point[[3, 1, 2, 1, 2, 3, 0]]
    drafts = torch.tensor([[1, 2, 3]] * 3)
    q = torch.eye(4)[drafts]
    return p, q, drafts, torch.tensor([1, 2, 4]), [0, 1, 3], [3, 2, 0]
