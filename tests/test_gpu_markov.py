"""DSpark's Markov rows on the GPU against the oracle (oracle/markov.py), through nvs_markov_draw.

The Markov bias is a lookup table by previous token (as the reference's tests/test_dspark_propose.py passes it),
so the GPU and the CPU oracle add identical biases whenever they drew identical tokens.
Bar: drafts bit-exact, candidate ids bit-exact, the number of kept candidates equal, probabilities within 1e-5 of
their value (the kernel's exp and its sum order differ from torch's softmax). Cases: the reference's propose tests,
random rows at V = 4,096 (fp32), 151,936 (bf16) and 32,000 (fp16) with mixed temperatures / top-k / top-p,
vocabularies that end inside a 16-byte piece (padded and unpadded rows), rows cut into 11 and 62 segments, ties at
the cut inside and beyond the candidates (the kernel's ordered tie pass), a dense batch (a row without top-k), and
the sparse rows scattered back to the reference's dense q.
"""
import pytest
import torch

from conftest import log_case
from nvs_amd.layers import markov as nm
from nvs_amd.layers import spec_sampler as ns
from oracle import markov as om
from oracle import spec_sampler as ss

pytestmark = pytest.mark.gpu


def sampling(device, temps, top_k, top_p):
    t = None if temps is None else torch.tensor(temps, dtype=torch.float32, device=device)
    k = torch.tensor(top_k, dtype=torch.int64, device=device)
    p = torch.tensor(top_p, dtype=torch.float32, device=device)
    return ns.SamplingTensors(t, k, p, int(k.max()), bool((p < 1).any()), bool((k > 0).all()))


def run_both(device, logits, anchors, table, st, seed=0, pad=0):
    """The product's sample_markov on the GPU and the oracle on the CPU with the same noise. With pad > 0 the
    device logits and bias rows sit in rows pad elements wider (row strides the vocabulary does not give)."""
    bias = lambda prev: table[prev % table.shape[0]]
    gen = torch.Generator(device=device).manual_seed(seed)
    if pad:
        lg = torch.zeros(*logits.shape[:-1], logits.shape[-1] + pad, dtype=logits.dtype, device=device)
        lg = lg[..., :logits.shape[-1]]
        lg.copy_(logits)
        tab = torch.zeros(table.shape[0], table.shape[1] + pad, dtype=table.dtype, device=device)
        tab = tab[:, :table.shape[1]]
        tab.copy_(table)
    else:
        lg = logits.to(device)
        tab = table.to(device)
    drafts, q = nm.sample_markov(lg, anchors.to(device), st, lambda prev: tab[prev % tab.shape[0]], gen)
    torch.cuda.synchronize()
    batch, k, vocab = logits.shape
    cands = nm.num_candidates(st.max_top_k, st.all_top_k, vocab)
    noise = None
    if st.temperatures is not None:
        gen.manual_seed(seed)                        # the product's draw, replayed for the oracle
        noise = ns.exponential_noise_(torch.empty(batch, k, cands or vocab, device=device), gen).cpu()
    cpu = lambda t: None if t is None else t.cpu()
    want = om.markov_rows(logits, anchors, bias, cpu(st.temperatures), cpu(st.top_k), cpu(st.top_p), st.max_top_k,
                          st.has_top_p, st.all_top_k, noise)
    return drafts.cpu(), q, want


def check_candidates(q, want, what):
    _, _, ids_ref, probs_ref = want
    ids, probs = q.ids.cpu().long(), q.probs.cpu()
    live = ids >= 0
    kept_ref = probs_ref > 0
    assert torch.equal(live.sum(-1), kept_ref.sum(-1)), f"{what}: kept counts differ"
    assert torch.equal(ids[live], ids_ref[live]), f"{what}: candidate ids differ"
    assert bool((probs[~live] == 0).all())
    assert torch.allclose(probs, probs_ref, rtol=1e-5, atol=1e-7), \
        f"{what}: max prob diff {float((probs - probs_ref).abs().max()):.3e}"


def test_reference_propose_cases(device):
    log_case("markov rows: reference propose cases")
    bias = torch.tensor([[0.0, 2.0, 0.0], [0.0, 0.0, 0.0], [0.0, 0.0, 0.0]])
    logits = torch.tensor([2.0, 1.0, 0.0]).expand(2, 3, 3).contiguous()
    drafts, q, _ = run_both(device, logits, torch.tensor([0, 1]), bias, sampling(device, None, [0, 0], [1.0, 1.0]))
    assert drafts.tolist() == [[1, 0, 1], [0, 1, 0]] and q is None
    # every row truncates: candidate rows over 84 of 200 tokens, thirty ties at the cut value 3
    vocab = 200
    logits = torch.randn(2, 4, vocab, generator=torch.Generator().manual_seed(5))
    logits[0] = logits[0].clamp(max=2.5)
    logits[0, :, :32] = torch.tensor([5.0, 4.0] + [3.0] * 30)
    st = sampling(device, [0.7, 1.0], [3, 20], [1.0, 0.8])
    drafts, q, want = run_both(device, logits, torch.tensor([2, 0]), torch.zeros(1, vocab), st)
    assert isinstance(q, nm.CandidateRows) and q.ids.shape == (2, 4, 84)
    assert torch.equal(drafts, want[0])
    check_candidates(q, want, "ties at the cut")
    dense = q.to_dense(vocab).cpu()
    assert torch.equal(dense > 0, want[1] > 0) and torch.allclose(dense, want[1], rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("vocab, dtype, batch", [(4096, torch.float32, 16), (151936, torch.bfloat16, 8),
                                                 (32000, torch.float16, 8)])
def test_random_rows_match_the_oracle(device, vocab, dtype, batch):
    log_case(f"markov rows: random V={vocab} {dtype} B={batch}")
    g = torch.Generator().manual_seed(vocab)
    logits = (torch.randn(batch, 7, vocab, generator=g) * 3).to(dtype)
    table = (torch.randn(16, vocab, generator=g) * 2).to(dtype)
    temps = [1.0, 0.7, 1.3, 1.0] * (batch // 4)
    top_k = [20, 5, 50, 1] * (batch // 4)
    top_p = [1.0, 0.8, 0.95, 1.0] * (batch // 4)
    st = sampling(device, temps, top_k, top_p)
    anchors = torch.randint(0, vocab, (batch,), generator=g)
    drafts, q, want = run_both(device, logits, anchors, table, st, seed=1)
    assert torch.equal(drafts, want[0]), f"drafts differ at {(drafts != want[0]).nonzero()[:5].tolist()}"
    check_candidates(q, want, "random rows")


def test_segments_near_the_limit_match_the_oracle(device):
    """V = 1,200,000 cuts each row into 62 segments (the split draw allows 64, and segments x candidates <= 4,096,
    so top-k <= 2 here): the merge's counts run over eight groups of lists."""
    vocab = 1_200_000
    log_case(f"markov rows: V={vocab} bf16, 62 segments")
    g = torch.Generator().manual_seed(62)
    batch = 4
    logits = (torch.randn(batch, 2, vocab, generator=g) * 3).to(torch.bfloat16)
    table = (torch.randn(4, vocab, generator=g) * 2).to(torch.bfloat16)
    st = sampling(device, [1.0, 0.8, 1.0, 1.3], [2, 1, 2, 2], [1.0, 1.0, 0.9, 1.0])
    anchors = torch.randint(0, vocab, (batch,), generator=g)
    drafts, q, want = run_both(device, logits, anchors, table, st, seed=4)
    assert torch.equal(drafts, want[0]), f"drafts differ at {(drafts != want[0]).nonzero()[:5].tolist()}"
    check_candidates(q, want, "62 segments")


@pytest.mark.parametrize("vocab, dtype, pad", [
    (32003, torch.bfloat16, 5),    # element loads (V is no whole number of 16-byte pieces); the last segment
    (32003, torch.bfloat16, 0),    # ends inside a piece of 8, with rows padded to 32,008 and unpadded
    (4099, torch.float32, 5),      # one segment ending inside a piece of 4
    (4099, torch.float16, 0),
    (32000, torch.bfloat16, 8),    # whole pieces: 16-byte loads at a row stride other than V
])
def test_vocabulary_ending_inside_a_piece_and_padded_rows(device, vocab, dtype, pad):
    log_case(f"markov rows: V={vocab} {dtype} row pad {pad}")
    g = torch.Generator().manual_seed(vocab + pad)
    batch = 8
    logits = (torch.randn(batch, 4, vocab, generator=g) * 3).to(dtype)
    logits[:, :, -2:] += 12.0   # the last elements, past the final whole piece, among the candidates
    table = (torch.randn(16, vocab, generator=g) * 2).to(dtype)
    st = sampling(device, [1.0, 0.7, 1.3, 1.0] * 2, [20, 5, 50, 1] * 2, [1.0, 0.8, 0.95, 1.0] * 2)
    anchors = torch.randint(0, vocab, (batch,), generator=g)
    drafts, q, want = run_both(device, logits, anchors, table, st, seed=3, pad=pad)
    assert torch.equal(drafts, want[0]), f"drafts differ at {(drafts != want[0]).nonzero()[:5].tolist()}"
    check_candidates(q, want, f"V={vocab} pad {pad}")
    ids = q.ids.cpu()
    assert bool(((ids == vocab - 1) | (ids == vocab - 2)).any()), "the last elements were never candidates"


@pytest.mark.parametrize("vocab, dtype, top_k", [
    (151936, torch.bfloat16, [100, 200, 64, 150]),   # 264 candidates, windows past 64: the workgroup finish
    (200000, torch.float32, [20, 5, 50, 1]),         # 11 segments: the merge's searches in two groups of lists
])
def test_wide_windows_and_many_segments_match_the_oracle(device, vocab, dtype, top_k):
    log_case(f"markov rows: V={vocab} {dtype} top_k={top_k}")
    g = torch.Generator().manual_seed(vocab + top_k[0])
    batch = 8
    logits = (torch.randn(batch, 3, vocab, generator=g) * 3).to(dtype)
    table = (torch.randn(16, vocab, generator=g) * 2).to(dtype)
    st = sampling(device, [1.0, 0.7, 1.3, 1.0] * 2, top_k * 2, [1.0, 0.8, 0.95, 1.0] * 2)
    anchors = torch.randint(0, vocab, (batch,), generator=g)
    drafts, q, want = run_both(device, logits, anchors, table, st, seed=3)
    assert torch.equal(drafts, want[0]), f"drafts differ at {(drafts != want[0]).nonzero()[:5].tolist()}"
    check_candidates(q, want, "wide windows / many segments")


@pytest.mark.parametrize("ties", [5000, 20000])
def test_ties_beyond_the_candidates(device, ties):
    # ten distinct top values, then `ties` copies of the 11th; top-k 11 keeps them all, the candidates keep the
    # first 65 of them in index order (20,000 ties exceed the kernel's pair list: its ordered tie pass)
    log_case(f"markov rows: {ties} ties at the cut")
    vocab = 151936
    g = torch.Generator().manual_seed(ties)
    logits = torch.randn(2, 2, vocab, generator=g).clamp(max=3.0)
    where = torch.randperm(vocab, generator=g)
    logits[:, :, where[:10]] = torch.arange(20.0, 10.0, -1.0)
    logits[:, :, where[10:10 + ties]] = 5.0
    st = sampling(device, [1.0, 0.9], [11, 11], [1.0, 1.0])
    drafts, q, want = run_both(device, logits, torch.tensor([0, 1]), torch.zeros(1, vocab), st, seed=2)
    assert torch.equal(drafts, want[0])
    check_candidates(q, want, f"{ties} ties")
    assert int((q.ids[0, 0] >= 0).sum()) == 75


def test_dense_rows_when_some_row_does_not_truncate(device):
    log_case("markov rows: dense batch")
    vocab = 3000
    g = torch.Generator().manual_seed(7)
    logits = torch.randn(4, 3, vocab, generator=g) * 2
    table = torch.randn(8, vocab, generator=g)
    st = sampling(device, [1.0, 0.8, 1.0, 1.2], [0, 10, 40, 5], [1.0, 0.9, 1.0, 1.0])
    drafts, q, want = run_both(device, logits, torch.tensor([1, 2, 3, 4]), table, st, seed=3)
    assert torch.equal(drafts, want[0])
    assert torch.allclose(q.cpu(), want[1], rtol=1e-5, atol=1e-7)


def test_markov_draw_rejects_bad_arguments(device):
    st = sampling(device, [1.0], [20], [1.0])
    lg = torch.zeros(1, 100, device=device)
    ids = torch.empty(1, 84, dtype=torch.int32, device=device)
    probs = torch.empty(1, 84, device=device)
    noise = torch.ones(1, 84, device=device)
    draws = torch.empty(1, dtype=torch.int64, device=device)
    with pytest.raises(Exception):
        nm.markov_draw(lg, st, 10, noise, ids, probs, draws)          # fewer candidates than max_top_k
    with pytest.raises(ValueError):
        nm.markov_draw(lg, st, 84, noise, ids.long(), probs, draws)
    with pytest.raises(ValueError):
        nm.markov_draw(lg, sampling(device, None, [20], [1.0]), 84, noise, ids, probs, draws)


@pytest.mark.parametrize("top_k, top_p, varlen, dtype", [
    (20, 1.0, False, torch.float32),      # the wave-0 finish
    (20, 0.8, True, torch.bfloat16),
    (100, 0.9, True, torch.float32),     # top-p with rank > 64: the workgroup finish, candidate hash in LDS
    (600, 1.0, False, torch.float32),    # 664 candidates: more than the hash holds, the row is scanned
])
def test_accept_on_candidate_rows_equals_the_dense_q(device, top_k, top_p, varlen, dtype):
    """A DSpark round: drafts and candidate rows from sample_markov, then the fused accept on the candidate rows
    and on the q they scatter to, with the same uniforms and noise: the same (n_accept, tail) bit for bit, and
    the oracle's accept on the dense q agrees."""
    log_case(f"accept on candidate rows: top_k={top_k} top_p={top_p} varlen={varlen} {dtype}")
    batch, k, vocab = 16, 7, 32000
    g = torch.Generator().manual_seed(top_k)
    target = torch.randn(batch, k + 1, vocab, generator=g) * 3
    draft_logits = target[:, :k] + torch.randn(batch, k, vocab, generator=g)
    table = torch.randn(16, vocab, generator=g) * 0.5
    st = sampling(device, [1.0, 0.8] * (batch // 2), [top_k] * batch, [top_p] * batch)
    gen = torch.Generator(device=device).manual_seed(9)
    tab = table.to(device)
    drafts, rows = nm.sample_markov(draft_logits.to(device), torch.arange(batch, device=device), st,
                                    lambda prev: tab[prev % 16], gen)
    assert isinstance(rows, nm.CandidateRows)
    lens = torch.randint(1, k + 2, (batch,), generator=g) if varlen else None
    logits = torch.cat([target[b, :int(lens[b])] for b in range(batch)]) if varlen else target.reshape(-1, vocab)
    lg = logits.to(dtype).to(device)
    uniforms = torch.rand(batch, k, generator=g).to(device)
    noise = ss.exponential_noise((batch, vocab), g).to(device)
    lens_d = None if lens is None else lens.to(device)
    dense = rows.to_dense(vocab)
    n_d, t_d = ns.spec_accept_with_draws(lg, dense, drafts, st, lens_d, uniforms, noise)
    n_s, t_s = ns.spec_accept_with_draws(lg, rows, drafts, st, lens_d, uniforms, noise)
    torch.cuda.synchronize()
    assert torch.equal(n_s, n_d) and torch.equal(t_s, t_d), "candidate rows and dense q disagree"
    cpu = st.temperatures.cpu()
    per_pos = cpu.repeat_interleave(lens if varlen else torch.full((batch,), k + 1))
    tk = st.top_k.cpu().repeat_interleave(lens if varlen else torch.full((batch,), k + 1))
    tp = st.top_p.cpu().repeat_interleave(lens if varlen else torch.full((batch,), k + 1))
    p = ss.probs_from_logits(lg.cpu(), per_pos, tk, tp, st.max_top_k, st.has_top_p)
    if varlen:
        want = ss.accept_random_varlen(p, dense.cpu(), drafts.cpu(), lens, uniforms.cpu(), noise.cpu())
    else:
        want = ss.accept_random(p.view(batch, k + 1, vocab), dense.cpu(), drafts.cpu(), uniforms.cpu(), noise.cpu())
    assert torch.equal(n_s.cpu(), want[0]) and torch.equal(t_s.cpu(), want[1]), "the oracle disagrees"
    print(f"mean accepted {float(n_s.float().mean()):.2f}")


def test_markov_rows_replay_in_a_graph(device):
    """The rows as the reference's sampling graphs run them: captured once, replayed with the noise refreshed
    outside the graph, eager work between the replays, every replay equal to the eager rows on the same noise."""
    log_case("markov rows: HIP graph replay")
    batch, k, vocab = 8, 7, 151936
    g = torch.Generator(device=device).manual_seed(31)
    logits = (torch.randn(batch, k, vocab, device=device, generator=g) * 3).to(torch.bfloat16)
    w1 = torch.randn(vocab, 16, device=device, generator=g, dtype=torch.bfloat16) * 0.1
    w2 = torch.randn(vocab, 16, device=device, generator=g, dtype=torch.bfloat16) * 0.1
    bias = lambda prev: torch.nn.functional.linear(torch.nn.functional.embedding(prev, w1), w2)
    st = sampling(device, [1.0, 0.7] * (batch // 2), [20, 5] * (batch // 2), [1.0, 0.9] * (batch // 2))
    C = nm.num_candidates(st.max_top_k, st.all_top_k, vocab)
    anchors = torch.arange(batch, device=device)
    noise = torch.empty(batch, k, C, device=device)
    drafts = torch.empty(batch, k, dtype=torch.int64, device=device)
    ns.exponential_noise_(noise, g)
    rows = nm.markov_rows(logits, anchors, st, bias, noise, drafts, C)   # warm-up, outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rows = nm.markov_rows(logits, anchors, st, bias, noise, drafts, C)
    for replay in range(3):
        ns.exponential_noise_(noise, g)
        graph.replay()
        torch.cuda.synchronize()
        got = (drafts.clone(), rows.ids.clone(), rows.probs.clone())
        want_drafts = torch.empty_like(drafts)
        want = nm.markov_rows(logits, anchors, st, bias, noise, want_drafts, C)
        torch.cuda.synchronize()
        assert torch.equal(got[0], want_drafts), f"replay {replay}: drafts differ from the eager rows"
        assert torch.equal(got[1], want.ids) and torch.equal(got[2], want.probs), f"replay {replay}: candidate rows"


def test_wide_window_rows_follow_the_oracle(device):
    """max_top_k above the draw kernel's 1024: each row's candidates come from torch's topk and are drawn with this
    library's probs_from_logits and race (speculative.py:178-181). The draws equal the oracle's and the candidate
    rows scatter to the oracle's dense q."""
    log_case("markov wide window (top-k 1500-3000)")
    gen = torch.Generator().manual_seed(7)
    batch, k, vocab = 4, 3, 151936
    logits = torch.randn(batch, k, vocab, generator=gen) * 3
    table = torch.randn(64, vocab, generator=gen)
    anchors = torch.randint(0, vocab, (batch,), generator=gen)
    st = sampling(device, [1.0, 0.8, 1.0, 1.2], [2000, 1500, 3000, 2000], [1.0, 0.9, 1.0, 0.95])
    drafts, q, want = run_both(device, logits, anchors, table, st)
    assert torch.equal(drafts, want[0])
    torch.testing.assert_close(q.to_dense(vocab).cpu(), want[1], rtol=1e-5, atol=1e-7)
