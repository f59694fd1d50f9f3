"""The decoder-layer elementwise kernels against the oracle, a whole verify forward of a small Qwen3-shaped target
against an eager CPU forward built from the oracle's ops, and the captured verify graph against the eager run of
the same kernels.

Tolerances.
  rms_norm, silu_and_mul: outputs are bf16 / fp16. The only differences from the oracle are the summation order
  of the squares (norm) and the last bits of exp (silu): at least 99% of the elements bit-identical; the new
  residual (a rounded sum) bit-exact. A one-ulp change of the fp32 scale can move dtype(x * scale) by one unit in
  the last place, which the weight product carries through a second rounding: norm outputs within 2^-6 of their
  magnitude (two roundings), silu outputs within 2^-7 (one).
  Forward: hipBLASLt and the CPU accumulate the GEMMs in different orders, so bf16 roundings drift apart layer by
  layer: relative L2 error of the final hidden states and of the cached keys / values at most 2e-2.
  Graph: the replay runs the same kernels on the same inputs as the eager forward: bit-identical.
"""
import pytest
import torch
import torch.nn.functional as F

from conftest import log_case
from nvs_amd import verify_round as vr
from nvs_amd.layers import activation as nact
from nvs_amd.layers import layernorm as nln
from oracle import attention as ref_attn
from oracle import layernorm as ref_ln
from oracle import qk_norm_rope as ref_qk

pytestmark = pytest.mark.gpu

SMALL = vr.Qwen3Shape(hidden_size=1024, num_layers=2, num_heads=8, num_kv_heads=2, head_dim=128,
                      intermediate_size=2048, vocab_size=2048, max_position=4096)


def close(got, want, what, min_same=0.99, rel=2.0 ** -7):
    g, w = got.float().cpu(), want.float().cpu()
    diff = (g - w).abs()
    bound = torch.maximum(g.abs(), w.abs()) * rel
    assert bool((diff <= bound).all()), f"{what}: max excess {float((diff - bound).max())}"
    same = float((g == w).float().mean())
    print(f"{what}: {100 * same:.3f}% bit-identical")
    assert same >= min_same, f"{what}: only {100 * same:.2f}% bit-identical"


@pytest.mark.parametrize("rows, hidden, dtype", [(1, 4096, torch.bfloat16), (288, 4096, torch.bfloat16),
                                                 (37, 1024, torch.float16), (5, 8192, torch.bfloat16),
                                                 (3, 136, torch.bfloat16)])
def test_rms_norm_matches_the_oracle(device, rows, hidden, dtype):
    log_case(f"rms_norm rows={rows} hidden={hidden} {dtype}")
    g = torch.Generator().manual_seed(rows + hidden)
    x = (torch.randn(rows, hidden, generator=g) * 3).to(dtype)
    r = torch.randn(rows, hidden, generator=g).to(dtype)
    w = (1 + 0.2 * torch.randn(hidden, generator=g)).to(dtype)
    out = nln.rms_norm(x.to(device), w.to(device), 1e-6)
    close(out, ref_ln.rms_forward(x, w, 1e-6), "rms_forward", rel=2.0 ** -6)
    res = r.to(device)
    xd = x.to(device)
    out, res2 = nln.rms_norm(xd, w.to(device), 1e-6, residual=res, out=xd)   # in place over x, as the layer calls it
    want, want_res = ref_ln.add_rms_forward(x, r, w, 1e-6)
    assert res2 is res and torch.equal(res.cpu(), want_res), "the new residual is the rounded sum, bit for bit"
    assert out.data_ptr() == xd.data_ptr()
    close(out, want, "add_rms_forward", rel=2.0 ** -6)


@pytest.mark.parametrize("rows, width, dtype", [(1, 12288, torch.bfloat16), (288, 12288, torch.bfloat16),
                                                (7, 2048, torch.float16), (3, 8, torch.bfloat16)])
def test_silu_and_mul_matches_the_oracle(device, rows, width, dtype):
    log_case(f"silu_and_mul rows={rows} width={width} {dtype}")
    g = torch.Generator().manual_seed(rows + width)
    x = (torch.randn(rows, 2 * width, generator=g) * 2).to(dtype)
    out = nact.silu_and_mul(x.to(device))
    close(out, ref_ln.silu_and_mul(x), "silu_and_mul")


def test_elementwise_ops_reject_bad_arguments(device):
    x = torch.zeros(4, 4100, dtype=torch.bfloat16, device=device)
    with pytest.raises(Exception):
        nln.rms_norm(x, torch.ones(4100, dtype=torch.bfloat16, device=device), 1e-6)    # not a multiple of 8
    with pytest.raises(ValueError):
        nln.rms_norm(x.float(), torch.ones(4100, device=device), 1e-6)
    with pytest.raises(ValueError):
        nact.silu_and_mul(torch.zeros(4, 7, dtype=torch.bfloat16, device=device))


def small_setup(device, seed=0):
    batch = vr.random_verify_batch(6, (1, 8), (20, 700), seed_lengths=seed + 3, seed_blocks=seed + 4)
    target = vr.Qwen3VerifyTarget(SMALL, batch.num_blocks, device=device, seed=seed, init_std=0.05)
    ids = torch.randint(0, SMALL.vocab_size, (batch.num_tokens,), generator=torch.Generator().manual_seed(seed))
    return batch, target, ids


def reference_forward(target, k_caches, v_caches, batch, ids):
    """Qwen3Model.forward on the CPU from the oracle's ops, the GEMMs as CPU bf16 linear layers. Writes the new
    keys and values into the given CPU caches."""
    s = target.shape
    cpu = lambda t: t.detach().cpu()
    md = vr.verify_varlen_metadata(batch, len(batch.q_lens), batch.num_tokens, 16, 8)
    positions = torch.tensor(md.positions)
    slots = torch.tensor(md.slot_mapping, dtype=torch.int32)
    rows = ref_attn.row_layout(md.cu_seqlens_q, md.cu_seqlens_k)
    tables = torch.tensor(md.block_tables, dtype=torch.int32)
    table = cpu(target.cos_sin_cache)
    T, eps = ids.shape[0], s.rms_norm_eps
    h = F.embedding(ids, cpu(target.embed))
    residual = None
    for i, lw in enumerate(target.layers):
        if residual is None:
            residual, h = h, ref_ln.rms_forward(h, cpu(lw.input_norm), eps)
        else:
            h, residual = ref_ln.add_rms_forward(h, residual, cpu(lw.input_norm), eps)
        qkv = F.linear(h, cpu(lw.qkv))
        q = qkv[:, :s.q_size].reshape(T, s.num_heads, s.head_dim)
        k = qkv[:, s.q_size:s.q_size + s.kv_size].reshape(T, s.num_kv_heads, s.head_dim)
        v = qkv[:, s.q_size + s.kv_size:].reshape(T, s.num_kv_heads, s.head_dim)
        q, _ = ref_qk.qk_norm_rope_store(positions, q, k, v, cpu(lw.q_norm), cpu(lw.k_norm), eps, table,
                                         k_caches[i], v_caches[i], slots)
        o = ref_attn.paged_attention_t32(q, k_caches[i], v_caches[i], tables, rows, target.scale, True)
        h = F.linear(o.to(h.dtype).reshape(T, s.q_size), cpu(lw.o))
        h, residual = ref_ln.add_rms_forward(h, residual, cpu(lw.post_norm), eps)
        h = F.linear(ref_ln.silu_and_mul(F.linear(h, cpu(lw.gate_up))), cpu(lw.down))
    h, _ = ref_ln.add_rms_forward(h, residual, cpu(target.norm), eps)
    return h, slots


def rel_l2(got, want):
    g, w = got.float().cpu(), want.float().cpu()
    return float((g - w).norm() / w.norm())


def test_forward_matches_the_cpu_oracle(device):
    log_case("verify forward, 2 small Qwen3 layers, 6 rows")
    batch, target, ids = small_setup(device)
    # the target's caches are head-major; the CPU copies are token-major, equal element for element
    assert target.k_caches.stride(-2) == SMALL.head_dim * 256 and not target.k_caches.is_contiguous()
    k0, v0 = target.k_caches.cpu().contiguous(), target.v_caches.cpu().contiguous()
    graphs = vr.VerifyGraphs(target, max_batch_size=8, query_len=8, max_model_len=1024)
    got = graphs.run_eager(batch, ids.to(device)).clone()
    torch.cuda.synchronize()
    want, slots = reference_forward(target, k0, v0, batch, ids)
    err = rel_l2(got, want)
    print(f"hidden: relative L2 error {err:.2e}")
    assert err <= 2e-2
    for name, mine, ref in (("keys", target.k_caches, k0), ("values", target.v_caches, v0)):
        flat_m = mine.cpu().contiguous().view(SMALL.num_layers, -1, SMALL.num_kv_heads, SMALL.head_dim)
        flat_r = ref.view_as(flat_m)
        live = slots[slots >= 0].long()
        err = rel_l2(flat_m[:, live], flat_r[:, live])
        print(f"cached {name}: relative L2 error {err:.2e}")
        assert err <= 2e-2
        untouched = torch.ones(flat_m.shape[1], dtype=torch.bool)
        untouched[live] = False
        assert torch.equal(flat_m[:, untouched], flat_r[:, untouched]), f"{name}: a slot outside the batch changed"
    logits = target.compute_logits(got)
    assert logits.shape == (batch.num_tokens, SMALL.vocab_size) and bool(torch.isfinite(logits).all())


def test_graph_replay_matches_eager(device):
    log_case("verify graph replay vs eager, 2 small Qwen3 layers")
    batch, target, ids = small_setup(device, seed=1)
    graphs = vr.VerifyGraphs(target, max_batch_size=8, query_len=8, max_model_len=1024)
    ids = ids.to(device)
    eager = graphs.run_eager(batch, ids).clone()
    rows, tokens = graphs.shape_for(batch.num_tokens)
    graphs.capture([tokens])
    for replay in range(3):   # eager work and synchronisation between the replays
        got = graphs.run(batch, ids).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {replay} differs from the eager forward"
        graphs.run_eager(batch, ids)
    # another batch of the same token count replays the same graph with its own metadata
    other = vr.VerifyBatch(batch.q_lens[::-1], batch.k_lens[::-1], batch.block_tables[::-1], batch.num_blocks)
    assert graphs.shape_for(other.num_tokens) == (rows, tokens)
    got = graphs.run(other, ids).clone()
    assert torch.equal(got, graphs.run_eager(other, ids))
    assert len(graphs.graphs) == 1


@pytest.mark.gpu
def test_run_drafts_places_the_drafts_like_the_host_layout(device):
    log_case("verify graph with drafts placed from the metadata, 2 small Qwen3 layers")
    batch, target, _ = small_setup(device, seed=2)
    k = 7
    gen = torch.Generator().manual_seed(5)
    batch.last_tokens = torch.randint(0, SMALL.vocab_size, (len(batch.q_lens),), generator=gen).tolist()
    drafts = torch.randint(0, SMALL.vocab_size, (len(batch.q_lens), k), generator=gen)
    md = vr.verify_varlen_metadata(batch, len(batch.q_lens), batch.num_tokens, 16, k + 1)
    ids = torch.tensor(md.input_ids)
    vr.place_drafts(ids, drafts, md)
    start = 0
    for r, q_len in enumerate(batch.q_lens):   # each row: its last token, then its first q_len - 1 drafts
        assert ids[start:start + q_len].tolist() == [batch.last_tokens[r]] + drafts[r, :q_len - 1].tolist()
        start += q_len
    graphs = vr.VerifyGraphs(target, max_batch_size=8, query_len=k + 1, max_model_len=1024)
    want = graphs.run(batch, ids.to(device)).clone()
    for _ in range(2):
        got = graphs.run_drafts(batch, drafts.to(device)).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_qwen3_8b_round_at_batch_64(device):
    """The fifth benchmark configuration as a test: 36 Qwen3-8B-shaped layers (random bf16 weights, paged
    head-major KV) over 64 rows of 1..8 verified tokens at 2,800-3,200-token contexts, captured as one HIP graph,
    then the LM head and the accept (speculative.py:411-448 for the round, :450-462 for the accept).
    The drafts partly follow the target (workloads.partly_accepted_drafts), so rows accept all their drafts (the
    bonus token), stop at a rejection (the residual), or reject at once. Checked: the graph replay equals the eager
    forward bit for bit; the fused accept (top-k 64, temperature 1) and the greedy accept on the round's bf16 logits
    equal the oracle's, bit for bit, given the same uniforms and noise; the generator is left where the
    reference's accept_random_varlen leaves it; acceptances, bonus tokens and residuals all occur."""
    import nvs_amd.workloads as wl
    from nvs_amd.layers import spec_sampler as ns
    from oracle import spec_sampler as ref_s

    log_case("verify round: 36 Qwen3-8B layers, B 64, q 1-8, ctx 2800-3200, fused and greedy accept")
    shape = vr.QWEN3_8B
    batch = vr.random_verify_batch(64)
    target = vr.Qwen3VerifyTarget(shape, batch.num_blocks, device=device)
    graphs = vr.VerifyGraphs(target, max_batch_size=512, query_len=8, max_model_len=4096)
    B, T, V = len(batch.q_lens), batch.num_tokens, shape.vocab_size
    st = ns.SamplingTensors(torch.ones(B, device=device), torch.full((B,), 64, dtype=torch.int64, device=device),
                            torch.ones(B, device=device), 64, False, True)
    rd = wl.partly_accepted_drafts(graphs, batch, st)
    hidden = graphs.run_drafts(batch, rd.drafts).clone()
    ids = graphs.input_ids[:T].clone()
    eager = graphs.run_eager(batch, ids).clone()
    torch.cuda.synchronize()
    assert torch.equal(hidden, eager), "graph replay differs from the eager forward"
    logits = target.compute_logits(hidden)
    lens = torch.tensor(batch.q_lens, dtype=torch.int64)
    ours = torch.Generator(device=device).manual_seed(12)
    n, tail = ns.accept(logits, rd.drafts, rd.q, st, batch.q_lens, ours)
    theirs = torch.Generator(device=device).manual_seed(12)
    uniforms = torch.rand(B, 7, device=device, generator=theirs)
    noise = torch.empty(B, V, device=device).exponential_(1.0, generator=theirs).clamp_min_(1e-10)
    assert torch.equal(ours.get_state(), theirs.get_state())
    logits_cpu = logits.float().cpu()
    n_want, tail_want = ref_s.accept_from_logits(logits_cpu, rd.q.cpu(), rd.drafts.cpu(), torch.ones(B),
                                                 torch.full((B,), 64, dtype=torch.int64), torch.ones(B), 64, False,
                                                 lens, uniforms.cpu(), noise.cpu())
    n, tail = n.cpu(), tail.cpu()
    assert torch.equal(n, n_want) and torch.equal(tail, tail_want)
    bonus = n == lens - 1
    print(f"fused accept: mean accepted {float(n.float().mean()):.2f}, bonus rows {int(bonus.sum())}, "
          f"rows with a residual {int((~bonus).sum())}, rows following the target {sum(f > 0 for f in rd.follow)}")
    assert float(n.float().mean()) > 0 and bool(bonus.any()) and bool((~bonus).any())
    follow = torch.tensor(rd.follow)
    assert bool((n >= follow).all()), "a draft that follows the target with q = p was rejected"
    greedy = ns.SamplingTensors(None, st.top_k, st.top_p, 64, False, True)
    n_g, tail_g = ns.accept(logits, rd.drafts, None, greedy, batch.q_lens, ours)
    n_gw, tail_gw = ref_s.accept_greedy_varlen(logits_cpu, rd.drafts.cpu(), lens)
    assert torch.equal(n_g.cpu(), n_gw) and torch.equal(tail_g.cpu(), tail_gw)
    assert bool((n_g.cpu() >= follow).all())
    assert torch.equal(ours.get_state(), theirs.get_state()), "the greedy accept drew random numbers"
