"""Parity of the HIP paged attention and KV store with the CPU oracle (fp64 brute force on the same bf16 inputs).

Tolerance: bf16 output, max |out - oracle| <= 2e-2 (the bar of the verify-attention contract). Each test also
reports the error of the oracle's own bf16-input fp32 path against fp64 (the rounding floor of an fp32 reference).
"""
import numpy as np
import pytest
import torch

import nvs_amd.workloads as wl
from conftest import log_case
from nvs_amd import _lib
from nvs_amd.layers import attention as nattn
from nvs_amd.utils.context import reset_context, set_context
from oracle import attention as ref

pytestmark = pytest.mark.gpu
TOL = 2e-2


def run_varlen(c, dev, max_seqlen_k=None):
    g = c.to(dev)
    out = nattn.paged_attention_varlen(g.q, g.k_cache, g.v_cache, max_seqlen_q=g.max_seqlen_q,
                                       cu_seqlens_q=g.cu_seqlens_q, max_seqlen_k=max_seqlen_k or g.max_seqlen_k,
                                       cu_seqlens_k=g.cu_seqlens_k, softmax_scale=g.scale, causal=True,
                                       block_table=g.block_tables)
    torch.cuda.synchronize()
    return out.float().cpu()


def check(out, c, causal=True, tol=TOL, rows=None):
    rows = c.rows if rows is None else rows
    want = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, rows, c.scale, causal)
    tokens = np.concatenate([np.arange(q0, q0 + lq) for q0, lq, _ in rows if lq > 0])
    err = np.abs(out.numpy()[tokens] - want[tokens]).max()
    t32 = ref.paged_attention_t32(c.q, c.k_cache, c.v_cache, c.block_tables, rows, c.scale, causal)
    own = np.abs(t32.numpy()[tokens] - want[tokens]).max()
    print(f"max|hip - fp64| = {err:.3e}   max|oracle fp32 - fp64| = {own:.3e}")
    assert np.isfinite(out.numpy()[tokens]).all()
    assert err <= tol, err
    return err


def test_c1_shape_bf16(device):
    log_case("attention c1 shape 16/8 heads ctx 1024")
    c = wl.verify_attention_case([8], [1024], 16, 8, 128)
    check(run_varlen(c, device), c)


def test_c2_shape(device):
    log_case("attention c2 shape b8 ctx 900-1200")
    c = wl.config_c2()
    check(run_varlen(c, device), c)


@pytest.mark.parametrize("block_size", [32, 64, 256])
def test_ragged_rows_and_padding(device, block_size):
    log_case(f"attention ragged bs={block_size}")
    q_lens = [1, 8, 3, 5, 2, 7, 4, 6, 8, 1]
    k_lens = [1, 8, 31, 32, 33, 255, 256, 257, 700, 1500]
    c = wl.verify_attention_case(q_lens, k_lens, 32, 8, 128, block_size=block_size)
    check(run_varlen(c, device), c)


def test_rows_with_no_queries_and_graph_sized_bounds(device):
    log_case("attention empty rows, max_seqlen_k 4096")
    c = wl.verify_attention_case([3, 0, 8, 0, 2], [40, 0, 900, 0, 300], 32, 8, 128, pad_tokens_to=1,
                                 table_width=16)
    out = run_varlen(c, device, max_seqlen_k=4096)
    check(out, c)


def test_long_context_splits(device):
    """Two rows split over many key ranges: each unit's last split to finish merges the partials in the launch,
    and leaves the unit counters at zero for the next call."""
    log_case("attention long context 4096 split-K")
    c = wl.verify_attention_case([8, 4], [4096, 3001], 32, 8, 128)
    check(run_varlen(c, device), c)
    c = wl.verify_attention_case([1], [4000], 32, 8, 128)
    check(run_varlen(c, device), c)
    counters = _lib.persistent_workspace("attention_unit_counters", 4, torch.device(device))
    torch.cuda.synchronize()
    assert int(counters.view(torch.int32).abs().sum()) == 0


def test_sixty_two_splits_of_one_long_row(device):
    """One 16,000-key row planned for 32k keys: 8 units, so the plan takes its 64-split maximum and the row is cut
    into 62 equal splits, all merged by the last one to finish."""
    log_case("attention one row, 16000 keys, max_seqlen_k 32768 (62 splits)")
    c = wl.verify_attention_case([3], [16000], 32, 8, 128, pad_tokens_to=1)
    check(run_varlen(c, device, max_seqlen_k=32768), c)


def test_units_longer_than_64_block_table_pages(device):
    """32-key blocks. 34 rows of 2,080-2,608 keys (272 units: unsplit) span 65-82 pages per unit: the kernel holds
    a unit's first 64 block ids in its lanes and reads the table for the pages past them. Two rows of 4,096 and
    3,000 keys are split, so each split starts at a later page of its row's table."""
    log_case("attention 32-key blocks: 34 unsplit rows of 65-82 pages; 2 split rows of 128 and 94 pages")
    k_lens = [2080 + 16 * r for r in range(34)]
    q_lens = [1 + (r % 4 == 0) for r in range(34)]
    c = wl.verify_attention_case(q_lens, k_lens, 32, 8, 128, block_size=32)
    check(run_varlen(c, device), c)
    c = wl.verify_attention_case([8, 5], [4096, 3000], 32, 8, 128, block_size=32)
    check(run_varlen(c, device), c)


@pytest.mark.parametrize("seed", range(8))
def test_random_shapes_across_split_plans(device, seed):
    """Seeded random batches (1-16 rows, 0-8 verify tokens, up to 4,000 keys, GQA groups 1/4/8) under graph-sized
    max_seqlen_k values that give unsplit, split and maximally split plans: every output against the fp64
    oracle, and the split merge's counters back at zero afterwards."""
    import random
    rng = random.Random(1000 + seed)
    rows = rng.randint(1, 16)
    hkv = 8
    hq = hkv * rng.choice([1, 4, 8])
    k_lens = [rng.randint(1, 4000) for _ in range(rows)]
    q_lens = [min(rng.randint(0, 8), lk) for lk in k_lens]
    q_lens[0] = max(q_lens[0], 1)
    max_k = rng.choice([max(k_lens), 4096, 16384])
    log_case(f"attention random shapes seed={seed} rows={rows} heads={hq}/{hkv} max_k={max_k} "
             f"q={q_lens} k={k_lens}")
    c = wl.verify_attention_case(q_lens, k_lens, hq, hkv, 128, pad_tokens_to=1, seed_qkv=seed)
    check(run_varlen(c, device, max_seqlen_k=max_k), c)
    counters = _lib.persistent_workspace("attention_unit_counters", 4, torch.device(device))
    torch.cuda.synchronize()
    assert int(counters.view(torch.int32).abs().sum()) == 0


def test_c3_full_size(device):
    log_case("attention c3 b64 varlen ctx 2800-3200")
    c = wl.config_c3()
    check(run_varlen(c, device, max_seqlen_k=4096), c)


@pytest.mark.parametrize("shape", ["c2", "c3", "split"])
def test_fp16_caches(device, shape):
    """A model built in fp16 (model_runner.py:55-57 takes hf_config.dtype) runs the same kernel on fp16 q / K / V
    with the fp16 32x32x16 MFMA and fp16 output: the batch-8 and batch-64 verify layers, and two long rows whose
    keys are split and merged in the launch, against the fp64 oracle of the same fp16 inputs."""
    log_case(f"attention fp16 {shape}")
    if shape == "c2":
        c = wl.config_c2(torch.float16)
        out = run_varlen(c, device)
    elif shape == "c3":
        c = wl.config_c3(torch.float16)
        out = run_varlen(c, device, max_seqlen_k=4096)
    else:
        c = wl.verify_attention_case([8, 4], [4096, 3001], 32, 8, 128, dtype=torch.float16)
        out = run_varlen(c, device)
    check(out, c)


def test_fp16_decode_branch(device):
    log_case("attention fp16 decode branch lq=7 non-causal")
    ctx = [12, 300, 1025, 64]
    c = wl.verify_attention_case([7] * 4, ctx, 32, 8, 128, pad_tokens_to=1, dtype=torch.float16)
    g = c.to(device)
    out = nattn.paged_attention_with_kvcache(g.q.view(4, 7, 32, 128), g.k_cache, g.v_cache,
                                             cache_seqlens=torch.tensor(ctx, dtype=torch.int32, device=device),
                                             block_table=g.block_tables, softmax_scale=g.scale, causal=False)
    assert out.dtype == torch.float16
    check(out.view(-1, 32, 128).float().cpu(), c, causal=False,
          rows=ref.row_layout(context_lens=ctx, query_len_per_seq=7))


def test_gqa_group_8_uses_two_query_tiles(device):
    log_case("attention group 8 (64 q heads / 8 kv) lq 8")
    c = wl.verify_attention_case([8, 5], [600, 129], 64, 8, 128)
    check(run_varlen(c, device), c)


def test_mha_group_1(device):
    log_case("attention group 1 (8/8 heads)")
    c = wl.verify_attention_case([8, 3], [333, 64], 8, 8, 128)
    check(run_varlen(c, device), c)


def test_strided_q_view_of_fused_qkv(device):
    log_case("attention q as a view of qkv")
    c = wl.verify_attention_case([4, 6], [100, 513], 32, 8, 128)
    g = c.to(device)
    T = g.q.shape[0]
    qkv = torch.randn(T, (32 + 16) * 128, dtype=torch.bfloat16, device=device)
    qkv[:, :32 * 128] = g.q.reshape(T, -1)
    q_view = qkv[:, :32 * 128].view(T, 32, 128)
    assert q_view.stride(0) == 48 * 128
    out = nattn.paged_attention_varlen(q_view, g.k_cache, g.v_cache, g.max_seqlen_q, g.cu_seqlens_q, g.max_seqlen_k,
                                       g.cu_seqlens_k, g.scale, True, g.block_tables)
    check(out.float().cpu(), c)


@pytest.mark.parametrize("causal, lq", [(True, 1), (True, 7), (False, 7)])
def test_decode_branch_fixed_query_length(device, causal, lq):
    log_case(f"attention decode branch causal={causal} lq={lq}")
    ctx = [lq + 5, 300, 1025, 64]
    c = wl.verify_attention_case([lq] * 4, ctx, 32, 8, 128, pad_tokens_to=1)
    g = c.to(device)
    B = len(ctx)
    q4 = g.q.view(B, lq, 32, 128)
    out = nattn.paged_attention_with_kvcache(q4, g.k_cache, g.v_cache, cache_seqlens=torch.tensor(
        ctx, dtype=torch.int32, device=device), block_table=g.block_tables, softmax_scale=g.scale, causal=causal)
    rows = ref.row_layout(context_lens=ctx, query_len_per_seq=lq)
    check(out.view(-1, 32, 128).float().cpu(), c, causal=causal, rows=rows)


def test_deterministic(device):
    log_case("attention determinism")
    c = wl.verify_attention_case([8, 3, 6], [2000, 700, 1800], 32, 8, 128)
    a = run_varlen(c, device)
    b = run_varlen(c, device)
    assert torch.equal(a, b)


def test_attention_forward_stores_then_attends(device):
    """Attention.forward on a Context, as Qwen3Attention calls it: the verified tokens' own K/V are stored through
    slot_mapping first and then attended to (attention.py:59-70)."""
    log_case("Attention.forward varlen with store")
    c = wl.verify_attention_case([3, 5], [77, 300], 32, 8, 128)
    bs = c.k_cache.shape[1]
    T = c.q.shape[0]
    gen = torch.Generator().manual_seed(5)
    k_new = torch.randn(T, 8, 128, generator=gen).to(torch.bfloat16)
    v_new = torch.randn(T, 8, 128, generator=gen).to(torch.bfloat16)
    slots = []
    for r, (q0, lq, lk) in enumerate(c.rows):
        for i in range(lq):
            pos = lk - lq + i
            slots.append(int(c.block_tables[r, pos // bs]) * bs + pos % bs if r < c.real_rows else -1)
    slot_mapping = torch.tensor(slots, dtype=torch.int32)
    want_k, want_v = c.k_cache.clone(), c.v_cache.clone()
    ref.store_kvcache(k_new, v_new, want_k, want_v, slot_mapping)
    g = c.to(device)
    layer = nattn.Attention(32, 128, c.scale, 8)
    layer.k_cache, layer.v_cache = g.k_cache, g.v_cache
    set_context(True, g.cu_seqlens_q, g.cu_seqlens_k, g.max_seqlen_q, 4096, slot_mapping.to(device), None,
                g.block_tables)
    try:
        out = layer(g.q, k_new.to(device), v_new.to(device))
    finally:
        reset_context()
    torch.cuda.synchronize()
    assert torch.equal(g.k_cache.cpu(), want_k) and torch.equal(g.v_cache.cpu(), want_v)
    c.k_cache, c.v_cache = want_k, want_v
    check(out.float().cpu(), c)


def test_graph_capture_replays_match_eager(device):
    log_case("attention hip graph capture and replays")
    c = wl.verify_attention_case([8, 2, 5], [900, 1700, 64], 32, 8, 128)
    g = c.to(device)
    eager = run_varlen(c, device, max_seqlen_k=4096)

    def fwd():
        return nattn.paged_attention_varlen(g.q, g.k_cache, g.v_cache, g.max_seqlen_q, g.cu_seqlens_q, 4096,
                                            g.cu_seqlens_k, g.scale, True, g.block_tables)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fwd()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = fwd()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out.float().cpu(), eager)
        _ = run_varlen(c, device)   # eager work between replays


def test_store_kvcache_bit_exact_strided_value_and_padding(device):
    log_case("store_kvcache strided value, padding slots")
    N, hkv, d, bs, blocks = 37, 8, 128, 256, 5
    gen = torch.Generator().manual_seed(3)
    qkv = torch.randn(N, (32 + 2 * hkv) * d, generator=gen).to(torch.bfloat16)
    key = qkv[:, 32 * d:(32 + hkv) * d].reshape(N, hkv, d)
    value = qkv[:, (32 + hkv) * d:].reshape(N, hkv, d)
    assert value.stride(0) == 48 * d
    slots = torch.randperm(blocks * bs, generator=gen)[:N].to(torch.int32)
    slots[[3, 10, 36]] = -1
    k_cache = torch.zeros(blocks, bs, hkv, d, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    want_k, want_v = k_cache.clone(), v_cache.clone()
    ref.store_kvcache(key, value, want_k, want_v, slots)
    gk, gv = k_cache.to(device), v_cache.to(device)
    qkv_d = qkv.to(device)
    nattn.store_kvcache(qkv_d[:, 32 * d:(32 + hkv) * d].view(N, hkv, d), qkv_d[:, (32 + hkv) * d:].view(N, hkv, d),
                        gk, gv, slots.to(device))
    torch.cuda.synchronize()
    assert torch.equal(gk.cpu(), want_k) and torch.equal(gv.cpu(), want_v)


@pytest.mark.parametrize("layout", ["token_major", "head_major", "kv_interleaved"])
@pytest.mark.parametrize("dtype, head_dim", [(torch.float32, 64), (torch.float16, 128), (torch.bfloat16, 4)])
def test_store_kvcache_other_dtypes_and_unaligned_rows(device, dtype, head_dim, layout):
    log_case(f"store_kvcache {dtype} head_dim {head_dim} {layout}")
    N, hkv, bs, blocks = 11, 2, 32, 3
    key = torch.randn(N, hkv, head_dim).to(dtype)
    value = torch.randn(N, hkv, head_dim).to(dtype)
    slots = torch.tensor([0, 5, -1, 95, 40, 41, 7, -1, 64, 3, 90], dtype=torch.int64)
    want_k = torch.zeros(blocks, bs, hkv, head_dim, dtype=dtype)
    want_v = torch.zeros_like(want_k)
    ref.store_kvcache(key, value, want_k, want_v, slots)
    if layout == "head_major":
        gk = wl.head_major_empty(*want_k.shape, dtype=dtype, device=device).zero_()
        gv = wl.head_major_empty(*want_v.shape, dtype=dtype, device=device).zero_()
    elif layout == "kv_interleaved":
        gk, gv = wl.kv_cache_empty(*want_k.shape, dtype=dtype, device=device)
        gk.zero_()
        gv.zero_()
    else:
        gk, gv = torch.zeros_like(want_k, device=device), torch.zeros_like(want_v, device=device)
    nattn.store_kvcache(key.to(device), value.to(device), gk, gv, slots.to(device))
    torch.cuda.synchronize()
    assert torch.equal(gk.cpu(), want_k) and torch.equal(gv.cpu(), want_v)


def test_store_kvcache_head_major_strided_value(device):
    log_case("store_kvcache into head-major caches, strided value, padding slots")
    N, hkv, d, bs, blocks = 37, 8, 128, 256, 5
    gen = torch.Generator().manual_seed(4)
    qkv = torch.randn(N, (32 + 2 * hkv) * d, generator=gen).to(torch.bfloat16)
    slots = torch.randperm(blocks * bs, generator=gen)[:N].to(torch.int32)
    slots[[0, 17]] = -1
    want_k = torch.zeros(blocks, bs, hkv, d, dtype=torch.bfloat16)
    want_v = torch.zeros_like(want_k)
    ref.store_kvcache(qkv[:, 32 * d:(32 + hkv) * d].reshape(N, hkv, d), qkv[:, (32 + hkv) * d:].reshape(N, hkv, d),
                      want_k, want_v, slots)
    gk = wl.head_major_empty(blocks, bs, hkv, d, dtype=torch.bfloat16, device=device).zero_()
    gv = wl.head_major_empty(blocks, bs, hkv, d, dtype=torch.bfloat16, device=device).zero_()
    assert gk.stride() == (hkv * bs * d, d, bs * d, 1)
    qkv_d = qkv.to(device)
    nattn.store_kvcache(qkv_d[:, 32 * d:(32 + hkv) * d].view(N, hkv, d), qkv_d[:, (32 + hkv) * d:].view(N, hkv, d),
                        gk, gv, slots.to(device))
    torch.cuda.synchronize()
    assert torch.equal(gk.cpu(), want_k) and torch.equal(gv.cpu(), want_v)


@pytest.mark.parametrize("layout", ["head_major", "kv_interleaved"])
@pytest.mark.parametrize("shape", ["c2_split", "c3", "draft_block"])
def test_head_major_cache_gives_the_token_major_result(device, shape, layout):
    """The kernel reads a cache through its strides: head-major memory, and K and V interleaved in one buffer (each
    block and kv head's keys and then values one run), give bit for bit the token-major result."""
    log_case(f"attention {layout} vs token-major {shape}")
    if shape == "draft_block":
        c = wl.verify_attention_case([7] * 16, [900 + 37 * i for i in range(16)], 32, 8, 128, pad_tokens_to=1)
    else:
        c = wl.config_c2() if shape == "c2_split" else wl.config_c3()
    g = c.to(device)
    h = c.head_major().to(device) if layout == "head_major" else c.kv_interleaved(device)
    assert h.k_cache.stride(1) == 128 and torch.equal(h.k_cache, g.k_cache) and torch.equal(h.v_cache, g.v_cache)
    if layout == "kv_interleaved":
        assert h.v_cache.data_ptr() - h.k_cache.data_ptr() == 256 * 128 * h.k_cache.element_size()
    if shape == "draft_block":
        ctx = torch.tensor(c.k_lens, dtype=torch.int32, device=device)
        outs = [nattn._paged_attention(x.q, x.k_cache, x.v_cache, x.block_tables, None, None, ctx, 7, 16, 7, 4096,
                                       x.scale, False) for x in (g, h)]
    else:
        outs = [nattn._paged_attention(x.q, x.k_cache, x.v_cache, x.block_tables, x.cu_seqlens_q, x.cu_seqlens_k,
                                       None, 0, len(c.q_lens), x.max_seqlen_q, 4096, x.scale, True) for x in (g, h)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    if shape == "c2_split":
        check(outs[1].float().cpu(), c)
