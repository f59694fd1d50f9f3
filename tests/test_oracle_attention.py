"""Pins the CPU attention oracle (oracle/attention.py): closed forms, an independent dense brute force with an
explicit mask, GQA mapping, block-table invariances, and the fp32 torch restatement against fp64. CPU only."""
import numpy as np
import pytest
import torch

import nvs_amd.workloads as wl
from oracle import attention as ref


def case(q_lens, k_lens, h=4, hkv=2, d=16, bs=8, seed=0, dtype=torch.float32, pad_to=1):
    return wl.verify_attention_case(q_lens, k_lens, h, hkv, d, block_size=bs, dtype=dtype, pad_tokens_to=pad_to,
                                    seed_qkv=seed)


def dense_bruteforce(c, causal=True):
    """Independent formulation: materialise every row's K/V by walking slots one key at a time, build the full
    [Lq, Lk] mask from absolute positions (query i sits at position Lk - Lq + i), loop over heads."""
    q = c.q.double().numpy()
    kc = c.k_cache.double().numpy()
    vc = c.v_cache.double().numpy()
    bs = kc.shape[1]
    T, H, D = q.shape
    group = H // kc.shape[2]
    out = np.zeros((T, H, D))
    for r, (q0, lq, lk) in enumerate(c.rows):
        table = c.block_tables[r].tolist()
        K = np.stack([kc[table[j // bs], j % bs] for j in range(lk)])
        V = np.stack([vc[table[j // bs], j % bs] for j in range(lk)])
        for i in range(lq):
            pos = lk - lq + i
            for h in range(H):
                s = np.array([q[q0 + i, h] @ K[j, h // group] for j in range(lk)]) * c.scale
                if causal:
                    s[np.arange(lk) > pos] = -np.inf
                w = np.exp(s - s.max())
                out[q0 + i, h] = (w / w.sum()) @ V[:, h // group]
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_f64_matches_dense_bruteforce(causal):
    c = case([3, 1, 5, 2], [20, 9, 31, 2])
    got = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, causal)
    np.testing.assert_allclose(got, dense_bruteforce(c, causal), rtol=1e-12, atol=1e-12)


def test_single_visible_key_returns_its_value_row():
    # causal, Lq = Lk: query 0 sees only key 0
    c = case([4], [4])
    got = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    v0 = c.v_cache[c.block_tables[0, 0], 0].double().numpy()    # [Hkv, D]
    group = c.q.shape[1] // c.k_cache.shape[2]
    np.testing.assert_allclose(got[0], np.repeat(v0, group, axis=0), rtol=1e-12)


def test_equal_keys_average_the_visible_values():
    c = case([3], [10])
    c.k_cache[:] = 1.0
    got = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    keys = ref.gather_keys(c.v_cache.double().numpy(), c.block_tables[0].tolist(), 10)   # [10, Hkv, D]
    group = c.q.shape[1] // c.k_cache.shape[2]
    for i in range(3):
        visible = 10 - 3 + i + 1
        np.testing.assert_allclose(got[i], np.repeat(keys[:visible].mean(0), group, axis=0), rtol=1e-10)


def test_gqa_head_mapping_uses_integer_division():
    # change kv head 1 only: query heads 2, 3 (group 2) move, heads 0, 1 do not
    c = case([2], [12])
    base = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    c.v_cache[:, :, 1] += 1.0
    moved = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    np.testing.assert_allclose(moved[:, :2], base[:, :2], rtol=1e-12)
    np.testing.assert_allclose(moved[:, 2:], base[:, 2:] + 1.0, atol=1e-6)  # fp32 cache + 1 rounds


def test_block_permutation_invariance():
    c = case([3, 4], [17, 30], bs=4)
    base = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    n = c.k_cache.shape[0]
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(n)
    tables = inv[c.block_tables.long()].to(torch.int32)
    got = ref.paged_attention_f64(c.q, c.k_cache[perm], c.v_cache[perm], tables, c.rows, c.scale, True)
    np.testing.assert_allclose(got, base, rtol=1e-12)


def test_decode_lq1_equals_full_attention_and_rows_with_no_queries_are_untouched():
    c = case([1, 0, 2], [9, 0, 6])
    causal = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    full = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, False)
    np.testing.assert_allclose(causal[0], full[0], rtol=1e-12)     # Lq = 1 sees every key either way
    assert not np.allclose(causal[1:], full[1:])                    # Lq = 2 differs under the mask


def test_fixed_mode_layout_equals_varlen():
    c = case([3, 3], [7, 12])
    varlen = ref.row_layout(c.cu_seqlens_q, c.cu_seqlens_k)
    fixed = ref.row_layout(context_lens=torch.tensor(c.k_lens), query_len_per_seq=3)
    assert varlen == fixed


def test_torch_fp32_restatement_matches_f64():
    c = case([8, 3, 5], [40, 17, 64], h=8, hkv=2, d=32, bs=16)
    got = ref.paged_attention_t32(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    want = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-5)


def test_config_c1_fp32_through_the_oracle():
    """C1 as specified: fp32 q/K/V, 16 q / 8 kv heads, one row of 8 verify positions over 1,024 keys in four
    permuted 256-key blocks plus the zero pad block. The fp32 restatement (the CPU baseline's path) against the fp64
    brute force, and the row's first position (which sees keys 0..1016) against the dense brute force."""
    c = wl.config_c1()
    assert c.q.dtype == torch.float32 and c.k_cache.shape == (5, 256, 8, 128)
    assert sorted(c.block_tables[0, :4].tolist()) == [0, 1, 2, 3] and c.block_tables[0, :4].tolist() != [0, 1, 2, 3]
    want = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    got = ref.paged_attention_t32(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    np.testing.assert_allclose(got.numpy()[:8], want[:8], rtol=1e-5, atol=1e-5)
    one = case([1], [1017], h=16, hkv=8, d=128, bs=256)
    one.q, one.k_cache, one.v_cache, one.block_tables = c.q[:1], c.k_cache, c.v_cache, c.block_tables
    np.testing.assert_allclose(want[:1], dense_bruteforce(one), rtol=1e-10, atol=1e-12)


def test_padding_rows_read_the_zero_pad_block():
    c = wl.verify_attention_case([3, 2], [10, 20], 4, 2, 16, block_size=8, pad_tokens_to=8, max_query_len=8)
    assert c.real_rows == 2 and len(c.q_lens) == 3 and sum(c.q_lens) == 8
    out = ref.paged_attention_f64(c.q, c.k_cache, c.v_cache, c.block_tables, c.rows, c.scale, True)
    pad_q0 = c.cu_seqlens_q[2].item()
    assert (c.block_tables[2] == c.pad_block).all()
    np.testing.assert_array_equal(out[pad_q0:], 0.0)   # zero V rows -> zero output, finite


def test_store_kvcache_copies_rows_to_slots_and_skips_padding():
    k_cache = torch.zeros(3, 4, 2, 8)
    v_cache = torch.zeros(3, 4, 2, 8)
    key = torch.randn(5, 2, 8)
    value = torch.randn(5, 2, 8)
    slots = torch.tensor([5, -1, 0, 11, -1], dtype=torch.int32)
    ref.store_kvcache(key, value, k_cache, v_cache, slots)
    flat_k = k_cache.view(-1, 2, 8)
    assert torch.equal(flat_k[5], key[0]) and torch.equal(flat_k[0], key[2]) and torch.equal(flat_k[11], key[3])
    assert torch.equal(v_cache.view(-1, 2, 8)[11], value[3])
    assert int((flat_k.abs().sum((1, 2)) > 0).sum()) == 3


def test_workload_layout_matches_verify_metadata():
    # the design example of test_batch_metadata.py:124-134 in this generator's terms: rows of 5 and 3 verified
    # tokens, padded to 8 tokens -> no padding row; cu_seqlens_k are the contexts
    c = wl.verify_attention_case([5, 3], [104, 39], 4, 2, 16, block_size=256, pad_tokens_to=8)
    assert c.cu_seqlens_q.tolist() == [0, 5, 8] and c.cu_seqlens_k.tolist() == [0, 104, 143]
    # one row of 3 in 9 tokens: padding rows of at most 4 tokens (k = 3) fill the rest (test_batch_metadata.py:137-146)
    c = wl.verify_attention_case([3], [7], 4, 2, 16, block_size=8, pad_tokens_to=9, max_query_len=4)
    assert c.cu_seqlens_q.tolist() == [0, 3, 7, 9] and c.cu_seqlens_k.tolist() == [0, 7, 11, 13]


def test_workload_byte_counts():
    c = wl.verify_attention_case([2, 1], [100, 50], 4, 2, 16, block_size=8, dtype=torch.bfloat16, pad_tokens_to=1)
    assert c.kv_bytes() == (100 + 50) * 2 * 16 * 2 * 2
    assert c.qo_bytes() == 2 * 3 * 4 * 16 * 2
    assert c.flops() == 4 * 4 * 16 * ((99 + 100) + 50)
