"""Host logic of the verify round, no GPU: the graphs' token counts (verify_schedule.py:18-23, with the known
answers of the reference's tests/test_verify_schedule.py:54-55), the row-slot metadata (batch_metadata.py:149-181)
on a hand-worked example, and the weight bytes of the Qwen3-8B shape."""
import pytest
import torch

from nvs_amd import verify_round as vr


def test_token_counts_known_answers():
    assert vr.verify_token_counts(4, 8) == [1, 2, 4, 8, 16, 24, 32]
    assert all(b * 8 in vr.verify_token_counts(64, 8) for b in range(1, 65))
    assert vr.verify_token_counts(3, 4) == [1, 2, 4, 8, 12]      # 4 is not below query_len 4: listed once
    assert vr.verify_token_counts(2, 1) == [1, 2]


def test_graph_shapes_cap_the_rows():
    counts = vr.verify_token_counts(512, 8)
    shapes = [(min(n, 512), n) for n in counts]
    assert shapes[-1] == (512, 4096) and (288, 288) in shapes and (512, 520) in shapes


def test_metadata_hand_worked():
    # row 0 verifies 3 tokens at the end of 300 (positions 297..299 in its second block, physical block 2);
    # row 1 verifies 1 token of 5 (position 4 in block 7). 8 token slots: one padding row of 4 tokens on the pad
    # block (8), then an empty row.
    batch = vr.VerifyBatch(q_lens=[3, 1], k_lens=[300, 5], block_tables=[[5, 2], [7]], num_blocks=8)
    md = vr.verify_varlen_metadata(batch, num_rows=4, num_tokens=8, width=3, query_len=8)
    assert md.positions == [297, 298, 299, 4, 0, 1, 2, 3]
    assert md.slot_mapping == [2 * 256 + 41, 2 * 256 + 42, 2 * 256 + 43, 7 * 256 + 4, -1, -1, -1, -1]
    assert md.cu_seqlens_q == [0, 3, 4, 8, 8]
    assert md.cu_seqlens_k == [0, 300, 305, 309, 309]
    assert md.block_tables == [[5, 2, 8], [7, 8, 8], [8, 8, 8], [8, 8, 8]]


def test_metadata_padding_rows_hold_at_most_query_len():
    batch = vr.VerifyBatch(q_lens=[1], k_lens=[10], block_tables=[[0]], num_blocks=1)
    md = vr.verify_varlen_metadata(batch, num_rows=4, num_tokens=12, width=1, query_len=4)
    assert md.cu_seqlens_q == [0, 1, 5, 9, 12]
    assert md.slot_mapping[1:] == [-1] * 11
    capture = vr.verify_varlen_metadata(None, num_rows=3, num_tokens=20, width=2, query_len=8, pad_block=5)
    assert capture.cu_seqlens_q == [0, 8, 16, 20] and capture.block_tables == [[5, 5]] * 3


def test_metadata_rejects_what_does_not_fit():
    batch = vr.VerifyBatch(q_lens=[8, 8], k_lens=[100, 100], block_tables=[[0], [1]], num_blocks=2)
    with pytest.raises(ValueError):
        vr.verify_varlen_metadata(batch, num_rows=2, num_tokens=8, width=1, query_len=8)    # 16 tokens in 8
    with pytest.raises(ValueError):
        vr.verify_varlen_metadata(batch, num_rows=2, num_tokens=24, width=1, query_len=8)   # no padding row left
    with pytest.raises(ValueError):
        vr.verify_varlen_metadata(batch, num_rows=1, num_tokens=16, width=1, query_len=8)   # two rows, one slot
    with pytest.raises(ValueError):
        vr.verify_varlen_metadata(vr.VerifyBatch([9], [100], [[0]], 1), num_rows=2, num_tokens=16, width=1,
                                  query_len=8)                                               # 9 > query_len


def test_random_batch_and_weight_bytes():
    batch = vr.random_verify_batch(64)
    assert len(batch.q_lens) == 64 and all(1 <= q <= 8 for q in batch.q_lens)
    assert all(2800 <= k <= 3200 for k in batch.k_lens)
    blocks = sorted(b for t in batch.block_tables for b in t)
    assert blocks == list(range(batch.num_blocks))                  # a permutation: every block used once
    assert all(len(t) * 256 >= k for t, k in zip(batch.block_tables, batch.k_lens))
    assert vr.QWEN3_8B.streamed_weight_bytes() == 15_136_194_560   # 36 layers + LM head in bf16


def reference_row(length: int, table: list[int], verified: int):
    """A sequence of `length` tokens verifying `verified` of them from position length - 1, as the reference's
    tests build it (make_sequence): in this layout q_len = verified and k_len = length - 1 + verified."""
    return verified, length - 1 + verified, table


def test_reference_verify_metadata_known_answers():
    # tests/test_batch_metadata.py:68-77: len 5 on blocks [7, 8, 9], k = 2, two slots of 3 tokens, block size 4
    q, k, t = reference_row(5, [7, 8, 9], 3)
    md = vr.verify_varlen_metadata(vr.VerifyBatch([q], [k], [t], num_blocks=99, block_size=4, last_tokens=[4]),
                                   num_rows=2, num_tokens=6, width=3, query_len=3)
    assert md.input_ids == [4, 0, 0, 0, 0, 0]
    assert md.positions == [4, 5, 6, 0, 1, 2]
    assert md.slot_mapping == [32, 33, 34, -1, -1, -1]
    assert md.cu_seqlens_q == [0, 3, 6] and md.cu_seqlens_k == [0, 7, 10]
    assert md.block_tables == [[7, 8, 9], [99, 99, 99]]
    # :80-84: a short block table is padded with the pad block
    q, k, t = reference_row(2, [4], 2)
    md = vr.verify_varlen_metadata(vr.VerifyBatch([q], [k], [t], num_blocks=99, block_size=4),
                                   num_rows=1, num_tokens=2, width=2, query_len=2)
    assert md.block_tables == [[4, 99]]


def test_reference_varlen_metadata_known_answers():
    # tests/test_batch_metadata.py:124-134: rows of len 100 (block 7) and 37 (block 3) verify 5 and 3 tokens, k = 7
    rows = [reference_row(100, [7], 5), reference_row(37, [3], 3)]
    batch = vr.VerifyBatch([r[0] for r in rows], [r[1] for r in rows], [r[2] for r in rows], num_blocks=99,
                           block_size=256, last_tokens=[99, 36])
    md = vr.verify_varlen_metadata(batch, num_rows=2, num_tokens=8, width=1, query_len=8)
    assert md.input_ids == [99, 0, 0, 0, 0, 36, 0, 0]
    assert md.positions == [99, 100, 101, 102, 103, 36, 37, 38]
    assert md.slot_mapping == [1891, 1892, 1893, 1894, 1895, 804, 805, 806]
    assert md.cu_seqlens_q == [0, 5, 8] and md.cu_seqlens_k == [0, 104, 143]
    assert md.draft_index == [1, 2, 3, 4, 6, 7] and md.draft_source == [0, 1, 2, 3, 7, 8]
    # :137-146: one row of 3 in 9 tokens and 4 slots, k = 3: padding rows of 4 and 2, then an empty slot
    q, k, t = reference_row(5, [7, 8], 3)
    md = vr.verify_varlen_metadata(vr.VerifyBatch([q], [k], [t], num_blocks=99, block_size=4),
                                   num_rows=4, num_tokens=9, width=2, query_len=4)
    assert md.positions == [4, 5, 6, 0, 1, 2, 3, 0, 1]
    assert md.slot_mapping == [32, 33, 34] + [vr.PAD_SLOT] * 6
    assert md.cu_seqlens_q == [0, 3, 7, 9, 9] and md.cu_seqlens_k == [0, 7, 11, 13, 13]
    assert md.block_tables == [[7, 8], [99, 99], [99, 99], [99, 99]]


def test_reference_verify_round_layout_known_answers():
    # tests/test_speculative_decoder.py:16-17,124-133: block size 4, k = 3; prompt [8, 9, 10] + 11 on blocks [3, 4]
    # verifies 11 and the drafts 12, 13, 14
    q, k, t = reference_row(4, [3, 4], 4)
    batch = vr.VerifyBatch([q], [k], [t], num_blocks=99, block_size=4, last_tokens=[11])
    md = vr.verify_varlen_metadata(batch, num_rows=1, num_tokens=4, width=2, query_len=4)
    ids = torch.tensor(md.input_ids)
    vr.place_drafts(ids, torch.tensor([[12, 13, 14]]), md)
    assert ids.tolist() == [11, 12, 13, 14]
    assert md.positions == [3, 4, 5, 6] and md.slot_mapping == [15, 16, 17, 18]
    assert md.cu_seqlens_q == [0, 4] and md.cu_seqlens_k == [0, 7] and md.block_tables == [[3, 4]]
    # :160-173: the same row verifying 2, and [1, 2, 3] + 4 on blocks [8, 9] verifying 4; drafts [5, 0, 1]
    rows = [reference_row(4, [3, 4], 2), reference_row(4, [8, 9], 4)]
    batch = vr.VerifyBatch([r[0] for r in rows], [r[1] for r in rows], [r[2] for r in rows], num_blocks=99,
                           block_size=4, last_tokens=[11, 4])
    md = vr.verify_varlen_metadata(batch, num_rows=2, num_tokens=6, width=2, query_len=4)
    ids = torch.tensor(md.input_ids)
    vr.place_drafts(ids, torch.tensor([[12, 13, 14], [5, 0, 1]]), md)
    assert ids.tolist() == [11, 12, 4, 5, 0, 1] and md.positions == [3, 4, 3, 4, 5, 6]
    assert md.slot_mapping == [15, 16, 35, 36, 37, 38]
    assert md.cu_seqlens_q == [0, 2, 6] and md.cu_seqlens_k == [0, 5, 12]


def test_reference_graph_inputs_known_answer():
    # tests/test_speculative_decoder.py:176-189: a graph of 8 tokens and 4 slots, rows verifying 2 and 3
    rows = [reference_row(4, [3, 4], 2), reference_row(4, [8, 9], 3)]
    batch = vr.VerifyBatch([r[0] for r in rows], [r[1] for r in rows], [r[2] for r in rows], num_blocks=99,
                           block_size=4, last_tokens=[11, 4])
    md = vr.verify_varlen_metadata(batch, num_rows=4, num_tokens=8, width=2, query_len=4)
    ids = torch.zeros(32, dtype=torch.int64)
    ids[:8] = torch.tensor(md.input_ids)
    vr.place_drafts(ids, torch.tensor([[12, 13, 14], [5, 0, 1]]), md)
    assert ids[:8].tolist() == [11, 12, 4, 5, 0, 0, 0, 0]
    assert md.cu_seqlens_q[:5] == [0, 2, 5, 8, 8]
    assert md.block_tables == [[3, 4], [8, 9], [99, 99], [99, 99]]
