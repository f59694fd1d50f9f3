"""Synthetic inputs of the verify hot path in the reference's memory layout.

Verify attention: the layout of verify_varlen_metadata (nanovllm/engine/batch_metadata.py:149-181) -- rows of
1..k+1 query tokens at the end of their context, cu_seqlens_q/k, padded block tables; padding rows of at most k+1
tokens on a zeroed pad block fill the token count up to a multiple of 8 -- over a per-layer paged cache
[blocks + 1, block_size, Hkv, D] whose last block is the pad block (model_runner.py:158-163). Physical blocks are
handed to rows in a random permutation.

Sampler: target logits ~ N(0, sigma^2), draft logits = target + N(0, 1) at the draft positions, draft probs q from
the draft logits, drafts sampled from q, uniforms and race noise from a seeded generator.

Seeds: Q/K/V 0, lengths 1, block permutation 2, target logits 10, draft noise 11, sampling generator 12.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class AttentionCase:
    q: torch.Tensor               # [T, H, D]
    k_cache: torch.Tensor         # [blocks + 1, bs, Hkv, D]
    v_cache: torch.Tensor
    block_tables: torch.Tensor    # [R, W] int32
    cu_seqlens_q: torch.Tensor    # [R + 1] int32
    cu_seqlens_k: torch.Tensor    # [R + 1] int32
    q_lens: list[int]
    k_lens: list[int]
    max_seqlen_q: int
    max_seqlen_k: int
    scale: float
    pad_block: int
    real_rows: int                # rows before the padding rows

    @property
    def rows(self) -> list[tuple[int, int, int]]:
        starts = self.cu_seqlens_q.tolist()
        return [(starts[r], self.q_lens[r], self.k_lens[r]) for r in range(len(self.q_lens))]

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes one attention pass reads: every visible key row of every kv head, once."""
        hkv, d = self.k_cache.shape[2], self.k_cache.shape[3]
        es = self.k_cache.element_size()
        return sum(lk for lq, lk in zip(self.q_lens, self.k_lens) if lq > 0) * hkv * d * es * 2

    def qo_bytes(self) -> int:
        es = self.q.element_size()
        return 2 * sum(self.q_lens) * self.q.shape[1] * self.q.shape[2] * es

    def flops(self) -> int:
        """2 FLOPs per multiply-add over the visible (query, key) pairs of QK^T and PV, all query heads."""
        h, d = self.q.shape[1], self.q.shape[2]
        pairs = 0
        for lq, lk in zip(self.q_lens, self.k_lens):
            pairs += sum(min(lk, lk - lq + i + 1) for i in range(lq))
        return 4 * h * d * pairs

    def to(self, device) -> "AttentionCase":
        fields = {name: getattr(self, name) for name in self.__dataclass_fields__}
        for name, value in fields.items():
            if isinstance(value, torch.Tensor):
                fields[name] = value.to(device)
        return AttentionCase(**fields)

    def head_major(self) -> "AttentionCase":
        """The same case with both caches stored head-major (head_major below)."""
        fields = {name: getattr(self, name) for name in self.__dataclass_fields__}
        fields["k_cache"] = head_major(self.k_cache)
        fields["v_cache"] = head_major(self.v_cache)
        return AttentionCase(**fields)

    def kv_interleaved(self, device=None) -> "AttentionCase":
        """The same case on `device` with both caches interleaved (kv_cache_empty). Built on the device directly:
        .to() would not keep the caches' strides."""
        fields = {name: getattr(self, name) for name in self.__dataclass_fields__}
        for name, value in fields.items():
            if isinstance(value, torch.Tensor):
                fields[name] = value.to(device)
        k, v = kv_cache_empty(*self.k_cache.shape, dtype=self.k_cache.dtype, device=device)
        k.copy_(self.k_cache)
        v.copy_(self.v_cache)
        fields["k_cache"], fields["v_cache"] = k, v
        return AttentionCase(**fields)


def head_major_empty(*shape: int, dtype: torch.dtype, device=None) -> torch.Tensor:
    """An uninitialised cache [..., blocks, block_size, Hkv, D] whose memory is [..., blocks, Hkv, block_size, D]:
    every (block, kv head) is one contiguous run of block_size * D elements."""
    *lead, block_size, hkv, d = shape
    return torch.empty(*lead, hkv, block_size, d, dtype=dtype, device=device).transpose(-3, -2)


def kv_cache_empty(*shape: int, dtype: torch.dtype, device=None) -> tuple[torch.Tensor, torch.Tensor]:
    """Uninitialised K and V caches, each [..., blocks, block_size, Hkv, D], interleaved: the memory is [..., blocks,
    Hkv, 2, block_size, D], so every (block, kv head) holds its block_size keys and then their values as one
    contiguous run. The kernels read and write it through its strides like any other layout; on the batch-64 verify
    layer it measured within about 1% of separate head-major caches (faster in variant sweeps, not in the bench's
    fixed order)."""
    *lead, block_size, hkv, d = shape
    buf = torch.empty(*lead, hkv, 2, block_size, d, dtype=dtype, device=device)
    return buf.select(-3, 0).transpose(-3, -2), buf.select(-3, 1).transpose(-3, -2)


def head_major(cache: torch.Tensor) -> torch.Tensor:
    """A head-major copy of a [..., blocks, block_size, Hkv, D] cache, equal to it element for element."""
    out = head_major_empty(*cache.shape, dtype=cache.dtype, device=cache.device)
    out.copy_(cache)
    return out


def verify_attention_case(q_lens: list[int], k_lens: list[int], num_heads: int, num_kv_heads: int, head_dim: int,
                          block_size: int = 256, dtype: torch.dtype = torch.bfloat16, pad_tokens_to: int = 8,
                          max_query_len: int = 8, table_width: int | None = None, device="cpu",
                          seed_qkv: int = 0, seed_blocks: int = 2, max_seqlen_k: int | None = None) -> AttentionCase:
    """Rows r < len(q_lens) verify q_lens[r] tokens against k_lens[r] keys (the verified tokens are the last
    q_lens[r] of them). The token count is padded to a multiple of pad_tokens_to with padding rows of at most
    max_query_len tokens that read the pad block from position 0 (batch_metadata.py:170-179)."""
    assert len(q_lens) == len(k_lens)
    for lq, lk in zip(q_lens, k_lens):
        assert 0 <= lq <= lk or (lq == 0 and lk == 0)
    q_lens = list(q_lens)
    k_lens = list(k_lens)
    real_rows = len(q_lens)
    total = sum(q_lens)
    padded = -(-total // pad_tokens_to) * pad_tokens_to if pad_tokens_to > 1 else total
    left = padded - total
    while left > 0:
        n = min(left, max_query_len)
        q_lens.append(n)
        k_lens.append(n)
        left -= n
    blocks_per_row = [math.ceil(lk / block_size) for lk in k_lens[:real_rows]]
    n_blocks = sum(blocks_per_row)
    pad_block = n_blocks
    width = table_width or max(1, max(blocks_per_row + [math.ceil(max(k_lens) / block_size)]))
    gen_blocks = torch.Generator().manual_seed(seed_blocks)
    perm = torch.randperm(n_blocks, generator=gen_blocks).tolist()
    tables = []
    at = 0
    for r in range(len(q_lens)):
        if r < real_rows:
            ids = perm[at:at + blocks_per_row[r]]
            at += blocks_per_row[r]
        else:
            ids = []
        tables.append(ids + [pad_block] * (width - len(ids)))
    gen = torch.Generator().manual_seed(seed_qkv)
    T = sum(q_lens)
    q = torch.randn(T, num_heads, head_dim, generator=gen).to(dtype)
    k_cache = torch.randn(n_blocks + 1, block_size, num_kv_heads, head_dim, generator=gen).to(dtype)
    v_cache = torch.randn(n_blocks + 1, block_size, num_kv_heads, head_dim, generator=gen).to(dtype)
    k_cache[pad_block] = 0
    v_cache[pad_block] = 0
    cu_q = [0]
    cu_k = [0]
    for lq, lk in zip(q_lens, k_lens):
        cu_q.append(cu_q[-1] + lq)
        cu_k.append(cu_k[-1] + lk)
    case = AttentionCase(
        q=q, k_cache=k_cache, v_cache=v_cache,
        block_tables=torch.tensor(tables, dtype=torch.int32),
        cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32),
        cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32),
        q_lens=q_lens, k_lens=k_lens,
        max_seqlen_q=max(max(q_lens), 1), max_seqlen_k=max_seqlen_k or max(max(k_lens), 1),
        scale=head_dim ** -0.5, pad_block=pad_block, real_rows=real_rows)
    return case.to(device) if device != "cpu" else case


def random_lengths(batch: int, q_range: tuple[int, int], k_range: tuple[int, int], seed: int = 1):
    """Verify lengths uniform in q_range and contexts uniform in k_range (both inclusive)."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randint(q_range[0], q_range[1] + 1, (batch,), generator=gen).tolist()
    k = torch.randint(k_range[0], k_range[1] + 1, (batch,), generator=gen).tolist()
    return q, [max(kk, qq) for qq, kk in zip(q, k)]


# The attention configurations (Qwen3-shaped: head_dim 128, 256-token blocks).
def config_c1(dtype=torch.float32) -> AttentionCase:
    """Qwen3-0.6B shape: 16 q / 8 kv heads, batch 1, 8 verify positions, 1,024-token context."""
    return verify_attention_case([8], [1024], 16, 8, 128, dtype=dtype)


def config_c2(dtype=torch.bfloat16) -> AttentionCase:
    """Qwen3-8B shape: 32 q / 8 kv heads, batch 8, 8 positions, contexts uniform in [900, 1200]."""
    q, k = random_lengths(8, (8, 8), (900, 1200))
    return verify_attention_case(q, k, 32, 8, 128, dtype=dtype)


def config_c3(dtype=torch.bfloat16, max_seqlen_k: int | None = None) -> AttentionCase:
    """Qwen3-8B shape at batch 64: verify lengths uniform in {1..8}, contexts uniform in [2800, 3200]."""
    q, k = random_lengths(64, (1, 8), (2800, 3200))
    return verify_attention_case(q, k, 32, 8, 128, dtype=dtype, max_seqlen_k=max_seqlen_k)


@dataclass
class SamplerCase:
    logits: torch.Tensor          # [T, V] target logits
    q: torch.Tensor               # [B, k, V] draft probabilities
    drafts: torch.Tensor          # [B, k] int64
    verified_lens: torch.Tensor | None   # [B] int64 or None (all k+1)
    temperatures: torch.Tensor    # [B]
    top_k: torch.Tensor           # [B] int64
    top_p: torch.Tensor           # [B]
    max_top_k: int
    has_top_p: bool
    uniforms: torch.Tensor        # [B, k]
    noise: torch.Tensor           # [B, V]

    def to(self, device) -> "SamplerCase":
        fields = {name: getattr(self, name) for name in self.__dataclass_fields__}
        for name, value in fields.items():
            if isinstance(value, torch.Tensor):
                fields[name] = value.to(device)
        return SamplerCase(**fields)


def sampler_case(batch: int, num_drafts: int, vocab: int, top_k: int | list[int] = 64,
                 top_p: float | list[float] = 1.0, temperature: float | list[float] = 1.0, sigma: float = 3.0,
                 verified_lens: list[int] | None = None, logits_dtype: torch.dtype = torch.float32,
                 draft_probs_fn=None, device="cpu") -> SamplerCase:
    """Target logits [T, V] ~ N(0, sigma^2) (seed 10); draft logits = target at the k draft positions + N(0, 1)
    (seed 11); q = draft_probs_fn(draft logits, temperatures, top_k, top_p) (the caller's probs_from_logits);
    drafts ~ q, then uniforms and noise, from one generator (seed 12) in the reference's order."""
    def per_row(v, dtype):
        vals = v if isinstance(v, list) else [v] * batch
        return torch.tensor(vals, dtype=dtype)
    temps = per_row(temperature, torch.float32)
    tk = per_row(top_k, torch.int64)
    tp = per_row(top_p, torch.float32)
    lens = None if verified_lens is None else torch.tensor(verified_lens, dtype=torch.int64)
    n_pos = batch * (num_drafts + 1) if lens is None else int(lens.sum())
    g_target = torch.Generator().manual_seed(10)
    full = torch.randn(batch, num_drafts + 1, vocab, generator=g_target) * sigma
    g_noise = torch.Generator().manual_seed(11)
    draft_logits = full[:, :num_drafts] + torch.randn(batch, num_drafts, vocab, generator=g_noise)
    if lens is None:
        logits = full.reshape(-1, vocab)
    else:
        logits = torch.cat([full[b, :int(lens[b])] for b in range(batch)])
    q = draft_probs_fn(draft_logits, temps, tk, tp)
    gen = torch.Generator().manual_seed(12)
    e_draft = torch.empty(batch, num_drafts, vocab).exponential_(1.0, generator=gen).clamp_min_(1e-10)
    drafts = (q / e_draft).argmax(dim=-1)
    uniforms = torch.rand(batch, num_drafts, generator=gen)
    noise = torch.empty(batch, vocab).exponential_(1.0, generator=gen).clamp_min_(1e-10)
    case = SamplerCase(logits=logits.to(logits_dtype), q=q.float().contiguous(), drafts=drafts,
                       verified_lens=lens, temperatures=temps, top_k=tk, top_p=tp,
                       max_top_k=int(tk.max()), has_top_p=bool((tp < 1.0).any()), uniforms=uniforms, noise=noise)
    return case.to(device) if device != "cpu" else case


@dataclass
class QkRopeCase:
    """Inputs of the q/k norm + rotary + KV store step of one layer: the fused qkv projection output
    [T, (Hq + 2 Hkv) * D] (q, k, v are views of it, as qwen3.py:79-81 splits it), token positions, the q/k norm
    weights, the rotary table, and a paged cache with the slots of the tokens (-1 for padding tokens)."""
    qkv: torch.Tensor             # [T, (Hq + 2 Hkv) * D]
    positions: torch.Tensor       # [T] int64
    q_norm_weight: torch.Tensor   # [D]
    k_norm_weight: torch.Tensor   # [D]
    table: torch.Tensor           # [P, D] fp32 cos | sin
    slot_mapping: torch.Tensor    # [T] int32
    k_cache: torch.Tensor         # [blocks, bs, Hkv, D]
    v_cache: torch.Tensor
    num_heads: int
    num_kv_heads: int
    head_dim: int
    eps: float = 1e-6

    def split(self):
        """(q, k, v) views [T, H, D] of the fused projection output."""
        hq, hkv, d = self.num_heads, self.num_kv_heads, self.head_dim
        q, k, v = self.qkv.split([hq * d, hkv * d, hkv * d], dim=-1)
        return q.view(-1, hq, d), k.view(-1, hkv, d), v.view(-1, hkv, d)

    def to(self, device) -> "QkRopeCase":
        fields = {name: getattr(self, name) for name in self.__dataclass_fields__}
        for name, value in fields.items():
            if isinstance(value, torch.Tensor):
                fields[name] = value.to(device)
        return QkRopeCase(**fields)

    def bytes_moved(self) -> int:
        """HBM bytes of the fused step: read q, k, v, positions, slots, the table rows and the weights; write the
        rotated q and the K/V rows of every stored token."""
        T = self.qkv.shape[0]
        es = self.qkv.element_size()
        d, hq, hkv = self.head_dim, self.num_heads, self.num_kv_heads
        stored = int((self.slot_mapping >= 0).sum())
        return (T * (hq + 2 * hkv) * d * es + T * (8 + 4) + T * d * 4 + 2 * d * es
                + T * hq * d * es + stored * 2 * hkv * d * es)


def qk_rope_case(num_tokens: int, num_heads: int = 32, num_kv_heads: int = 8, head_dim: int = 128,
                 num_padding: int = 8, max_position: int = 40960, rope_theta: float = 1e6, block_size: int = 256,
                 dtype=torch.bfloat16, seed: int = 0) -> QkRopeCase:
    """Qwen3-8B-shaped by default (rope_theta 1e6, 40,960 positions). The last num_padding tokens carry slot -1; the
    others go to distinct random slots of a cache with room for all of them."""
    from .layers.qk_norm_rope import rope_cos_sin_cache
    g = torch.Generator().manual_seed(seed)
    width = (num_heads + 2 * num_kv_heads) * head_dim
    qkv = (torch.randn(num_tokens, width, generator=g) * 2).to(dtype)
    positions = torch.randint(0, max_position, (num_tokens,), generator=g)
    q_w = (1 + 0.1 * torch.randn(head_dim, generator=g)).to(dtype)
    k_w = (1 + 0.1 * torch.randn(head_dim, generator=g)).to(dtype)
    table = rope_cos_sin_cache(head_dim, max_position, rope_theta, torch.device("cpu"))
    blocks = (num_tokens + block_size - 1) // block_size + 1
    slots = torch.randperm(blocks * block_size, generator=g)[:num_tokens].to(torch.int32)
    if num_padding:
        slots[-num_padding:] = -1
    k_cache = torch.zeros(blocks, block_size, num_kv_heads, head_dim, dtype=dtype)
    return QkRopeCase(qkv, positions, q_w, k_w, table, slots, k_cache, torch.zeros_like(k_cache), num_heads,
                      num_kv_heads, head_dim)


@dataclass
class RoundDrafts:
    """The draft side of a synthetic verify round: drafts [B, k] int64, their dense draft probabilities q [B, k, V]
    fp32, and per row how many leading drafts follow the target (follow[b] <= q_lens[b] - 1)."""
    drafts: torch.Tensor
    q: torch.Tensor
    follow: list[int]


def partly_accepted_drafts(graphs, batch, sampling, num_drafts: int = 7, seed: int = 13) -> RoundDrafts:
    """Drafts for one verify round on `graphs` (verify_round.VerifyGraphs) that the target partly accepts, so the
    accept's every branch runs: rows whose verified drafts all follow the target (the bonus token), rows that
    follow it up to a cut and then carry a random draft (a rejection, then the residual), and rows of random drafts.

    The random drafter draws from a top-64 softmax of N(0, 9) logits. A draft that follows the target is the
    target's argmax at its position, and its q row is the target's own probabilities there (sampling's per-row
    parameters), so u * q(d) < p(d) for every u < 1. The forward is causal, so position j's logits depend only on
    the drafts before j: the drafts are fixed position by position, one forward each. Sets batch.last_tokens."""
    import random

    from .layers import spec_sampler as ns

    target = graphs.target
    dev, vocab = target.device, target.shape.vocab_size
    rows, k = len(batch.q_lens), num_drafts
    rng = random.Random(seed)
    follow = []
    for L in batch.q_lens:
        kind = rng.choice(("all", "cut", "none"))
        follow.append(L - 1 if kind == "all" else (rng.randint(0, L - 2) if kind == "cut" and L >= 2 else 0))
    g = torch.Generator(device=dev).manual_seed(seed)
    batch.last_tokens = torch.randint(0, vocab, (rows,), generator=torch.Generator().manual_seed(seed)).tolist()
    q = torch.randn(rows, k, vocab, device=dev, generator=g).mul_(3.0)
    kth = q.topk(64, dim=-1).values[..., -1:]
    q = torch.softmax(q.masked_fill_(q < kth, float("-inf")), dim=-1)
    drafts = (q / torch.empty_like(q).exponential_(generator=g)).argmax(-1)
    starts = [sum(batch.q_lens[:b]) for b in range(rows)]
    for j in range(k):
        chosen = [b for b in range(rows) if j < follow[b]]
        if not chosen:
            continue
        logits = target.compute_logits(graphs.run_drafts(batch, drafts))
        at = torch.tensor([starts[b] + j for b in chosen], device=dev)
        drafts[torch.tensor(chosen, device=dev), j] = logits[at].argmax(-1)
    logits = target.compute_logits(graphs.run_drafts(batch, drafts))
    lens = torch.tensor(batch.q_lens, dtype=torch.int64, device=dev)
    p = ns.probs_from_logits(logits, ns.sampling_per_token(sampling, lens, logits.shape[0]))
    for b in range(rows):
        for j in range(follow[b]):
            q[b, j] = p[starts[b] + j]
    return RoundDrafts(drafts, q, follow)
