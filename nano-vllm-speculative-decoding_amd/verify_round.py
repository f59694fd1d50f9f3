"""A whole verify round of a Qwen3-shaped target: the forward of every decoder layer over the verify batch, the
logits at the verified positions, and the fused accept. The forward is captured as one HIP graph per
(row slots, tokens) shape, and each round loads its metadata into the graph's buffers and replays it.

Reference (the structure mirrored):
  SpeculativeDecoder.verify_logits / _verify_graph / _load_graph_inputs / capture_graphs   speculative.py:470-572
  verify_varlen_metadata (row slots: the batch, padding rows, empty rows)                  batch_metadata.py:149-181
  verify_token_counts (the graphs' token counts)                                           verify_schedule.py:18-23
  Qwen3DecoderLayer / Qwen3Model / Qwen3ForCausalLM.compute_logits                        qwen3.py:146-160,174-191,221-226
Each step of a layer runs on this library except the projections and the LM head, which are plain GEMMs
(torch.nn.functional.linear, served by hipBLASLt):
  input RMSNorm (+ residual add)   nvs_rms_norm              qwen3.py:152-155
  qkv projection                   GEMM                      qwen3.py:78
  q/k norm, RoPE, paged KV store   nvs_qk_norm_rope_store    qwen3.py:82-85, attention.py:63-64
  paged verify attention           nvs_paged_attention       attention.py:65-70
  o projection                     GEMM                      qwen3.py:87
  post-attention RMSNorm           nvs_rms_norm              qwen3.py:157
  gate_up projection               GEMM                      qwen3.py:114
  SiLU-and-mul                     nvs_silu_and_mul          qwen3.py:115
  down projection                  GEMM                      qwen3.py:116
Weights are random (no checkpoint is loaded): they set the bytes and FLOPs of a round, not its numbers.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from .layers import attention as nattn
from .layers.activation import silu_and_mul
from .layers.layernorm import rms_norm
from .layers.qk_norm_rope import qk_norm_rope_store, rope_cos_sin_cache
from .workloads import head_major_empty

PAD_SLOT = -1


@dataclass(frozen=True)
class Qwen3Shape:
    hidden_size: int = 4096
    num_layers: int = 36
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 12288
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_position: int = 40960

    @property
    def q_size(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_kv_heads * self.head_dim

    def layer_weight_elements(self) -> int:
        """qkv, o, gate_up and down projections of one layer (the norms are a few KB)."""
        h, i = self.hidden_size, self.intermediate_size
        return h * (self.q_size + 2 * self.kv_size) + self.q_size * h + h * 2 * i + i * h

    def streamed_weight_bytes(self, element_size: int = 2) -> int:
        """Weight bytes one forward reads from HBM: every projection and the LM head (the embedding is gathered
        per token). 15.14 GB for Qwen3-8B in bf16."""
        return (self.num_layers * self.layer_weight_elements() + self.vocab_size * self.hidden_size) * element_size


QWEN3_8B = Qwen3Shape()


def verify_token_counts(max_batch_size: int, query_len: int) -> list[int]:
    """Token counts of the variable-length verify graphs (verify_schedule.py:18-23): the powers 1, 2, 4 that are
    below query_len, then each multiple of query_len up to max_batch_size rows of query_len tokens."""
    return [n for n in (1, 2, 4) if n < query_len] + [query_len * b for b in range(1, max_batch_size + 1)]


@dataclass
class VerifyBatch:
    """The rows of one verify round: row r verifies q_lens[r] tokens (its last token and q_lens[r] - 1 drafts),
    the last q_lens[r] of a context of k_lens[r] tokens held in blocks block_tables[r] of the paged caches."""
    q_lens: list[int]
    k_lens: list[int]
    block_tables: list[list[int]]
    num_blocks: int               # blocks in use; the pad block (zeros) is block num_blocks
    block_size: int = 256
    last_tokens: list[int] | None = None   # each row's last token (the first verified input), when known

    @property
    def pad_block(self) -> int:
        return self.num_blocks

    @property
    def num_tokens(self) -> int:
        return sum(self.q_lens)

    def kv_bytes(self, num_kv_heads: int, head_dim: int, element_size: int = 2) -> int:
        """K and V bytes one attention layer reads: every key of every row once."""
        return sum(self.k_lens) * num_kv_heads * head_dim * element_size * 2


def random_verify_batch(batch: int, q_range: tuple[int, int] = (1, 8), k_range: tuple[int, int] = (2800, 3200),
                        block_size: int = 256, seed_lengths: int = 1, seed_blocks: int = 2) -> VerifyBatch:
    """Verify lengths and contexts uniform in the ranges (inclusive); each row's blocks drawn from one random
    permutation of the physical blocks."""
    g = torch.Generator().manual_seed(seed_lengths)
    q = torch.randint(q_range[0], q_range[1] + 1, (batch,), generator=g).tolist()
    k = torch.randint(k_range[0], k_range[1] + 1, (batch,), generator=g).tolist()
    k = [max(kk, qq) for qq, kk in zip(q, k)]
    per_row = [math.ceil(kk / block_size) for kk in k]
    perm = torch.randperm(sum(per_row), generator=torch.Generator().manual_seed(seed_blocks)).tolist()
    tables, at = [], 0
    for n in per_row:
        tables.append(perm[at:at + n])
        at += n
    return VerifyBatch(q, k, tables, sum(per_row), block_size)


@dataclass
class VerifyMetadata:
    """One verify forward over its row slots (batch_metadata.py:127-139). input_ids holds each row's last token
    (0 when unknown) and 0 at the draft positions, which draft_index / draft_source fill from the drafts [B, k]."""
    input_ids: list[int] = field(default_factory=list)
    positions: list[int] = field(default_factory=list)
    slot_mapping: list[int] = field(default_factory=list)
    cu_seqlens_q: list[int] = field(default_factory=lambda: [0])
    cu_seqlens_k: list[int] = field(default_factory=lambda: [0])
    block_tables: list[list[int]] = field(default_factory=list)
    draft_index: list[int] = field(default_factory=list)
    draft_source: list[int] = field(default_factory=list)


def verify_varlen_metadata(batch: VerifyBatch | None, num_rows: int, num_tokens: int, width: int,
                           query_len: int, pad_block: int | None = None) -> VerifyMetadata:
    """The row slots of a verify forward (batch_metadata.py:149-181): the batch's rows first (positions
    k_len - q_len .. k_len - 1 and their cache slots), then padding rows of at most query_len tokens at positions
    0.. of the pad block with slot -1, until num_tokens tokens are placed, then empty rows up to num_rows.
    batch None: every row slot is padding (what a graph is captured on)."""
    if pad_block is None:
        assert batch is not None, "a capture batch needs the pad block"
        pad_block = batch.pad_block
    block_size = 256 if batch is None else batch.block_size
    real = [] if batch is None else list(zip(batch.q_lens, batch.k_lens, batch.block_tables))
    if len(real) > num_rows:
        raise ValueError(f"{len(real)} rows do not fit {num_rows} row slots")
    # What the batch leaves of num_tokens is shared out over the padding rows, query_len tokens at most each.
    spare = num_tokens - sum(q_len for q_len, _, _ in real)
    if spare < 0:
        raise ValueError(f"{num_tokens - spare} tokens do not fit a graph of {num_tokens}")
    pad_rows = num_rows - len(real)
    if spare > pad_rows * query_len:
        raise ValueError(f"{spare} tokens beyond the batch need more than {pad_rows} padding rows of {query_len}")
    pad_lens = [min(query_len, max(0, spare - i * query_len)) for i in range(pad_rows)]

    md = VerifyMetadata()

    def add_row(first_position: int, n: int, n_keys: int, slots: list[int], table_row: list[int]) -> None:
        md.positions.extend(range(first_position, first_position + n))
        md.slot_mapping.extend(slots)
        md.cu_seqlens_q.append(md.cu_seqlens_q[-1] + n)
        md.cu_seqlens_k.append(md.cu_seqlens_k[-1] + n_keys)
        md.block_tables.append(table_row)

    num_drafts = query_len - 1
    for r, (q_len, k_len, table) in enumerate(real):
        if not 1 <= q_len <= query_len or len(table) > width or len(table) * block_size < k_len:
            raise ValueError("a row's verify length, context or block table does not fit the graph")
        first = len(md.input_ids)
        md.input_ids.append(batch.last_tokens[r] if batch.last_tokens is not None else 0)
        md.input_ids.extend([0] * (q_len - 1))
        md.draft_index.extend(range(first + 1, first + q_len))          # the row's drafts follow its last token
        md.draft_source.extend(range(r * num_drafts, r * num_drafts + q_len - 1))
        start = k_len - q_len
        add_row(start, q_len, k_len, [table[p // block_size] * block_size + p % block_size for p in range(start, k_len)],
                table + [pad_block] * (width - len(table)))
    for n in pad_lens:   # padding rows attend to their own tokens on the pad block; empty rows have none
        md.input_ids.extend([0] * n)
        add_row(0, n, n, [PAD_SLOT] * n, [pad_block] * width)
    return md


@dataclass
class VerifyContext:
    """What Attention.forward reads from get_context() on the verify branch (context.py:5-16)."""
    cu_seqlens_q: torch.Tensor
    cu_seqlens_k: torch.Tensor
    max_seqlen_q: int
    max_seqlen_k: int
    slot_mapping: torch.Tensor
    block_tables: torch.Tensor


@dataclass
class LayerWeights:
    qkv: torch.Tensor         # [q + 2 kv, hidden]
    o: torch.Tensor           # [hidden, q]
    gate_up: torch.Tensor     # [2 intermediate, hidden]
    down: torch.Tensor        # [hidden, intermediate]
    input_norm: torch.Tensor  # [hidden]
    post_norm: torch.Tensor   # [hidden]
    q_norm: torch.Tensor      # [head_dim]
    k_norm: torch.Tensor      # [head_dim]


class Qwen3VerifyTarget:
    """Random-init weights of a Qwen3 shape and one paged KV cache per layer, [num_blocks + 1, block_size, Hkv, D]
    with the pad block last and zero (model_runner.py:158-169). The caches start with random keys and values."""

    def __init__(self, shape: Qwen3Shape, num_blocks: int, block_size: int = 256, device="cuda",
                 dtype: torch.dtype = torch.bfloat16, seed: int = 0, init_std: float = 0.02):
        self.shape, self.dtype, self.device = shape, dtype, torch.device(device)
        self.block_size, self.num_blocks = block_size, num_blocks
        g = torch.Generator(device=self.device).manual_seed(seed)
        s = shape

        def weight(*size):
            return torch.randn(*size, generator=g, device=self.device, dtype=dtype).mul_(init_std)

        def ones(n):
            return torch.ones(n, device=self.device, dtype=dtype)

        self.embed = weight(s.vocab_size, s.hidden_size)
        self.layers = [LayerWeights(qkv=weight(s.q_size + 2 * s.kv_size, s.hidden_size),
                                    o=weight(s.hidden_size, s.q_size),
                                    gate_up=weight(2 * s.intermediate_size, s.hidden_size),
                                    down=weight(s.hidden_size, s.intermediate_size),
                                    input_norm=ones(s.hidden_size), post_norm=ones(s.hidden_size),
                                    q_norm=ones(s.head_dim), k_norm=ones(s.head_dim))
                       for _ in range(s.num_layers)]
        self.norm = ones(s.hidden_size)
        self.lm_head = weight(s.vocab_size, s.hidden_size)
        # Per layer a [num_blocks + 1, block_size, Hkv, D] view of head-major memory: the attention streams every
        # (block, kv head) as one contiguous run (the reference's token-major layout works too, only slower).
        cache = (s.num_layers, num_blocks + 1, block_size, s.num_kv_heads, s.head_dim)
        self.k_caches = head_major_empty(*cache, dtype=dtype, device=self.device)
        self.v_caches = head_major_empty(*cache, dtype=dtype, device=self.device)
        self.k_caches.normal_(generator=g)
        self.v_caches.normal_(generator=g)
        self.k_caches[:, num_blocks].zero_()
        self.v_caches[:, num_blocks].zero_()
        self.cos_sin_cache = rope_cos_sin_cache(s.head_dim, s.max_position, s.rope_theta, self.device)
        self.scale = s.head_dim ** -0.5

    @property
    def pad_block(self) -> int:
        return self.num_blocks

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, ctx: VerifyContext) -> torch.Tensor:
        """Qwen3Model.forward (qwen3.py:174-191) over T tokens -> the final-normed hidden states [T, hidden]."""
        s = self.shape
        T = input_ids.shape[0]
        eps = s.rms_norm_eps
        qs, kvs = s.q_size, s.kv_size
        h = F.embedding(input_ids, self.embed)
        residual = None
        for i, lw in enumerate(self.layers):
            if residual is None:
                residual = h
                h = rms_norm(h, lw.input_norm, eps)
            else:
                h, residual = rms_norm(h, lw.input_norm, eps, residual=residual, out=h)
            qkv = F.linear(h, lw.qkv)
            q = qkv[:, :qs].view(T, s.num_heads, s.head_dim)
            k = qkv[:, qs:qs + kvs].view(T, s.num_kv_heads, s.head_dim)
            v = qkv[:, qs + kvs:].view(T, s.num_kv_heads, s.head_dim)
            q = qk_norm_rope_store(positions, q, k, v, lw.q_norm, lw.k_norm, eps, self.cos_sin_cache,
                                   self.k_caches[i], self.v_caches[i], ctx.slot_mapping, q_out=q)
            o = nattn.paged_attention_varlen(q, self.k_caches[i], self.v_caches[i], ctx.max_seqlen_q,
                                             ctx.cu_seqlens_q, ctx.max_seqlen_k, ctx.cu_seqlens_k, self.scale,
                                             causal=True, block_table=ctx.block_tables)
            h = F.linear(o.view(T, qs), lw.o)
            h, residual = rms_norm(h, lw.post_norm, eps, residual=residual, out=h)
            h = F.linear(silu_and_mul(F.linear(h, lw.gate_up)), lw.down)
        h, _ = rms_norm(h, self.norm, eps, residual=residual, out=h)
        return h

    def compute_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """ParallelLMHead.forward with all_logits (embed_head.py:56-61): [T, hidden] -> [T, vocab]."""
        return F.linear(hidden, self.lm_head)


def place_drafts(input_ids: torch.Tensor, drafts: torch.Tensor, md: VerifyMetadata) -> None:
    """The verified drafts into the flat input ids where the metadata puts them (speculative.py:514-517):
    input_ids[draft_index] = drafts.flatten()[draft_source]."""
    if not md.draft_index:
        return
    dev = input_ids.device
    index = torch.tensor(md.draft_index, dtype=torch.int64).to(dev, non_blocking=True)
    source = torch.tensor(md.draft_source, dtype=torch.int64).to(dev, non_blocking=True)
    input_ids[index] = drafts.reshape(-1).to(input_ids.dtype)[source]


class VerifyGraphs:
    """One HIP graph of the target's forward per (row slots, tokens) shape of verify_token_counts, over static
    device buffers, all in one memory pool (speculative.py:530-572). A round builds its metadata on the host,
    copies it into the buffers, replays the smallest graph holding its tokens and returns the hidden states of the
    verified tokens; the logits and the accept follow outside the graph, as in the reference."""

    def __init__(self, target: Qwen3VerifyTarget, max_batch_size: int = 512, query_len: int = 8,
                 max_model_len: int = 4096):
        self.target = target
        self.max_batch_size, self.query_len, self.max_model_len = max_batch_size, query_len, max_model_len
        self.width = math.ceil(max_model_len / target.block_size)
        self.shapes = [(min(n, max_batch_size), n) for n in verify_token_counts(max_batch_size, query_len)]
        max_tokens, max_rows = max_batch_size * query_len, max_batch_size
        dev = target.device
        self.input_ids = torch.zeros(max_tokens, dtype=torch.int64, device=dev)
        self.positions = torch.zeros(max_tokens, dtype=torch.int64, device=dev)
        self.slot_mapping = torch.full((max_tokens,), PAD_SLOT, dtype=torch.int32, device=dev)
        self.cu_seqlens_q = torch.zeros(max_rows + 1, dtype=torch.int32, device=dev)
        self.cu_seqlens_k = torch.zeros(max_rows + 1, dtype=torch.int32, device=dev)
        self.block_tables = torch.full((max_rows, self.width), target.pad_block, dtype=torch.int32, device=dev)
        self.outputs = torch.zeros(max_tokens, target.shape.hidden_size, dtype=target.dtype, device=dev)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.pool = None

    def shape_for(self, num_tokens: int) -> tuple[int, int]:
        """The smallest graph shape with at least num_tokens tokens."""
        for shape in self.shapes:
            if shape[1] >= num_tokens:
                return shape
        raise ValueError(f"{num_tokens} tokens exceed the largest verify graph")

    def _context(self, num_rows: int, num_tokens: int) -> VerifyContext:
        return VerifyContext(self.cu_seqlens_q[:num_rows + 1], self.cu_seqlens_k[:num_rows + 1], self.query_len,
                             self.max_model_len, self.slot_mapping[:num_tokens], self.block_tables[:num_rows])

    @torch.inference_mode()
    def run_drafts(self, batch: VerifyBatch, drafts: torch.Tensor) -> torch.Tensor:
        """run() with the input ids built from the metadata (speculative.py:502-512): each row's last token
        (batch.last_tokens) and its verified drafts from drafts [B, k], placed by draft_index / draft_source."""
        if batch.last_tokens is None:
            raise ValueError("run_drafts needs each row's last token")
        num_rows, num_tokens = self.shape_for(batch.num_tokens)
        if num_tokens not in self.graphs:
            self.capture([num_tokens])
        md = verify_varlen_metadata(batch, num_rows, num_tokens, self.width, self.query_len)
        self._load(md, num_rows, num_tokens)
        self.input_ids[:num_tokens].copy_(torch.tensor(md.input_ids, dtype=torch.int64,
                                                       pin_memory=self.target.device.type == "cuda"),
                                          non_blocking=True)
        place_drafts(self.input_ids, drafts, md)
        self.graphs[num_tokens].replay()
        return self.outputs[:batch.num_tokens]

    def _load(self, md: VerifyMetadata, num_rows: int, num_tokens: int) -> None:
        """Host metadata into the buffers (speculative.py:519-529): pinned host tensors, asynchronous copies."""
        pin = self.target.device.type == "cuda"

        def host(values, dtype):
            return torch.tensor(values, dtype=dtype, pin_memory=pin)

        self.positions[:num_tokens].copy_(host(md.positions, torch.int64), non_blocking=True)
        self.slot_mapping[:num_tokens].copy_(host(md.slot_mapping, torch.int32), non_blocking=True)
        self.cu_seqlens_q[:num_rows + 1].copy_(host(md.cu_seqlens_q, torch.int32), non_blocking=True)
        self.cu_seqlens_k[:num_rows + 1].copy_(host(md.cu_seqlens_k, torch.int32), non_blocking=True)
        self.block_tables[:num_rows].copy_(host(md.block_tables, torch.int32), non_blocking=True)

    def _forward(self, num_rows: int, num_tokens: int) -> torch.Tensor:
        return self.target.forward(self.input_ids[:num_tokens], self.positions[:num_tokens],
                                   self._context(num_rows, num_tokens))

    @torch.inference_mode()
    def capture(self, token_counts: list[int] | None = None) -> None:
        """Capture the graphs of the given token counts (every shape when None), largest first, each on padding
        rows only, after one eager warm-up run of the same shape."""
        shapes = [s for s in self.shapes if token_counts is None or s[1] in token_counts]
        for num_rows, num_tokens in reversed(shapes):
            if num_tokens in self.graphs:
                continue
            md = verify_varlen_metadata(None, num_rows, num_tokens, self.width, self.query_len, self.target.pad_block)
            self._load(md, num_rows, num_tokens)
            self.outputs[:num_tokens] = self._forward(num_rows, num_tokens)   # warm-up
            torch.cuda.synchronize(self.target.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, self.pool):
                self.outputs[:num_tokens] = self._forward(num_rows, num_tokens)
            if self.pool is None:
                self.pool = graph.pool()
            self.graphs[num_tokens] = graph
            torch.cuda.synchronize(self.target.device)

    @torch.inference_mode()
    def run(self, batch: VerifyBatch, input_ids: torch.Tensor) -> torch.Tensor:
        """Hidden states [batch.num_tokens, hidden] of the batch's verified tokens, through the captured graph of
        the smallest shape holding them (captured here if it is missing)."""
        n = batch.num_tokens
        num_rows, num_tokens = self.shape_for(n)
        if num_tokens not in self.graphs:
            self.capture([num_tokens])
        md = verify_varlen_metadata(batch, num_rows, num_tokens, self.width, self.query_len)
        self._load(md, num_rows, num_tokens)
        self.input_ids[:n].copy_(input_ids)
        self.input_ids[n:num_tokens].zero_()
        self.graphs[num_tokens].replay()
        return self.outputs[:n]

    @torch.inference_mode()
    def run_eager(self, batch: VerifyBatch, input_ids: torch.Tensor) -> torch.Tensor:
        """The same forward without the graph (speculative.py:484-498), on the same padded shape and buffers."""
        n = batch.num_tokens
        num_rows, num_tokens = self.shape_for(n)
        md = verify_varlen_metadata(batch, num_rows, num_tokens, self.width, self.query_len)
        self._load(md, num_rows, num_tokens)
        self.input_ids[:n].copy_(input_ids)
        self.input_ids[n:num_tokens].zero_()
        return self._forward(num_rows, num_tokens)[:n]
