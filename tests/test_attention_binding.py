"""The attention binding on the CPU, in the style of the reference's tests/test_attention_modes.py: the module
names Attention.forward calls are swapped by bind(), and each call is followed to where it lands.

Prefill without a block table (model_runner.py:176-185: no cached prefix; speculative decoding turns the prefix
cache off, so every prompt and the warm-up take this branch) must reach the function bound before the swap,
unchanged. Verify rows (prefill context with a block table) and decode / draft-block rows must reach
nvs_paged_attention, and the KV store nvs_store_kvcache. The library is replaced by a recorder of its C entry
points, so no GPU is needed: what is checked is the dispatch and the arguments handed to the C ABI."""
import ctypes
import types

import pytest
import torch

from nvs_amd import _lib
from nvs_amd.layers import attention as nattn
from nvs_amd.utils.context import reset_context, set_context

HEADS, KV_HEADS, HEAD_DIM, BLOCK = 4, 2, 128, 32


class Recorder:
    """Stands in for a flash-attn function: remembers the call and returns q unchanged."""

    def __init__(self):
        self.calls = []

    def __call__(self, q, k, v, **kwargs):
        self.calls.append((q, k, v, kwargs))
        return q.clone()


class FakeLib:
    """Stands in for libnvs_amd.so: records each C entry point called with its arguments and returns NVS_OK."""

    def __init__(self):
        self.calls = []

    def nvs_paged_attention_workspace_size(self, *args):
        args[-1]._obj.value = 0          # an unsplit plan: no workspace
        return _lib.NVS_OK

    def __getattr__(self, name):
        if not name.startswith("nvs_"):
            raise AttributeError(name)

        def entry(*args):
            self.calls.append((name, args))
            return _lib.NVS_OK
        return entry

    def named(self, name):
        return [args for called, args in self.calls if called == name]


@pytest.fixture
def bound(monkeypatch):
    """nvs_amd's attention module bound over a stand-in prefill function, with the C library recorded."""
    lib, prefill = FakeLib(), Recorder()
    monkeypatch.setattr(_lib, "load", lambda path=None: lib)
    monkeypatch.setattr(_lib, "require_device", lambda *tensors: None)
    monkeypatch.setattr(_lib, "stream_of", lambda t: 0)
    for name in ("store_kvcache", "flash_attn_varlen_func", "flash_attn_with_kvcache"):
        monkeypatch.setattr(nattn, name, getattr(nattn, name))     # restored after the test
    monkeypatch.setattr(nattn, "flash_attn_varlen_func", prefill)  # what the module held before the swap
    nattn.bind(nattn)
    yield lib, prefill
    reset_context()


def layer(blocks=3):
    attn = nattn.Attention(HEADS, HEAD_DIM, 0.125, KV_HEADS)
    attn.k_cache = torch.zeros(blocks, BLOCK, KV_HEADS, HEAD_DIM, dtype=torch.bfloat16)
    attn.v_cache = torch.zeros_like(attn.k_cache)
    return attn


def rows(n):
    q = torch.randn(n, HEADS, HEAD_DIM).to(torch.bfloat16)
    k = torch.randn(n, KV_HEADS, HEAD_DIM).to(torch.bfloat16)
    return q, k, k.clone()


def test_prefill_without_block_table_reaches_the_previous_function(bound):
    lib, prefill = bound
    cu = torch.tensor([0, 5, 9], dtype=torch.int32)
    set_context(True, cu, cu, 5, 5, torch.arange(9, dtype=torch.int32))
    q, k, v = rows(9)
    out = layer()(q, k, v)
    assert len(prefill.calls) == 1 and not lib.named("nvs_paged_attention")
    pq, pk, pv, kwargs = prefill.calls[0]
    # the prompt's own new rows, unpaged, with the reference's keyword arguments
    assert pq is q and pk is k and pv is v
    assert kwargs == dict(max_seqlen_q=5, cu_seqlens_q=cu, max_seqlen_k=5, cu_seqlens_k=cu, softmax_scale=0.125,
                          causal=True, block_table=None)
    assert torch.equal(out, q)
    # the new rows were stored into the cache first (attention.py:63-64)
    assert len(lib.named("nvs_store_kvcache")) == 1


def test_verify_rows_reach_nvs_paged_attention(bound):
    lib, prefill = bound
    cu_q = torch.tensor([0, 3, 8], dtype=torch.int32)
    cu_k = torch.tensor([0, 40, 90], dtype=torch.int32)
    bt = torch.tensor([[0, 1], [2, 1]], dtype=torch.int32)
    set_context(True, cu_q, cu_k, 5, 64, torch.arange(8, dtype=torch.int32), None, bt)
    attn = layer()
    out = attn(*rows(8))
    assert not prefill.calls
    (args,) = lib.named("nvs_paged_attention")
    assert out.shape == (8, HEADS, HEAD_DIM)
    # q, k_cache, v_cache, block tables, cu_seqlens_q/k handed over as device pointers; varlen mode (no context_lens)
    assert args[4] == attn.k_cache.data_ptr() and args[5] == attn.v_cache.data_ptr()
    assert args[10] == bt.data_ptr() and args[13] == cu_q.data_ptr() and args[14] == cu_k.data_ptr()
    assert args[15] is None
    n_rows, max_q, max_k, h, hkv, d, bs, scale, causal = args[17:26]
    assert (n_rows, max_q, max_k, h, hkv, d, bs, causal) == (2, 5, 64, HEADS, KV_HEADS, HEAD_DIM, BLOCK, 1)
    assert scale == pytest.approx(0.125)


@pytest.mark.parametrize("lq, causal", [(1, True), (7, False)])
def test_decode_and_draft_block_reach_nvs_paged_attention(bound, lq, causal):
    lib, prefill = bound
    ctx_lens = torch.tensor([40, 17, 60], dtype=torch.int32)
    bt = torch.tensor([[0, 1], [2, 0], [1, 2]], dtype=torch.int32)
    set_context(False, slot_mapping=torch.arange(3 * lq, dtype=torch.int32), context_lens=ctx_lens,
                block_tables=bt, query_len_per_seq=lq, causal=causal)
    out = layer()(*rows(3 * lq))
    assert not prefill.calls
    (args,) = lib.named("nvs_paged_attention")
    assert out.shape == (3 * lq, HEADS, HEAD_DIM)
    # fixed-Lq mode: no cu_seqlens, the context lengths, query_len_per_seq queries per row, the context's causal flag
    assert args[13] is None and args[14] is None and args[15] == ctx_lens.data_ptr()
    assert (args[16], args[17], args[18]) == (lq, 3, lq)
    assert args[25] == int(causal)


def test_bind_on_a_module_keeps_its_prefill_and_unbinds():
    """bind() on any module holding the reference's three names (as nanovllm.layers.attention does)."""
    module = types.ModuleType("attention")
    prefill, decode, store = Recorder(), Recorder(), Recorder()
    module.flash_attn_varlen_func, module.flash_attn_with_kvcache, module.store_kvcache = prefill, decode, store
    previous = nattn.bind(module)
    assert module.store_kvcache is nattn.store_kvcache
    assert module.flash_attn_with_kvcache is nattn.paged_attention_with_kvcache
    assert module.flash_attn_varlen_func.prefill is prefill
    nattn.bind(module)                                  # binding again keeps the first prefill function
    assert module.flash_attn_varlen_func.prefill is prefill
    cu = torch.tensor([0, 2], dtype=torch.int32)
    q = torch.zeros(2, HEADS, HEAD_DIM)
    module.flash_attn_varlen_func(q, q, q, max_seqlen_q=2, cu_seqlens_q=cu, max_seqlen_k=2, cu_seqlens_k=cu,
                                  softmax_scale=1.0, causal=True, block_table=None)
    assert len(prefill.calls) == 1
    nattn.unbind(module, previous)
    assert (module.flash_attn_varlen_func, module.flash_attn_with_kvcache, module.store_kvcache) == \
        (prefill, decode, store)


def test_set_prefill_attention_serves_this_modules_attention(monkeypatch):
    prefill = Recorder()
    monkeypatch.setattr(nattn, "flash_attn_varlen_func", nattn.flash_attn_varlen_func)
    nattn.set_prefill_attention(prefill)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    set_context(True, cu, cu, 4, 4, torch.arange(4, dtype=torch.int32))
    try:
        attn = nattn.Attention(HEADS, HEAD_DIM, 1.0, KV_HEADS)     # no cache bound: nothing stored
        attn(*rows(4))
    finally:
        reset_context()
    assert len(prefill.calls) == 1 and prefill.calls[0][3]["block_table"] is None
