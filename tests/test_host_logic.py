"""Host-side logic of the drop-in layer, on the CPU: the context mirror, SamplingTensors construction, and the
guarantee that no op silently runs on the CPU."""
from types import SimpleNamespace

import pytest
import torch

from nvs_amd.layers import attention as nattn
from nvs_amd.layers import spec_sampler as ns
from nvs_amd.utils import context as ctx


def test_context_defaults_and_round_trip():
    ctx.reset_context()
    c = ctx.get_context()
    assert (c.is_prefill, c.max_seqlen_q, c.query_len_per_seq, c.causal) == (False, 0, 1, True)
    ctx.set_context(False, context_lens=torch.ones(3, dtype=torch.int32), query_len_per_seq=7, causal=False)
    c = ctx.get_context()
    assert c.query_len_per_seq == 7 and c.causal is False and c.context_lens.tolist() == [1, 1, 1]
    ctx.reset_context()
    assert ctx.get_context().context_lens is None


def rows(*params):
    return ns.sampling_tensors([SimpleNamespace(temperature=t, top_k=k, top_p=p) for t, k, p in params],
                               torch.device("cpu"))


def test_sampling_tensors_greedy_batch_has_no_temperatures():
    # test_spec_sampler.py:35-39
    s = rows((0, 0, 1.0), (0, 0, 1.0))
    assert s.temperatures is None and s.max_top_k == 0 and s.has_top_p is False


def test_sampling_tensors_rejects_mixed_greedy_and_random():
    # test_spec_sampler.py:42-44
    with pytest.raises(ValueError):
        rows((0, 0, 1.0), (0.7, 0, 1.0))


def test_sampling_tensors_flags_and_per_token_expansion():
    s = rows((0.7, 3, 0.9), (1.0, 0, 1.0))
    assert (s.max_top_k, s.has_top_p, s.all_top_k) == (3, True, False)
    per = ns.sampling_per_token(s, torch.tensor([2, 3]), 5)
    assert per.top_k.tolist() == [3, 3, 0, 0, 0] and per.max_top_k == 3
    torch.testing.assert_close(per.temperatures, torch.tensor([0.7, 0.7, 1.0, 1.0, 1.0]))


def test_ops_refuse_cpu_tensors():
    s = rows((1.0, 2, 1.0))
    with pytest.raises(ValueError, match="ROCm device"):
        ns.probs_from_logits(torch.randn(1, 8), s)
    with pytest.raises(ValueError, match="ROCm device"):
        ns.race(torch.rand(2, 8), torch.rand(2, 8))
    with pytest.raises(ValueError, match="ROCm device"):
        ns.accept_greedy(torch.randn(1, 2, 8), torch.tensor([[1]]))
    key = torch.zeros(2, 2, 4)
    cache = torch.zeros(1, 4, 2, 4)
    with pytest.raises(ValueError, match="ROCm device"):
        nattn.store_kvcache(key, key, cache, cache.clone(), torch.tensor([0, 1], dtype=torch.int32))


def test_store_kvcache_keeps_the_reference_preconditions():
    # attention.py:36-39: strided heads are rejected before anything else
    key = torch.zeros(2, 4, 2, 8)[:, :, 0]       # stride(1) != head_dim
    cache = torch.zeros(1, 4, 2, 4)
    with pytest.raises(AssertionError):
        nattn.store_kvcache(key, key, cache, cache, torch.tensor([0, 1], dtype=torch.int32))


def test_unbound_prefill_without_block_table_raises():
    """With no prefill attention bound, a call without a block table is refused (never run as paged attention);
    the binding tests (test_attention_binding.py) show where a bound one sends it."""
    with pytest.raises(NotImplementedError):
        nattn.paged_attention_varlen(torch.zeros(1), torch.zeros(1), torch.zeros(1), 1, torch.zeros(2), 1,
                                     torch.zeros(2), 1.0, True, None)
    with pytest.raises(NotImplementedError):
        nattn.varlen_func(None)(torch.zeros(1), torch.zeros(1), torch.zeros(1), max_seqlen_q=1,
                                cu_seqlens_q=torch.zeros(2), max_seqlen_k=1, cu_seqlens_k=torch.zeros(2),
                                softmax_scale=1.0, causal=True)


def test_truncate_without_top_k_returns_the_input():
    s = rows((1.0, 0, 1.0))
    x = torch.randn(2, 5)
    assert ns.truncate_logits(x, s) is x


def test_outgrown_persistent_buffers_stay_allocated(monkeypatch):
    """A counter buffer replaced by a larger one is kept referenced (a graph captured with it still holds its
    address), and the name now maps to the larger buffer."""
    from nvs_amd import _lib
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setattr(_lib, "_persistent", {})
    monkeypatch.setattr(_lib, "_superseded", [])
    dev = torch.device("cpu")
    small = _lib.persistent_workspace("test_counters", 1000, dev)
    assert _lib.persistent_workspace("test_counters", 500, dev) is small
    big = _lib.persistent_workspace("test_counters", 100000, dev)
    assert big is not small and big.numel() >= 100000 and int(big.sum()) == 0
    assert any(buf is small for buf in _lib._superseded)
