"""nvs_spec_accept_noalloc, the fused accept with its records and row counters in the library's fixed device
scratch, called through the C ABI and checked against nvs_spec_accept (the entry point with a caller workspace):
accepted lengths and tails bit for bit, on two calls in a row, the second smaller, for a batch that truncates and one
that does not (dense races, whose state also lives in the scratch); and sizes past the scratch refused before any
launch."""
import pytest
import torch

import nvs_amd.workloads as wl
from conftest import log_case
from nvs_amd import _lib
from nvs_amd.layers import spec_sampler as ns
from oracle import spec_sampler as ref

pytestmark = pytest.mark.gpu


def draft_probs(draft_logits, temps, tk, tp):
    return ref.probs_from_logits(draft_logits, temps, tk, tp, int(tk.max()), bool((tp < 1).any()))


def noalloc(case, device):
    g = case.to(device)
    B, k = case.drafts.shape
    T, V = case.logits.shape
    n = torch.full((B,), -7, dtype=torch.int64, device=device)
    tail = torch.full((B,), -7, dtype=torch.int64, device=device)
    lib = _lib.load()
    lens = None if g.verified_lens is None else g.verified_lens.contiguous()
    _lib.check(lib.nvs_spec_accept_noalloc(
        g.logits.data_ptr(), _lib.dtype_code(g.logits.dtype), g.logits.stride(0), g.temperatures.data_ptr(),
        g.top_k.data_ptr(), g.top_p.data_ptr(), case.max_top_k, int(case.has_top_p), g.q.data_ptr(),
        g.drafts.data_ptr(), _lib.ptr(lens), g.uniforms.data_ptr(), g.noise.data_ptr(), B, k, T, V, n.data_ptr(),
        tail.data_ptr(), _lib.stream_of(g.logits)), "spec_accept_noalloc")
    return n.cpu(), tail.cpu()


def with_workspace(case, device):
    g = case.to(device)
    st = ns.SamplingTensors(g.temperatures, g.top_k, g.top_p, case.max_top_k, case.has_top_p,
                            bool((case.top_k > 0).all()))
    n, tail = ns.spec_accept_with_draws(g.logits, g.q, g.drafts, st, g.verified_lens, g.uniforms, g.noise)
    return n.cpu(), tail.cpu()


@pytest.mark.parametrize("top_k", [64, 0], ids=["truncating", "dense"])
def test_noalloc_matches_the_workspace_entry_point(device, top_k):
    big = wl.sampler_case(48, 7, 151936, top_k=top_k, verified_lens=[1, 8, 3, 5, 2, 7, 4, 6] * 6,
                          draft_probs_fn=draft_probs)
    small = wl.sampler_case(5, 3, 32000, top_k=top_k, top_p=[0.9, 1.0, 0.8, 1.0, 1.0],
                            temperature=[0.7, 1.0, 1.3, 1.0, 1.0], draft_probs_fn=draft_probs)
    for name, case in (("48 rows varlen V 151936", big), ("5 rows fixed V 32000", small)):
        log_case(f"spec_accept_noalloc top_k={top_k}: {name}")
        got = noalloc(case, device)
        want = with_workspace(case, device)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), name


def test_noalloc_refuses_sizes_past_its_scratch(device):
    log_case("spec_accept_noalloc size limits")
    lib = _lib.load()
    p = 1 << 20    # never dereferenced: the checks return before any launch
    st = lib.nvs_spec_accept_noalloc(p, _lib.DTYPE_F32, 100, p, p, p, 64, 0, p, p, None, p, p, 1025, 7, 1025 * 8,
                                     100, p, p, None)
    assert st == _lib.NVS_ERR_UNSUPPORTED and b"1024" in lib.nvs_last_error()
    st = lib.nvs_spec_accept_noalloc(p, _lib.DTYPE_F32, 100, p, p, p, 64, 0, p, p, p, p, p, 1000, 7, 40000, 100,
                                     p, p, None)
    assert st == _lib.NVS_ERR_UNSUPPORTED
