"""Parity of the fused q/k RMSNorm + rotary + KV store kernel with the eager CPU oracle.

Tolerance: outputs are bf16 (or fp16). The kernel follows the oracle's op order and roundings element by element
(correctly rounded sqrt and division, products and sums rounded separately); the only difference is the summation
order of the 128 squares inside the RMSNorm, which can move a normalised value by one unit in the last place
before the rotation mixes it into its pair. So: every element within 2^-7 of (its magnitude + the norm of its
rotated pair), at least 99% of them bit-identical, values copied to the cache bit-exact, slots of padding tokens
(slot -1) untouched.
"""
import numpy as np
import pytest
import torch

import nvs_amd.workloads as wl
from conftest import log_case
from nvs_amd.layers import qk_norm_rope as nrope
from oracle import qk_norm_rope as ref

pytestmark = pytest.mark.gpu


def pair_norm(y: torch.Tensor) -> torch.Tensor:
    """Norm of each rotated (y[i], y[i + 64]) pair, repeated on both halves."""
    y = y.float()
    half = y.shape[-1] // 2
    n = torch.sqrt(y[..., :half] ** 2 + y[..., half:] ** 2)
    return torch.cat([n, n], dim=-1)


def close_to_oracle(got: torch.Tensor, want: torch.Tensor, what: str, rotated: torch.Tensor | None = None):
    """rotated: the oracle's normalised input of the rotation. One ulp of a normalised value moves both outputs of
    its pair by up to 2^-8 of the pair's norm, however small the output itself is after the rotation."""
    g, w = got.float().cpu(), want.float().cpu()
    diff = (g - w).abs()
    scale = torch.maximum(g.abs(), w.abs())
    if rotated is not None:
        scale = scale + pair_norm(rotated.cpu())
    bound = scale * 2.0 ** -7
    assert bool((diff <= bound).all()), f"{what}: max excess {float((diff - bound).max())}"
    same = float((g == w).float().mean())
    print(f"{what}: {100 * same:.3f}% bit-identical, max |diff| {float(diff.max()):.3e}")
    assert same >= 0.99, f"{what}: only {100 * same:.2f}% bit-identical"


def run_case(case: wl.QkRopeCase, device, keys_only=False, norms=True, in_place=False, head_major=False,
             kv_interleaved=False):
    g = case.to(device)
    q, k, v = g.split()
    if head_major:
        kc, vc = wl.head_major(g.k_cache), wl.head_major(g.v_cache)
    elif kv_interleaved:
        kc, vc = wl.kv_cache_empty(*g.k_cache.shape, dtype=g.k_cache.dtype, device=device)
        kc.copy_(g.k_cache)
        vc.copy_(g.v_cache)
    else:
        kc, vc = g.k_cache.clone(), g.v_cache.clone()
    qw = g.q_norm_weight if norms else None
    kw = g.k_norm_weight if norms else None
    q_in = None if keys_only else q
    q_out = q if in_place else None
    out = nrope.qk_norm_rope_store(g.positions, q_in, k, v, qw, kw, case.eps, g.table, kc, vc, g.slot_mapping,
                                   q_out=q_out)
    torch.cuda.synchronize()
    qc, kcpu, vcpu = case.split()
    kc_ref, vc_ref = case.k_cache.clone(), case.v_cache.clone()
    q_ref, k_ref = ref.qk_norm_rope_store(case.positions, None if keys_only else qc, kcpu, vcpu,
                                          case.q_norm_weight if norms else None,
                                          case.k_norm_weight if norms else None, case.eps, case.table,
                                          kc_ref, vc_ref, case.slot_mapping)
    q_norm = ref.rms_norm(qc, case.q_norm_weight, case.eps) if norms else qc
    k_norm = ref.rms_norm(kcpu, case.k_norm_weight, case.eps) if norms else kcpu
    return out, kc, vc, q_ref, (kc_ref, vc_ref, k_norm), q_norm


def check_caches(case, kc, vc, refs):
    kc_ref, vc_ref, k_norm = refs
    live = case.slot_mapping >= 0
    slots = case.slot_mapping[live].long()
    flat_k = kc.cpu().contiguous().view(-1, case.num_kv_heads, case.head_dim)   # logical [slot, head, dim] order
    flat_v = vc.cpu().contiguous().view(-1, case.num_kv_heads, case.head_dim)
    ref_k, ref_v = kc_ref.view_as(flat_k), vc_ref.view_as(flat_v)
    close_to_oracle(flat_k[slots], ref_k[slots], "k in cache", k_norm[live])
    assert torch.equal(flat_v[slots], ref_v[slots]), "v copies must be bit-exact"
    untouched = torch.ones(flat_k.shape[0], dtype=torch.bool)
    untouched[slots] = False
    assert torch.count_nonzero(flat_k[untouched]) == 0 and torch.count_nonzero(flat_v[untouched]) == 0


@pytest.mark.parametrize("num_tokens", [1, 296, 2048])
def test_qwen3_8b_shape(device, num_tokens):
    log_case(f"qk norm rope store qwen3-8b T={num_tokens}")
    case = wl.qk_rope_case(num_tokens, num_padding=min(8, num_tokens - 1))
    out, kc, vc, q_ref, refs, q_norm = run_case(case, device)
    close_to_oracle(out, q_ref, "q", q_norm)
    check_caches(case, kc, vc, refs)


def test_head_major_cache(device):
    """Caches stored head-major ([blocks, Hkv, block_size, D] memory behind the [blocks, block_size, Hkv, D] view):
    the same values land in the same logical slots, and nothing else is written."""
    log_case("qk norm rope store into head-major caches, qwen3-8b T=296")
    case = wl.qk_rope_case(296, num_padding=8, seed=6)
    out, kc, vc, q_ref, refs, q_norm = run_case(case, device, head_major=True)
    assert kc.stride(1) == case.head_dim and not kc.is_contiguous()
    close_to_oracle(out, q_ref, "q", q_norm)
    check_caches(case, kc, vc, refs)


def test_kv_interleaved_cache(device):
    """K and V interleaved in one buffer (each block and kv head's keys, then its values, one contiguous run): the
    same values land in the same logical slots, and nothing else is written."""
    log_case("qk norm rope store into kv-interleaved caches, qwen3-8b T=296")
    case = wl.qk_rope_case(296, num_padding=8, seed=7)
    out, kc, vc, q_ref, refs, q_norm = run_case(case, device, kv_interleaved=True)
    assert kc.stride(2) == 2 * kc.shape[1] * case.head_dim and not kc.is_contiguous()
    close_to_oracle(out, q_ref, "q", q_norm)
    check_caches(case, kc, vc, refs)


def test_f64_mathematics(device):
    """The kernel's result against the fp64 formula (RMSNorm then the complex rotation), one rounding budget per
    bf16 step."""
    log_case("qk norm rope store vs fp64")
    case = wl.qk_rope_case(64, num_padding=0, seed=4)
    out, *_ = run_case(case, device)
    qc, _, _ = case.split()
    y = ref.rms_norm_f64(qc.float().numpy(), case.q_norm_weight.float().numpy(), case.eps)
    want = ref.rope_f64(case.positions.numpy(), y, case.table.numpy().astype(np.float64))
    got = out.float().cpu().numpy()
    # the two roundings before the rotation move each value of a (y1, y2) pair by up to 2^-8 of it, the rotation
    # carries that onto both outputs in proportion to the pair's norm, and the last rounding adds 2^-9 of the output
    half = y.shape[-1] // 2
    norm = np.sqrt(y[..., :half] ** 2 + y[..., half:] ** 2)
    norm = np.concatenate([norm, norm], axis=-1)
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * (np.abs(want) + norm))


def test_keys_only_draft_path_and_no_norm(device):
    log_case("qk norm rope store keys only / no norm")
    case = wl.qk_rope_case(100, num_heads=16, num_kv_heads=8, seed=2)
    out, kc, vc, _, refs, _ = run_case(case, device, keys_only=True)
    assert out is None
    check_caches(case, kc, vc, refs)
    out, kc, vc, q_ref, refs, q_norm = run_case(case, device, norms=False)
    close_to_oracle(out, q_ref, "q without norm", q_norm)
    check_caches(case, kc, vc, refs)


def test_in_place_fp16_and_gqa_shapes(device):
    log_case("qk norm rope store in place, fp16, 64/8 heads")
    case = wl.qk_rope_case(77, num_heads=64, num_kv_heads=8, dtype=torch.float16, seed=3)
    out, kc, vc, q_ref, refs, q_norm = run_case(case, device, in_place=True)
    close_to_oracle(out, q_ref, "q fp16 in place", q_norm)
    check_caches(case, kc, vc, refs)


def test_rejects_bad_arguments(device):
    case = wl.qk_rope_case(4, num_padding=0).to(device)
    q, k, v = case.split()
    with pytest.raises(ValueError):
        nrope.qk_norm_rope_store(case.positions, q, k, v, case.q_norm_weight, case.k_norm_weight, 1e-6,
                                 case.table.double(), case.k_cache, case.v_cache, case.slot_mapping)
    with pytest.raises(ValueError):
        nrope.qk_norm_rope_store(case.positions.int(), q, k, v, case.q_norm_weight, case.k_norm_weight, 1e-6,
                                 case.table, case.k_cache, case.v_cache, case.slot_mapping)
