"""The q/k RMSNorm + rotary + store oracle against closed forms and fp64 mathematics (CPU only).

Each check fails for a plausible mistake: a missing eps or mean (instead of sum), the interleaved instead of the
split-halves rotation, a sign flip in either rotated half, cos/sin swapped, or a wrong frequency exponent.
"""
import math

import numpy as np
import pytest
import torch

from oracle import qk_norm_rope as ref

D = 128


def test_rms_norm_closed_forms():
    w = torch.linspace(0.5, 1.5, D)
    # a constant vector c normalises to sign(c) * |c| / sqrt(c^2 + eps) times the weight
    c, eps = -3.0, 1e-6
    y = ref.rms_norm(torch.full((1, D), c), w, eps)
    torch.testing.assert_close(y[0], w * (c / math.sqrt(c * c + eps)), rtol=1e-6, atol=0)
    # one non-zero entry a: var = a^2 / D, so that entry becomes sqrt(D) * sign(a) * w_i (eps aside)
    x = torch.zeros(1, D)
    x[0, 17] = 0.25
    y = ref.rms_norm(x, w, 0.0)
    assert y[0, 17].item() == pytest.approx(math.sqrt(D) * w[17].item(), rel=1e-6)
    assert torch.count_nonzero(y) == 1


def test_rms_norm_matches_f64_and_rounds_like_the_reference():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(64, 4, D, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    y = ref.rms_norm(x, w, 1e-6)
    assert y.dtype == torch.bfloat16
    want = ref.rms_norm_f64(x.float().numpy(), w.float().numpy(), 1e-6)
    # two bf16 roundings (after the normalisation and after the weight): within 2^-7 relative
    np.testing.assert_array_less(np.abs(y.float().numpy() - want), np.abs(want) * 2.0 ** -7 + 1e-30)


def test_rope_table_matches_the_frequency_formula():
    table = ref.rope_table(D, 4096, 1e6)
    want = ref.rope_table_f64(D, 4096, 1e6)
    np.testing.assert_allclose(table.numpy(), want, atol=2e-3, rtol=0)   # fp32 angle products up to 4095
    assert table.shape == (4096, D)
    np.testing.assert_array_equal(table[0, : D // 2].numpy(), np.ones(D // 2, dtype=np.float32))
    np.testing.assert_array_equal(table[0, D // 2:].numpy(), np.zeros(D // 2, dtype=np.float32))
    # frequency i is base^(-2i/D): at position 1 the angle of the last frequency is 1e6^(-126/128)
    assert table[1, D // 2 - 1].item() == pytest.approx(math.cos(1e6 ** (-126 / 128)), rel=1e-6)


def test_rope_is_the_split_halves_complex_rotation():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(40, 3, D, generator=g)
    pos = torch.randint(0, 4096, (40,), generator=g)
    table = torch.tensor(ref.rope_table_f64(D, 4096, 1e4), dtype=torch.float32)
    got = ref.rope(pos, x, table)
    want = ref.rope_f64(pos.numpy(), x.numpy(), table.numpy().astype(np.float64))
    np.testing.assert_allclose(got.numpy(), want, rtol=0, atol=1e-5)
    # the interleaved convention (pairs 2i, 2i+1) is a different rotation
    cos, sin = table[pos].unsqueeze(1).chunk(2, dim=-1)
    xe, xo = x[..., 0::2], x[..., 1::2]
    inter = torch.stack([xe * cos - xo * sin, xo * cos + xe * sin], -1).reshape(x.shape)
    assert not torch.allclose(inter, got, atol=1e-3)


def test_rope_position_zero_is_identity_and_rotations_compose_and_keep_norms():
    table = ref.rope_table_f64(D, 8192, 1e4)
    g = np.random.default_rng(7)
    x = g.standard_normal((6, 2, D))
    zero = np.zeros(6, dtype=np.int64)
    np.testing.assert_allclose(ref.rope_f64(zero, x, table), x, atol=1e-15)
    a, b = g.integers(0, 4000, 6), g.integers(0, 4000, 6)
    np.testing.assert_allclose(ref.rope_f64(b, ref.rope_f64(a, x, table), table), ref.rope_f64(a + b, x, table),
                               atol=1e-9)
    y = ref.rope_f64(a, x, table)
    h = D // 2
    np.testing.assert_allclose(y[..., :h] ** 2 + y[..., h:] ** 2, x[..., :h] ** 2 + x[..., h:] ** 2, rtol=1e-12)
    # attention scores depend only on the relative position
    q, k = g.standard_normal((1, 1, D)), g.standard_normal((1, 1, D))
    s1 = np.sum(ref.rope_f64(np.array([900]), q, table) * ref.rope_f64(np.array([100]), k, table))
    s2 = np.sum(ref.rope_f64(np.array([1800]), q, table) * ref.rope_f64(np.array([1000]), k, table))
    assert s1 == pytest.approx(s2, rel=1e-9)


def test_fused_sequence_stores_rotated_keys_and_raw_values():
    g = torch.Generator().manual_seed(9)
    T, hq, hkv = 5, 4, 2
    q = torch.randn(T, hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(T, hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(T, hkv, D, generator=g).to(torch.bfloat16)
    w = torch.ones(D, dtype=torch.bfloat16)
    table = ref.rope_table(D, 64, 1e4)
    pos = torch.tensor([0, 3, 9, 9, 63])
    slots = torch.tensor([7, -1, 0, 2, 5], dtype=torch.int32)
    kc = torch.zeros(8, hkv, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    q_rot, k_rot = ref.qk_norm_rope_store(pos, q, k, v, w, w, 1e-6, table, kc, vc, slots)
    assert torch.equal(k_rot, ref.rope(pos, ref.rms_norm(k, w, 1e-6), table))
    assert torch.equal(q_rot, ref.rope(pos, ref.rms_norm(q, w, 1e-6), table))
    for t, s in enumerate(slots.tolist()):
        if s >= 0:
            assert torch.equal(kc[s], k_rot[t]) and torch.equal(vc[s], v[t])
    assert torch.count_nonzero(kc[[1, 3, 4, 6]]) == 0    # untouched slots; slot -1 wrote nothing
    _, k_only = ref.qk_norm_rope_store(pos, None, k, v, None, w, 1e-6, table, None, None, None)
    assert torch.equal(k_only, k_rot)


def test_the_package_table_is_the_oracle_table():
    from nvs_amd.layers.qk_norm_rope import rope_cos_sin_cache
    assert torch.equal(rope_cos_sin_cache(D, 4096, 1e6, torch.device("cpu")), ref.rope_table(D, 4096, 1e6))
