"""Pinning of oracle.layernorm: closed forms, the fp64 mathematics, and the residual semantics of
add_rms_forward (layernorm.py:26-40). Each check fails for a dropped residual, a sum instead of a mean, a missing
eps, a swapped gate and up half, or sigmoid in place of silu."""
import numpy as np
import torch

from oracle import layernorm as ref


def test_constant_row_normalises_to_the_weight():
    # mean(c^2) = c^2, so x / sqrt(c^2 + eps) = sign(c) up to eps; the output is sign(c) * weight
    x = torch.full((3, 64), -2.5, dtype=torch.bfloat16)
    w = torch.linspace(-1, 1, 64).to(torch.bfloat16)
    out = ref.rms_forward(x, w, 1e-6)
    assert torch.equal(out, (-w.float()).to(torch.bfloat16).expand_as(out))


def test_known_vector_and_eps():
    # x = (3, 4): mean of squares 12.5; with eps 0 the scale is 1/sqrt(12.5); eps = 12.5 halves the variance term
    x = torch.tensor([[3.0, 4.0]])
    w = torch.ones(2)
    assert torch.allclose(ref.rms_forward(x, w, 0.0), x / 12.5 ** 0.5)
    assert torch.allclose(ref.rms_forward(x, w, 12.5), x / 25.0 ** 0.5)


def test_matches_the_fp64_mathematics():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16, 4096, generator=g).to(torch.bfloat16)
    r = torch.randn(16, 4096, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16)
    want = ref.rms_norm_f64(x.float().numpy(), w.float().numpy(), 1e-6)
    got = ref.rms_forward(x, w, 1e-6).float().numpy()
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)
    out, res = ref.add_rms_forward(x, r, w, 1e-6)
    want = ref.rms_norm_f64(x.float().numpy(), w.float().numpy(), 1e-6, r.float().numpy())
    assert np.all(np.abs(out.float().numpy() - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)
    # the new residual is the rounded sum, and the norm is of the unrounded sum: rms of (x + r), not of x
    assert torch.equal(res, (x.float() + r.float()).to(torch.bfloat16))
    assert not torch.equal(out, ref.rms_forward(x, w, 1e-6))


def test_silu_and_mul_halves_and_closed_forms():
    # gate 0 -> 0; gate large -> gate * up; the gate is the first half
    x = torch.tensor([[0.0, 20.0, -20.0, 3.0, 5.0, 7.0]])
    out = ref.silu_and_mul(x)
    assert out[0, 0] == 0.0
    assert abs(float(out[0, 1]) - 20.0 * 5.0) < 1e-4
    assert abs(float(out[0, 2])) < 1e-6
    g = torch.Generator().manual_seed(1)
    x = torch.randn(8, 256, generator=g).to(torch.bfloat16)
    want = ref.silu_and_mul_f64(x.float().numpy())
    got = ref.silu_and_mul(x).float().numpy()
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-30)
    swapped = torch.cat(x.chunk(2, -1)[::-1], -1)
    assert not torch.equal(ref.silu_and_mul(swapped), ref.silu_and_mul(x))
