"""The differentiable Torch expressions of the radial and harmonic bases
(``ye3t_amd.runtime.basis_torch``, used for second derivatives through the
``ye3t_runtime`` operators): values and first derivatives (by autograd) equal
the oracle's tables and derivatives, which are pinned against the reference's
core bit for bit."""

import numpy as np
import pytest
import torch

import oracle
from ye3t_amd.runtime import basis_torch


@pytest.mark.parametrize("l_max", [0, 2, 3, 6, 8])
def test_harmonics_and_gradient_match_the_oracle(l_max):
    rng = np.random.default_rng(l_max)
    v = rng.normal(size=(120, 3)) * rng.uniform(0.3, 3.0, size=(120, 1))
    x = torch.from_numpy(v).requires_grad_(True)
    y = basis_torch.real_harmonics(x, l_max)
    ref_y, ref_g = oracle.real_sph_table(v, l_max)
    np.testing.assert_allclose(y.detach().numpy(), ref_y, rtol=0, atol=5e-14)
    if not y.requires_grad:  # l_max = 0: a constant
        assert not np.any(ref_g)
        return
    for k in range(y.shape[1]):
        (g,) = torch.autograd.grad(y[:, k].sum(), x, retain_graph=True)
        np.testing.assert_allclose(g.numpy(), ref_g[:, k, :], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("n_max", [0, 1, 2, 8, 15])
def test_radial_and_derivative_match_the_oracle(n_max):
    rng = np.random.default_rng(n_max)
    r = rng.uniform(0.2, 6.0, size=150)
    x = torch.from_numpy(r).requires_grad_(True)
    c = torch.full((150,), 5.0, dtype=torch.float64)
    lam = torch.full((150,), 1.5, dtype=torch.float64)
    R = basis_torch.cheb_exp_cos_radial(x, c, lam, n_max)
    ref_v, ref_d = oracle.radial_table(r, np.full(150, 5.0), np.full(150, 1.5), n_max)
    np.testing.assert_allclose(R.detach().numpy(), ref_v, rtol=0, atol=5e-15)
    if not R.requires_grad:  # n_max = 0: a constant inside the cutoff
        assert not np.any(ref_d)
        return
    for n in range(n_max + 1):
        (g,) = torch.autograd.grad(R[:, n].sum(), x, retain_graph=True)
        np.testing.assert_allclose(g.numpy(), ref_d[:, n], rtol=1e-12, atol=1e-12)
