"""Complex output of ``spherical_harmonics_table_with_derivative`` (``real_output=False``).

The device op forms the reference's complex table from the HIP real table with
a fixed unitary per ``l`` (``ye3t_amd.runtime.complex_from_real_table``).  These
CPU checks feed the oracle's real table through that conversion and pin the
result against SciPy's complex harmonics (Condon-Shortley phase, orthonormal,
the reference's convention: ``core/spherical.py:20-60,170-187``) for the
values, against central differences of SciPy's values for the gradient, and
against the reference's own real-from-complex map (``execution_plan.py:6943-6963``)
for the round trip.  SciPy is independent of both the oracle and this package,
so a wrong sign, a swapped ``m``/``-m`` column or a dropped ``1/sqrt2`` fails.
"""

import numpy as np
import pytest

import oracle


def _directions(n, seed):
    rng = np.random.default_rng(seed)
    v = rng.normal(size=(n, 3)) * rng.uniform(0.5, 3.0, size=(n, 1))
    # off-axis directions on both hemispheres and every azimuth quadrant
    extra = np.array([[1.0, 2.0, 0.5], [-1.0, 0.3, -2.0], [0.2, -1.5, 1.0], [-0.7, -0.4, 0.1]])
    return np.concatenate([v, extra])


def _scipy_table(v, l_max):
    from scipy.special import sph_harm_y

    r = np.linalg.norm(v, axis=1)
    u = v / r[:, None]
    theta = np.arctan2(np.linalg.norm(u[:, :2], axis=1), u[:, 2])
    phi = np.arctan2(u[:, 1], u[:, 0])
    cols = [sph_harm_y(l, m, theta, phi) for l in range(l_max + 1) for m in range(-l, l + 1)]
    return np.stack(cols, axis=1)


def _convert(v, l_max, dtype=None):
    import torch

    from ye3t_amd.runtime import complex_from_real_table

    val, grad = oracle.real_sph_table(v, l_max)
    tv, tg = torch.from_numpy(val), torch.from_numpy(grad)
    if dtype is not None:
        tv, tg = tv.to(dtype), tg.to(dtype)
    y, g = complex_from_real_table(tv, tg, l_max)
    return y, g


@pytest.mark.parametrize("l_max", [0, 1, 3, 6])
def test_complex_values_match_scipy(l_max):
    v = _directions(200, l_max)
    y, g = _convert(v, l_max)
    assert y.shape == (v.shape[0], (l_max + 1) ** 2) and g.shape == (v.shape[0], (l_max + 1) ** 2, 3)
    ref = _scipy_table(v, l_max)
    np.testing.assert_allclose(y.numpy(), ref, rtol=0, atol=1e-12)


@pytest.mark.parametrize("l_max", [1, 4])
def test_complex_gradient_matches_central_differences(l_max):
    v = _directions(60, 10 + l_max)
    _, g = _convert(v, l_max)
    h = 1e-6
    fd = np.zeros(g.shape, dtype=np.complex128)
    for k in range(3):
        step = np.zeros(3)
        step[k] = h
        fd[:, :, k] = (_scipy_table(v + step, l_max) - _scipy_table(v - step, l_max)) / (2 * h)
    scale = max(1.0, float(np.abs(fd).max()))
    np.testing.assert_allclose(g.numpy(), fd, rtol=0, atol=2e-7 * scale)


def test_round_trip_through_the_reference_real_map():
    """The reference's real rows taken from the complex table (its own map)
    give back the real table the conversion started from."""
    l_max = 5
    v = _directions(50, 99)
    real, _ = oracle.real_sph_table(v, l_max)
    y = _convert(v, l_max)[0].numpy()
    rows = []
    for l in range(l_max + 1):
        for m in range(-l, l + 1):
            c = y[:, l * l + l + abs(m)]
            if m < 0:
                rows.append(np.sqrt(2.0) * (1.0 if (-m) % 2 else -1.0) * c.imag)
            elif m == 0:
                rows.append(c.real)
            else:
                rows.append(np.sqrt(2.0) * (-1.0 if m % 2 else 1.0) * c.real)
    np.testing.assert_allclose(np.stack(rows, axis=1), real, rtol=0, atol=1e-13)


def test_conjugate_symmetry_and_dtypes():
    """``Y_l,-m = (-1)^m conj(Y_lm)`` for values and gradient; float32 tables
    give complex64, float64 complex128."""
    import torch

    l_max = 4
    v = _directions(30, 7)
    y, g = _convert(v, l_max)
    assert y.dtype == torch.complex128 and g.dtype == torch.complex128
    for l in range(l_max + 1):
        for m in range(1, l + 1):
            s = (-1) ** m
            assert torch.allclose(y[:, l * l + l - m], s * y[:, l * l + l + m].conj(), rtol=0, atol=1e-15)
            assert torch.allclose(g[:, l * l + l - m], s * g[:, l * l + l + m].conj(), rtol=0, atol=1e-15)
        assert torch.all(y[:, l * l + l].imag == 0)
    y32, g32 = _convert(v, l_max, torch.float32)
    assert y32.dtype == torch.complex64 and g32.dtype == torch.complex64
