"""The factorized-angular and symmetric-power restatements in ``oracle/`` pinned.

* factorized angular (forward, adjoint, linear readout and its adjoint): the
  closed-form known-answer case of the reference's installed-CUDA smoke test
  (``cmake/smoke_installed_cuda.py:106-240``) with Torch autograd for the
  gradients, and bit-for-bit equality with the reference's own CPU core
  (``oracle/_ref``, compiled from its sources) on random DAGs, real and complex;
* symmetric-power monomial adjoint and shared monomials: the reference fixture
  ``shared_monomial_plan_v1`` (expected outputs and input adjoint), the core,
  and central differences of the forward.
"""

import json
import os

import numpy as np
import pytest
import torch

import oracle
from tests._dag import (KAT_LINEAR_BIAS, KAT_LINEAR_WEIGHT, KAT_OUTPUT_ADJOINT, KAT_PACKED, KAT_SOURCES,
                        KAT_TABLES, kat_closed_form, random_dag)

HAVE_REF = oracle.ref_lib() is not None and hasattr(oracle.ref_lib(), "ref_factorized_angular_f64")
needs_ref = pytest.mark.skipif(not HAVE_REF, reason="reference core not built (oracle/_ref)")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "shared_monomial_plan_v1.json")


def _torch_kat(packed):
    """The smoke test's Torch reference, differentiable."""
    src = packed.reshape(2, 2, 6)
    c = torch.as_tensor(KAT_TABLES["coefficient_values"])
    roots = (src[:, :, :3] * src[:, :, 3:] * c.conj().reshape(1, 1, 3)).sum(dim=2)
    return roots @ torch.as_tensor(KAT_TABLES["projection_values"]).reshape(2, 2)


def test_kat_forward_closed_form():
    packed = KAT_PACKED.astype(np.complex128)
    got = oracle.factorized_angular(packed, KAT_TABLES, KAT_SOURCES)
    np.testing.assert_allclose(got, kat_closed_form(packed), rtol=0, atol=1e-15)


def test_kat_adjoint_matches_torch_autograd():
    x = torch.as_tensor(KAT_PACKED.astype(np.complex128)).requires_grad_(True)
    g = torch.as_tensor(KAT_OUTPUT_ADJOINT)
    (expected,) = torch.autograd.grad(_torch_kat(x), x, g)
    got = oracle.factorized_angular_adjoint(KAT_OUTPUT_ADJOINT, KAT_PACKED.astype(np.complex128), KAT_TABLES,
                                            KAT_SOURCES)
    np.testing.assert_allclose(got, expected.numpy(), rtol=0, atol=1e-14)


def test_kat_linear_and_its_adjoint_match_torch_autograd():
    x = torch.as_tensor(KAT_PACKED.astype(np.complex128)).requires_grad_(True)
    w = torch.as_tensor(KAT_LINEAR_WEIGHT).requires_grad_(True)
    b = torch.tensor(KAT_LINEAR_BIAS, dtype=torch.complex128).requires_grad_(True)
    lin = _torch_kat(x) @ w + b
    got = oracle.factorized_angular_linear(KAT_PACKED.astype(np.complex128), KAT_TABLES, KAT_SOURCES,
                                           KAT_LINEAR_WEIGHT, KAT_LINEAR_BIAS)
    np.testing.assert_allclose(got, lin.detach().numpy(), rtol=0, atol=1e-14)
    g = torch.as_tensor(KAT_OUTPUT_ADJOINT[:, 0])
    ex, ew, eb = torch.autograd.grad(lin, (x, w, b), g)
    gx, gw, gb = oracle.factorized_angular_linear_adjoint(KAT_OUTPUT_ADJOINT[:, 0], KAT_PACKED.astype(np.complex128),
                                                          KAT_TABLES, KAT_SOURCES, KAT_LINEAR_WEIGHT)
    np.testing.assert_allclose(gx, ex.numpy(), rtol=0, atol=1e-14)
    np.testing.assert_allclose(gw, ew.numpy(), rtol=0, atol=1e-14)
    assert abs(gb - complex(eb)) < 1e-14


@needs_ref
@pytest.mark.parametrize("complex_data", [False, True])
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_dag_restatement_is_the_reference_core_bitwise(complex_data, seed):
    tables, S, D = random_dag(seed, complex_data=complex_data)
    rng = np.random.default_rng(100 + seed)
    B = 5
    x = rng.normal(size=(B, S * D))
    if complex_data:
        x = x + 1j * rng.normal(size=x.shape)
    out = oracle.factorized_angular(x, tables, S)
    ref = oracle.factorized_angular(x, tables, S, use_reference=True)
    assert np.array_equal(out, ref)
    g = rng.normal(size=out.shape) + (1j * rng.normal(size=out.shape) if complex_data else 0)
    adj = oracle.factorized_angular_adjoint(g, x, tables, S)
    assert np.array_equal(adj, oracle.factorized_angular_adjoint(g, x, tables, S, use_reference=True))
    w = rng.normal(size=out.shape[1]) + (1j * rng.normal(size=out.shape[1]) if complex_data else 0)
    bias = complex(0.3, -0.2) if complex_data else 0.3
    lin = oracle.factorized_angular_linear(x, tables, S, w, bias)
    assert np.array_equal(lin, oracle.factorized_angular_linear(x, tables, S, w, bias, use_reference=True))
    ga = rng.normal(size=B) + (1j * rng.normal(size=B) if complex_data else 0)
    mine = oracle.factorized_angular_linear_adjoint(ga, x, tables, S, w)
    theirs = oracle.factorized_angular_linear_adjoint(ga, x, tables, S, w, use_reference=True)
    for a, b in zip(mine, theirs):
        assert np.array_equal(np.asarray(a), np.asarray(b))


@pytest.mark.parametrize("seed", [4, 5])
def test_dag_adjoint_is_the_transpose_of_the_directional_derivative(seed):
    """Real data: <adjoint(g), v> equals <g, J v>, J v from an exact five-point
    stencil (the output is a polynomial of degree <= 4 in the input along v for
    these depths... checked against a small step instead where deeper)."""
    tables, S, D = random_dag(seed, complex_data=False, max_nodes=7)
    rng = np.random.default_rng(200 + seed)
    x = rng.normal(size=(3, S * D))
    v = rng.normal(size=x.shape)
    g = rng.normal(size=oracle.factorized_angular(x, tables, S).shape)
    h = 1e-3
    f = [oracle.factorized_angular(x + k * h * v, tables, S) for k in (-2, -1, 1, 2)]
    jv = (f[0] - 8 * f[1] + 8 * f[2] - f[3]) / (12 * h)
    lhs = float(np.sum(oracle.factorized_angular_adjoint(g, x, tables, S) * v))
    rhs = float(np.sum(g * jv))
    assert abs(lhs - rhs) <= 1e-8 * max(1.0, abs(rhs))


def _fixture():
    with open(GOLDEN) as fh:
        d = json.load(fh)
    D, M, B = int(d["input_dimension"]), int(d["monomial_count"]), int(d["batch_size"])
    return d, np.array(d["monomial_counts"]).reshape(M, D), np.array(d["input"], dtype=np.float64).reshape(B, D)


def test_shared_monomial_fixture_forward_and_adjoint():
    d, counts, x = _fixture()
    out = oracle.symmetric_power_shared_monomial(x, counts, d["output_offsets"], d["coefficient_terms"],
                                                 d["coefficient_values"])
    np.testing.assert_allclose(out.ravel(), d["expected_output"], rtol=1e-15, atol=1e-15)
    gin = oracle.symmetric_power_shared_monomial_adjoint(d["output_adjoint"], x, counts, d["output_offsets"],
                                                         d["coefficient_terms"], d["coefficient_values"])
    np.testing.assert_allclose(gin.ravel(), d["expected_input_adjoint"], rtol=1e-15, atol=1e-15)


def _grouped_from_shared(d, counts):
    """The fixture's table as a grouped (per-output) monomial table: one term
    per coefficient, counts of its monomial, its output index."""
    terms = np.array(d["coefficient_terms"])
    return counts[terms], np.array(d["output_offsets"]), np.array(d["coefficient_outputs"]), \
        np.array(d["coefficient_values"])


def test_monomial_adjoint_on_the_fixture():
    """The grouped monomial table built from the fixture gives the fixture's
    expected output (forward) and expected input adjoint (adjoint)."""
    d, counts, x = _fixture()
    g_counts, offs, idx, vals = _grouped_from_shared(d, counts)
    out = oracle.symmetric_power_monomial(x, g_counts, offs, vals)
    np.testing.assert_allclose(out.ravel(), d["expected_output"], rtol=1e-15, atol=1e-15)
    gin = oracle.symmetric_power_monomial_adjoint(d["output_adjoint"], x, g_counts, idx, vals, len(offs) - 1)
    np.testing.assert_allclose(gin.ravel(), d["expected_input_adjoint"], rtol=1e-15, atol=1e-15)


@needs_ref
def test_monomial_operators_are_the_reference_core_bitwise():
    rng = np.random.default_rng(9)
    B, D, M, O = 7, 5, 11, 4
    counts = rng.integers(0, 3, (M, D))
    x = rng.normal(size=(B, D))
    x[2, 1] = 0.0  # one zero factor
    x[3, 1] = x[3, 3] = 0.0  # two zero factors
    coef_terms = rng.integers(0, M, 17)
    offs = np.array([0, 4, 9, 13, 17])
    vals = rng.normal(size=17)
    a = oracle.symmetric_power_shared_monomial(x, counts, offs, coef_terms, vals)
    assert np.array_equal(a, oracle.symmetric_power_shared_monomial(x, counts, offs, coef_terms, vals,
                                                                    use_reference=True))
    g = rng.normal(size=(B, O))
    a = oracle.symmetric_power_shared_monomial_adjoint(g, x, counts, offs, coef_terms, vals)
    assert np.array_equal(a, oracle.symmetric_power_shared_monomial_adjoint(g, x, counts, offs, coef_terms, vals,
                                                                            use_reference=True))
    idx = np.repeat(np.arange(O), np.diff(offs))
    gc = counts[coef_terms]
    a = oracle.symmetric_power_monomial_adjoint(g, x, gc, idx, vals, O)
    assert np.array_equal(a, oracle.symmetric_power_monomial_adjoint(g, x, gc, idx, vals, O, use_reference=True))


def test_monomial_adjoint_is_the_gradient_of_the_forward():
    rng = np.random.default_rng(10)
    B, D, T, O = 3, 4, 9, 3
    counts = rng.integers(0, 3, (T, D))
    offs = np.array([0, 2, 6, 9])
    idx = np.repeat(np.arange(O), np.diff(offs))
    vals = rng.normal(size=T)
    x = rng.normal(size=(B, D))
    g = rng.normal(size=(B, O))
    gin = oracle.symmetric_power_monomial_adjoint(g, x, counts, idx, vals, O)
    h = 1e-4
    for c in range(D):
        e = np.zeros_like(x)
        e[:, c] = h
        f = [oracle.symmetric_power_monomial(x + k * e, counts, offs, vals) for k in (-2, -1, 1, 2)]
        d = (f[0] - 8 * f[1] + 8 * f[2] - f[3]) / (12 * h)  # exact for degree <= 4
        np.testing.assert_allclose(gin[:, c], np.sum(g * d, axis=1), rtol=1e-9, atol=1e-9)
