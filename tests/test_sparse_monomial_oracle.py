"""Oracle of the sparse shared-monomial operators, pinned without the reference's CUDA.

The reference implements ``symmetric_power_shared_sparse_monomial`` and its
adjoint and double backward only in CUDA (``execution_plan_cuda.cu:5720-5955,
11012-11330``), so nothing compiles here to compare with.  The restatement
(``oracle/ye3t_oracle_dag.c``) is pinned instead by:

* the dense shared-monomial operators, which are bit-exact against the
  reference's CPU core (``tests/test_oracle_dag.py``) and its fixture: a sparse
  table built from dense exponent rows (supports in component order, optionally
  with a component split into two entries) gives the same bits forward and
  backward, including rows with exact zeros (the zero-degree rules);
* five-point directional derivatives: the double backward's output tangent is
  the forward's derivative along the tangent, and its input tangent is the
  adjoint's derivative along the tangent at fixed output adjoint (the monomials
  are polynomials of degree <= 4 here, so the stencil is exact up to rounding),
  at generic points and at points with one or two exact zeros.
"""

import numpy as np
import pytest

import oracle


def _dense_table(rng, D=5, M=7, O=4, max_degree=4):
    counts = np.zeros((M, D), dtype=np.int64)
    for t in range(M):
        deg = int(rng.integers(1, max_degree + 1))
        for _ in range(deg):
            counts[t, int(rng.integers(0, D))] += 1
    per_out = rng.integers(1, 4, size=O)
    offs = np.concatenate([[0], np.cumsum(per_out)]).astype(np.int64)
    terms = rng.integers(0, M, size=int(offs[-1])).astype(np.int64)
    vals = rng.normal(size=int(offs[-1]))
    return counts, offs, terms, vals


def _sparse_from_dense(counts, split=False):
    toff, comp, ex = [0], [], []
    for row in counts:
        for c, e in enumerate(row):
            if e == 0:
                continue
            if split and e >= 2:
                comp += [c, c]
                ex += [e - 1, 1]
            else:
                comp.append(c)
                ex.append(int(e))
        toff.append(len(comp))
    return (np.array(toff, dtype=np.int64), np.array(comp, dtype=np.int64), np.array(ex, dtype=np.int64))


def _inputs(rng, B, D, zeros):
    x = rng.normal(size=(B, D))
    for b in range(B):
        for _ in range(zeros if b % 3 else 0):
            x[b, int(rng.integers(0, D))] = 0.0
    return x


@pytest.mark.parametrize("seed", range(4))
def test_sparse_equals_the_dense_shared_form_bitwise(seed):
    rng = np.random.default_rng(seed)
    counts, offs, terms, vals = _dense_table(rng)
    B, D, O = 40, counts.shape[1], offs.shape[0] - 1
    x = _inputs(rng, B, D, zeros=1 + seed % 2)
    g = rng.normal(size=(B, O))
    toff, comp, ex = _sparse_from_dense(counts)
    dense = oracle.symmetric_power_shared_monomial(x, counts, offs, terms, vals)
    sparse = oracle.symmetric_power_shared_sparse_monomial(x, toff, comp, ex, offs, terms, vals)
    assert np.array_equal(dense, sparse)
    dadj = oracle.symmetric_power_shared_monomial_adjoint(g, x, counts, offs, terms, vals)
    sadj = oracle.symmetric_power_shared_sparse_monomial_adjoint(g, x, toff, comp, ex, offs, terms, vals)
    assert np.array_equal(dadj, sadj)
    # a repeated component in one support is the same monomial
    toff2, comp2, ex2 = _sparse_from_dense(counts, split=True)
    assert comp2.size > comp.size
    np.testing.assert_allclose(oracle.symmetric_power_shared_sparse_monomial(x, toff2, comp2, ex2, offs, terms, vals),
                               dense, rtol=1e-13, atol=1e-13)


def _five_point(f, h=1e-3):
    return (-f(2 * h) + 8 * f(h) - 8 * f(-h) + f(-2 * h)) / (12 * h)


@pytest.mark.parametrize("seed,zeros", [(0, 0), (1, 0), (2, 1), (3, 2), (4, 1)])
def test_double_backward_is_the_derivative_of_forward_and_adjoint(seed, zeros):
    rng = np.random.default_rng(100 + seed)
    counts, offs, terms, vals = _dense_table(rng, max_degree=4)
    toff, comp, ex = _sparse_from_dense(counts, split=bool(seed % 2))
    B, D, O = 24, counts.shape[1], offs.shape[0] - 1
    x = _inputs(rng, B, D, zeros)
    v = rng.normal(size=(B, D))
    g = rng.normal(size=(B, O))
    ot, it = oracle.symmetric_power_shared_sparse_monomial_double_backward(v, g, x, toff, comp, ex, offs, terms, vals)
    fwd = lambda s: oracle.symmetric_power_shared_sparse_monomial(x + s * v, toff, comp, ex, offs, terms, vals)  # noqa: E731
    adj = lambda s: oracle.symmetric_power_shared_sparse_monomial_adjoint(  # noqa: E731
        g, x + s * v, toff, comp, ex, offs, terms, vals)
    ot_fd, it_fd = _five_point(fwd), _five_point(adj)
    assert np.max(np.abs(ot - ot_fd)) <= 1e-8 * max(1.0, np.max(np.abs(ot_fd)))
    assert np.max(np.abs(it - it_fd)) <= 1e-8 * max(1.0, np.max(np.abs(it_fd)))
    # not a vacuous check: the tangents carry signal
    assert np.max(np.abs(ot)) > 1e-3 and np.max(np.abs(it)) > 1e-3


def test_zero_degree_rules_at_exact_zeros():
    """x^2 y at x = 0: no gradient (degree 2), Hessian x-x entry 2 y; x y at
    x = 0: cofactor y to x, cross terms of the Hessian."""
    toff = np.array([0, 2, 4], dtype=np.int64)
    comp = np.array([0, 1, 0, 1], dtype=np.int64)
    ex = np.array([2, 1, 1, 1], dtype=np.int64)
    offs = np.array([0, 1, 2], dtype=np.int64)
    terms = np.array([0, 1], dtype=np.int64)
    vals = np.array([1.0, 1.0])
    x = np.array([[0.0, 3.0]])
    g = np.array([[1.0, 1.0]])
    v = np.array([[0.5, 2.0]])
    assert np.array_equal(oracle.symmetric_power_shared_sparse_monomial(x, toff, comp, ex, offs, terms, vals),
                          [[0.0, 0.0]])
    adj = oracle.symmetric_power_shared_sparse_monomial_adjoint(g, x, toff, comp, ex, offs, terms, vals)
    assert np.array_equal(adj, [[3.0, 0.0]])  # d(x^2 y) = 0; d(x y)/dx = y = 3
    ot, it = oracle.symmetric_power_shared_sparse_monomial_double_backward(v, g, x, toff, comp, ex, offs, terms, vals)
    # directional derivatives: x^2 y -> 0, x y -> y v_x = 1.5
    assert np.array_equal(ot, [[0.0, 1.5]])
    # Hessians along v: x^2 y -> (2 y v_x, 0) = (3, 0); x y -> (v_y, v_x) = (2, 0.5)
    assert np.array_equal(it, [[5.0, 0.5]])
