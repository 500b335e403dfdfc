"""Symmetric-power monomial ops on the GPU through the reference-shaped mirror.

* ``symmetric_power_shared_monomial_contraction`` and the grouped
  ``symmetric_power_monomial_contraction`` on the reference's fixture
  ``shared_monomial_plan_v1``: expected outputs, and the fixture's
  ``expected_input_adjoint`` from Torch autograd through the library's
  adjoint kernels;
* random tables with zero inputs (the reference's zero-factor rules) against
  the pinned oracle, fp64 at 1e-12 and fp32 at 2e-5.
"""

import json
import os

import numpy as np
import pytest

import oracle
from tests._util import TOL, column_rel_error, flush

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "shared_monomial_plan_v1.json")


def _fixture():
    with open(GOLDEN) as fh:
        d = json.load(fh)
    D, M, B = int(d["input_dimension"]), int(d["monomial_count"]), int(d["batch_size"])
    return d, np.array(d["monomial_counts"], dtype=np.int64).reshape(M, D), \
        np.array(d["input"], dtype=np.float64).reshape(B, D)


def test_shared_and_grouped_contractions_on_the_fixture(gpu):
    flush("monomial contractions on the shared_monomial_plan_v1 fixture")
    import torch

    from ye3t_amd.runtime import symmetric_power_monomial_contraction, symmetric_power_shared_monomial_contraction

    d, counts, x = _fixture()
    g = torch.as_tensor(np.array(d["output_adjoint"], dtype=np.float64).reshape(x.shape[0], -1), device=gpu)
    expect_out = np.array(d["expected_output"], dtype=np.float64)
    expect_adj = np.array(d["expected_input_adjoint"], dtype=np.float64)
    xs = torch.as_tensor(x, device=gpu).requires_grad_(True)
    out = symmetric_power_shared_monomial_contraction(xs, counts, d["output_offsets"], d["coefficient_terms"],
                                                      d["coefficient_outputs"], d["coefficient_values"])
    np.testing.assert_allclose(out.detach().cpu().numpy().ravel(), expect_out, rtol=1e-14, atol=1e-14)
    (gx,) = torch.autograd.grad(out, xs, g)
    np.testing.assert_allclose(gx.cpu().numpy().ravel(), expect_adj, rtol=1e-14, atol=1e-14)
    # the same table grouped per output: one term per coefficient
    terms = np.array(d["coefficient_terms"], dtype=np.int64)
    xg = torch.as_tensor(x, device=gpu).requires_grad_(True)
    out2 = symmetric_power_monomial_contraction(xg, counts[terms], d["output_offsets"], d["coefficient_outputs"],
                                                d["coefficient_values"])
    np.testing.assert_allclose(out2.detach().cpu().numpy().ravel(), expect_out, rtol=1e-14, atol=1e-14)
    (gx2,) = torch.autograd.grad(out2, xg, g)
    np.testing.assert_allclose(gx2.cpu().numpy().ravel(), expect_adj, rtol=1e-14, atol=1e-14)
    # leading dimensions are kept
    x3 = torch.as_tensor(x, device=gpu).reshape(1, *x.shape)
    out3 = symmetric_power_shared_monomial_contraction(x3, counts, d["output_offsets"], d["coefficient_terms"],
                                                       d["coefficient_outputs"], d["coefficient_values"])
    assert tuple(out3.shape) == (1, x.shape[0], 3)


def _random_tables(seed, D=5, M=13, O=6, C=29):
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, 3, (M, D))
    per = np.diff(np.sort(np.concatenate([[0, C], rng.integers(0, C, O - 1)])))
    offs = np.concatenate([[0], np.cumsum(per)])
    terms = rng.integers(0, M, C)
    outs = np.repeat(np.arange(O), per)
    vals = rng.normal(size=C)
    return counts, offs, terms, outs, vals


@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_random_tables_against_the_oracle(gpu, dtype):
    flush(f"monomial contractions, random tables, {dtype}")
    import torch

    from ye3t_amd.runtime import symmetric_power_monomial_contraction, symmetric_power_shared_monomial_contraction

    counts, offs, terms, outs, vals = _random_tables(5)
    rng = np.random.default_rng(6)
    B = 300
    x = rng.normal(size=(B, counts.shape[1]))
    x[3, 2] = 0.0  # one zero factor
    x[7, 1] = x[7, 4] = 0.0  # two zero factors
    x[9, :] = 0.0
    real = torch.float64 if dtype == "f64" else torch.float32
    xd = torch.as_tensor(x, dtype=real, device=gpu)
    xr = xd.double().cpu().numpy()
    vr = torch.as_tensor(vals, dtype=real).double().numpy()
    g = rng.normal(size=(B, len(offs) - 1))
    gd = torch.as_tensor(g, dtype=real, device=gpu)
    gr = gd.double().cpu().numpy()
    xs = xd.clone().requires_grad_(True)
    out = symmetric_power_shared_monomial_contraction(xs, counts, offs, terms, outs, vals)
    ref = oracle.symmetric_power_shared_monomial(xr, counts, offs, terms, vr)
    (gx,) = torch.autograd.grad(out, xs, gd)
    gref = oracle.symmetric_power_shared_monomial_adjoint(gr, xr, counts, offs, terms, vr)
    xg = xd.clone().requires_grad_(True)
    out2 = symmetric_power_monomial_contraction(xg, counts[terms], offs, outs, vals)
    (gx2,) = torch.autograd.grad(out2, xg, gd)
    gref2 = oracle.symmetric_power_monomial_adjoint(gr, xr, counts[terms], outs, vr, len(offs) - 1)
    errs = [column_rel_error(out.detach().cpu().numpy(), ref), column_rel_error(gx.cpu().numpy(), gref),
            column_rel_error(out2.detach().cpu().numpy(), ref), column_rel_error(gx2.cpu().numpy(), gref2)]
    flush("  " + " ".join(f"{e:.2e}" for e in errs))
    assert max(errs) < TOL[dtype]
    assert np.allclose(gref, gref2)  # the two forms are one contraction


def test_inconsistent_tables_are_refused(gpu):
    import torch

    from ye3t_amd.runtime import symmetric_power_monomial_contraction, symmetric_power_shared_monomial_contraction

    counts, offs, terms, outs, vals = _random_tables(7)
    x = torch.zeros((4, counts.shape[1]), dtype=torch.float64, device=gpu)
    bad_outs = outs.copy()
    bad_outs[0] = len(offs) - 2
    with pytest.raises(ValueError, match="output_indices"):
        symmetric_power_monomial_contraction(x, counts[terms], offs, bad_outs, vals)
    bad_terms = terms.copy()
    bad_terms[3] = counts.shape[0]
    with pytest.raises(ValueError, match="coefficient_terms"):
        symmetric_power_shared_monomial_contraction(x, counts, offs, bad_terms, outs, vals)
    with pytest.raises(NotImplementedError, match="reference"):
        symmetric_power_monomial_contraction(x, counts[terms], offs, outs, vals, backend="reference")


def _sparse_tables(seed, D=6, M=11, O=5, C=23):
    """Random sparse supports (a component may appear twice in one support)."""
    rng = np.random.default_rng(seed)
    toff, comp, ex = [0], [], []
    for _ in range(M):
        for _ in range(int(rng.integers(1, 4))):
            comp.append(int(rng.integers(0, D)))
            ex.append(int(rng.integers(1, 3)))
        toff.append(len(comp))
    per = np.diff(np.sort(np.concatenate([[0, C], rng.integers(0, C, O - 1)])))
    offs = np.concatenate([[0], np.cumsum(per)])
    terms = rng.integers(0, M, C)
    outs = np.repeat(np.arange(O), per)
    return (np.array(toff), np.array(comp), np.array(ex), offs, terms, outs, rng.normal(size=C))


@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_sparse_shared_monomials_against_the_oracle(gpu, dtype):
    """Forward, adjoint (autograd through the mirror) and double backward
    (autograd of the Torch adjoint operator) against the pinned oracle, with
    rows holding one, two and all-zero factors."""
    flush(f"sparse shared monomials, random tables, {dtype}")
    import torch

    from ye3t_amd.runtime import symmetric_power_shared_sparse_monomial_contraction, torch_ops

    toff, comp, ex, offs, terms, outs, vals = _sparse_tables(11)
    rng = np.random.default_rng(12)
    B, D, O = 257, 6, len(offs) - 1
    x = rng.normal(size=(B, D))
    x[3, 2] = 0.0
    x[7, 1] = x[7, 4] = 0.0
    x[9, :] = 0.0
    real = torch.float64 if dtype == "f64" else torch.float32
    xd = torch.as_tensor(x, dtype=real, device=gpu)
    xr = xd.double().cpu().numpy()
    vr = torch.as_tensor(vals, dtype=real).double().numpy()
    gd = torch.as_tensor(rng.normal(size=(B, O)), dtype=real, device=gpu)
    gr = gd.double().cpu().numpy()
    vd = torch.as_tensor(rng.normal(size=(B, D)), dtype=real, device=gpu)
    tables = (toff, comp, ex, offs, terms, outs, vals)
    xs = xd.clone().requires_grad_(True)
    out = symmetric_power_shared_sparse_monomial_contraction(xs, *tables)
    (gx,) = torch.autograd.grad(out, xs, gd)
    ref = oracle.symmetric_power_shared_sparse_monomial(xr, toff, comp, ex, offs, terms, vr)
    gref = oracle.symmetric_power_shared_sparse_monomial_adjoint(gr, xr, toff, comp, ex, offs, terms, vr)
    # the Torch operators: the adjoint is differentiable through the double backward
    torch_ops.register()
    ops = torch.ops.ye3t_runtime
    dev_tables = [torch.as_tensor(a, dtype=torch.int64, device=gpu) for a in (toff, comp, ex, offs, terms, outs)]
    dev_tables.append(torch.as_tensor(vals, dtype=real, device=gpu))
    g_req = gd.clone().requires_grad_(True)
    x_req = xd.clone().requires_grad_(True)
    adj = ops.symmetric_power_shared_sparse_monomial_adjoint(g_req, x_req, *dev_tables)
    ot, it = torch.autograd.grad(adj, (g_req, x_req), vd)
    ot_ref, it_ref = oracle.symmetric_power_shared_sparse_monomial_double_backward(
        vd.double().cpu().numpy(), gr, xr, toff, comp, ex, offs, terms, vr)
    errs = [column_rel_error(out.detach().cpu().numpy(), ref), column_rel_error(gx.cpu().numpy(), gref),
            column_rel_error(adj.detach().cpu().numpy(), gref), column_rel_error(ot.cpu().numpy(), ot_ref),
            column_rel_error(it.cpu().numpy(), it_ref)]
    flush("  " + " ".join(f"{e:.2e}" for e in errs))
    assert max(errs) < TOL[dtype]
    # the operators pass Torch's operator checks (schema, fake, autograd registration)
    if dtype == "f64":
        for op, args in ((ops.symmetric_power_shared_sparse_monomial.default, (xd, *dev_tables)),
                         (ops.symmetric_power_shared_sparse_monomial_adjoint.default, (gd, xd, *dev_tables)),
                         (ops.symmetric_power_shared_sparse_monomial_double_backward.default,
                          (vd, gd, xd, *dev_tables))):
            result = torch.library.opcheck(op, args, raise_exception=False)
            assert all(v == "SUCCESS" for v in result.values()), result


def test_sparse_tables_are_refused_on_bad_indices(gpu):
    import torch

    from ye3t_amd.runtime import symmetric_power_shared_sparse_monomial_contraction

    toff, comp, ex, offs, terms, outs, vals = _sparse_tables(13)
    x = torch.zeros((4, 6), dtype=torch.float64, device=gpu)
    bad = comp.copy()
    bad[0] = 6
    with pytest.raises(ValueError, match="term_components"):
        symmetric_power_shared_sparse_monomial_contraction(x, toff, bad, ex, offs, terms, outs, vals)
    bad = ex.copy()
    bad[1] = 0
    with pytest.raises(ValueError, match="positive"):
        symmetric_power_shared_sparse_monomial_contraction(x, toff, comp, bad, offs, terms, outs, vals)
    with pytest.raises(ValueError, match="equal length"):
        symmetric_power_shared_sparse_monomial_contraction(x, toff, comp[:-1], ex, offs, terms, outs, vals)
