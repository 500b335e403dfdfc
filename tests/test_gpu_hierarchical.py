"""The hierarchical repeated-block runtime on the GPU against the reference's values.

``tests/golden/hierarchical_v1.json`` holds the reference Torch branch's
forward, gradient of ``sum |out|^2`` and Hessian-vector product (complex128, on
seeded float64 inputs) for the plans of the reference's
``tests/test_hierarchical_runtime.py`` (v1 one- and two-block plans, v2
three-block plans, ranks 3 to 12) and for module groups (shared block powers,
shared-monomial power evaluation).  Here the block powers run on the library's
complex sparse shared-monomial kernels (forward, adjoint, double backward) and
a group's destination-segmented schedule on the segmented factorized-angular
kernel; the bars are the reference tests' own (1e-12 forward, 1e-10 gradient
and HVP).  The complex sparse kernels are also checked directly against a
numpy restatement of the reference kernels' conjugation rules.
"""

import json
import os

import numpy as np
import pytest

from tests._util import flush

pytestmark = pytest.mark.gpu
FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "hierarchical_v1.json")


def _fixture():
    with open(FIXTURE) as fh:
        return json.load(fh)


def _complex(pairs):
    a = np.asarray(pairs, dtype=np.float64)
    return a[..., 0] + 1j * a[..., 1]


def _close(actual, expected, tol):
    import torch

    e = torch.as_tensor(expected, device=actual.device)
    assert actual.shape == e.shape, (tuple(actual.shape), tuple(e.shape))
    assert torch.allclose(actual, e.to(actual.dtype), atol=tol, rtol=tol), \
        float((actual - e.to(actual.dtype)).abs().max())


def _derivatives(out, inputs, direction):
    import torch

    grads = torch.autograd.grad(out.abs().square().sum(), inputs, create_graph=True)
    hvp = torch.autograd.grad(sum((g * d).sum() for g, d in zip(grads, direction)), inputs)
    return grads, hvp


CASES = [c["name"] for c in _fixture()["cases"]]


@pytest.mark.parametrize("name", CASES)
def test_module_matches_the_reference(gpu, name):
    import torch

    from ye3t_amd.runtime.hierarchical import YE3THierarchicalRepeatedBlockModule

    case = next(c for c in _fixture()["cases"] if c["name"] == name)
    flush(f"hierarchical module {name}")
    module = YE3THierarchicalRepeatedBlockModule(case["plan"], dtype=torch.complex128, device=gpu)
    facts = case["facts"]
    for key in ("block_count", "route_count", "channel_count", "tableau_count", "magnetic_count",
                "output_dimension", "target_L", "lr_multiplicity", "hierarchical_schema"):
        assert getattr(module, key) == facts[key], key
    inputs = tuple(torch.tensor(v, dtype=torch.float64, device=gpu, requires_grad=True) for v in case["inputs"])
    out = module(*inputs)
    _close(out, _complex(case["output"]), 1e-12)
    direction = tuple(torch.tensor(d, dtype=torch.float64, device=gpu) for d in case["direction"])
    grads, hvp = _derivatives(out, inputs, direction)
    for got, want in zip(grads, case["gradient"]):
        _close(got, np.asarray(want), 1e-10)
    for got, want in zip(hvp, case["hvp"]):
        _close(got, np.asarray(want), 1e-10)
    ro = case["readout"]
    y = module.linear_readout(tuple(i.detach() for i in inputs), torch.tensor(ro["weight"], dtype=torch.float64, device=gpu),
                               ro["bias"])
    _close(y, _complex(ro["output"]), 1e-12)
    report = module.runtime_report()
    assert report["supports_autograd_vjp_hvp"] and report["runtime_path_discovery"] is False
    assert report["last_backend"].startswith("shared_monomial_then_")
    want = [dict(r, powers=tuple(r["powers"])) for r in case["report"]["block_power_table_reports"]]
    assert [dict(r) for r in report["block_power_table_reports"]] == want


GROUPS = list(range(len(_fixture()["groups"])))


@pytest.mark.parametrize("index", GROUPS)
@pytest.mark.parametrize("parent", ["reference", "destination_segmented"])
def test_group_matches_the_reference(gpu, index, parent):
    import torch

    from ye3t_amd.runtime.hierarchical import (YE3THierarchicalRepeatedBlockModule,
                                               YE3THierarchicalRepeatedBlockModuleGroup)

    fx = _fixture()
    group_fx = fx["groups"][index]
    cases = {c["name"]: c for c in fx["cases"]}
    flush(f"hierarchical group {group_fx['members']} powers {group_fx['block_power_policy']} parent {parent}")
    modules = tuple(YE3THierarchicalRepeatedBlockModule(cases[m]["plan"], dtype=torch.complex128, device=gpu)
                    for m in group_fx["members"])
    group = YE3THierarchicalRepeatedBlockModuleGroup(modules, group_fx["bindings"], parent_execution_policy=parent,
                                                     block_power_execution_policy=group_fx["block_power_policy"])
    inputs = tuple(torch.tensor(v, dtype=torch.float64, device=gpu, requires_grad=True)
                   for v in group_fx["inputs"])
    out = group.forward_packed(inputs)
    _close(out, _complex(group_fx["output"]), 1e-12)
    direction = tuple(torch.tensor(d, dtype=torch.float64, device=gpu) for d in group_fx["direction"])
    grads, hvp = _derivatives(out, inputs, direction)
    for got, want in zip(grads, group_fx["gradient"]):
        _close(got, np.asarray(want), 1e-10)
    for got, want in zip(hvp, group_fx["hvp"]):
        _close(got, np.asarray(want), 1e-10)
    report = group.runtime_report()
    for key, value in group_fx["report_counts"].items():
        assert report[key] == value, key
    assert report["destination_native_enabled"] is (parent == "destination_segmented")
    if parent == "destination_segmented":
        assert report["destination_native_call_count"] == 1 and report["destination_segment_reports"]
        # without gradients the forward is the segmented kernel alone
        with torch.no_grad():
            _close(group.forward_packed(tuple(i.detach() for i in inputs)), _complex(group_fx["output"]), 1e-12)
    logical = group.forward(tuple(i.detach() for i in inputs))
    assert len(logical) == len(modules)
    flat = torch.cat([o.reshape(o.shape[0], -1) for o in logical], dim=1)
    _close(flat, _complex(group_fx["output"]), 1e-12)


def _np_sparse(x, toff, comp, ex, offs, terms, vals):
    """Forward and adjoint of a sparse shared monomial table in numpy: the
    reference kernels' rules (adjoint g conj(c) conj(dm/dx_c); inputs without
    zeros here)."""
    B, D = x.shape
    O = len(offs) - 1
    out = np.zeros((B, O), dtype=complex)
    jac = np.zeros((B, O, D), dtype=complex)
    for o in range(O):
        for k in range(offs[o], offs[o + 1]):
            t = terms[k]
            m = np.ones(B, dtype=complex)
            for q in range(toff[t], toff[t + 1]):
                m = m * x[:, comp[q]] ** ex[q]
            out[:, o] += vals[k] * m
            for q in range(toff[t], toff[t + 1]):
                jac[:, o, comp[q]] += vals[k] * ex[q] * m / x[:, comp[q]]
    return out, jac


def test_complex_sparse_monomial_kernels(gpu):
    import torch

    from ye3t_amd.runtime import native

    rng = np.random.default_rng(71)
    B, D = 6, 4
    toff, comp, ex = [0, 2, 3, 6], [0, 2, 1, 0, 1, 3], [2, 1, 3, 1, 1, 2]
    offs, terms = [0, 2, 4, 5], [0, 2, 1, 2, 0]
    vals = rng.normal(size=5) + 1j * rng.normal(size=5)
    x = rng.normal(size=(B, D)) + 1j * rng.normal(size=(B, D))
    table = native.SparseMonomialTable(D, toff, comp, ex, offs, terms, [0, 0, 1, 1, 2], vals, gpu,
                                       torch.complex128)
    xt = torch.tensor(x, device=gpu)
    want, jac = _np_sparse(x, toff, comp, ex, offs, terms, vals)
    got = table.forward(xt).cpu().numpy()
    assert np.allclose(got, want, atol=1e-13, rtol=1e-13)
    g = rng.normal(size=(B, 3)) + 1j * rng.normal(size=(B, 3))
    adj = table.adjoint(torch.tensor(g, device=gpu), xt).cpu().numpy()
    assert np.allclose(adj, np.einsum("bo,bod->bd", g, np.conj(jac)), atol=1e-13, rtol=1e-13)
    # double backward: output tangent = J v; input tangent = sum g conj(c)
    # conj(H v), the five-point derivative of the adjoint along v
    v = rng.normal(size=(B, D)) + 1j * rng.normal(size=(B, D))
    out_t, in_t = table.double_backward(torch.tensor(v, device=gpu), torch.tensor(g, device=gpu), xt)
    assert np.allclose(out_t.cpu().numpy(), np.einsum("bod,bd->bo", jac, v), atol=1e-12, rtol=1e-12)

    def adj_at(s):
        return table.adjoint(torch.tensor(g, device=gpu), torch.tensor(x + s * v, device=gpu)).cpu().numpy()

    h = 1e-3
    fd = (-adj_at(2 * h) + 8 * adj_at(h) - 8 * adj_at(-h) + adj_at(-2 * h)) / (12 * h)
    assert np.allclose(in_t.cpu().numpy(), fd, atol=1e-8, rtol=1e-8)
