"""Segmented factorized-angular DAGs: several plans in one op (CPU checks).

The reference's ``factorized_angular_segmented`` (schema
``execution_plan_torch.cpp:7666-7679``, CPU core
``ye3t_runtime_core.cpp:6977-7070``) runs one DAG per segment over disjoint
column ranges of the packed input and the output, with explicit per-root
projection metadata.  Checked here:

* the oracle's restatement against the reference's compiled core
  (``oracle/_ref``), bit for bit, on random segments whose roots have any
  dimension and project onto random projection intervals into shuffled output
  blocks, real and complex, forward and adjoint;
* on the four reference-written plans of ``tests/golden/
  execution_plan_factorized_v1.json`` grouped as the reference's segmented
  group groups them: the segmented result is the concatenation of the
  single-plan results (bit for bit) and matches the reference branch's
  outputs (1e-12);
* the adjoint against an exact five-point directional derivative;
* the HIP library's host validation refuses planted table errors (no device
  call is reached).
"""

import types

import numpy as np
import pytest

import oracle
from tests._dag import SEGMENT_KEYS, random_segmented
from tests.test_execution_plan_loader import DATA, _arr, _packed, _unpack
from ye3t_amd.runtime.execution_plan import ExecutionPlan


def _fixture_members(cplx):
    members = []
    for name in sorted(DATA["plans"]):
        rec = DATA["plans"][name]
        tables, meta = ExecutionPlan.from_json(rec["plan_json"]).factorized_angular_buffers(complex_values=cplx)
        members.append((name, types.SimpleNamespace(
            **tables, source_dimension=meta["source_dimension"], input_dimension=meta["input_dimension"],
            workspace_dimension=meta["workspace_dimension"], output_dimension=meta["output_dimension"],
            magnetic_dimension=meta["magnetic_dimension"]), tables, meta))
    return members


@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_segmented_oracle_matches_reference_core(seed, cplx):
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    tables, (D, _S, _W, F) = random_segmented(seed, complex_data=cplx, count=int(2 + seed % 3))
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(5, D)) + (1j * rng.normal(size=(5, D)) if cplx else 0)
    g = rng.normal(size=(5, F)) + (1j * rng.normal(size=(5, F)) if cplx else 0)
    out = oracle.factorized_angular_segmented(x, tables, F)
    ref = oracle.factorized_angular_segmented(x, tables, F, use_reference=True)
    assert np.array_equal(out, ref)
    adj = oracle.factorized_angular_segmented_adjoint(g, x, tables)
    adj_ref = oracle.factorized_angular_segmented_adjoint(g, x, tables, use_reference=True)
    assert np.array_equal(adj, adj_ref)
    assert np.any(out != 0) and np.any(adj != 0)


@pytest.mark.parametrize("dtype", ["float64", "complex128"])
def test_segmented_fixture_plans_are_the_concatenation(dtype):
    from ye3t_amd.runtime.dag import segmented_tables

    cplx = dtype == "complex128"
    members = _fixture_members(cplx)
    tables, (D, S, W, F) = segmented_tables([m for _, m, _, _ in members])
    cases = {c["plan"]: c for c in DATA["cases"] if c["dtype"] == dtype}
    packed = [_packed(cases[name], meta["source_dimension"]) for name, _, _, meta in members]
    x = np.concatenate(packed, axis=1)
    assert x.shape[1] == D and S == sum(m.source_dimension for _, m, _, _ in members)
    out = oracle.factorized_angular_segmented(x, tables, F)
    pieces = [oracle.factorized_angular(p, t, meta["source_dimension"]) for p, (_, _, t, meta) in zip(packed, members)]
    assert np.array_equal(out, np.concatenate(pieces, axis=1))
    cursor = 0
    gs = []
    for (name, m, t, meta), piece in zip(members, pieces):
        expected = _arr(cases[name]["output"], dtype).reshape(piece.shape)
        assert np.max(np.abs(out[:, cursor:cursor + piece.shape[1]] - expected)) <= 1e-12
        gs.append(_arr(cases[name]["output_cotangent"], dtype).reshape(piece.shape))
        cursor += piece.shape[1]
    g = np.concatenate(gs, axis=1)
    adj = oracle.factorized_angular_segmented_adjoint(g, x, tables)
    plain = [oracle.factorized_angular_adjoint(gg, p, t, meta["source_dimension"])
             for gg, p, (_, _, t, meta) in zip(gs, packed, members)]
    assert np.array_equal(adj, np.concatenate(plain, axis=1))
    col = 0
    for (name, m, t, meta), p in zip(members, packed):
        for a, e in zip(_unpack(adj[:, col:col + p.shape[1]], cases[name], meta["source_dimension"]),
                        cases[name]["slot_adjoints"]):
            assert np.max(np.abs(a - _arr(e, dtype))) <= 1e-12
        col += p.shape[1]


def test_segmented_adjoint_is_the_directional_derivative():
    tables, (D, _S, _W, F) = random_segmented(11, complex_data=False, count=3)
    rng = np.random.default_rng(5)
    x, dx, g = rng.normal(size=(4, D)), rng.normal(size=(4, D)), rng.normal(size=(4, F))
    f = lambda t: float(np.sum(g * oracle.factorized_angular_segmented(x + t * dx, tables, F)))  # noqa: E731
    h = 1e-3  # five-point stencil: truncation O(h^4), rounding O(eps / h)
    fd = (f(-2 * h) - 8 * f(-h) + 8 * f(h) - f(2 * h)) / (12 * h)
    adj = float(np.sum(oracle.factorized_angular_segmented_adjoint(g, x, tables) * dx))
    assert abs(fd - adj) <= 1e-8 * max(1.0, abs(adj))
    # a planted mistake in the oracle's adjoint (one segment's cotangent block
    # shifted by one column) is caught by the same check
    g2 = g.copy()
    g2[:, 1:] = g[:, :-1]
    bad = float(np.sum(oracle.factorized_angular_segmented_adjoint(g2, x, tables) * dx))
    assert abs(fd - bad) > 1e-6 * max(1.0, abs(adj))


def _handle(tables, dims, dtype="float64"):
    import torch

    from ye3t_amd.runtime import native

    dt = {"float64": torch.float64, "complex128": torch.complex128}[dtype]
    return native.FactorizedAngularSegmentedPlanHandle(tables, *dims, dt)


@pytest.mark.parametrize("mistake,message", [
    ("input_offsets", "partition packed input"),
    ("root_overlap", "root output"),
    ("child_order", "children must precede"),
    ("coefficient_row", "coefficient row"),
    ("projection_interval", "root projection interval"),
    ("total_sources", "total_source_count"),
    ("workspace", "workspace dimension"),
])
def test_segmented_validation_refuses_planted_errors(mistake, message):
    from ye3t_amd.runtime import native

    if not native.available():
        pytest.skip("HIP library not built")
    tables, dims = random_segmented(7, complex_data=False, count=3)
    dims = list(dims)
    t = {k: v.copy() for k, v in tables.items()}
    if mistake == "input_offsets":
        t["segment_input_offsets"][1] += 1
    elif mistake == "root_overlap":
        r0, r1 = t["segment_root_offsets"][0], t["segment_root_offsets"][1]
        if r1 - r0 < 2:
            t["root_output_offsets"][r0] += 1
        else:
            t["root_output_offsets"][r0 + 1] = t["root_output_offsets"][r0]
    elif mistake == "child_order":
        n0, n1 = t["segment_node_offsets"][0], t["segment_node_offsets"][1]
        merge = next(n for n in range(n0, n1) if t["node_leaf_offsets"][n] < 0)
        t["node_left"][merge] = merge - n0
    elif mistake == "coefficient_row":
        t["coefficient_rows"][0] = 10 ** 6
    elif mistake == "projection_interval":
        t["root_projection_dimensions"][0] += t["segment_projection_dimensions"][0]
    elif mistake == "total_sources":
        dims[1] += 1
    elif mistake == "workspace":
        dims[2] += 1
    with pytest.raises(RuntimeError, match=message):
        _handle(t, dims)
