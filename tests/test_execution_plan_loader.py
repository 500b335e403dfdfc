"""The execution-plan loader against documents the reference wrote.

``tests/golden/execution_plan_factorized_v1.json`` holds four factorized-angular
plans built by the reference's own native-test helpers and serialized by its
``to_json``, with their hashes, the reference's ``_factorized_plan_buffers`` of
each, and the reference Torch branch's forward / adjoint / linear readout on
seeded slots (``tests/golden/make_execution_plan_fixtures.py``).  Checked here:

* ``from_json`` reproduces ``plan_hash`` and ``coefficient_hash``; ``to_json``
  rewrites the document byte for byte; the round trip keeps the hash
  (``scalar_ace_export.py:10-19``);
* the derived tables equal the reference's buffers exactly, and the subtree
  identity hashes match;
* the pinned oracle run on those tables reproduces the reference branch's
  outputs and gradients (1e-12), so the tables mean what the reference means;
* planted mistakes (an edited coefficient, an edited provenance field, a node
  out of topological order, a dangling table id) are refused; the v1 schema
  migrates as the reference's ``from_dict`` does and v3 is refused.
"""

import copy
import json
import os

import numpy as np
import pytest

import oracle
from ye3t_amd.runtime.execution_plan import (EXECUTION_PLAN_LEGACY_SCHEMA, EXECUTION_PLAN_SCHEMA, ExecutionPlan,
                                             canonical_json, stable_hash)

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "execution_plan_factorized_v1.json")
INT_TABLES = ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
              "node_coefficient_offsets", "coefficient_rows", "coefficient_columns", "root_nodes")


def _data():
    with open(FIXTURE) as f:
        return json.load(f)


DATA = _data()
PLANS = sorted(DATA["plans"])


def _c(pairs):
    a = np.asarray(pairs, dtype=np.float64)
    return a[..., 0] + 1j * a[..., 1]


def _arr(values, dtype):
    a = np.asarray(values, dtype=np.float64)
    return a[..., 0] + 1j * a[..., 1] if dtype == "complex128" else a


def _packed(case, source_dimension):
    slots = [_arr(s, case["dtype"]) for s in case["slots"]]
    if source_dimension == 1:
        slots = [s[:, None, :] for s in slots]
    x = np.concatenate(slots, axis=-1)
    return x.reshape(x.shape[0], -1)


def _unpack(adj, case, source_dimension):
    B = adj.shape[0]
    dims = [2 * L + 1 for L in case["input_Ls"]]
    adj = adj.reshape(B, source_dimension, sum(dims))
    out, o = [], 0
    for d in dims:
        part = adj[:, :, o:o + d]
        out.append(part[:, 0, :] if source_dimension == 1 else part)
        o += d
    return out


@pytest.mark.parametrize("name", PLANS)
def test_reference_document_hash_and_round_trip(name):
    rec = DATA["plans"][name]
    plan = ExecutionPlan.from_json(rec["plan_json"])
    assert plan.plan_hash == rec["plan_hash"]
    assert plan.coefficient_hash == rec["coefficient_hash"]
    text = plan.to_json(indent=2) + "\n"
    assert text == rec["plan_json"]
    assert ExecutionPlan.from_json(text).plan_hash == plan.plan_hash
    # the hash is SHA-256 of the compact sorted JSON of the payload without plan_hash
    payload = json.loads(rec["plan_json"])
    del payload["plan_hash"]
    import hashlib

    assert hashlib.sha256(json.dumps(payload, sort_keys=True, separators=(",", ":")).encode()).hexdigest() == \
        rec["plan_hash"]
    assert stable_hash(payload) == rec["plan_hash"]


@pytest.mark.parametrize("name", PLANS)
def test_reference_buffers_and_subtree_identity(name):
    rec = DATA["plans"][name]
    plan = ExecutionPlan.from_json(rec["plan_json"])
    tables, meta = plan.factorized_angular_buffers(rec["factorized_angular_plan_id"])
    ref = rec["buffers"]
    for k in INT_TABLES:
        assert tables[k].tolist() == ref[k], k
    assert np.array_equal(tables["coefficient_values"], _c(ref["coefficient_values"]))
    assert np.array_equal(tables["projection_values"], _c(ref["projection_values"]))
    for k in ("input_dimension", "source_dimension", "workspace_dimension", "output_dimension",
              "logical_channel_tableau_dimension", "magnetic_dimension", "reference_dense_synthesis_element_count"):
        assert meta[k] == ref[k], k
    assert list(meta["node_operator_hashes"]) == ref["node_operator_hashes"]
    assert list(meta["node_subtree_hashes"]) == ref["node_subtree_hashes"]
    real_tables, _ = plan.factorized_angular_buffers(complex_values=False)
    assert real_tables["coefficient_values"].dtype == np.float64
    assert np.array_equal(real_tables["coefficient_values"], tables["coefficient_values"].real)


@pytest.mark.parametrize("case", DATA["cases"], ids=lambda c: f"{c['plan']}-{c['dtype']}")
def test_oracle_on_loaded_tables_reproduces_reference_branch(case):
    rec = DATA["plans"][case["plan"]]
    plan = ExecutionPlan.from_json(rec["plan_json"])
    tables, meta = plan.factorized_angular_buffers(complex_values=case["dtype"] == "complex128")
    S = meta["source_dimension"]
    x = _packed(case, S)
    out = oracle.factorized_angular(x, tables, S)
    expected = _arr(case["output"], case["dtype"]).reshape(out.shape)
    assert np.max(np.abs(out - expected)) <= 1e-12
    cot = _arr(case["output_cotangent"], case["dtype"]).reshape(out.shape)
    adj = _unpack(oracle.factorized_angular_adjoint(cot, x, tables, S), case, S)
    for a, e in zip(adj, case["slot_adjoints"]):
        assert np.max(np.abs(a - _arr(e, case["dtype"]))) <= 1e-12
    w = _arr(case["readout_weight"], case["dtype"])
    b = _arr(case["readout_bias"], case["dtype"])
    lin = oracle.factorized_angular_linear(x, tables, S, w, b)
    assert np.max(np.abs(lin.reshape(-1) - _arr(case["readout"], case["dtype"]).reshape(-1))) <= 1e-12


def _payload(name):
    return json.loads(DATA["plans"][name]["plan_json"])


def test_planted_mistakes_are_refused():
    name = PLANS[0]
    p = _payload(name)
    p["synthesis_tables"][1]["values"][0][0] += 1e-9  # coefficient no longer matches its table hash
    with pytest.raises(ValueError, match="coefficient hash"):
        ExecutionPlan.from_dict(p)
    p = _payload(name)
    p["provenance"]["api"] = "edited"  # payload no longer matches plan_hash
    with pytest.raises(ValueError, match="execution-plan hash"):
        ExecutionPlan.from_dict(p)
    p["plan_hash"] = ""
    assert ExecutionPlan.from_dict(p).plan_hash != DATA["plans"][name]["plan_hash"]
    p = _payload(name)
    nodes = p["factorized_angular_plans"][0]["nodes"]
    merge = next(i for i, n in enumerate(nodes) if n["kind"] == "merge")
    nodes.insert(0, nodes.pop(merge))  # a merge before its children
    with pytest.raises(ValueError, match="topological"):
        ExecutionPlan.from_dict(p)
    p = _payload(name)
    p["factorized_angular_plans"][0]["young_synthesis_table_id"] = "missing"
    with pytest.raises(ValueError, match="Young synthesis table"):
        ExecutionPlan.from_dict(p)
    p = _payload(name)
    p["synthesis_tables"][0]["row_indices"][0] = p["synthesis_tables"][0]["input_dimension"]
    with pytest.raises(ValueError, match="row index"):
        ExecutionPlan.from_dict(p)


def test_schema_versions():
    name = PLANS[1]
    p = _payload(name)
    legacy = dict(p, schema_version=EXECUTION_PLAN_LEGACY_SCHEMA)
    migrated = ExecutionPlan.from_dict(legacy)
    assert migrated.schema_version == EXECUTION_PLAN_SCHEMA
    assert migrated.provenance["migrated_from_schema"] == EXECUTION_PLAN_LEGACY_SCHEMA
    assert migrated.provenance["legacy_plan_hash"] == p["plan_hash"]
    assert migrated.plan_hash != p["plan_hash"]
    assert ExecutionPlan.from_json(migrated.to_json()).plan_hash == migrated.plan_hash
    with pytest.raises(NotImplementedError):
        ExecutionPlan.from_dict(dict(p, schema_version="ye3t_execution_plan_v3"))
    with pytest.raises(ValueError, match="unsupported"):
        ExecutionPlan.from_dict(dict(p, schema_version="ye3t_execution_plan_v9"))


def test_plan_selection_and_canonical_json():
    p = _payload(PLANS[0])
    plan = ExecutionPlan.from_dict(p)
    assert plan.factorized_angular_plan().plan_id == p["factorized_angular_plans"][0]["plan_id"]
    two = copy.deepcopy(p)
    extra = copy.deepcopy(two["factorized_angular_plans"][0])
    extra["plan_id"] = "second"
    two["factorized_angular_plans"].append(extra)
    two["plan_hash"] = ""
    both = ExecutionPlan.from_dict(two)
    with pytest.raises(ValueError, match="required"):
        both.factorized_angular_plan()
    assert both.factorized_angular_plan("second").plan_id == "second"
    # canonical form: sorted keys, tuples as lists, complex as pairs
    assert canonical_json({"b": (1, 2), "a": 1 + 2j}) == '{"a":[1.0,2.0],"b":[1,2]}'
