"""On-disk product plans: JSON round trip, hash checks and validation (CPU)."""

import json

import numpy as np
import pytest

import oracle
from ye3t_amd.ace import plan_io
from ye3t_amd.ace import workloads as W
from ye3t_amd.ace.plan import ACEFeatureSpec, ProductPlan
from ye3t_amd.ace.program import compile_program


def _small_rank4_spec():
    # config-3 shaped (species-folded channels, ranks 1-4) at a test-sized truncation
    return ACEFeatureSpec(channel_count=44, l_max=4, nu_max=4, targets=(0,), parity="even",
                          radial_per_species=11, caps={1: (11, 0), 2: (3, 4), 3: (2, 2), 4: (1, 2)})


@pytest.fixture(scope="module", params=["config4", "rank4"])
def plan(request):
    spec = W.config(4).feature_spec if request.param == "config4" else _small_rank4_spec()
    return ProductPlan(spec)


def test_round_trip_is_exact(plan):
    text = plan_io.to_json(plan)
    back = plan_io.from_json(text)
    assert plan_io.plan_hash(back) == plan_io.plan_hash(plan) == json.loads(text)["plan_hash"]
    assert back.convention_hash() == plan.convention_hash()
    assert back.features == plan.features and back.outputs == plan.outputs
    assert back.label_records == plan.label_records and back.contents == plan.contents
    # coefficients bit for bit, so the compiled programs are identical
    for a, b in zip(plan.nodes, back.nodes):
        assert a["key"] == b["key"] and a["deps"] == b["deps"]
        if a["kind"] != "leaf":
            assert [(c, np.float64(v).tobytes(), f) for c, v, f in a["terms"]] == \
                   [(c, np.float64(v).tobytes(), f) for c, v, f in b["terms"]]
    for dtype in ("f32", "f64"):
        pa, pb = compile_program(plan, dtype), compile_program(back, dtype)
        for key, value in pa.items():
            if isinstance(value, np.ndarray):
                assert np.array_equal(value, pb[key]), key
            else:
                assert value == pb[key], key
    # the oracle evaluates the loaded plan to the same bits
    A = np.random.default_rng(3).normal(size=(37, plan.a_width))
    assert np.array_equal(oracle.ace_product_flat(A, back.flat_arrays()), oracle.ace_product_flat(A, plan.flat_arrays()))


def test_the_compiler_is_deterministic(plan):
    again = ProductPlan(plan.spec)
    assert plan_io.to_json(again) == plan_io.to_json(plan)


def test_save_and_load(plan, tmp_path):
    path = tmp_path / "plan.json"
    digest = plan_io.save_plan(plan, path)
    assert digest == plan_io.plan_hash(plan)
    first = path.read_bytes()
    plan_io.save_plan(plan_io.load_plan(path), path)
    assert path.read_bytes() == first


def test_tampering_and_bad_documents_are_rejected(plan):
    doc = plan_io.plan_to_dict(plan)
    # a changed coefficient without a new hash
    bad = json.loads(json.dumps(doc))
    node = next(nd for nd in bad["nodes"] if nd["kind"] == "pair")
    node["terms"][0][1] += 1e-9
    with pytest.raises(ValueError, match="hash mismatch"):
        plan_io.plan_from_dict(bad)
    # a wrong schema
    bad = dict(doc, schema="ye3t_amd_product_plan_v0")
    with pytest.raises(ValueError, match="not a ye3t_amd_product_plan_v1"):
        plan_io.plan_from_dict(bad)

    # structural corruption re-signed with a valid hash is still caught
    def resign(d):
        body = {k: v for k, v in d.items() if k != "plan_hash"}
        d["plan_hash"] = "sha256:" + __import__("hashlib").sha256(plan_io._canonical(body)).hexdigest()
        return d

    bad = json.loads(json.dumps(doc))
    bad["outputs"][0][0] = len(bad["nodes"])
    with pytest.raises(ValueError, match="output map"):
        plan_io.plan_from_dict(resign(bad))
    bad = json.loads(json.dumps(doc))
    node = next(nd for nd in bad["nodes"] if nd["kind"] == "pair")
    node["terms"][0][2][0] = 99
    with pytest.raises(ValueError, match="factor out of range"):
        plan_io.plan_from_dict(resign(bad))
    bad = json.loads(json.dumps(doc))
    leaf = next(nd for nd in bad["nodes"] if nd["kind"] == "leaf")
    leaf["a_offset"] = bad["a_width"]
    with pytest.raises(ValueError, match="leaf outside"):
        plan_io.plan_from_dict(resign(bad))
    bad = json.loads(json.dumps(doc))
    bad["label_records"][0][2] = ["leaf", 99, 0]
    with pytest.raises(ValueError, match="convention hash"):
        plan_io.plan_from_dict(resign(bad))
    with pytest.raises(ValueError):
        plan_io.from_json(plan_io.to_json(plan).replace('"a_width":', '"a_width":1000,"x":', 1))
