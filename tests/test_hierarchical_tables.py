"""Host side of the hierarchical runtime, pinned by the reference's own values.

``tests/golden/hierarchical_v1.json`` (written by
``tests/golden/make_hierarchical_fixtures.py`` from the reference) holds, for the
plans the reference's ``tests/test_hierarchical_runtime.py`` builds, every block
power's ``SymmetricPowerProductPlan`` payload, plan key, grouped and shared
count tables and table report.  These tests check on the CPU that the plan
records round-trip with their convention hash, that
``symmetric_power_plan_key`` is the reference's string, and that the lowering
reproduces the tables entry for entry (the complex coefficients bit for bit:
the same sums in the same order).  The sparse supports are checked against the
dense exponent rows they encode.
"""

import copy
import json
import os

import numpy as np
import pytest

from ye3t_amd.runtime import hierarchical as H

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "hierarchical_v1.json")


def _fixture():
    with open(FIXTURE) as fh:
        return json.load(fh)


def _powers():
    for case in _fixture()["cases"]:
        for power in case["block_powers"]:
            yield case["name"], power


@pytest.mark.parametrize("name,power", list(_powers()), ids=lambda v: v if isinstance(v, str) else "")
def test_power_plan_lowering_matches_the_reference(name, power):
    plan = H.SymmetricPowerProductPlan.from_dict(power["plan"])
    assert plan.to_dict() == power["plan"]
    assert H.symmetric_power_plan_key(plan) == power["plan_key"]
    rows, offsets, index, values = H.product_plan_count_table(plan)
    g = power["grouped"]
    assert [list(r) for r in rows] == g["monomial_counts"]
    assert offsets == g["output_offsets"]
    assert index == g["output_index"]
    assert [[v.real, v.imag] for v in values] == g["monomial_values"]
    unique, offs, terms, outs, vals = H.shared_table(rows, offsets, index, values)
    s = power["shared"]
    assert [list(u) for u in unique] == s["monomial_counts"]
    assert offs == s["output_offsets"] and terms == s["coefficient_terms"] and outs == s["coefficient_outputs"]
    assert [[v.real, v.imag] for v in vals] == s["coefficient_values"]
    report = H.symmetric_power_product_plan_table_report(plan)
    want = dict(power["table_report"])
    want["powers"] = tuple(want["powers"])
    assert report == want
    # sparse supports rebuild the dense rows
    toff, comp, ex = H.sparse_supports(unique)
    dense = np.zeros((len(unique), plan.channel_count), dtype=np.int64)
    for t in range(len(unique)):
        for q in range(toff[t], toff[t + 1]):
            dense[t, comp[q]] += ex[q]
    assert dense.tolist() == s["monomial_counts"]


def test_plan_hash_check_and_key_identity():
    """A changed coefficient changes the key; provenance does not (the
    reference's ``test_hierarchical_power_identity_uses_exact_numeric_contraction``);
    a payload whose convention hash disagrees is refused."""
    power = _fixture()["cases"][0]["block_powers"][0]
    plan = H.SymmetricPowerProductPlan.from_dict(power["plan"])
    meta = copy.deepcopy(plan.to_dict())
    meta["target"] = {"permutation": "different_parent_provenance",
                      "rotation": {"L_R": int(plan.entries[0].output_L)}}
    meta["label_source"] = "different_parent_label"
    meta["validation_report"] = {"different": True}
    meta["provenance"] = {"different_parent": True}
    meta["convention_hash"] = ""
    assert H.symmetric_power_plan_key(H.SymmetricPowerProductPlan.from_dict(meta)) == \
        H.symmetric_power_plan_key(plan)
    changed = copy.deepcopy(meta)
    changed["entries"][0]["component_terms"][0]["coefficient"][0] += 1.0e-6
    assert H.symmetric_power_plan_key(H.SymmetricPowerProductPlan.from_dict(changed)) != \
        H.symmetric_power_plan_key(plan)
    bad = copy.deepcopy(power["plan"])
    bad["entries"][0]["component_terms"][0]["coefficient"][0] += 1.0
    with pytest.raises(ValueError, match="convention hash"):
        H.SymmetricPowerProductPlan.from_dict(bad)


def test_module_refuses_cpu_and_the_torch_branch():
    import torch

    case = _fixture()["cases"][0]
    with pytest.raises(NotImplementedError):
        H.YE3THierarchicalRepeatedBlockModule(case["plan"], device="cpu")
    with pytest.raises(NotImplementedError):
        H.YE3THierarchicalRepeatedBlockModule(case["plan"], backend="reference", device="cpu")
    with pytest.raises(ValueError, match="complex"):
        H.YE3THierarchicalRepeatedBlockModule(case["plan"], dtype=torch.float64, device="cpu")
