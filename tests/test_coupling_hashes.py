"""``count`` / ``plan`` / ``compile_ace_factorized_schedules_by_L`` against the reference's literal output.

``tests/golden/coupling_hashes_v1.json`` was written by the reference itself
(``tests/golden/make_coupling_fixtures.py``): for every config-1 and config-4
content, every config-2 content of rank <= 2, seeded samples of configs 2, 3
and 5 and a few non-default requests, it holds the 16-hex ``convention_hash``
of ``count`` and of ``plan``, the label payloads in report order and, for the
requests the reference refuses, its error message.  The ``count`` hash covers
the label payloads, so an equal hash pins the label list and its order.
"""

import hashlib
import json
import os

import pytest

from ye3t_amd.core.basis import CompactLabel
from ye3t_amd.couplings import compile_ace_factorized_schedules_by_L, count, plan

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = json.load(open(os.path.join(HERE, "golden", "coupling_hashes_v1.json")))


def _labels_json(report, L):
    return json.loads(json.dumps([lab.payload() for lab in report.labels_for_target(L)]))


@pytest.mark.parametrize("chunk", range(8))
def test_count_and_plan_hashes_equal_the_reference(chunk):
    cases = FIXTURE["cases"][chunk::8]
    assert cases
    for case in cases:
        req = dict(case["request"])
        if "error" in case:
            with pytest.raises(ValueError) as info:
                count(carrier="ACE_density", **req)
            assert str(info.value) == case["message"]
            continue
        report = count(carrier="ACE_density", **req)
        L = req.get("target_L")
        labels = _labels_json(report, L)
        assert labels == case["labels"], req
        assert hashlib.sha256(json.dumps(labels).encode()).hexdigest() == case["labels_sha256"]
        assert report.counts_by_target[report.spec.target_rotation.L_R if L is None else L] == case["count"]
        assert report.backend == case["backend"]
        assert report.convention_hash == case["count_hash"], req
        p = plan(report)
        assert p.convention_hash == case["plan_hash"], req
        assert p.backend_plan.reason == case["plan_backend_reason"]
        if "plan_hash_kwargs" in case:
            assert plan(carrier="ACE_density", **req).convention_hash == case["plan_hash_kwargs"]


def test_fixture_covers_the_benchmark_contents():
    from ye3t_amd.ace import workloads as W

    reqs = {(tuple(c["request"]["content"]), tuple(c["request"]["input_Ls"]), c["request"].get("target_L"))
            for c in FIXTURE["cases"]}
    for n, l in W.config(4).feature_spec.contents():
        assert all((n, l, L) in reqs for L in (0, 1, 2))
    assert ((1, 1, 2), (1, 1, 0), 0) in reqs and ((1, 1, 2), (1, 1, 0), 2) in reqs
    assert sum(1 for c in FIXTURE["cases"] if "count_hash" in c) > 700


def test_compile_hashes_equal_the_reference():
    for case in FIXTURE["compile"]:
        rep = compile_ace_factorized_schedules_by_L(content=case["content"], input_Ls=case["input_Ls"],
                                                    **case["kwargs"])
        assert rep.convention_hash == case["convention_hash"], case
        assert sorted(rep.schedules_by_target) == case["targets"]
        assert json.loads(json.dumps(rep.validation_report)) == case["validation_report"]


def test_planted_mistakes_change_the_hash():
    """A wrong field in any hashed part of the payload gives another string."""
    case = FIXTURE["cases"][0]
    req = dict(case["request"])
    base = count(carrier="ACE_density", **req)
    assert base.convention_hash == case["count_hash"]
    # a different spec field (readout aggregation) and a different label order
    other = count({"readout": {"aggregation": "site_sum"}}, carrier="ACE_density", **req)
    assert other.convention_hash != case["count_hash"]
    many = next(c for c in FIXTURE["cases"] if c.get("count", 0) >= 3)
    report = count(carrier="ACE_density", **many["request"])
    L = many["request"]["target_L"]
    from ye3t_amd.couplings import _convention_hash

    def payload(labels):
        return {"spec": report.spec.to_dict(), "input_Ls": tuple(many["request"]["input_Ls"]),
                "target": report.target, "backend": report.backend, "labels": [lab.payload() for lab in labels]}

    labels = list(report.labels_for_target(L))
    assert _convention_hash(payload(labels)) == many["count_hash"]
    assert _convention_hash(payload(labels[::-1])) != many["count_hash"]


def test_report_labels_are_compact_label_records():
    report = count(content=(1, 1, 2), input_Ls=(1, 1, 0), target_L=0)
    (lab,) = report.labels_for_target(0)
    assert isinstance(lab, CompactLabel)
    assert lab.L_R == 0 and lab.rank == 3
    assert lab.basis_key == ("node", ("sym", 0, 0), ())
    assert CompactLabel.from_dict(lab.to_dict()) == lab
    assert CompactLabel.from_tuple(lab.payload()) == lab
    assert report.require_label(lab.compact_label(), target_L=0) == lab
    with pytest.raises(ValueError, match="Invalid descriptor label"):
        report.require_label(((1, 1, 2), (1, 1, 0), (2, 2)), target_L=0)
    with pytest.raises(ValueError, match="only the globally trivial Young sector"):
        count(content=(1, 2), input_Ls=(1, 1), target_permutation="antisymmetric")
    with pytest.raises(ValueError, match="natural product parity"):
        count({"target_rotation": {"L_R": 0, "parity": "odd"}}, content=(1, 2), input_Ls=(1, 1))
