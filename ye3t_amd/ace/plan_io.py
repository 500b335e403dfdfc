"""On-disk form of a compiled :class:`~ye3t_amd.ace.plan.ProductPlan`.

A plan is written as one JSON document (schema ``ye3t_amd_product_plan_v1``)
holding everything the product kernels and the oracle need: the feature spec,
the contents and labels in column order, and the hash-consed DAG (leaf,
symmetric-block and pair-coupling nodes with their coefficient terms) with
the output column map.  Loading it rebuilds the plan without running the
coupling compiler.

``plan_hash`` is ``"sha256:"`` + the SHA-256 of the canonical JSON of the
document without that field (sorted keys, ``(",", ":")`` separators, no NaN),
the scheme the reference applies to its typed factor tables
(``ye3t/execution_plan.py:6670-6673``).  As in the reference's plan export
(``ye3t/scalar_ace_export.py:10-19``), writing checks that the JSON round
trip keeps the hash, and loading recomputes it and rejects a document whose
hash does not match.  Floats are written with Python's shortest round-trip
representation, so coefficients load back bit for bit.

This is this backend's plan format, not the reference's ``YE3TExecutionPlan``
schema (``ye3t/execution_plan.py:6566``): the two hash different payloads.
"""

import hashlib
import json

from ye3t_amd.ace.plan import ACEFeatureSpec, ProductPlan

SCHEMA = "ye3t_amd_product_plan_v1"


def _canonical(obj):
    return json.dumps(obj, sort_keys=True, separators=(",", ":"), allow_nan=False).encode("utf-8")


def _tuplify(value):
    """JSON lists back to the tuples labels and node keys are made of."""
    if isinstance(value, list):
        return tuple(_tuplify(v) for v in value)
    return value


def _listify(value):
    if isinstance(value, tuple) or isinstance(value, list):
        return [_listify(v) for v in value]
    if isinstance(value, bool) or value is None or isinstance(value, str):
        return value
    if isinstance(value, float):
        return float(value)
    if hasattr(value, "item"):  # numpy scalars
        return value.item()
    return value


def _node_to_json(nd):
    out = {"kind": nd["kind"], "key": _listify(nd["key"]), "dim": int(nd["dim"]),
           "deps": [int(d) for d in nd["deps"]]}
    if nd["kind"] == "leaf":
        out["a_offset"] = int(nd["a_offset"])
    else:
        out["terms"] = [[int(c), float(v), [int(f) for f in factors]] for c, v, factors in nd["terms"]]
        if nd["kind"] == "sym":
            out["k"] = int(nd["k"])
    return out


def _node_from_json(d):
    nd = {"kind": d["kind"], "key": _tuplify(d["key"]), "dim": int(d["dim"]),
          "deps": tuple(int(x) for x in d["deps"])}
    if d["kind"] == "leaf":
        nd["a_offset"] = int(d["a_offset"])
    else:
        nd["terms"] = [(int(c), float(v), tuple(int(f) for f in factors)) for c, v, factors in d["terms"]]
        if d["kind"] == "sym":
            nd["k"] = int(d["k"])
    return nd


def plan_to_dict(plan):
    """The document of ``plan`` with its ``plan_hash``."""
    doc = {
        "schema": SCHEMA,
        "spec": plan.spec.to_dict(),
        "a_width": int(plan.a_width),
        "feature_count": int(plan.feature_count),
        "contents": [[list(map(int, n)), list(map(int, l))] for n, l in plan.contents],
        "label_records": [[int(L), int(ci), _listify(lab), int(first)] for L, ci, lab, first in plan.label_records],
        "nodes": [_node_to_json(nd) for nd in plan.nodes],
        "outputs": [[int(n), int(c)] for n, c in plan.outputs],
        "convention_hash": plan.convention_hash(),
    }
    doc["plan_hash"] = "sha256:" + hashlib.sha256(_canonical(doc)).hexdigest()
    return doc


def plan_hash(plan):
    return plan_to_dict(plan)["plan_hash"]


def _spec_from_dict(d):
    return ACEFeatureSpec(channel_count=int(d["channel_count"]), l_max=int(d["l_max"]), nu_max=int(d["nu_max"]),
                          targets=tuple(int(t) for t in d["targets"]), parity=str(d["parity"]),
                          nu_min=int(d["nu_min"]), radial_per_species=int(d["radial_per_species"]),
                          caps={int(k): tuple(int(x) for x in v) for k, v in d["caps"].items()},
                          channel_ids=tuple(int(x) for x in d["channel_ids"]))


def plan_from_dict(doc):
    """Rebuild a plan from its document; the hash and the structure are checked."""
    if not isinstance(doc, dict) or doc.get("schema") != SCHEMA:
        raise ValueError(f"not a {SCHEMA} document (schema {doc.get('schema') if isinstance(doc, dict) else None!r})")
    body = {k: v for k, v in doc.items() if k != "plan_hash"}
    digest = "sha256:" + hashlib.sha256(_canonical(body)).hexdigest()
    if doc.get("plan_hash") != digest:
        raise ValueError(f"plan hash mismatch: the document says {doc.get('plan_hash')!r}, its content hashes "
                         f"to {digest!r}")
    plan = ProductPlan.__new__(ProductPlan)
    plan.spec = _spec_from_dict(doc["spec"])
    plan.a_width = int(doc["a_width"])
    if plan.a_width != plan.spec.row_width():
        raise ValueError("a_width does not match the spec")
    plan.contents = [(tuple(n), tuple(l)) for n, l in doc["contents"]]
    plan.label_records = [(int(L), int(ci), _tuplify(lab), int(first)) for L, ci, lab, first in doc["label_records"]]
    plan.features = []
    seen = {}  # label index within its (L, content) schedule
    for L, ci, lab, first in plan.label_records:
        if first != len(plan.features) or not 0 <= ci < len(plan.contents):
            raise ValueError("label records out of order")
        li = seen.get((L, ci), 0)
        seen[(L, ci)] = li + 1
        for comp in range(2 * L + 1):
            plan.features.append((L, ci, li, comp))
    plan.feature_count = int(doc["feature_count"])
    if plan.feature_count != len(plan.features):
        raise ValueError("feature_count does not match the label records")
    plan.nodes = [_node_from_json(d) for d in doc["nodes"]]
    plan.node_index = {nd["key"]: i for i, nd in enumerate(plan.nodes)}
    for i, nd in enumerate(plan.nodes):
        if any(not 0 <= dep < i for dep in nd["deps"]):
            raise ValueError(f"node {i}: dependencies must precede it")
        if nd["kind"] == "leaf":
            if not (0 <= nd["a_offset"] and nd["a_offset"] + nd["dim"] <= plan.a_width):
                raise ValueError(f"node {i}: leaf outside the density row")
        else:
            ins = [plan.nodes[dep]["dim"] for dep in nd["deps"]]
            for c, _v, factors in nd["terms"]:
                if not 0 <= c < nd["dim"]:
                    raise ValueError(f"node {i}: term component out of range")
                limits = ins * len(factors) if nd["kind"] == "sym" else ins
                if any(not 0 <= f < lim for f, lim in zip(factors, limits)):
                    raise ValueError(f"node {i}: term factor out of range")
    plan.outputs = [(int(n), int(c)) for n, c in doc["outputs"]]
    if len(plan.outputs) != plan.feature_count or any(
            not 0 <= n < len(plan.nodes) or not 0 <= c < plan.nodes[n]["dim"] for n, c in plan.outputs):
        raise ValueError("output map out of range")
    plan._flat = None
    if plan.convention_hash() != doc["convention_hash"]:
        raise ValueError("convention hash mismatch")
    return plan


def to_json(plan, indent=None):
    return json.dumps(plan_to_dict(plan), sort_keys=True, indent=indent, allow_nan=False)


def from_json(text):
    return plan_from_dict(json.loads(text))


def save_plan(plan, path):
    """Write ``plan``; the JSON round trip must keep its hash.  Returns the hash."""
    text = to_json(plan) + "\n"
    restored = from_json(text)
    if plan_hash(restored) != plan_hash(plan):
        raise RuntimeError("the plan JSON round trip changed the plan hash")
    with open(path, "w", encoding="utf-8") as f:
        f.write(text)
    return json.loads(text)["plan_hash"]


def load_plan(path):
    with open(path, "r", encoding="utf-8") as f:
        return from_json(f.read())
