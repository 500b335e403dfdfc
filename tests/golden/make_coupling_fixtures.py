"""Write the reference's literal convention hashes and label lists for the benchmark contents.

Nothing in the reference tree holds the 16-hex ``convention_hash`` strings of
``ye3t.couplings.count`` / ``plan`` / ``compile_ace_factorized_schedules_by_L``
(``ye3t/couplings/__init__.py:2617-2706, 2709-2965, 2967-3077``) for the
benchmark configurations' contents, nor their full label lists.  This script
imports the reference (from ``/root/reference``, in the build container only)
and records, per request:

* ``count``: the report's ``convention_hash``, its label count and (for the
  smaller requests) the label payloads exactly as ``_report_label_payload``
  writes them into the hash payload;
* ``plan``: the plan's ``convention_hash`` (it hashes ``report.to_dict()`` and
  the backend plan), its selected backend and reason;
* ``compile``: the ``convention_hash`` of the schedule report and its summary;
* for a request the reference refuses, the exception type and message.

Requests: the config-1 quick-start content at every target, every config-4
content at L = 0, 1, 2, every config-2 content of rank <= 2 plus a seeded
sample of rank 3, and seeded samples of config-3 and config-5 contents; a few
requests with ``tree_schedule="left"`` / ``"right"``, an explicit
``coefficient_backend`` and ``fast_path_policy="disable"``.  The output
``coupling_hashes_v1.json`` is data only; run this once where the reference
tree is mounted and commit the JSON.
"""
import json
import sys

import numpy as np

REF = "/root/reference"


def _label_payload(label):
    return json.loads(json.dumps(label))


def _requests():
    sys.path.insert(0, __file__.rsplit("/tests/", 1)[0])
    from ye3t_amd.ace import workloads as W

    reqs = []
    for L in (0, 1, 2, 3):
        reqs.append(dict(content=(1, 1, 2), input_Ls=(1, 1, 0), target_L=L))
    for n, l in W.config(4).feature_spec.contents():
        for L in (0, 1, 2):
            reqs.append(dict(content=n, input_Ls=l, target_L=L))
    rng = np.random.default_rng(20261202)
    c2 = list(W.config(2).feature_spec.contents())
    reqs += [dict(content=n, input_Ls=l, target_L=0) for n, l in c2 if len(n) <= 2]
    r3 = [c for c in c2 if len(c[0]) == 3]
    reqs += [dict(content=r3[i][0], input_Ls=r3[i][1], target_L=0)
             for i in sorted(rng.choice(len(r3), 120, replace=False))]
    for cid, per_rank in ((3, {2: 20, 3: 30, 4: 30}), (5, {2: 20, 3: 20, 4: 20})):
        cs = list(W.config(cid).feature_spec.contents())
        for rank, k in per_rank.items():
            pool = [c for c in cs if len(c[0]) == rank]
            for i in sorted(rng.choice(len(pool), k, replace=False)):
                for L in ((0,) if cid == 3 else (0, 1, 2)):
                    reqs.append(dict(content=pool[i][0], input_Ls=pool[i][1], target_L=L))
    # unsorted leaves: the spec keeps the caller's order, the labels are canonical
    reqs.append(dict(content=(2, 1, 1), input_Ls=(0, 1, 1), target_L=0))
    reqs.append(dict(content=(3, 1, 2, 1), input_Ls=(1, 2, 1, 2), target_L=1))
    for tree in ("left", "right"):
        reqs.append(dict(content=(1, 1, 2, 2), input_Ls=(1, 1, 2, 2), target_L=0, tree_schedule=tree))
        reqs.append(dict(content=(1, 2, 3), input_Ls=(1, 2, 3), target_L=2, tree_schedule=tree))
    reqs.append(dict(content=(1, 1, 2), input_Ls=(1, 1, 0), target_L=0,
                     coefficient_backend="symmetric_power_fast_path"))
    reqs.append(dict(content=(1, 1, 2), input_Ls=(1, 1, 0), target_L=0, fast_path_policy="disable"))
    reqs.append(dict(content=(1, 1, 2), input_Ls=(1, 1, 0), target_L=2,
                     fast_path_policy="force:global_coupler"))
    reqs.append(dict(content=(1, 1, 2), input_Ls=(1, 1, 0)))
    return reqs


def _plain(req):
    return {k: (list(v) if isinstance(v, tuple) else v) for k, v in req.items()}


def main(dst="tests/golden/coupling_hashes_v1.json"):
    reqs = _requests()
    sys.path.insert(0, REF)
    from ye3t import couplings as C
    from ye3t.couplings import _report_label_payload

    cases = []
    for i, req in enumerate(reqs):
        try:
            report = C.count(carrier="ACE_density", **req)
        except ValueError as exc:
            cases.append({"request": _plain(req), "error": "ValueError", "message": str(exc)})
            continue
        plan = C.plan(report)
        L = int(report.spec.target_rotation.L_R) if req.get("target_L") is None else int(req["target_L"])
        labels = [_label_payload(_report_label_payload(lab)) for lab in report.labels_by_target.get(L, ())]
        case = {
            "request": _plain(req),
            "count_hash": report.convention_hash,
            "count": int(report.counts_by_target.get(L, 0)),
            "backend": report.backend,
            "plan_hash": plan.convention_hash,
            "plan_backend_reason": plan.backend_plan.reason,
            "labels_sha256": __import__("hashlib").sha256(json.dumps(labels).encode()).hexdigest(),
        }
        if len(labels) <= 40:
            case["labels"] = labels
        # the same plan through the keyword form
        if i % 17 == 0:
            case["plan_hash_kwargs"] = C.plan(carrier="ACE_density", **req).convention_hash
        cases.append(case)
        if i % 50 == 0:
            print(i, len(reqs), case["count_hash"], case["plan_hash"], case["count"], flush=True)
    compiles = []
    comp_reqs = [((1, 1, 2), (1, 1, 0), {}), ((1, 1, 2), (1, 1, 0), {"cache_policy": "cold"}),
                 ((1, 1, 2), (1, 1, 0), {"tree_schedule": "left"}),
                 ((1, 1, 2), (1, 1, 0), {"coeff_tol": 1e-12})]
    comp_reqs += [(n, l, {}) for n, l in __import__("ye3t_amd.ace.workloads", fromlist=["x"]).config(4)
                  .feature_spec.contents()]
    comp_reqs += [((1, 2, 3), (1, 1, 2), {}), ((1, 1, 1, 1), (2, 2, 2, 2), {}), ((1, 2, 2, 3), (1, 2, 2, 3), {})]
    for n, l, kw in comp_reqs:
        rep = C.compile_ace_factorized_schedules_by_L(content=n, input_Ls=l, **kw)
        compiles.append({"content": list(n), "input_Ls": list(l), "kwargs": kw,
                         "convention_hash": rep.convention_hash,
                         "targets": sorted(int(t) for t in rep.schedules_by_target),
                         "validation_report": json.loads(json.dumps(rep.validation_report))})
    json.dump({"_source": "reference ye3t (imported by tests/golden/make_coupling_fixtures.py)",
               "cases": cases, "compile": compiles}, open(dst, "w"), indent=None, separators=(",", ":"))
    print("wrote", dst, len(cases), "count/plan cases,", len(compiles), "compile cases")


if __name__ == "__main__":
    main(*sys.argv[1:])
