"""Write golden vectors for the execution-plan loader and the factorized-angular module.

The reference tree holds no serialized execution plan, so nothing it ships pins
``YE3TExecutionPlan.to_json`` / ``plan_hash`` (``ye3t/execution_plan.py:116-145,
7137-7245``) or the buffers ``_factorized_plan_buffers`` derives from a plan
(``ye3t/runtime/execution_plan.py:12918-13151``).  This script imports the
reference (from ``/root/reference``, in the build container only) and writes,
for the factorized-angular plans its own native tests build
(``tests/test_execution_plan_native.py:138-173`` through
``tests/_legacy_algebraic_plan.py``):

* the plan document exactly as ``to_json(indent=2)`` writes it, and its hash;
* the node tables, coefficient COO and projection of ``_factorized_plan_buffers``;
* the reference Torch branch's forward, fused linear readout and slot adjoints on
  seeded inputs (``backend="reference"``, float64 or complex128, CPU).

The output ``execution_plan_factorized_v1.json`` is data only; run this once
where the reference tree is mounted and commit the JSON.
"""
import json
import sys

REF = "/root/reference"


def _pairs(t):
    import torch

    t = t.detach().cpu()
    if t.is_complex():
        t = torch.view_as_real(t.resolve_conj())
    return t.tolist()


def _case(name, plan, dtype_name, seed, batch=3):
    import torch
    from ye3t.execution_plan import YE3TExecutionPlan
    from ye3t.runtime.execution_plan import YE3TFactorizedAngularModule, _factorized_plan_buffers

    dtype = {"float64": torch.float64, "complex128": torch.complex128}[dtype_name]
    text = plan.to_json(indent=2) + "\n"
    restored = YE3TExecutionPlan.from_json(text)
    assert restored.plan_hash == plan.plan_hash
    angular = plan.factorized_angular_plans[0]
    buffers = _factorized_plan_buffers(plan, angular, dtype, torch.device("cpu"),
                                       materialize_reference_dense_tables=False)
    module = YE3TFactorizedAngularModule(plan, backend="reference", dtype=dtype)
    gen = torch.Generator().manual_seed(seed)
    src = int(module.source_dimension)
    slots = []
    for L in module.input_Ls:
        shape = (batch, 2 * L + 1) if src == 1 else (batch, src, 2 * L + 1)
        re = torch.randn(shape, generator=gen, dtype=torch.float64)
        if dtype.is_complex:
            re = torch.complex(re, torch.randn(shape, generator=gen, dtype=torch.float64))
        slots.append(re.to(dtype).requires_grad_(True))
    out = module(tuple(slots))
    cot = torch.randn(out.shape, generator=gen, dtype=torch.float64)
    if dtype.is_complex:
        cot = torch.complex(cot, torch.randn(out.shape, generator=gen, dtype=torch.float64))
    cot = cot.to(dtype)
    grads = torch.autograd.grad((out * cot.conj()).real.sum() if dtype.is_complex else (out * cot).sum(),
                                tuple(slots))
    weight = torch.randn(int(module.output_dimension), generator=gen, dtype=torch.float64).to(dtype)
    bias = torch.tensor(0.375, dtype=torch.float64).to(dtype)
    readout = module.linear_readout(tuple(s.detach() for s in slots), weight, bias)
    ints = ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
            "node_coefficient_offsets", "coefficient_rows", "coefficient_columns", "root_nodes")
    plan_record = {
        "plan_json": text,
        "plan_hash": plan.plan_hash,
        "coefficient_hash": plan.coefficient_hash,
        "factorized_angular_plan_id": angular.plan_id,
        "buffers": {
            **{k: buffers[k].tolist() for k in ints},
            "coefficient_values": _pairs(buffers["coefficient_values"]),
            "projection_values": _pairs(buffers["projection_values"]),
            "input_dimension": int(buffers["input_dimension"]),
            "source_dimension": int(buffers["source_dimension"]),
            "workspace_dimension": int(buffers["workspace_dimension"]),
            "output_dimension": int(buffers["output_dimension"]),
            "logical_channel_tableau_dimension": int(buffers["logical_channel_tableau_dimension"]),
            "magnetic_dimension": int(buffers["magnetic_dimension"]),
            "reference_dense_synthesis_element_count": int(buffers["reference_dense_synthesis_element_count"]),
            "node_operator_hashes": list(buffers["node_operator_hashes"]),
            "node_subtree_hashes": list(buffers["node_subtree_hashes"]),
        },
    }
    return plan_record, {
        "plan": name,
        "dtype": dtype_name,
        "input_Ls": list(module.input_Ls),
        "slots": [_pairs(s) for s in slots],
        "output": _pairs(out),
        "output_cotangent": _pairs(cot),
        "slot_adjoints": [_pairs(g) for g in grads],
        "readout_weight": _pairs(weight),
        "readout_bias": _pairs(bias),
        "readout": _pairs(readout),
    }


def main(dst="tests/golden/execution_plan_factorized_v1.json"):
    sys.path[:0] = [REF, REF + "/tests"]
    from _legacy_algebraic_plan import algebraic_young_angular_plan

    specs = [
        ("rank3_l121_L2", dict(content=(1, 2, 3), input_Ls=(1, 2, 1), target_L=2), {}),
        ("rank3_role_l121_L2", dict(content=(1, 2, 3), input_Ls=(1, 2, 1), target_L=2),
         dict(target_partition=(2, 1), role_labels=("role_0", "role_1", "role_2"))),
        ("rank4_homogeneous_role_L2", dict(content=(1, 1, 1, 1), input_Ls=(1, 1, 1, 1), target_L=2),
         dict(role_labels=("role_0",) * 4)),
        ("rank4_two_block_role_L1", dict(content=(1, 1, 2, 2), input_Ls=(1, 1, 1, 1), target_L=1),
         dict(target_partition=(3, 1), subgroup_partitions=((2,), (2,)),
              role_labels=("role_0", "role_0", "role_1", "role_1"))),
    ]
    plans, cases = {}, []
    for i, (name, args, kw) in enumerate(specs):
        plan = algebraic_young_angular_plan(args["content"], args["input_Ls"], args["target_L"], **kw)[1]
        for dtype_name in ("float64", "complex128"):
            plans[name], case = _case(name, plan, dtype_name, seed=1000 + 10 * i + (dtype_name == "complex128"))
            cases.append(case)
            print(name, dtype_name, plans[name]["plan_hash"][:16], len(plans[name]["plan_json"]), flush=True)
    json.dump({"_source": "reference ye3t (imported by tests/golden/make_execution_plan_fixtures.py)",
               "plans": plans, "cases": cases}, open(dst, "w"), indent=None, separators=(",", ":"))


if __name__ == "__main__":
    main(*sys.argv[1:])
