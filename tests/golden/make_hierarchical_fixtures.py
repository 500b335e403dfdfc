"""Write golden vectors for the hierarchical repeated-block runtime.

The reference ships no hierarchical plan document, and nothing in its tree pins
the values of ``YE3THierarchicalRepeatedBlockModule`` /
``YE3THierarchicalRepeatedBlockModuleGroup`` (``ye3t/runtime/hierarchical.py:
79-1540``) or of the block-power lowering they call
(``ye3t/runtime/symmetric_power.py:95-142, 144-193, 740-876``).  This script
imports the reference (from ``/root/reference``, in the build container only)
and writes, for the plans its own tests build with
``execution_plan_from_repeated_angular_blocks`` (``tests/test_hierarchical_
runtime.py:7-203, 469-555``):

* the plan document (``to_dict()``) and the module's shape facts;
* for every block power: its ``SymmetricPowerProductPlan`` payload, the plan
  key, the grouped and shared count tables and the table report;
* the reference Torch branch's (``backend="reference"``, complex128, CPU)
  forward on seeded float64 inputs, the gradient of ``sum |out|^2`` and its
  Hessian-vector product along a seeded direction, and a linear readout;
* for module groups: ``forward_packed``, gradient, HVP and report counts.

The output ``hierarchical_v1.json`` is data only; run this once where the
reference tree is mounted and commit the JSON.
"""
import json
import sys

REF = "/root/reference"
OUT = "tests/golden/hierarchical_v1.json"


def _pairs(t):
    import torch

    t = t.detach().cpu()
    if t.is_complex():
        t = torch.view_as_real(t.resolve_conj())
    return t.tolist()


def _source(kind, rank, content, role_labels=None):
    from ye3t.execution_plan import YE3TSourceRealization

    if role_labels is None:
        return YE3TSourceRealization(kind=kind, rank=rank, content=content)
    return YE3TSourceRealization(kind=kind, rank=rank, content=content, role_labels=role_labels,
                                 retain_role_order=True)


def _plans():
    """(name, plan) for the reference test helpers' plans."""
    from ye3t.couplings import blockwise_symmetric_power_labels, execution_plan_from_repeated_angular_blocks as build

    out = []
    for target_L in (1, 2):
        out.append((f"rank3_L{target_L}", build(
            ({"power": 2, "input_L": 1, "slot_indices": (0, 1)}, {"power": 1, "input_L": 1, "slot_indices": (2,)}),
            parent_partition=(2, 1), target_L=target_L,
            source_realization=_source("lifted_density_roles", 3, (1, 1, 2), ("branch_a", "branch_a", "branch_b")),
            spatial_symmetry="O3", expected_multiplicity=(2 if target_L == 1 else None))))
    out.append(("ordinary_rank4", build(
        ({"power": 2, "input_L": 1, "slot_indices": (0, 1), "source_binding": {"binding_id": "channel_a_L1", "input_L": 1}},
         {"power": 2, "input_L": 1, "slot_indices": (2, 3), "source_binding": {"binding_id": "channel_b_L1", "input_L": 1}}),
        id_prefix="ordinary_r4", parent_partition=(4,), target_L=0,
        source_realization=_source("ordinary_density", 4, ("channel_a", "channel_a", "channel_b", "channel_b")),
        spatial_symmetry="O3", expected_multiplicity=2)))
    report = blockwise_symmetric_power_labels(content=(1, 1, 2, 2, 3, 3), input_Ls=(1,) * 6, target_L=0,
                                              tree_schedule="balanced", label_strategy="exhaustive")
    labels = tuple(lab for lab in report["labels"] if tuple(lab.internal_Ls) == (2, 2, 2, 2, 0))
    out.append(("ordinary_rank6_three_block", build(
        tuple({"power": 2, "input_L": 1, "slot_indices": (2 * i, 2 * i + 1),
               "source_binding": {"binding_id": f"{c}_L1", "input_L": 1}} for i, c in enumerate("abc")),
        id_prefix="ordinary_r6_three_block", parent_partition=(6,), target_L=0,
        source_realization=_source("ordinary_density", 6, ("a", "a", "b", "b", "c", "c")),
        spatial_symmetry="O3", expected_multiplicity=1, compiler_labels=labels, coefficient_materialization="exact")))
    report = blockwise_symmetric_power_labels(content=(1, 1, 1, 2, 2, 3), input_Ls=(3, 3, 3, 1, 1, 0), target_L=1,
                                              tree_schedule="balanced", label_strategy="exhaustive")
    out.append(("ordinary_rank6_uneven", build(
        ({"power": 3, "input_L": 3, "slot_indices": (0, 1, 2), "source_binding": {"binding_id": "a_L3", "input_L": 3}},
         {"power": 2, "input_L": 1, "slot_indices": (3, 4), "source_binding": {"binding_id": "b_L1", "input_L": 1}},
         {"power": 1, "input_L": 0, "slot_indices": (5,), "source_binding": {"binding_id": "c_L0", "input_L": 0}}),
        id_prefix="ordinary_r6_uneven_three_block", parent_partition=(6,), target_L=1,
        source_realization=_source("ordinary_density", 6, ("a", "a", "a", "b", "b", "c")),
        spatial_symmetry="O3", expected_multiplicity=4, compiler_labels=tuple(report["labels"]),
        coefficient_materialization="exact")))
    out.append(("rank9", build(
        ({"power": 9, "input_L": 2, "slot_indices": tuple(range(9))},), parent_partition=(9,), target_L=0,
        source_realization=_source("lifted_density_roles", 9, (1,) * 9, ("repeated_branch",) * 9),
        expected_multiplicity=2)))
    out.append(("rank12", build(
        ({"power": 8, "input_L": 1, "slot_indices": tuple(range(8))},
         {"power": 4, "input_L": 1, "slot_indices": tuple(range(8, 12))}),
        parent_partition=(8, 4), target_L=0,
        source_realization=_source("lifted_density_roles", 12, (1,) * 8 + (2,) * 4,
                                   ("branch_a",) * 8 + ("branch_b",) * 4),
        spatial_symmetry="O3")))
    return out


def _tables(plan):
    import torch
    from ye3t.runtime.hierarchical import _symmetric_power_plan_key
    from ye3t.runtime.symmetric_power import (_symmetric_power_product_plan_count_table,
                                              symmetric_power_product_plan_table_report)

    grouped, shared, out_dtype = _symmetric_power_product_plan_count_table(
        plan, device=torch.device("cpu"), dtype=torch.complex128, imag_tol=1.0e-12)
    return {
        "plan": plan.to_dict(),
        "plan_key": _symmetric_power_plan_key(plan),
        "grouped": {"monomial_counts": grouped[0].tolist(), "output_offsets": grouped[1].tolist(),
                    "output_index": grouped[2].tolist(), "monomial_values": _pairs(grouped[3])},
        "shared": {"monomial_counts": shared[0].tolist(), "output_offsets": shared[1].tolist(),
                   "coefficient_terms": shared[2].tolist(), "coefficient_outputs": shared[3].tolist(),
                   "coefficient_values": _pairs(shared[4])},
        "output_dtype": str(out_dtype),
        "table_report": dict(symmetric_power_product_plan_table_report(plan, device="cpu",
                                                                        dtype=torch.complex128)),
    }


def _derivatives(outputs, inputs, gen):
    import torch

    grads = torch.autograd.grad(outputs.abs().square().sum(), inputs, create_graph=True)
    direction = tuple(torch.randn(g.shape, generator=gen, dtype=torch.float64) for g in grads)
    hvp = torch.autograd.grad(sum((g * d).sum() for g, d in zip(grads, direction)), inputs)
    return grads, direction, hvp


def _jsonable(report):
    return json.loads(json.dumps(report, default=lambda v: list(v) if isinstance(v, tuple) else str(v)))


def main():
    sys.path.insert(0, REF)
    import torch
    from ye3t.runtime import YE3THierarchicalRepeatedBlockModule, YE3THierarchicalRepeatedBlockModuleGroup

    cases, modules = [], {}
    for index, (name, plan) in enumerate(_plans()):
        module = YE3THierarchicalRepeatedBlockModule(plan, backend="reference", dtype=torch.complex128)
        modules[name] = module
        gen = torch.Generator().manual_seed(1000 + index)
        batch = 4
        inputs = tuple(torch.randn((batch, 2 * int(b["input_L"]) + 1), generator=gen, dtype=torch.float64)
                       .requires_grad_(True) for b in module._blocks)
        out = module(*inputs)
        grads, direction, hvp = _derivatives(out, inputs, gen)
        weight = torch.randn(module.output_dimension, generator=gen, dtype=torch.float64)
        readout = module.linear_readout(tuple(i.detach() for i in inputs), weight, 0.25)
        cases.append({
            "name": name,
            "plan": plan.to_dict(),
            "instruction_id": str(module.instruction_id),
            "facts": {"block_count": module.block_count, "route_count": module.route_count,
                      "channel_count": module.channel_count, "tableau_count": module.tableau_count,
                      "magnetic_count": module.magnetic_count, "output_dimension": module.output_dimension,
                      "target_L": module.target_L, "lr_multiplicity": module.lr_multiplicity,
                      "hierarchical_schema": module.hierarchical_schema,
                      "block_input_Ls": [int(b["input_L"]) for b in module._blocks]},
            "block_powers": [dict({"block_index": int(r["block_index"]), "output_L": int(r["output_L"])},
                                  **_tables(r["plan"])) for r in module.block_power_requests()],
            "inputs": [i.detach().tolist() for i in inputs],
            "output": _pairs(out),
            "gradient": [g.detach().tolist() for g in grads],
            "direction": [d.tolist() for d in direction],
            "hvp": [h.tolist() for h in hvp],
            "readout": {"weight": weight.tolist(), "bias": 0.25, "output": _pairs(readout)},
            "report": _jsonable(module.runtime_report()),
        })
        print(name, tuple(out.shape), file=sys.stderr)

    groups = []
    for gi, (members, bindings, policy) in enumerate((
            (("rank3_L1", "rank3_L2"), ((0, 1), (0, 1)), "individual"),
            (("rank3_L1", "rank3_L2"), ((0, 1), (0, 1)), "shared_monomial"),
            (("rank9",), ((0,),), "shared_monomial"),
            (("rank12", "ordinary_rank4"), ((0, 1), (1, 0)), "individual"))):
        mods = tuple(modules[m] for m in members)
        group = YE3THierarchicalRepeatedBlockModuleGroup(mods, bindings, block_power_execution_policy=policy)
        gen = torch.Generator().manual_seed(2000 + gi)
        width = {}
        for mod, row in zip(mods, bindings):
            for blk, b in zip(mod._blocks, row):
                width[b] = 2 * int(blk["input_L"]) + 1
        inputs = tuple(torch.randn((5, width[b]), generator=gen, dtype=torch.float64).requires_grad_(True)
                       for b in range(len(width)))
        out = group.forward_packed(inputs)
        grads, direction, hvp = _derivatives(out, inputs, gen)
        report = group.runtime_report()
        groups.append({
            "members": list(members), "bindings": [list(r) for r in bindings], "block_power_policy": policy,
            "inputs": [i.detach().tolist() for i in inputs], "output": _pairs(out),
            "gradient": [g.detach().tolist() for g in grads], "direction": [d.tolist() for d in direction],
            "hvp": [h.tolist() for h in hvp],
            "report_counts": {k: report[k] for k in ("member_plan_count", "block_power_request_count",
                                                     "block_power_evaluation_count", "block_power_reuse_count",
                                                     "shared_power_group_count", "output_dimension")
                              if k in report},
        })
        print("group", members, policy, tuple(out.shape), file=sys.stderr)

    with open(OUT, "w") as fh:
        json.dump({"schema": "ye3t_amd_hierarchical_fixture_v1", "cases": cases, "groups": groups}, fh)
        fh.write("\n")


if __name__ == "__main__":
    main()
