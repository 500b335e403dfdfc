"""Hierarchical repeated-block runtime on the device.

The reference's ``ye3t.runtime.hierarchical`` (``ye3t/runtime/hierarchical.py``)
evaluates one ``block_symmetric_power`` instruction of an execution plan whose
metadata follows ``ye3t_hierarchical_repeated_angular_blocks_v1`` or ``_v2``:

1. **block powers** -- each compiler-factored block's input multiplet
   (``2 input_L + 1`` complex values) goes through a
   ``SymmetricPowerProductPlan``: descriptors are sparse combinations of
   degree-``power`` monomials (``symmetric_power_product_plan_contraction``,
   ``ye3t/runtime/symmetric_power.py:879-927``);
2. **routes** -- products of block outputs coupled by angular synthesis
   tables applied as ``C^dagger`` (two blocks: grouped binary CG; v2: a sparse
   factorized outer product over any number of blocks);
3. **LR analysis** -- every route times the conjugate LR synthesis row of each
   tableau.

Here the block powers run on the library's sparse shared-monomial kernels
(real or complex, with adjoint and double backward, so gradients and
Hessian-vector products stay on the device), the routes and LR analysis on
device tensor ops, and a module group's destination-segmented schedule on the
segmented factorized-angular kernel.  Nothing runs on the CPU: a CPU device
raises, and ``backend="reference"`` (the reference's Torch branch) is not
carried.
"""

import json
import math
import os
from dataclasses import dataclass, field

from ye3t_amd.couplings import _convention_hash
from ye3t_amd.runtime import native
from ye3t_amd.runtime.execution_plan import ExecutionPlan

HIERARCHICAL_SCHEMAS = ("ye3t_hierarchical_repeated_angular_blocks_v1",
                        "ye3t_hierarchical_repeated_angular_blocks_v2")
_V2 = HIERARCHICAL_SCHEMAS[1]


# ---- compiler power plans (ye3t/couplings/__init__.py:2275-2440) ------------------------------------------

@dataclass(frozen=True)
class SymmetricPowerBlockPlan:
    """One descriptor of a symmetric-power plan (reference
    ``SymmetricPowerBlockPlan``, ``couplings/__init__.py:2275-2336``):
    ``component_terms`` are ``{"exponents": tuple, "coefficient": complex}``
    over ``channel_indices``."""

    descriptor_index: int
    channel_indices: tuple
    power: int
    input_L: int
    output_L: int
    multiplicity_index: int
    component_index: int
    component_terms: tuple
    lower_degree_exponents: tuple = ()
    coefficient_entry_count: int = 0
    validation_report: dict = field(default_factory=dict)

    def to_dict(self):
        return {
            "descriptor_index": int(self.descriptor_index),
            "channel_indices": [int(v) for v in self.channel_indices],
            "power": int(self.power), "input_L": int(self.input_L), "output_L": int(self.output_L),
            "multiplicity_index": int(self.multiplicity_index), "component_index": int(self.component_index),
            "component_terms": [{"exponents": [int(v) for v in t["exponents"]],
                                 "coefficient": [float(t["coefficient"].real), float(t["coefficient"].imag)]}
                                for t in self.component_terms],
            "lower_degree_exponents": [[int(v) for v in e] for e in self.lower_degree_exponents],
            "coefficient_entry_count": int(self.coefficient_entry_count),
            "validation_report": dict(self.validation_report),
        }

    @classmethod
    def from_dict(cls, p):
        return cls(descriptor_index=int(p["descriptor_index"]),
                   channel_indices=tuple(int(v) for v in p["channel_indices"]), power=int(p["power"]),
                   input_L=int(p["input_L"]), output_L=int(p["output_L"]),
                   multiplicity_index=int(p["multiplicity_index"]), component_index=int(p["component_index"]),
                   component_terms=tuple({"exponents": tuple(int(v) for v in t["exponents"]),
                                          "coefficient": complex(*t["coefficient"])}
                                         for t in p.get("component_terms", ())),
                   lower_degree_exponents=tuple(tuple(int(v) for v in e)
                                                for e in p.get("lower_degree_exponents", ())),
                   coefficient_entry_count=int(p.get("coefficient_entry_count", 0)),
                   validation_report=dict(p.get("validation_report", {})))


@dataclass(frozen=True)
class SymmetricPowerProductPlan:
    """Compiler-owned exponent-vector plan of one block power (reference
    ``SymmetricPowerProductPlan``, ``couplings/__init__.py:2339-2422``);
    ``from_dict`` checks ``convention_hash`` as the reference does."""

    entries: tuple
    descriptor_count: int
    channel_count: int
    carrier: str
    target: dict
    factor_basis: str
    normalization_convention: str
    coefficient_source: str
    label_source: str
    backend: str
    convention_hash: str = ""
    validation_report: dict = field(default_factory=dict)
    provenance: dict = field(default_factory=dict)

    @property
    def active_descriptor_indices(self):
        return tuple(sorted(int(e.descriptor_index) for e in self.entries))

    def to_dict(self):
        return {
            "entries": [e.to_dict() for e in self.entries], "descriptor_count": int(self.descriptor_count),
            "channel_count": int(self.channel_count),
            "active_descriptor_indices": list(self.active_descriptor_indices), "carrier": str(self.carrier),
            "target": dict(self.target), "factor_basis": str(self.factor_basis),
            "normalization_convention": str(self.normalization_convention),
            "coefficient_source": str(self.coefficient_source), "label_source": str(self.label_source),
            "backend": str(self.backend), "convention_hash": str(self.convention_hash),
            "validation_report": dict(self.validation_report), "provenance": dict(self.provenance),
        }

    @classmethod
    def from_dict(cls, p):
        entries = tuple(SymmetricPowerBlockPlan.from_dict(e) for e in p.get("entries", ()))
        plan = cls(entries=entries, descriptor_count=int(p["descriptor_count"]),
                   channel_count=int(p["channel_count"]), carrier=str(p["carrier"]), target=dict(p["target"]),
                   factor_basis=str(p["factor_basis"]), normalization_convention=str(p["normalization_convention"]),
                   coefficient_source=str(p["coefficient_source"]), label_source=str(p["label_source"]),
                   backend=str(p["backend"]), convention_hash=str(p.get("convention_hash", "")),
                   validation_report=dict(p.get("validation_report", {})), provenance=dict(p.get("provenance", {})))
        expected = _convention_hash({
            "entries": [e.to_dict() for e in entries], "descriptor_count": plan.descriptor_count,
            "channel_count": plan.channel_count, "carrier": plan.carrier, "target": dict(plan.target),
            "factor_basis": plan.factor_basis, "normalization_convention": plan.normalization_convention,
            "basis_convention": str(plan.validation_report.get("basis_convention", "real_tesseral")),
            "backend": plan.backend})
        if plan.convention_hash and plan.convention_hash != expected:
            raise ValueError("symmetric-power plan convention hash does not match payload")
        return plan


def symmetric_power_plan_key(plan):
    """Numeric identity of a power contraction (reference
    ``_symmetric_power_plan_key``, ``runtime/hierarchical.py:40-76``): equal
    keys evaluate the same descriptors whatever their provenance."""
    payload = {
        "descriptor_count": int(plan.descriptor_count), "channel_count": int(plan.channel_count),
        "carrier": str(plan.carrier), "factor_basis": str(plan.factor_basis),
        "normalization_convention": str(plan.normalization_convention),
        "entries": [{"descriptor_index": int(e.descriptor_index),
                     "channel_indices": [int(v) for v in e.channel_indices], "power": int(e.power),
                     "input_L": int(e.input_L), "output_L": int(e.output_L),
                     "multiplicity_index": int(e.multiplicity_index), "component_index": int(e.component_index),
                     "component_terms": [{"exponents": [int(v) for v in t["exponents"]],
                                          "coefficient": [float(complex(t["coefficient"]).real),
                                                          float(complex(t["coefficient"]).imag)]}
                                         for t in e.component_terms]}
                    for e in plan.entries],
    }
    return json.dumps(payload, sort_keys=True, separators=(",", ":"))


# ---- lowering to monomial tables (ye3t/runtime/symmetric_power.py:144-193, 740-876) -----------------------

def product_plan_count_table(plan, imag_tol=1.0e-12, complex_output=True):
    """The grouped table of a power plan: entries' terms on the full channel
    axis, equal (descriptor, exponent row) pairs summed, coefficients at or
    below ``imag_tol`` in modulus dropped, rows by descriptor then exponent
    row.  Returns ``(counts, offsets, output_index, values)`` as host lists
    (reference ``_symmetric_power_product_plan_count_table``)."""
    D, C = int(plan.descriptor_count), int(plan.channel_count)
    accumulated = {}
    for entry in plan.entries:
        d = int(entry.descriptor_index)
        if d < 0 or d >= D:
            raise ValueError("symmetric-power plan descriptor index is outside descriptor_count")
        channels = tuple(int(v) for v in entry.channel_indices)
        for term in entry.component_terms:
            exps = tuple(int(v) for v in term["exponents"])
            if len(exps) != len(channels):
                raise ValueError("symmetric-power plan exponent width does not match its channel indices")
            counts = [0] * C
            for local, e in enumerate(exps):
                c = channels[local]
                if c < 0 or c >= C:
                    raise ValueError("symmetric-power plan channel index is outside channel_count")
                counts[c] += e
            key = (d, tuple(counts))
            accumulated[key] = accumulated.get(key, 0.0 + 0.0j) + complex(term["coefficient"])
    by_descriptor = [[] for _ in range(D)]
    for (d, counts), coefficient in accumulated.items():
        if abs(coefficient) > float(imag_tol):
            by_descriptor[d].append((counts, coefficient))
    rows, offsets, index, values = [], [0], [], []
    for d in range(D):
        for counts, coefficient in sorted(by_descriptor[d], key=lambda item: item[0]):
            rows.append(counts)
            index.append(d)
            values.append(coefficient if complex_output else coefficient.real)
        offsets.append(len(rows))
    return rows, offsets, index, values


def shared_table(count_rows, output_offsets, coefficient_outputs, coefficient_values):
    """Unique monomials (first-appearance order) and, per coefficient, its
    monomial: ``(monomial_counts, output_offsets, coefficient_terms,
    coefficient_outputs, coefficient_values)`` (reference
    ``_shared_symmetric_power_table``)."""
    unique, lookup, terms = [], {}, []
    for row in count_rows:
        key = tuple(int(v) for v in row)
        if key not in lookup:
            lookup[key] = len(unique)
            unique.append(key)
        terms.append(lookup[key])
    return unique, list(output_offsets), terms, list(coefficient_outputs), list(coefficient_values)


def sparse_supports(monomial_counts):
    """Sparse supports of dense exponent rows: ``(term_offsets,
    term_components, term_exponents)`` with each row's nonzero exponents in
    component order (the product the dense rows define, without the x^0 factors)."""
    offsets, comps, exps = [0], [], []
    for row in monomial_counts:
        for c, e in enumerate(row):
            if e:
                comps.append(c)
                exps.append(int(e))
        offsets.append(len(comps))
    return offsets, comps, exps


def symmetric_power_product_plan_table_report(plan, imag_tol=1.0e-12, complex_output=True):
    """Size report of a plan's grouped and shared tables (reference
    ``symmetric_power_product_plan_table_report``, ``symmetric_power.py:95-142``):
    the byte count is that of the reference's int64 / complex128 tensors."""
    rows, offsets, index, values = product_plan_count_table(plan, imag_tol, complex_output)
    unique = shared_table(rows, offsets, index, values)[0]
    C, R, M = int(plan.channel_count), len(rows), len(unique)
    value_bytes = 16 if complex_output else 8
    grouped_bytes = R * C * 8 + len(offsets) * 8 + R * 8 + R * value_bytes
    shared_bytes = M * C * 8 + len(offsets) * 8 + R * 8 + R * 8 + R * value_bytes
    powers = tuple(sorted({int(e.power) for e in plan.entries}))
    return {
        "channel_count": C, "descriptor_count": int(plan.descriptor_count), "entry_count": len(plan.entries),
        "powers": powers, "maximum_power": max(powers) if powers else None, "coefficient_count": R,
        "unique_monomial_count": M, "coefficient_reuse": float(R) / float(M) if M else 0.0,
        "cached_grouped_and_shared_table_bytes": int(grouped_bytes + shared_bytes),
        "output_dtype": "torch.complex128" if complex_output else "torch.float64",
        "selection_policy": os.environ.get("YE3T_SYMMETRIC_POWER_SHARED_TABLE_POLICY", "auto"),
        "runtime_path_discovery": False,
    }


_TABLE_CACHE = {}


def _device_table(counts_rows, offsets, outputs, values, channel_count, device, dtype):
    """A ``native.SparseMonomialTable`` of a grouped table (cached by content)."""
    unique, offs, terms, outs, vals = shared_table(counts_rows, offsets, outputs, values)
    key = (tuple(unique), tuple(offs), tuple(terms), tuple(outs), tuple(vals), int(channel_count), str(device),
           str(dtype))
    table = _TABLE_CACHE.get(key)
    if table is None:
        toff, comp, ex = sparse_supports(unique)
        table = native.SparseMonomialTable(int(channel_count), toff, comp, ex, offs, terms, outs, vals, device,
                                           dtype)
        _TABLE_CACHE[key] = table
    return table


def _table_functions():
    import torch

    class _Apply(torch.autograd.Function):
        """Forward of a sparse monomial table; its backward is differentiable."""

        @staticmethod
        def forward(ctx, x, table):
            ctx.save_for_backward(x)
            ctx.table = table
            return table.forward(x)

        @staticmethod
        def backward(ctx, g):
            (x,) = ctx.saved_tensors
            return _Adjoint.apply(g.contiguous(), x, ctx.table), None

    class _Adjoint(torch.autograd.Function):
        """``A(g, x) = sum g conj(c) conj(dm/dx)``; its backward is the
        library's double backward: the forward's directional derivative for
        ``g`` and the Hessian term for ``x``."""

        @staticmethod
        def forward(ctx, g, x, table):
            ctx.save_for_backward(g, x)
            ctx.table = table
            return table.adjoint(g, x)

        @staticmethod
        def backward(ctx, t):
            g, x = ctx.saved_tensors
            out_t, in_t = ctx.table.double_backward(t.contiguous(), g, x)
            return out_t, in_t, None

    return _Apply


_APPLY = None


def apply_table(x, table):
    """``table`` applied to the rows of ``x`` (``[..., D]``), differentiable twice."""
    global _APPLY
    if _APPLY is None:
        _APPLY = _table_functions()
    flat = x.reshape(-1, int(x.shape[-1])).contiguous()
    out = _APPLY.apply(flat, table)
    return out.reshape(tuple(x.shape[:-1]) + (int(out.shape[-1]),))


def symmetric_power_product_plan_contraction(input, plan, *, backend="auto", imag_tol=1.0e-12):
    """Descriptors of a compiler power plan on the device (reference
    ``symmetric_power_product_plan_contraction``, ``symmetric_power.py:879-927``):
    the input is converted to the table's dtype (complex when the input is
    complex or the coefficients are) and contracted with the plan's shared
    monomial table in sparse form."""
    import torch

    if backend not in ("auto", "native"):
        raise ValueError("backend must be auto or native (the reference's Torch branch is not carried)")
    input = torch.as_tensor(input)
    if input.ndim < 1:
        raise ValueError("symmetric-power product-plan input requires a channel axis")
    if int(input.shape[-1]) != int(plan.channel_count):
        raise ValueError("symmetric-power plan channel_count does not match input")
    if input.device.type != "cuda":
        raise NotImplementedError("symmetric_power_product_plan_contraction runs on the GPU only")
    has_complex = any(abs(complex(t["coefficient"]).imag) > float(imag_tol)
                      for e in plan.entries for t in e.component_terms)
    if input.dtype in (torch.complex64, torch.complex128):
        out_dtype = input.dtype
    elif has_complex:
        out_dtype = torch.complex128 if input.dtype == torch.float64 else torch.complex64
    else:
        out_dtype = input.dtype
    rows, offsets, index, values = product_plan_count_table(plan, imag_tol, out_dtype.is_complex)
    table = _device_table(rows, offsets, index, values, plan.channel_count, input.device, out_dtype)
    return apply_table(input.to(out_dtype), table)


# ---- the module ----------------------------------------------------------------------------------------

def _dense_synthesis(table, dtype, device):
    import torch

    matrix = torch.zeros((int(table.input_dimension), int(table.output_dimension)), dtype=dtype, device=device)
    rows = torch.tensor(table.row_indices, dtype=torch.long, device=device)
    cols = torch.tensor(table.column_indices, dtype=torch.long, device=device)
    vals = torch.tensor(table.values, dtype=dtype, device=device)
    matrix.index_put_((rows, cols), vals, accumulate=True)
    return matrix


def _resolve_device(device):
    import torch

    if device is None:
        if not torch.cuda.is_available():
            raise NotImplementedError("the hierarchical runtime needs a GPU (no CPU path)")
        return torch.device("cuda", torch.cuda.current_device())
    device = torch.device(device)
    if device.type != "cuda":
        raise NotImplementedError("the hierarchical runtime runs on the GPU only")
    return device


def _torch_module_base():
    import torch

    return torch.nn.Module


class YE3THierarchicalRepeatedBlockModule(_torch_module_base()):
    """One factored Schur/LR repeated-angular instruction (reference
    ``YE3THierarchicalRepeatedBlockModule``, ``runtime/hierarchical.py:79-605``):
    same constructor, ``forward`` / ``forward_flat`` / ``linear_readout`` /
    ``runtime_report`` / ``block_power_requests``, same validation errors.
    Outputs are ``[..., channel_count, tableau_count, magnetic_count]``
    complex; gradients and Hessian-vector products run on the device."""

    def __init__(self, execution_plan, instruction_id=None, backend="auto", dtype=None, device=None):
        import torch

        super().__init__()
        if not isinstance(execution_plan, ExecutionPlan):
            execution_plan = ExecutionPlan.from_dict(execution_plan)
        instructions = {str(i["instruction_id"]): i for i in execution_plan.instructions}
        if instruction_id is None:
            if len(execution_plan.forward_schedule) != 1:
                raise ValueError("instruction_id is required for a multi-instruction plan")
            instruction_id = execution_plan.forward_schedule[0]
        instruction_id = str(instruction_id)
        if instruction_id not in instructions:
            raise ValueError("instruction_id is not present in the execution plan")
        instruction = instructions[instruction_id]
        metadata = dict(instruction.get("metadata", {}))
        if instruction.get("opcode") != "block_symmetric_power":
            raise ValueError("hierarchical repeated-block runtime requires block_symmetric_power")
        schema = metadata.get("schema")
        if schema not in HIERARCHICAL_SCHEMAS:
            raise ValueError("unsupported hierarchical repeated-block schema")
        if bool(metadata.get("runtime_path_discovery", True)):
            raise ValueError("hierarchical runtime forbids runtime path discovery")
        if bool(metadata.get("raw_angular_tree_forest_materialized", True)):
            raise ValueError("hierarchical runtime forbids raw angular tree forests")
        backend = str(backend)
        if backend not in {"auto", "native", "reference"}:
            raise ValueError("backend must be auto, native, or reference")
        if backend == "reference":
            raise NotImplementedError("the reference's Torch branch is not carried; use backend='auto' or 'native'")
        if dtype is None:
            dtype = torch.complex128
        if dtype not in (torch.complex64, torch.complex128):
            raise ValueError("hierarchical complex-magnetic plans require a complex dtype")
        device = _resolve_device(device)

        blocks = tuple(dict(b) for b in metadata["blocks"])
        power_plans = {}
        for record in metadata["block_power_plans"]:
            key = (int(record["block_index"]), int(record["output_L"]))
            if key in power_plans:
                raise ValueError("duplicate hierarchical block power plan")
            plan = SymmetricPowerProductPlan.from_dict(record["plan"])
            if int(plan.channel_count) != 2 * int(blocks[key[0]]["input_L"]) + 1:
                raise ValueError("hierarchical block power input width is inconsistent")
            power_plans[key] = plan
        if not power_plans:
            raise ValueError("hierarchical instruction has no block power plans")
        object.__setattr__(self, "_block_power_plans", power_plans)
        object.__setattr__(self, "_block_power_table_reports", tuple(
            dict({"block_index": k[0], "output_L": k[1]}, **symmetric_power_product_plan_table_report(p))
            for k, p in sorted(power_plans.items())))

        tables = {t.table_id: t for t in execution_plan.synthesis_tables}
        lr_id = str(metadata["lr_synthesis_table_id"])
        if lr_id not in tables:
            raise ValueError("hierarchical LR synthesis table is missing")
        self.register_buffer("lr_synthesis", _dense_synthesis(tables[lr_id], dtype, device), persistent=False)
        routes = tuple(dict(r) for r in metadata["routes"])
        if tuple(int(r["route_index"]) for r in routes) != tuple(range(len(routes))):
            raise ValueError("hierarchical routes must use canonical contiguous indices")
        cg_names, cg_sparse = {}, {}
        for table_id in sorted({str(r["angular_synthesis_table_id"]) for r in routes
                                if r.get("angular_synthesis_table_id") is not None}):
            if table_id not in tables:
                raise ValueError("hierarchical angular synthesis table is missing")
            t = tables[table_id]
            cg_sparse[table_id] = {"input_dimension": int(t.input_dimension),
                                   "output_dimension": int(t.output_dimension),
                                   "rows": tuple(int(v) for v in t.row_indices),
                                   "columns": tuple(int(v) for v in t.column_indices),
                                   "values": tuple(complex(v) for v in t.values)}
            if schema != _V2:
                name = "cg_synthesis_" + str(len(cg_names))
                self.register_buffer(name, _dense_synthesis(t, dtype, device), persistent=False)
                cg_names[table_id] = name
        object.__setattr__(self, "_cg_buffer_names", cg_names)
        object.__setattr__(self, "_cg_sparse_entries", cg_sparse)
        object.__setattr__(self, "_routes", routes)
        object.__setattr__(self, "_blocks", blocks)

        out_carrier = instruction.get("output_carrier")
        layouts = [layout for layout in execution_plan.carrier_layouts if layout.get("key") == out_carrier]
        if len(layouts) != 1:
            raise ValueError("hierarchical instruction must have one output layout")
        layout = layouts[0]
        self.instruction_id = instruction_id
        self.backend = backend
        self.plan_hash = str(execution_plan.plan_hash)
        self.coefficient_hash = str(execution_plan.coefficient_hash)
        self.channel_count = int(layout["channel_count"])
        self.tableau_count = int(layout["tableau_count"])
        self.magnetic_count = int(layout["magnetic_count"])
        self.output_dimension = int(layout["width"])
        self.target_L = int(metadata["target_L"])
        self.target_parity = metadata.get("target_parity")
        self.lr_multiplicity = int(metadata["lr_multiplicity"])
        self.block_count = len(blocks)
        self.route_count = len(routes)
        self.hierarchical_schema = str(schema)
        self.last_backend = None
        self.last_linear_readout_backend = None
        if schema != _V2 and self.block_count not in (1, 2):
            raise ValueError("hierarchical repeated-block runtime currently requires one or two compiler-factored "
                             "blocks")
        if self.channel_count != self.route_count * self.lr_multiplicity:
            raise ValueError("hierarchical route/LR count does not match output layout")
        if tuple(self.lr_synthesis.shape) != (self.lr_multiplicity, self.tableau_count):
            raise ValueError("hierarchical LR synthesis dimensions are inconsistent")

        def index_buffer(name, values):
            self.register_buffer(name, torch.tensor(tuple(int(v) for v in values), dtype=torch.long, device=device),
                                 persistent=False)

        generic, groups = [], []
        if schema == _V2:
            for ri, route in enumerate(routes):
                sparse = cg_sparse[str(route["angular_synthesis_table_id"])]
                out_Ls = tuple(int(v) for v in route["block_output_Ls"])
                mults = tuple(int(v) for v in route["block_multiplicity_indices"])
                widths = tuple(2 * v + 1 for v in out_Ls)
                columns = []
                for bi, width in enumerate(widths):
                    stride = math.prod(widths[bi + 1:])
                    name = f"generic_route_{ri}_block_{bi}"
                    index_buffer(name, (mults[bi] * width + (row // stride) % width for row in sparse["rows"]))
                    columns.append(name)
                index_buffer(f"generic_route_{ri}_output", sparse["columns"])
                self.register_buffer(f"generic_route_{ri}_coefficient",
                                     torch.tensor(tuple(v.conjugate() for v in sparse["values"]), dtype=dtype,
                                                  device=device), persistent=False)
                generic.append({"route_index": ri, "output_Ls": out_Ls, "component_columns": tuple(columns),
                                "output_indices": f"generic_route_{ri}_output",
                                "coefficients": f"generic_route_{ri}_coefficient"})
        elif self.block_count == 1:
            index_buffer("single_block_route_indices", (r["block_multiplicity_indices"][0] for r in routes))
        else:
            by_table = {}
            for route in routes:
                by_table.setdefault(str(route["angular_synthesis_table_id"]), []).append(route)
            for gi, table_id in enumerate(sorted(by_table)):
                members = by_table[table_id]
                index_buffer(f"route_left_indices_{gi}", (r["block_multiplicity_indices"][0] for r in members))
                index_buffer(f"route_right_indices_{gi}", (r["block_multiplicity_indices"][1] for r in members))
                index_buffer(f"route_output_indices_{gi}", (r["route_index"] for r in members))
                groups.append({"table_id": table_id, "left_L": int(members[0]["block_output_Ls"][0]),
                               "right_L": int(members[0]["block_output_Ls"][1]), "route_count": len(members),
                               "left_indices": f"route_left_indices_{gi}",
                               "right_indices": f"route_right_indices_{gi}",
                               "output_indices": f"route_output_indices_{gi}"})
        object.__setattr__(self, "_generic_routes", tuple(generic))
        object.__setattr__(self, "_route_groups", tuple(groups))

    def block_power_requests(self):
        return tuple({"block_index": int(b), "output_L": int(L), "plan_key": symmetric_power_plan_key(plan),
                      "plan": plan} for (b, L), plan in sorted(self._block_power_plans.items()))

    def _evaluate_block_plans(self, block_inputs):
        evaluated = {}
        for key, plan in self._block_power_plans.items():
            block_index, output_L = key
            value = symmetric_power_product_plan_contraction(block_inputs[block_index], plan, backend="auto")
            m = 2 * output_L + 1
            if int(plan.descriptor_count) % m:
                raise ValueError("block power descriptor layout is not multiplet-complete")
            evaluated[key] = value.reshape(tuple(value.shape[:-1]) + (int(plan.descriptor_count) // m, m))
        return evaluated

    def _evaluate_routes(self, evaluated, leading):
        import torch

        if self.hierarchical_schema == _V2:
            values = []
            for route in self._generic_routes:
                terms = getattr(self, route["coefficients"]).reshape((1,) * len(leading) + (-1,))
                for bi, L in enumerate(route["output_Ls"]):
                    block = evaluated[(bi, int(L))].reshape(tuple(leading) + (-1,))
                    terms = terms * block.index_select(-1, getattr(self, route["component_columns"][bi]))
                out = torch.zeros(tuple(leading) + (self.magnetic_count,), dtype=self.lr_synthesis.dtype,
                                  device=self.lr_synthesis.device)
                values.append(out.index_add(-1, getattr(self, route["output_indices"]), terms))
            return torch.stack(values, dim=-2)
        if self.block_count == 1:
            return evaluated[(0, self.target_L)].index_select(-2, self.single_block_route_indices)
        out = torch.zeros(tuple(leading) + (self.route_count, self.magnetic_count), dtype=self.lr_synthesis.dtype,
                          device=self.lr_synthesis.device)
        for group in self._route_groups:
            left = evaluated[(0, group["left_L"])].index_select(-2, getattr(self, group["left_indices"]))
            right = evaluated[(1, group["right_L"])].index_select(-2, getattr(self, group["right_indices"]))
            product = (left.unsqueeze(-1) * right.unsqueeze(-2)).reshape(tuple(leading) + (group["route_count"], -1))
            coupled = torch.matmul(product, getattr(self, self._cg_buffer_names[group["table_id"]]).conj())
            out = out.index_copy(len(leading), getattr(self, group["output_indices"]), coupled)
        return out

    def _forward_from_evaluated(self, evaluated, leading):
        routes = self._evaluate_routes(evaluated, leading)
        analysis = self.lr_synthesis.conj().reshape((1,) * len(leading) +
                                                    (1, self.lr_multiplicity, self.tableau_count, 1))
        output = routes.unsqueeze(-2).unsqueeze(-2) * analysis
        return output.reshape(tuple(leading) + (self.channel_count, self.tableau_count, self.magnetic_count))

    def _convert_inputs(self, block_inputs):
        import torch

        if len(block_inputs) == 1 and isinstance(block_inputs[0], (tuple, list)):
            block_inputs = tuple(block_inputs[0])
        if len(block_inputs) != self.block_count:
            raise ValueError("hierarchical input count does not match block count")
        converted, leading = [], None
        for block, value in zip(self._blocks, block_inputs):
            value = torch.as_tensor(value, dtype=self.lr_synthesis.dtype, device=self.lr_synthesis.device)
            if int(value.shape[-1]) != 2 * int(block["input_L"]) + 1:
                raise ValueError("hierarchical block input multiplet width is incorrect")
            current = tuple(value.shape[:-1])
            if leading is None:
                leading = current
            elif current != leading:
                raise ValueError("hierarchical block inputs require matching leading shapes")
            converted.append(value)
        return tuple(converted), leading

    def forward(self, *block_inputs):
        converted, leading = self._convert_inputs(block_inputs)
        output = self._forward_from_evaluated(self._evaluate_block_plans(converted), leading)
        self.last_backend = ("shared_monomial_then_sparse_factorized_outer_then_lr_analysis"
                             if self.hierarchical_schema == _V2
                             else "shared_monomial_then_grouped_binary_cg_then_lr_analysis")
        return output

    def forward_flat(self, *block_inputs):
        output = self.forward(*block_inputs)
        return output.reshape(tuple(output.shape[:-3]) + (self.output_dimension,))

    def linear_readout(self, source, weight, bias):
        import torch

        inputs = tuple(source) if isinstance(source, (tuple, list)) else (source,)
        features = self.forward_flat(*inputs)
        weight = torch.as_tensor(weight, dtype=features.dtype, device=features.device)
        bias = torch.as_tensor(bias, dtype=features.dtype, device=features.device).reshape(())
        if weight.ndim != 1 or int(weight.numel()) != self.output_dimension:
            raise ValueError("hierarchical readout weight has the wrong width")
        self.last_linear_readout_backend = "materialized_hierarchical_readout"
        return features @ weight + bias

    def runtime_report(self):
        v2 = self.hierarchical_schema == _V2
        return {
            "runtime": "YE3THierarchicalRepeatedBlockModule", "instruction_id": str(self.instruction_id),
            "plan_hash": self.plan_hash, "coefficient_hash": self.coefficient_hash,
            "block_count": self.block_count, "route_count": self.route_count,
            "channel_count": self.channel_count, "tableau_count": self.tableau_count,
            "magnetic_count": self.magnetic_count, "target_L": self.target_L, "target_parity": self.target_parity,
            "backend": self.backend, "last_backend": self.last_backend,
            "last_linear_readout_backend": self.last_linear_readout_backend,
            "runtime_path_discovery": False, "raw_angular_tree_forest_materialized": False,
            "composition": "shared_block_power_then_" + ("sparse_factorized_outer_C_dagger_then_LR_C_dagger" if v2
                                                         else "grouped_binary_C_dagger_then_LR_C_dagger"),
            "block_power_table_reports": tuple(dict(r) for r in self._block_power_table_reports),
            "supports_autograd_vjp_hvp": True,
            "device_kernels": "symmetric_power_shared_sparse_monomial (+ adjoint, double backward)",
        }


# ---- module groups (reference runtime/hierarchical.py:608-1650) -----------------------------------------

def _group_functions():
    import torch

    class _Destination(torch.autograd.Function):
        """Forward: block powers, then the destination-segmented
        factorized-angular kernel.  Backward: the same map recomputed as the
        members' routes and LR analysis on the device (differentiable again,
        so Hessian-vector products hold); the two agree to rounding."""

        @staticmethod
        def forward(ctx, group, *inputs):
            ctx.group = group
            ctx.save_for_backward(*inputs)
            with torch.no_grad():
                powers, leading = group._evaluate_unique_powers(inputs)
                return group._destination_segmented_output(powers, leading)

        @staticmethod
        def backward(ctx, g):
            inputs = ctx.saved_tensors
            needs = [i for i, t in enumerate(inputs) if t.requires_grad]
            grads = [None] * len(inputs)
            if needs:
                create = torch.is_grad_enabled()
                with torch.enable_grad():
                    out = ctx.group._composite_packed(inputs)
                    got = torch.autograd.grad(out, [inputs[i] for i in needs], g, create_graph=create,
                                              allow_unused=True)
                for i, v in zip(needs, got):
                    grads[i] = v
            return (None, *grads)

    return _Destination


_DESTINATION = None


class YE3THierarchicalRepeatedBlockModuleGroup(_torch_module_base()):
    """Several hierarchical modules sharing physical block inputs (reference
    ``YE3THierarchicalRepeatedBlockModuleGroup``, ``runtime/hierarchical.py:
    608-1650``): compiler-identical block powers are evaluated once
    (``block_power_execution_policy="shared_monomial"`` evaluates all powers
    of one binding as one shared monomial table), and with
    ``parent_execution_policy`` ``"auto"`` or ``"destination_segmented"`` the
    members' routes and LR analysis run as one segmented factorized-angular
    launch over the gathered powers (the library's segmented kernel)."""

    def __init__(self, modules, block_binding_indices_by_module, parent_execution_policy="reference",
                 block_power_execution_policy="individual"):
        super().__init__()
        modules = tuple(modules)
        if not modules:
            raise ValueError("hierarchical module group requires at least one module")
        if any(not isinstance(m, YE3THierarchicalRepeatedBlockModule) for m in modules):
            raise ValueError("hierarchical module group accepts only compiler-owned hierarchical modules")
        rows = tuple(tuple(int(v) for v in row) for row in block_binding_indices_by_module)
        if len(rows) != len(modules):
            raise ValueError("hierarchical block binding rows must match the module count")
        for module, row in zip(modules, rows):
            if len(row) != int(module.block_count):
                raise ValueError("hierarchical block binding count must match compiler blocks")
            if any(v < 0 for v in row):
                raise ValueError("hierarchical block binding indices must be nonnegative")
        bindings = tuple(sorted({v for row in rows for v in row}))
        if bindings != tuple(range(len(bindings))):
            raise ValueError("hierarchical block binding indices must be canonical and contiguous")
        first = modules[0]
        if any(m.lr_synthesis.dtype != first.lr_synthesis.dtype or m.lr_synthesis.device != first.lr_synthesis.device
               or m.backend != first.backend for m in modules[1:]):
            raise ValueError("hierarchical modules must share backend, dtype, and device")
        object.__setattr__(self, "_source_modules", modules)
        object.__setattr__(self, "_binding_rows", rows)

        records, lookup, per_module, requests = [], {}, [], 0
        for module, row in zip(modules, rows):
            current = {}
            for request in module.block_power_requests():
                b, L = int(request["block_index"]), int(request["output_L"])
                key = (row[b], str(request["plan_key"]))
                if key not in lookup:
                    lookup[key] = len(records)
                    records.append({"binding_index": row[b], "output_L": L, "plan": request["plan"],
                                    "plan_key": str(request["plan_key"])})
                current[(b, L)] = lookup[key]
                requests += 1
            per_module.append(current)
        object.__setattr__(self, "_unique_power_records", tuple(records))
        object.__setattr__(self, "_module_power_indices", tuple(per_module))

        parent_execution_policy = str(parent_execution_policy)
        if parent_execution_policy not in {"auto", "reference", "destination_segmented"}:
            raise ValueError("parent_execution_policy must be auto, reference, or destination_segmented")
        # the segmented kernel is part of the library this runtime already requires
        self.parent_execution_policy_requested = parent_execution_policy
        self.destination_native_capable = True
        self.destination_native_enabled = parent_execution_policy in {"auto", "destination_segmented"}
        block_power_execution_policy = str(block_power_execution_policy)
        if block_power_execution_policy not in {"individual", "shared_monomial"}:
            raise ValueError("block_power_execution_policy must be individual or shared_monomial")
        self.block_power_execution_policy = block_power_execution_policy

        slices, base = [], 0
        for mi, module in enumerate(modules):
            slices.append({"module_index": mi, "start": base, "stop": base + module.output_dimension,
                           "instruction_id": str(module.instruction_id), "plan_hash": str(module.plan_hash)})
            base += module.output_dimension
        self.output_slices = tuple(slices)
        self.output_dimension = int(base)
        self.unique_binding_count = len(bindings)
        self.power_request_count = int(requests)
        self.power_evaluation_count = len(records)
        self.shared_power_group_count = 0
        self.last_backend = None
        if block_power_execution_policy == "shared_monomial":
            self._prepare_shared_power_groups()
        if self.destination_native_enabled:
            self._prepare_destination_segmented_schedule()

    def _prepare_shared_power_groups(self):
        first = self._source_modules[0]
        by_binding = {}
        for index, record in enumerate(self._unique_power_records):
            by_binding.setdefault(int(record["binding_index"]), []).append(index)
        groups = []
        for binding in sorted(by_binding):
            indices = tuple(by_binding[binding])
            plans = tuple(self._unique_power_records[i]["plan"] for i in indices)
            widths = {int(p.channel_count) for p in plans}
            if len(widths) != 1:
                raise ValueError("shared hierarchical power bindings require one input channel dimension")
            rows, offsets, outputs, values, out_slices = [], [0], [], [], []
            term_base = out_base = 0
            for index, plan in zip(indices, plans):
                r, o, idx, v = product_plan_count_table(plan)
                rows.extend(r)
                offsets.extend(term_base + x for x in o[1:])
                outputs.extend(out_base + x for x in idx)
                values.extend(v)
                out_slices.append({"power_index": index, "start": out_base,
                                   "stop": out_base + int(plan.descriptor_count)})
                term_base += len(r)
                out_base += int(plan.descriptor_count)
            width = next(iter(widths))
            table = _device_table(rows, offsets, outputs, values, width, first.lr_synthesis.device,
                                  first.lr_synthesis.dtype)
            groups.append({"binding_index": binding, "power_indices": indices, "table": table,
                           "output_slices": tuple(out_slices), "input_dimension": width,
                           "output_dimension": out_base, "coefficient_count": len(values),
                           "unique_monomial_count": int(table.M)})
        object.__setattr__(self, "_shared_power_groups", tuple(groups))
        self.shared_power_group_count = len(groups)

    def _prepare_destination_segmented_schedule(self):
        """The members as one segmented factorized-angular DAG over the
        gathered block powers (reference ``runtime/hierarchical.py:892-1313``):
        segment k is member k; its sources are its routes, each packing the
        route's left (and right) block multiplet (absent components gather a
        zero sentinel column); a route group is a leaf, or a merge of a left
        and a right leaf by its CG table; every root projects each route
        source onto the member's (route, LR multiplicity, tableau) columns
        with the conjugate LR synthesis row, and a member's roots are summed
        after the launch."""
        import torch

        modules = self._source_modules
        first = modules[0]
        device, dtype = first.lr_synthesis.device, first.lr_synthesis.dtype
        power_offsets, width = [], 0
        for record in self._unique_power_records:
            power_offsets.append(width)
            width += int(record["plan"].descriptor_count)
        object.__setattr__(self, "_power_output_offsets", tuple(power_offsets))
        self.power_output_dimension = int(width)
        sentinel = width

        seg = {k: [] for k in ("source", "input", "input_dim", "ws", "ws_dim", "node", "root", "proj", "proj_dim",
                               "output")}
        seg["source"].append(0)
        seg["node"].append(0)
        seg["root"].append(0)
        seg["output"].append(0)
        nodes = {k: [] for k in ("offsets", "dims", "leaf", "left", "right")}
        coef_offsets, coef_rows, coef_cols, coef_vals = [], [], [], []
        roots, root_ps, root_pd, root_oo = [], [], [], []
        projections, gather, reports, expanded = [], [], [], []
        input_base = ws_base = coef_base = proj_base = out_base = 0

        for mi, (module, power_indices) in enumerate(zip(modules, self._module_power_indices)):
            S = int(module.route_count)
            logical = int(module.channel_count * module.tableau_count)
            if module.hierarchical_schema == _V2:
                raise NotImplementedError("destination-segmented execution covers the v1 schema's one- and two-block "
                                          "routes, as the reference's does")
            if module.block_count == 1:
                left_w, right_w = module.magnetic_count, 0
                route_groups = ({"routes": tuple(range(S)), "left_L": module.target_L, "right_L": None,
                                 "table_id": None},)
            else:
                left_w = max(2 * int(r["block_output_Ls"][0]) + 1 for r in module._routes)
                right_w = max(2 * int(r["block_output_Ls"][1]) + 1 for r in module._routes)
                route_groups = tuple({"routes": tuple(int(v) for v in
                                                      getattr(module, g["output_indices"]).cpu().tolist()),
                                      "left_L": g["left_L"], "right_L": g["right_L"], "table_id": g["table_id"]}
                                     for g in module._route_groups)
            W = left_w + right_w
            local_gather = [sentinel] * (S * W)
            for route in module._routes:
                ri = int(route["route_index"])
                for bi, (L, mult) in enumerate(zip(route["block_output_Ls"], route["block_multiplicity_indices"])):
                    m = 2 * int(L) + 1
                    src = power_offsets[power_indices[(bi, int(L))]] + int(mult) * m
                    dst = ri * W + (0 if bi == 0 else left_w)
                    for k in range(m):
                        local_gather[dst + k] = src + k
            gather.extend(local_gather)

            l_off, l_dim, l_leaf, l_left, l_right = [], [], [], [], []
            l_coef_off, l_rows, l_cols, l_vals, l_roots = [0], [], [], [], []
            cursor, leaves = 0, {}

            def leaf(offset, dim):
                nonlocal cursor
                key = (offset, dim)
                if key not in leaves:
                    leaves[key] = len(l_off)
                    l_off.append(cursor)
                    l_dim.append(dim)
                    l_leaf.append(offset)
                    l_left.append(-1)
                    l_right.append(-1)
                    l_coef_off.append(len(l_vals))
                    cursor += dim
                return leaves[key]

            for group in route_groups:
                ld = 2 * int(group["left_L"]) + 1
                left = leaf(0, ld)
                if group["right_L"] is None:
                    l_roots.append(left)
                    continue
                rd = 2 * int(group["right_L"]) + 1
                right = leaf(left_w, rd)
                sparse = module._cg_sparse_entries[str(group["table_id"])]
                if sparse["input_dimension"] != ld * rd or sparse["output_dimension"] != module.magnetic_count:
                    raise ValueError("hierarchical angular table dimensions do not match the compiled route")
                l_roots.append(len(l_off))
                l_off.append(cursor)
                l_dim.append(module.magnetic_count)
                l_leaf.append(-1)
                l_left.append(left)
                l_right.append(right)
                l_rows.extend(sparse["rows"])
                l_cols.extend(sparse["columns"])
                l_vals.extend(sparse["values"])
                l_coef_off.append(len(l_vals))
                cursor += module.magnetic_count

            stride = len(route_groups) * logical
            projection = torch.zeros((S, stride), dtype=dtype, device=device)
            analysis = module.lr_synthesis.conj()
            for root_index, group in enumerate(route_groups):
                root_ps.append(root_index * logical)
                root_pd.append(logical)
                root_oo.append(root_index * module.output_dimension)
                for ri in group["routes"]:
                    for mult in range(module.lr_multiplicity):
                        for tab in range(module.tableau_count):
                            col = (ri * module.lr_multiplicity + mult) * module.tableau_count + tab
                            projection[ri, root_index * logical + col] = analysis[mult, tab]
            shifted = [v + coef_base for v in l_coef_off]
            coef_offsets.extend(shifted if not coef_offsets else shifted[1:])
            coef_base += len(l_vals)
            for k, v in zip(("offsets", "dims", "leaf", "left", "right"), (l_off, l_dim, l_leaf, l_left, l_right)):
                nodes[k].extend(v)
            coef_rows.extend(l_rows)
            coef_cols.extend(l_cols)
            coef_vals.extend(l_vals)
            roots.extend(l_roots)
            projections.append(projection.reshape(-1))
            seg["source"].append(seg["source"][-1] + S)
            seg["input"].append(input_base)
            seg["input_dim"].append(W)
            seg["ws"].append(ws_base)
            seg["ws_dim"].append(cursor)
            seg["node"].append(seg["node"][-1] + len(l_off))
            seg["root"].append(seg["root"][-1] + len(l_roots))
            seg["proj"].append(proj_base)
            seg["proj_dim"].append(stride)
            wide = len(l_roots) * module.output_dimension
            seg["output"].append(out_base + wide)
            expanded.append({"module_index": mi, "start": out_base, "stop": out_base + wide,
                             "root_count": len(l_roots), "output_dimension": module.output_dimension})
            reports.append({"module_index": mi, "rank": int(sum(int(b["power"]) for b in module._blocks)),
                            "source_route_count": S, "input_dimension": W, "root_count": len(l_roots),
                            "node_count": len(l_off), "coefficient_count": len(l_vals),
                            "projection_nonzero_count": int(torch.count_nonzero(projection).item()),
                            "output_dimension": module.output_dimension, "expanded_output_dimension": wide})
            input_base += S * W
            ws_base += S * cursor
            proj_base += int(projection.numel())
            out_base += wide

        def ints(values):
            return torch.as_tensor(list(values), dtype=torch.int64, device=device).contiguous()

        self.register_buffer("destination_power_gather_indices", ints(gather), persistent=False)
        object.__setattr__(self, "_destination_tables", (
            ints(seg["source"]), ints(seg["input"]), ints(seg["input_dim"]), ints(seg["ws"]), ints(seg["ws_dim"]),
            ints(seg["node"]), ints(seg["root"]), ints(seg["proj"]), ints(seg["proj_dim"]), ints(seg["output"]),
            ints(nodes["offsets"]), ints(nodes["dims"]), ints(nodes["leaf"]), ints(nodes["left"]),
            ints(nodes["right"]), ints(coef_offsets), ints(coef_rows), ints(coef_cols),
            torch.as_tensor(coef_vals, dtype=dtype, device=device).contiguous(), ints(roots), ints(root_ps),
            ints(root_pd), ints(root_oo), torch.cat(tuple(projections)).contiguous()))
        self.destination_total_source_count = int(seg["source"][-1])
        self.destination_input_dimension = int(input_base)
        self.destination_workspace_dimension = int(ws_base)
        self.destination_output_dimension = int(out_base)
        object.__setattr__(self, "_destination_segment_reports", tuple(reports))
        object.__setattr__(self, "_destination_expanded_output_slices", tuple(expanded))

    def _destination_segmented_output(self, unique_powers, leading):
        import torch

        from ye3t_amd.runtime.dag import factorized_angular_segmented

        batch = math.prod(int(s) for s in leading)
        flat = torch.cat(tuple(v.reshape(batch, -1) for v in unique_powers), dim=1)
        if int(flat.shape[1]) != self.power_output_dimension:
            raise RuntimeError("hierarchical power arena width is inconsistent")
        padded = torch.cat((flat, flat.new_zeros((batch, 1))), dim=1)
        packed = padded.index_select(1, self.destination_power_gather_indices).contiguous()
        expanded = factorized_angular_segmented(packed, *self._destination_tables, self.destination_total_source_count,
                                                self.destination_workspace_dimension,
                                                self.destination_output_dimension)
        return torch.cat(tuple(expanded[:, r["start"]:r["stop"]].reshape(batch, r["root_count"],
                                                                          r["output_dimension"]).sum(dim=1)
                               for r in self._destination_expanded_output_slices), dim=1)

    def _evaluate_unique_powers(self, block_inputs):
        import torch

        block_inputs = tuple(block_inputs)
        if len(block_inputs) != self.unique_binding_count:
            raise ValueError("hierarchical grouped input count does not match physical bindings")
        first = self._source_modules[0]
        evaluated = [None] * len(self._unique_power_records)
        leading = None
        if self.block_power_execution_policy == "shared_monomial":
            for group in self._shared_power_groups:
                value = torch.as_tensor(block_inputs[group["binding_index"]], dtype=first.lr_synthesis.dtype,
                                        device=first.lr_synthesis.device)
                if int(value.shape[-1]) != group["input_dimension"]:
                    raise ValueError("hierarchical shared-power input width is incorrect")
                current = tuple(value.shape[:-1])
                if leading is None:
                    leading = current
                elif current != leading:
                    raise ValueError("hierarchical grouped inputs require matching leading shapes")
                packed = apply_table(value, group["table"])
                for piece in group["output_slices"]:
                    record = self._unique_power_records[piece["power_index"]]
                    m = 2 * int(record["output_L"]) + 1
                    evaluated[piece["power_index"]] = packed[..., piece["start"]:piece["stop"]].reshape(
                        current + (int(record["plan"].descriptor_count) // m, m))
            if any(v is None for v in evaluated):
                raise RuntimeError("hierarchical shared-power schedule omitted a request")
            return tuple(evaluated), tuple(leading)
        for index, record in enumerate(self._unique_power_records):
            value = torch.as_tensor(block_inputs[record["binding_index"]], dtype=first.lr_synthesis.dtype,
                                    device=first.lr_synthesis.device)
            plan = record["plan"]
            if int(value.shape[-1]) != int(plan.channel_count):
                raise ValueError("hierarchical grouped physical multiplet width is incorrect")
            current = tuple(value.shape[:-1])
            if leading is None:
                leading = current
            elif current != leading:
                raise ValueError("hierarchical grouped inputs require matching leading shapes")
            result = symmetric_power_product_plan_contraction(value, plan)
            m = 2 * int(record["output_L"]) + 1
            if int(plan.descriptor_count) % m:
                raise ValueError("hierarchical grouped power output is not multiplet-complete")
            evaluated[index] = result.reshape(current + (int(plan.descriptor_count) // m, m))
        return tuple(evaluated), tuple(leading)

    def _composite_outputs(self, block_inputs):
        powers, leading = self._evaluate_unique_powers(block_inputs)
        outputs = []
        for module, indices in zip(self._source_modules, self._module_power_indices):
            outputs.append(module._forward_from_evaluated({k: powers[i] for k, i in indices.items()}, leading))
        return tuple(outputs), leading

    def _composite_packed(self, block_inputs):
        import torch

        outputs, leading = self._composite_outputs(block_inputs)
        batch = math.prod(int(s) for s in leading)
        return torch.cat(tuple(o.reshape(batch, m.output_dimension) for o, m in zip(outputs, self._source_modules)),
                         dim=1)

    def _convert(self, block_inputs):
        import torch

        first = self._source_modules[0]
        return tuple(torch.as_tensor(v, dtype=first.lr_synthesis.dtype, device=first.lr_synthesis.device)
                     for v in block_inputs)

    def _destination_packed(self, block_inputs):
        global _DESTINATION
        import torch

        inputs = self._convert(block_inputs)
        if torch.is_grad_enabled() and any(t.requires_grad for t in inputs):
            if _DESTINATION is None:
                _DESTINATION = _group_functions()
            return _DESTINATION.apply(self, *inputs)
        powers, leading = self._evaluate_unique_powers(inputs)
        return self._destination_segmented_output(powers, leading)

    def forward(self, block_inputs):
        if self.destination_native_enabled:
            packed = self._destination_packed(block_inputs)
            leading = tuple(packed.shape[:-1])
            self.last_backend = "shared_block_powers_then_destination_segmented_schur_lr"
            return tuple(packed[:, r["start"]:r["stop"]].reshape(leading + (m.channel_count, m.tableau_count,
                                                                            m.magnetic_count))
                         for r, m in zip(self.output_slices, self._source_modules))
        outputs, _leading = self._composite_outputs(self._convert(block_inputs))
        self.last_backend = "shared_block_powers_then_compiler_parent_schur_lr"
        return outputs

    def forward_packed(self, block_inputs):
        if self.destination_native_enabled:
            self.last_backend = "shared_block_powers_then_destination_segmented_schur_lr"
            return self._destination_packed(block_inputs)
        self.last_backend = "shared_block_powers_then_compiler_parent_schur_lr"
        return self._composite_packed(self._convert(block_inputs))

    def runtime_report(self):
        shared = getattr(self, "_shared_power_groups", ())
        return {
            "runtime": "YE3THierarchicalRepeatedBlockModuleGroup",
            "member_plan_count": len(self._source_modules),
            "member_plan_hashes": tuple(str(m.plan_hash) for m in self._source_modules),
            "unique_physical_binding_count": self.unique_binding_count,
            "block_power_request_count": self.power_request_count,
            "block_power_evaluation_count": self.power_evaluation_count,
            "block_power_reuse_count": self.power_request_count - self.power_evaluation_count,
            "block_power_execution_policy": self.block_power_execution_policy,
            "shared_power_group_count": self.shared_power_group_count,
            "block_power_runtime_call_count": (self.shared_power_group_count
                                               if self.block_power_execution_policy == "shared_monomial"
                                               else self.power_evaluation_count),
            "shared_power_groups": tuple({k: (tuple(g[k]) if k == "power_indices" else g[k])
                                          for k in ("binding_index", "power_indices", "input_dimension",
                                                    "output_dimension", "coefficient_count",
                                                    "unique_monomial_count")} for g in shared),
            "block_power_table_reports": tuple(dict({"binding_index": r["binding_index"], "output_L": r["output_L"]},
                                                    **symmetric_power_product_plan_table_report(r["plan"]))
                                               for r in self._unique_power_records),
            "output_dimension": self.output_dimension,
            "parent_execution_policy_requested": self.parent_execution_policy_requested,
            "destination_native_capable": self.destination_native_capable,
            "destination_native_enabled": self.destination_native_enabled,
            "destination_native_call_count": 1 if self.destination_native_enabled else 0,
            "destination_power_output_dimension": int(getattr(self, "power_output_dimension", 0)),
            "destination_input_dimension": int(getattr(self, "destination_input_dimension", 0)),
            "destination_workspace_dimension": int(getattr(self, "destination_workspace_dimension", 0)),
            "destination_expanded_output_dimension": int(getattr(self, "destination_output_dimension", 0)),
            "destination_post_native_reduction_count": (len(self._source_modules)
                                                        if self.destination_native_enabled else 0),
            "destination_segment_reports": tuple(dict(r) for r in getattr(self, "_destination_segment_reports", ())),
            "destination_order": "compiler_module_order",
            "runtime_path_discovery": False,
            "supports_autograd_vjp_hvp": True,
            "last_backend": self.last_backend,
        }


__all__ = ["SymmetricPowerBlockPlan", "SymmetricPowerProductPlan", "symmetric_power_plan_key",
           "product_plan_count_table", "shared_table", "sparse_supports",
           "symmetric_power_product_plan_table_report", "symmetric_power_product_plan_contraction",
           "YE3THierarchicalRepeatedBlockModule", "YE3THierarchicalRepeatedBlockModuleGroup"]
