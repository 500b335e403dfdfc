"""Reference execution-plan documents: loader, plan hash and factorized-angular buffers.

A ``YE3TExecutionPlan`` (``ye3t/execution_plan.py:6566-7241``) is the
reference compiler's portable plan: a JSON document with carrier layouts,
source assemblies, synthesis tables, factorized-angular DAG plans, runtime
instructions and schedules, a coefficient hash over the tables and a plan hash
over the whole payload.  This module reads and writes such documents and
derives, for one factorized-angular plan, the tables the HIP
``factorized_angular`` op takes (the reference's ``_factorized_plan_buffers``,
``ye3t/runtime/execution_plan.py:12918-13151``).

Scope.  The records the factorized-angular runtime reads are parsed and
validated as the reference's constructors do (synthesis tables with their
coefficient hash, ``ye3t/execution_plan.py:5986-6087``; source assemblies,
``:5899-5983``; DAG nodes and plans, ``:6090-6300``).  Every other record
(carrier layouts, instructions, schedules, wiring, certificate, provenance,
the source realization inside an assembly) is carried through unchanged as
canonical JSON and enters the plan hash as written.  A document written by
the reference's ``to_json`` is in that form already, so its ``plan_hash``
reproduces here; the reference's own semantic checks of those other records
(instruction typing, wiring, hierarchical routes, ``:6600-7135``) are not
restated.  Schema ``ye3t_execution_plan_v1`` is migrated as the reference does
(``:7175-7190``); the coupled-product schema ``ye3t_execution_plan_v3`` (the
exact C-tilde DAG, ``:683-868``) is refused.

Hashing (``ye3t/execution_plan.py:116-145`` with
``ye3t/cache/graph_json.py:13-80``): a payload is made canonical (mappings
with string keys in sorted order, tuples as lists, complex numbers as
``[real, imag]``) and hashed as SHA-256 of its compact sorted JSON
(``separators=(",", ":")``).  ``to_json`` writes the canonical payload with
``sort_keys=True`` and ``indent=2``; ``from_json(to_json())`` returns a plan
with the same ``plan_hash`` (the round trip ``scalar_ace_export.py:10-19``
checks).
"""

import hashlib
import json
from dataclasses import dataclass, field

import numpy as np

EXECUTION_PLAN_SCHEMA = "ye3t_execution_plan_v2"
EXECUTION_PLAN_LEGACY_SCHEMA = "ye3t_execution_plan_v1"
EXECUTION_PLAN_COUPLED_PRODUCT_SCHEMA = "ye3t_execution_plan_v3"
PRIMARY_CONVENTION = "complex_condon_shortley_young_orthogonal_v1"
ANALYSIS_ORIENTATION = "conjugate_transpose"


def canonical_payload(value):
    """The canonical JSON value of ``value`` (reference ``_canonical_payload``,
    ``ye3t/execution_plan.py:116-137``)."""
    if hasattr(value, "to_dict"):
        return canonical_payload(value.to_dict())
    if isinstance(value, dict):
        return {str(k): canonical_payload(v) for k, v in sorted(value.items(), key=lambda kv: str(kv[0]))}
    if isinstance(value, (tuple, list)):
        return [canonical_payload(v) for v in value]
    if isinstance(value, complex):
        return [float(value.real), float(value.imag)]
    return value


def canonical_json(value):
    """Compact sorted JSON of the canonical payload: the bytes the hash reads."""
    return json.dumps(canonical_payload(value), sort_keys=True, separators=(",", ":"))


def stable_hash(value):
    """SHA-256 hex digest of :func:`canonical_json` (reference ``_stable_hash``,
    ``ye3t/execution_plan.py:140-144``)."""
    return hashlib.sha256(canonical_json(value).encode("utf-8")).hexdigest()


def _complex_tuple(values):
    out = []
    for v in values:
        if isinstance(v, (tuple, list)):
            if len(v) != 2:
                raise ValueError("complex values are stored as [real, imag] pairs")
            out.append(complex(float(v[0]), float(v[1])))
        else:
            out.append(complex(v))
    return tuple(out)


def _complex_payload(values):
    return [[float(v.real), float(v.imag)] for v in values]


def _int_tuple(values):
    return tuple(int(v) for v in values)


def _permutation(value, rank):
    perm = _int_tuple(value)
    if len(perm) != rank or tuple(sorted(perm)) != tuple(range(rank)):
        raise ValueError("coset representatives must be zero-based permutations of the input slots")
    return perm


@dataclass(frozen=True)
class SynthesisTable:
    """Sparse synthesis map ``C`` in COO form; runtimes apply ``C^dagger``
    (reference ``YE3TSynthesisTable``, ``ye3t/execution_plan.py:5986-6087``)."""

    table_id: str
    input_dimension: int
    output_dimension: int
    row_indices: tuple
    column_indices: tuple
    values: tuple
    orientation: str = "synthesis"
    convention_id: str = PRIMARY_CONVENTION
    coefficient_hash: str = ""
    validation_report: dict = field(default_factory=dict)
    provenance: dict = field(default_factory=dict)

    def __post_init__(self):
        n_in, n_out = int(self.input_dimension), int(self.output_dimension)
        if n_in <= 0 or n_out <= 0:
            raise ValueError("synthesis table dimensions must be positive")
        rows, cols, vals = _int_tuple(self.row_indices), _int_tuple(self.column_indices), _complex_tuple(self.values)
        if not (len(rows) == len(cols) == len(vals)):
            raise ValueError("synthesis table COO arrays must have equal length")
        if not vals:
            raise ValueError("synthesis table must contain at least one entry")
        if any(r < 0 or r >= n_in for r in rows):
            raise ValueError("synthesis table row index is out of bounds")
        if any(c < 0 or c >= n_out for c in cols):
            raise ValueError("synthesis table column index is out of bounds")
        if str(self.orientation) != "synthesis":
            raise ValueError("stored coefficient tables must use synthesis orientation")
        convention = str(self.convention_id)
        computed = stable_hash({"input_dimension": n_in, "output_dimension": n_out, "row_indices": rows,
                                "column_indices": cols, "values": _complex_payload(vals),
                                "orientation": "synthesis", "convention_id": convention})
        if str(self.coefficient_hash) and str(self.coefficient_hash) != computed:
            raise ValueError("synthesis-table coefficient hash does not match its payload")
        for name, value in (("table_id", str(self.table_id)), ("input_dimension", n_in),
                            ("output_dimension", n_out), ("row_indices", rows), ("column_indices", cols),
                            ("values", vals), ("orientation", "synthesis"), ("convention_id", convention),
                            ("coefficient_hash", computed), ("validation_report", dict(self.validation_report)),
                            ("provenance", dict(self.provenance))):
            object.__setattr__(self, name, value)

    def to_dict(self):
        return {"table_id": self.table_id, "input_dimension": self.input_dimension,
                "output_dimension": self.output_dimension, "row_indices": list(self.row_indices),
                "column_indices": list(self.column_indices), "values": _complex_payload(self.values),
                "orientation": "synthesis", "analysis_orientation": ANALYSIS_ORIENTATION,
                "convention_id": self.convention_id, "coefficient_hash": self.coefficient_hash,
                "validation_report": dict(self.validation_report), "provenance": dict(self.provenance)}

    @classmethod
    def from_dict(cls, p):
        return cls(table_id=p["table_id"], input_dimension=p["input_dimension"],
                   output_dimension=p["output_dimension"], row_indices=p["row_indices"],
                   column_indices=p["column_indices"], values=p["values"],
                   orientation=p.get("orientation", "synthesis"),
                   convention_id=p.get("convention_id", PRIMARY_CONVENTION),
                   coefficient_hash=p.get("coefficient_hash", ""),
                   validation_report=p.get("validation_report", {}), provenance=p.get("provenance", {}))


@dataclass(frozen=True)
class SourceAssemblyPlan:
    """Sparse source placement ``L_v`` (source coordinate -> induced basis
    row) in COO form (reference ``YE3TSourceAssemblyPlan``,
    ``ye3t/execution_plan.py:5899-5983``).  ``source_realization`` is kept as
    its canonical JSON record."""

    assembly_id: str
    source_realization: dict
    source_dimension: int
    induced_dimension: int
    row_indices: tuple
    column_indices: tuple
    values: tuple
    normalization: str = "compiler_explicit"
    validation_report: dict = field(default_factory=dict)
    provenance: dict = field(default_factory=dict)

    def __post_init__(self):
        n_src, n_ind = int(self.source_dimension), int(self.induced_dimension)
        if n_src <= 0 or n_ind <= 0:
            raise ValueError("source and induced dimensions must be positive")
        rows, cols, vals = _int_tuple(self.row_indices), _int_tuple(self.column_indices), _complex_tuple(self.values)
        if not (len(rows) == len(cols) == len(vals)):
            raise ValueError("source assembly COO arrays must have equal length")
        if not vals:
            raise ValueError("source assembly must contain at least one entry")
        if any(r < 0 or r >= n_ind for r in rows):
            raise ValueError("source assembly row index is out of bounds")
        if any(c < 0 or c >= n_src for c in cols):
            raise ValueError("source assembly column index is out of bounds")
        if not isinstance(self.source_realization, dict):
            raise ValueError("source assembly needs a source_realization record")
        for name, value in (("assembly_id", str(self.assembly_id)),
                            ("source_realization", canonical_payload(self.source_realization)),
                            ("source_dimension", n_src), ("induced_dimension", n_ind), ("row_indices", rows),
                            ("column_indices", cols), ("values", vals), ("normalization", str(self.normalization)),
                            ("validation_report", dict(self.validation_report)),
                            ("provenance", dict(self.provenance))):
            object.__setattr__(self, name, value)

    def to_dict(self):
        return {"assembly_id": self.assembly_id, "source_realization": self.source_realization,
                "source_dimension": self.source_dimension, "induced_dimension": self.induced_dimension,
                "row_indices": list(self.row_indices), "column_indices": list(self.column_indices),
                "values": _complex_payload(self.values), "normalization": self.normalization,
                "validation_report": dict(self.validation_report), "provenance": dict(self.provenance)}

    @classmethod
    def from_dict(cls, p):
        return cls(assembly_id=p["assembly_id"], source_realization=p["source_realization"],
                   source_dimension=p["source_dimension"], induced_dimension=p["induced_dimension"],
                   row_indices=p["row_indices"], column_indices=p["column_indices"], values=p["values"],
                   normalization=p.get("normalization", "compiler_explicit"),
                   validation_report=p.get("validation_report", {}), provenance=p.get("provenance", {}))


@dataclass(frozen=True)
class FactorizedAngularNode:
    """One leaf or binary CG merge of an angular DAG (reference
    ``YE3TFactorizedAngularNode``, ``ye3t/execution_plan.py:6090-6186``)."""

    node_id: str
    kind: str
    output_L: int
    leaf_index: int = None
    left_node_id: str = None
    right_node_id: str = None
    synthesis_table_id: str = None

    def __post_init__(self):
        kind, L = str(self.kind), int(self.output_L)
        if kind not in ("leaf", "merge"):
            raise ValueError("factorized angular node kind must be leaf or merge")
        if L < 0:
            raise ValueError("factorized angular node output_L must be nonnegative")
        leaf = None if self.leaf_index is None else int(self.leaf_index)
        left = None if self.left_node_id is None else str(self.left_node_id)
        right = None if self.right_node_id is None else str(self.right_node_id)
        table = None if self.synthesis_table_id is None else str(self.synthesis_table_id)
        if kind == "leaf":
            if leaf is None or leaf < 0:
                raise ValueError("leaf angular nodes require a nonnegative index")
            if any(v is not None for v in (left, right, table)):
                raise ValueError("leaf angular nodes cannot reference merge data")
        else:
            if leaf is not None:
                raise ValueError("merge angular nodes cannot carry a leaf index")
            if not left or not right or not table:
                raise ValueError("merge angular nodes require two children and a synthesis table")
        for name, value in (("node_id", str(self.node_id)), ("kind", kind), ("output_L", L), ("leaf_index", leaf),
                            ("left_node_id", left), ("right_node_id", right), ("synthesis_table_id", table)):
            object.__setattr__(self, name, value)

    def to_dict(self):
        return {"node_id": self.node_id, "kind": self.kind, "output_L": self.output_L,
                "leaf_index": self.leaf_index, "left_node_id": self.left_node_id,
                "right_node_id": self.right_node_id, "synthesis_table_id": self.synthesis_table_id}

    @classmethod
    def from_dict(cls, p):
        return cls(node_id=p["node_id"], kind=p["kind"], output_L=p["output_L"], leaf_index=p.get("leaf_index"),
                   left_node_id=p.get("left_node_id"), right_node_id=p.get("right_node_id"),
                   synthesis_table_id=p.get("synthesis_table_id"))


@dataclass(frozen=True)
class FactorizedAngularPlan:
    """A typed angular forest with its Young and source placement records
    (reference ``YE3TFactorizedAngularPlan``, ``ye3t/execution_plan.py:6189-6300``)."""

    plan_id: str
    input_Ls: tuple
    output_L: int
    bracketing: str
    nodes: tuple
    root_node_ids: tuple
    coset_representatives: tuple
    source_assembly_id: str
    young_synthesis_table_id: str
    convention_id: str = PRIMARY_CONVENTION
    validation_report: dict = field(default_factory=dict)
    provenance: dict = field(default_factory=dict)

    def __post_init__(self):
        input_Ls = _int_tuple(self.input_Ls)
        if not input_Ls or any(L < 0 for L in input_Ls):
            raise ValueError("factorized angular input_Ls must be nonempty")
        output_L = int(self.output_L)
        if output_L < 0:
            raise ValueError("factorized angular output_L must be nonnegative")
        nodes = tuple(n if isinstance(n, FactorizedAngularNode) else FactorizedAngularNode.from_dict(n)
                      for n in self.nodes)
        ids = {n.node_id for n in nodes}
        if len(ids) != len(nodes):
            raise ValueError("factorized angular node IDs must be unique")
        roots = tuple(str(r) for r in self.root_node_ids)
        if not roots or any(r not in ids for r in roots):
            raise ValueError("factorized angular roots must reference DAG nodes")
        seen = set()
        for n in nodes:
            if n.kind == "leaf":
                if n.leaf_index >= len(input_Ls):
                    raise ValueError("angular leaf index is outside input_Ls")
                if n.output_L != input_Ls[n.leaf_index]:
                    raise ValueError("angular leaf L does not match input_Ls")
            elif n.left_node_id not in seen or n.right_node_id not in seen:
                raise ValueError("factorized angular nodes must be in topological order")
            seen.add(n.node_id)
        reps = tuple(_permutation(r, len(input_Ls)) for r in self.coset_representatives)
        if not reps:
            raise ValueError("factorized angular plan requires coset placements")
        for name, value in (("plan_id", str(self.plan_id)), ("input_Ls", input_Ls), ("output_L", output_L),
                            ("bracketing", str(self.bracketing)), ("nodes", nodes), ("root_node_ids", roots),
                            ("coset_representatives", reps), ("source_assembly_id", str(self.source_assembly_id)),
                            ("young_synthesis_table_id", str(self.young_synthesis_table_id)),
                            ("convention_id", str(self.convention_id)),
                            ("validation_report", dict(self.validation_report)),
                            ("provenance", dict(self.provenance))):
            object.__setattr__(self, name, value)

    def to_dict(self):
        return {"plan_id": self.plan_id, "input_Ls": list(self.input_Ls), "output_L": self.output_L,
                "bracketing": self.bracketing, "nodes": [n.to_dict() for n in self.nodes],
                "root_node_ids": list(self.root_node_ids),
                "coset_representatives": [list(r) for r in self.coset_representatives],
                "source_assembly_id": self.source_assembly_id,
                "young_synthesis_table_id": self.young_synthesis_table_id, "convention_id": self.convention_id,
                "validation_report": dict(self.validation_report), "provenance": dict(self.provenance)}

    @classmethod
    def from_dict(cls, p):
        return cls(plan_id=p["plan_id"], input_Ls=p["input_Ls"], output_L=p["output_L"], bracketing=p["bracketing"],
                   nodes=p["nodes"], root_node_ids=p["root_node_ids"],
                   coset_representatives=p["coset_representatives"], source_assembly_id=p["source_assembly_id"],
                   young_synthesis_table_id=p["young_synthesis_table_id"],
                   convention_id=p.get("convention_id", PRIMARY_CONVENTION),
                   validation_report=p.get("validation_report", {}), provenance=p.get("provenance", {}))


def _records(values, cls, name):
    out = tuple(v if isinstance(v, cls) else cls.from_dict(v) for v in values)
    ids = [getattr(r, name) for r in out]
    if len(set(ids)) != len(ids):
        raise ValueError(f"execution-plan {name} values must be unique")
    return out


@dataclass(frozen=True)
class ExecutionPlan:
    """A reference execution-plan document (``YE3TExecutionPlan``,
    ``ye3t/execution_plan.py:6566-7241``) with its factorized-angular records
    parsed and the rest carried as canonical JSON.

    ``coefficient_hash`` and ``plan_hash`` are recomputed on construction; a
    supplied non-empty value that differs raises ``ValueError``, as the
    reference's constructor does (``:7107-7140``)."""

    schema_version: str = EXECUTION_PLAN_SCHEMA
    carrier_layouts: tuple = ()
    source_assemblies: tuple = ()
    synthesis_tables: tuple = ()
    factorized_angular_plans: tuple = ()
    instructions: tuple = ()
    forward_schedule: tuple = ()
    reverse_schedule: tuple = ()
    second_order_schedule: tuple = ()
    wiring: dict = None
    convention_id: str = PRIMARY_CONVENTION
    coefficient_hash: str = ""
    plan_hash: str = ""
    certificate: dict = field(default_factory=dict)
    provenance: dict = field(default_factory=dict)

    def __post_init__(self):
        schema = str(self.schema_version)
        if schema == EXECUTION_PLAN_COUPLED_PRODUCT_SCHEMA:
            raise NotImplementedError("ye3t_execution_plan_v3 (the coupled-product C-tilde DAG) is not read by "
                                      "this loader; it reads the factorized-angular records of v1/v2 plans")
        if schema != EXECUTION_PLAN_SCHEMA:
            raise ValueError(f"unsupported YE3T execution-plan schema {schema!r}")
        tables = _records(self.synthesis_tables, SynthesisTable, "table_id")
        assemblies = _records(self.source_assemblies, SourceAssemblyPlan, "assembly_id")
        angular = _records(self.factorized_angular_plans, FactorizedAngularPlan, "plan_id")
        table_ids = {t.table_id for t in tables}
        assembly_ids = {a.assembly_id for a in assemblies}
        for plan in angular:
            if plan.source_assembly_id not in assembly_ids:
                raise ValueError("factorized angular plan references an unknown source assembly")
            if plan.young_synthesis_table_id not in table_ids:
                raise ValueError("factorized angular plan references an unknown Young synthesis table")
            if any(n.kind == "merge" and n.synthesis_table_id not in table_ids for n in plan.nodes):
                raise ValueError("factorized angular merge references an unknown synthesis table")
        computed_coefficients = stable_hash([t.to_dict() for t in tables])
        if str(self.coefficient_hash) and str(self.coefficient_hash) != computed_coefficients:
            raise ValueError("execution-plan coefficient hash does not match its tables")
        for name, value in (("schema_version", schema),
                            ("carrier_layouts", tuple(canonical_payload(v) for v in self.carrier_layouts)),
                            ("source_assemblies", assemblies), ("synthesis_tables", tables),
                            ("factorized_angular_plans", angular),
                            ("instructions", tuple(canonical_payload(v) for v in self.instructions)),
                            ("forward_schedule", tuple(self.forward_schedule)),
                            ("reverse_schedule", tuple(self.reverse_schedule)),
                            ("second_order_schedule", tuple(self.second_order_schedule)),
                            ("wiring", None if self.wiring is None else canonical_payload(self.wiring)),
                            ("convention_id", str(self.convention_id)),
                            ("coefficient_hash", computed_coefficients),
                            ("certificate", canonical_payload(dict(self.certificate))),
                            ("provenance", canonical_payload(dict(self.provenance)))):
            object.__setattr__(self, name, value)
        computed = stable_hash(self._payload(include_plan_hash=False))
        if str(self.plan_hash) and str(self.plan_hash) != computed:
            raise ValueError("execution-plan hash does not match its payload")
        object.__setattr__(self, "plan_hash", computed)

    def _payload(self, include_plan_hash):
        payload = {
            "schema_version": self.schema_version,
            "carrier_layouts": list(self.carrier_layouts),
            "source_assemblies": [a.to_dict() for a in self.source_assemblies],
            "synthesis_tables": [t.to_dict() for t in self.synthesis_tables],
            "factorized_angular_plans": [p.to_dict() for p in self.factorized_angular_plans],
            "instructions": list(self.instructions),
            "forward_schedule": list(self.forward_schedule),
            "reverse_schedule": list(self.reverse_schedule),
            "second_order_schedule": list(self.second_order_schedule),
            "convention_id": self.convention_id,
            "coefficient_hash": self.coefficient_hash,
            "certificate": dict(self.certificate),
            "provenance": dict(self.provenance),
        }
        if self.wiring is not None:
            payload["wiring"] = self.wiring
        if include_plan_hash:
            payload["plan_hash"] = self.plan_hash
        return payload

    def to_dict(self):
        return self._payload(include_plan_hash=True)

    def to_json(self, indent=2):
        return json.dumps(canonical_payload(self.to_dict()), sort_keys=True, indent=indent)

    @classmethod
    def from_dict(cls, payload):
        """Reference ``YE3TExecutionPlan.from_dict`` (``ye3t/execution_plan.py:7166-7236``),
        including the ``ye3t_execution_plan_v1`` migration."""
        payload = dict(payload)
        schema = payload.get("schema_version", EXECUTION_PLAN_SCHEMA)
        if schema == EXECUTION_PLAN_LEGACY_SCHEMA:
            provenance = dict(payload.get("provenance", {}))
            provenance.update({"migrated_from_schema": EXECUTION_PLAN_LEGACY_SCHEMA,
                               "legacy_plan_hash": payload.get("plan_hash", ""),
                               "legacy_spatial_symmetry": "SO3", "spatial_symmetry": "SO3_legacy",
                               "parity_inferred": False})
            payload["schema_version"] = EXECUTION_PLAN_SCHEMA
            payload["provenance"] = provenance
            payload["plan_hash"] = ""
        return cls(schema_version=payload.get("schema_version", EXECUTION_PLAN_SCHEMA),
                   carrier_layouts=tuple(payload.get("carrier_layouts", ())),
                   source_assemblies=tuple(payload.get("source_assemblies", ())),
                   synthesis_tables=tuple(payload.get("synthesis_tables", ())),
                   factorized_angular_plans=tuple(payload.get("factorized_angular_plans", ())),
                   instructions=tuple(payload.get("instructions", ())),
                   forward_schedule=tuple(payload.get("forward_schedule", ())),
                   reverse_schedule=tuple(payload.get("reverse_schedule", ())),
                   second_order_schedule=tuple(payload.get("second_order_schedule", ())),
                   wiring=payload.get("wiring"), convention_id=payload.get("convention_id", PRIMARY_CONVENTION),
                   coefficient_hash=payload.get("coefficient_hash", ""), plan_hash=payload.get("plan_hash", ""),
                   certificate=payload.get("certificate", {}), provenance=payload.get("provenance", {}))

    @classmethod
    def from_json(cls, text):
        return cls.from_dict(json.loads(text))

    # ---- factorized-angular runtime tables -------------------------------------------------

    def factorized_angular_plan(self, plan_id=None):
        """The plan named ``plan_id``, or the only one when ``plan_id`` is None
        (the reference module's selection, ``ye3t/runtime/execution_plan.py:13563-13578``)."""
        plans = {p.plan_id: p for p in self.factorized_angular_plans}
        if plan_id is None:
            if len(plans) != 1:
                raise ValueError("factorized_angular_plan_id is required for zero or multiple angular plans")
            return next(iter(plans.values()))
        return plans[str(plan_id)]

    def factorized_angular_subtree_identity(self, plan_id=None, leaf_bindings=None):
        """Per-node operator and subtree hashes of one angular DAG (reference
        ``_factorized_angular_subtree_identity``, ``ye3t/execution_plan.py:6303-6422``)."""
        plan = self.factorized_angular_plan(plan_id)
        tables = {t.table_id: t for t in self.synthesis_tables}
        nodes = {n.node_id: n for n in plan.nodes}
        if leaf_bindings is None:
            leaf_bindings = tuple(("logical_slot", i) for i in range(len(plan.input_Ls)))
        elif len(tuple(leaf_bindings)) != len(plan.input_Ls):
            raise ValueError("factorized angular leaf bindings must cover every input slot")
        leaf_bindings = tuple(leaf_bindings)
        op_hash, sub_hash = {}, {}
        for n in plan.nodes:
            dim = 2 * n.output_L + 1
            if n.kind == "leaf":
                op = {"kind": "leaf", "output_L": n.output_L, "output_dimension": dim,
                      "convention_id": plan.convention_id}
                sub = {"operator": op, "physical_binding": leaf_bindings[n.leaf_index]}
            else:
                t = tables[n.synthesis_table_id]
                left, right = nodes[n.left_node_id], nodes[n.right_node_id]
                dl, dr = 2 * left.output_L + 1, 2 * right.output_L + 1
                if t.input_dimension != dl * dr or t.output_dimension != dim:
                    raise ValueError("factorized angular merge table dimensions do not match its child and "
                                     "output carriers")
                op = {"kind": "merge", "output_L": n.output_L, "output_dimension": dim, "left_dimension": dl,
                      "right_dimension": dr, "synthesis_coefficient_hash": t.coefficient_hash,
                      "synthesis_orientation": t.orientation, "analysis_orientation": ANALYSIS_ORIENTATION,
                      "table_convention_id": t.convention_id, "plan_convention_id": plan.convention_id}
                sub = {"operator": op, "left_subtree_hash": sub_hash[n.left_node_id],
                       "right_subtree_hash": sub_hash[n.right_node_id]}
            op_hash[n.node_id] = stable_hash(op)
            sub_hash[n.node_id] = stable_hash(sub)
        return {"node_operator_hashes": tuple(op_hash[n.node_id] for n in plan.nodes),
                "node_subtree_hashes": tuple(sub_hash[n.node_id] for n in plan.nodes)}

    def factorized_angular_buffers(self, plan_id=None, complex_values=True):
        """The HIP ``factorized_angular`` op's tables for one angular plan
        (reference ``_factorized_plan_buffers``,
        ``ye3t/runtime/execution_plan.py:12918-13151``), as numpy arrays.

        Node ``i`` owns workspace rows ``node_offsets[i] .. + node_dimensions[i]``;
        leaves copy input slot ``leaf_index`` (offset ``node_leaf_offsets``),
        merges read their children ``node_left``/``node_right`` through the
        synthesis table's COO (concatenated in node order, ranges
        ``node_coefficient_offsets``).  ``projection_values`` is the
        ``source_dimension x Young output`` matrix
        ``sum_r L_v[r, s] * conj(Y[r, t])`` composed from the source assembly
        and the Young table.  With ``complex_values=False`` the coefficient
        and projection arrays keep only their real parts, as the reference
        does for a real dtype (``:11392-11397``).

        Returns ``(tables, meta)``: ``tables`` has the op's table names,
        ``meta`` the dimensions, ``input_Ls``, ``output_L``, ``plan_id``, the
        dense-synthesis element count and the subtree identity hashes."""
        plan = self.factorized_angular_plan(plan_id)
        tables = {t.table_id: t for t in self.synthesis_tables}
        assembly = {a.assembly_id: a for a in self.source_assemblies}[plan.source_assembly_id]
        young = tables[plan.young_synthesis_table_id]
        n_src = assembly.source_dimension
        proj = np.zeros((n_src, young.output_dimension), dtype=np.complex128)
        young_by_row = {}
        for r, c, v in zip(young.row_indices, young.column_indices, young.values):
            young_by_row.setdefault(r, []).append((c, v))
        for r, s, v in zip(assembly.row_indices, assembly.column_indices, assembly.values):
            for c, yv in young_by_row.get(r, ()):
                proj[s, c] += v * yv.conjugate()
        input_offsets, run = [], 0
        for L in plan.input_Ls:
            input_offsets.append(run)
            run += 2 * L + 1
        index = {n.node_id: i for i, n in enumerate(plan.nodes)}
        offs, dims, leaf_offs, left, right, coef_offs = [], [], [], [], [], [0]
        rows, cols, vals = [], [], []
        ws = 0
        dense_elements = 0
        for n in plan.nodes:
            d = 2 * n.output_L + 1
            offs.append(ws)
            dims.append(d)
            ws += d
            if n.kind == "leaf":
                leaf_offs.append(input_offsets[n.leaf_index])
                left.append(-1)
                right.append(-1)
            else:
                t = tables[n.synthesis_table_id]
                leaf_offs.append(-1)
                left.append(index[n.left_node_id])
                right.append(index[n.right_node_id])
                rows.extend(t.row_indices)
                cols.extend(t.column_indices)
                vals.extend(t.values)
                dense_elements += t.input_dimension * t.output_dimension
            coef_offs.append(len(vals))
        values = np.asarray(vals, dtype=np.complex128)
        projection = proj.reshape(-1)
        if not complex_values:
            values, projection = values.real.copy(), projection.real.copy()
        i64 = lambda v: np.asarray(v, dtype=np.int64)  # noqa: E731
        out = {"node_offsets": i64(offs), "node_dimensions": i64(dims), "node_leaf_offsets": i64(leaf_offs),
               "node_left": i64(left), "node_right": i64(right), "node_coefficient_offsets": i64(coef_offs),
               "coefficient_rows": i64(rows), "coefficient_columns": i64(cols), "coefficient_values": values,
               "root_nodes": i64([index[r] for r in plan.root_node_ids]), "projection_values": projection}
        identity = self.factorized_angular_subtree_identity(plan.plan_id)
        meta = {"plan_id": plan.plan_id, "input_Ls": plan.input_Ls, "output_L": plan.output_L,
                "input_dimension": run, "source_dimension": n_src, "workspace_dimension": ws,
                "output_dimension": len(plan.root_node_ids) * young.output_dimension * (2 * plan.output_L + 1),
                "logical_channel_tableau_dimension": len(plan.root_node_ids) * young.output_dimension,
                "magnetic_dimension": 2 * plan.output_L + 1,
                "reference_dense_synthesis_element_count": dense_elements,
                "coefficient_complex": bool(any(v.imag != 0.0 for t in tables.values() for v in t.values)),
                **identity}
        return out, meta
