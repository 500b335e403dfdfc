"""Public compiler facade for the ACE_density (globally trivial) sector.

Mirrors the reference entry points used on the hot path:

* ``compile_ace_factorized_schedules_by_L`` / ``ACEFactorizedScheduleReport``
  (reference ``ye3t/couplings/__init__.py:2565-2706``), including the
  ``convention_hash`` payload (``:242-252, 2685-2697``);
* ``count`` / ``plan`` for ``carrier="ACE_density"`` (``:2709-3077``): the same
  request records (:mod:`ye3t_amd.spec`), labels, reports and
  ``convention_hash`` payloads, so the hash strings equal the reference's.
"""

import hashlib
import json
import math
from collections import Counter
from dataclasses import dataclass, field

from ye3t_amd.core import basis as _basis
from ye3t_amd.core import couplings as core_couplings
from ye3t_amd.spec import YE3TBackendPlan, YE3TSpec, coerce_spec, plan_backend, target_partition


def _json_default(value):
    if hasattr(value, "to_dict"):
        return value.to_dict()
    if isinstance(value, tuple):
        return list(value)
    return repr(value)


def _convention_hash(payload):
    """``sha256(json.dumps(payload, sort_keys=True))[:16]`` -- reference ``:242-252``."""
    encoded = json.dumps(dict(payload), sort_keys=True, default=_json_default).encode("utf-8")
    return hashlib.sha256(encoded).hexdigest()[:16]


@dataclass(frozen=True, eq=False)
class ACEFactorizedScheduleReport:
    """Provenance wrapper for ACE factorized schedules (reference ``:2565-2614``)."""

    content: tuple
    input_Ls: tuple
    target: dict
    backend: str
    schedules_by_target: dict
    convention_hash: str
    validation_report: dict
    provenance: dict = field(default_factory=dict)

    @property
    def schedules_by_L(self):
        return self.schedules_by_target

    def evaluate(self, block_values, *, target_L, backend="auto"):
        """Apply the compiled inter-block coefficients to adapted block values.

        ``block_values`` is ``[batch, basis, block, m]``; returns
        ``[batch, component_count]`` (reference ``:2574-2591``).
        """
        target_L = int(target_L)
        if target_L not in self.schedules_by_target:
            raise ValueError("target_L is not present in this ACE schedule report.")
        return core_couplings.evaluate_factorized_schedule_torch(
            block_values, self.schedules_by_target[target_L], backend=backend)

    def to_dict(self):
        summary = {}
        for L, s in sorted(self.schedules_by_target.items()):
            summary[int(L)] = {"rank": int(s.rank), "L_R": int(s.L_R), "basis_count": s.basis_count,
                               "component_count": s.component_count, "term_count": s.term_count,
                               "block_count": int(s.block_count), "tree_type": str(s.tree_type)}
        return {"content": list(self.content), "input_Ls": list(self.input_Ls), "target": dict(self.target),
                "backend": self.backend, "convention_hash": self.convention_hash,
                "validation_report": dict(self.validation_report), "schedule_summary": summary,
                "provenance": dict(self.provenance)}


def compile_ace_factorized_schedules_by_L(*, content=None, input_Ls=None, tree_schedule="balanced",
                                          constructor_backend="auto", coeff_tol=1.0e-14,
                                          cache_policy="reuse"):
    """Return ACE factorized schedules for every allowed ``L_R`` (reference ``:2617-2706``)."""
    if content is None or input_Ls is None:
        raise ValueError("content and input_Ls are required.")
    n_in = tuple(int(v) for v in content)
    l_in = tuple(int(v) for v in input_Ls)
    if len(n_in) != len(l_in):
        raise ValueError("content and input_Ls must have the same length.")
    cache_policy = str(cache_policy)
    if cache_policy not in {"reuse", "clear_before", "cold"}:
        raise ValueError("cache_policy must be 'reuse', 'clear_before', or 'cold'.")
    if cache_policy in {"clear_before", "cold"}:
        core_couplings._FACTORIZED_SCHEDULES_CACHE.clear()
    schedules = core_couplings.generate_factorized_coefficient_schedules_by_L(
        n_in, l_in, tree_type=str(tree_schedule), coeff_tol=float(coeff_tol),
        constructor_backend=str(constructor_backend))
    by_target = {int(L): s for L, s in sorted(schedules.items()) if s.basis_count > 0}
    target = {"permutation": "trivial",
              "rotation": {"L_R_values": tuple(sorted(by_target))}}
    validation_report = {
        "passed": True,
        "scope": "ACE_density_factorized_schedule_materialization",
        "carrier": "ACE_density",
        "valid_labels_from": "ye3t.couplings.count",
        "coefficient_source": "ye3t.core.couplings.generate_factorized_coefficient_schedules_by_L",
        "cache_policy": cache_policy,
        "target_count": int(len(by_target)),
        "total_basis_count": int(sum(s.basis_count for s in by_target.values())),
        "total_component_count": int(sum(s.component_count for s in by_target.values())),
        "total_term_count": int(sum(s.term_count for s in by_target.values())),
    }
    provenance = {
        "api": "ye3t.couplings.compile_ace_factorized_schedules_by_L",
        "compiler_owner": "ye3t",
        "lower_level_api": "ye3t.core.couplings.generate_factorized_coefficient_schedules_by_L",
        "label_source": "ye3t.couplings.count / fixed-content ACE globally trivial sector",
        "usage": "explicit compiler/materialization benchmark or cache precompile path",
    }
    convention_hash = _convention_hash({
        "content": n_in,
        "input_Ls": l_in,
        "tree_schedule": str(tree_schedule),
        "constructor_backend": str(constructor_backend),
        "coeff_tol": float(coeff_tol),
        "cache_policy": cache_policy,
        "targets": tuple(sorted(by_target)),
        "summary": validation_report,
    })
    return ACEFactorizedScheduleReport(
        content=n_in, input_Ls=l_in, target=target, backend="ace_factorized_coefficient_schedule",
        schedules_by_target=by_target, convention_hash=convention_hash,
        validation_report=validation_report, provenance=provenance)


@dataclass(frozen=True, eq=False)
class MultiplicityReport:
    """Valid labels and counts of one fixed-content request (reference ``:2117-2160``)."""

    spec: YE3TSpec
    counts_by_target: dict
    labels_by_target: dict
    content: tuple
    carrier: str
    target: dict
    backend: str
    convention_hash: str
    validation_report: dict
    provenance: dict = field(default_factory=dict)

    @property
    def labels(self):
        return tuple(lab for labs in self.labels_by_target.values() for lab in labs)

    def labels_for_target(self, target_L=None):
        if target_L is None:
            target_L = int(self.spec.target_rotation.L_R)
        return tuple(self.labels_by_target.get(int(target_L), ()))

    def contains_label(self, label, *, target_L=None):
        candidate = _basis.normalize_compact_label(label)
        pool = self.labels if target_L is None else self.labels_for_target(int(target_L))
        return candidate in set(pool)

    def require_label(self, label, *, target_L=None):
        candidate = _basis.normalize_compact_label(label)
        if not self.contains_label(candidate, target_L=target_L):
            where = "any target" if target_L is None else f"L_R={int(target_L)}"
            raise ValueError("Invalid descriptor label for this YE3T coupling request: "
                             f"{candidate!r} is not in the fixed-content multiplicity report for {where}.")
        return candidate

    def to_dict(self):
        return {
            "content": list(self.content),
            "carrier": self.carrier,
            "target": dict(self.target),
            "backend": self.backend,
            "convention_hash": self.convention_hash,
            "validation_report": dict(self.validation_report),
            "counts_by_target": {int(k): int(v) for k, v in self.counts_by_target.items()},
            "labels_by_target": {int(k): [lab.payload() for lab in labs]
                                 for k, labs in self.labels_by_target.items()},
            "provenance": dict(self.provenance),
        }


@dataclass(frozen=True, eq=False)
class CouplerPlan:
    """Backend plan plus the count it was made from (reference ``:2163-2215``)."""

    spec: YE3TSpec
    report: MultiplicityReport
    backend_plan: YE3TBackendPlan
    content: tuple
    carrier: str
    target: dict
    backend: str
    convention_hash: str
    validation_report: dict
    provenance: dict = field(default_factory=dict)


def _input_Ls_from_spec(spec, input_Ls=None):
    """``input_Ls`` argument, else the spec's metadata, else all zeros (reference ``:255-266``)."""
    values = spec.metadata.get("input_Ls", ()) if input_Ls is None else input_Ls
    values = tuple(int(v) for v in (values or ()))
    if not values:
        values = tuple(0 for _ in spec.content)
    if len(values) != len(spec.content):
        raise ValueError(f"input_Ls length {len(values)} must match content rank {len(spec.content)}.")
    return values


def _fixed_content_validation(content, input_Ls, tree_type):
    """The orbit-module summary of ``FixedContentModule.decompose`` (``fixed_content.py:222-293``).

    The stabilizer is the Young subgroup permuting equal ``(n, l)`` leaves
    (``generalized_irreps.py:69-83``), so its order is the product of the
    factorials of the leaf multiplicities; the orbit of the ordered leaves has
    ``rank! / order`` members, each carrying ``prod (2 l + 1)`` magnetic states.
    The global Young x rotation sectors decompose that same space, so their
    dimensions sum to it.
    """
    _basis.validate_tree_type(tree_type)
    if not content:
        raise ValueError("FixedContentSpec requires at least one content entry.")
    if len(content) != len(input_Ls):
        raise ValueError("content and input_Ls must have the same length, "
                         f"got {len(content)} and {len(input_Ls)}.")
    if any(L < 0 for L in input_Ls):
        raise ValueError(f"input_Ls must be nonnegative, got {tuple(input_Ls)!r}.")
    order = 1
    for mult in Counter(zip(content, input_Ls)).values():
        order *= math.factorial(mult)
    orbit = math.factorial(len(content)) // order
    dim = orbit
    for L in input_Ls:
        dim *= 2 * int(L) + 1
    return {
        "passed": True,
        "scope": "fixed_content_orbit_module_decomposition",
        "catalog_validation_passed": True,
        "orbit_module_dim": int(dim),
        "decomposed_dim": int(dim),
        "stabilizer_order": int(order),
        "orbit_dimension": int(orbit),
        "compact_labels_from": "ye3t.core.api.YE3TAPI.compact_labels_by_target_L",
        "global_sectors_from": "ye3t.fixed_content.FixedContentModule.decompose",
    }


_PRIMITIVE_MODES = {None, "exact", "full_exact_basis", "original_exact"}


def count(request=None, *, content=None, input_Ls=None, target_L=None, target_permutation=None, carrier=None,
          carrier_options=None, tree_schedule=None, coefficient_backend=None, fast_path_policy=None,
          validation_scope=None, runtime_status=None, metadata=None):
    """Valid compact labels and their count for a fixed-content ACE_density request.

    Reference ``ye3t/couplings/__init__.py:2709-2965`` on its ACE_density
    branch: the same spec merge, parity and Young-sector checks, label order,
    reports and ``convention_hash`` payload
    ``{spec, input_Ls, target, backend, labels}``.  Other carriers and the
    primitive basis modes belong to the reference's wider coupler and raise.
    """
    spec = coerce_spec(request, content=content, input_Ls=input_Ls, target_L=target_L,
                       target_permutation=target_permutation, carrier=carrier, carrier_options=carrier_options,
                       tree_schedule=tree_schedule, coefficient_backend=coefficient_backend,
                       fast_path_policy=fast_path_policy, validation_scope=validation_scope,
                       runtime_status=runtime_status, metadata=metadata)
    if spec.carrier != "ACE_density":
        raise ValueError(f"carrier={spec.carrier!r} is not served by this backend; it computes only "
                         "the ACE_density carrier.")
    l_in = _input_Ls_from_spec(spec, input_Ls=input_Ls)
    requested_parity = spec.target_rotation.parity
    natural = "odd" if sum(l_in) % 2 else "even"
    if requested_parity in {"even", "odd"} and requested_parity != natural:
        raise ValueError(f"Requested parity={requested_parity!r} is incompatible with the natural product parity "
                         f"{natural!r} for input_Ls={l_in!r}.")
    partition = target_partition(spec.target_permutation, len(spec.content))
    if partition != (len(spec.content),):
        raise ValueError("ACE_density supports only the globally trivial Young sector.")
    carrier_validation = {"carrier": spec.carrier, "passed": True, "scope": "generic_fixed_content_carrier"}
    n_in = tuple(int(v) for v in spec.content)
    fixed = _fixed_content_validation(n_in, l_in, spec.tree_schedule)
    tree_type = _basis.validate_tree_type(spec.tree_schedule)
    L = int(spec.target_rotation.L_R) if target_L is None else int(target_L)
    mode = spec.carrier_options.get("basis_mode", spec.carrier_options.get("primitive_mode", None))
    if mode not in _PRIMITIVE_MODES:
        raise ValueError(f"basis_mode={mode!r}: primitive compact basis modes are not served by this backend.")
    labels = tuple(_basis.CompactLabel.from_tuple(c)
                   for c in _basis.compact_labels_by_L(n_in, l_in, tree_type).get(L, ()))
    backend_plan = plan_backend(spec, input_Ls=l_in)
    target = {"permutation": spec.target_permutation, "rotation": spec.target_rotation.to_dict()}
    validation_report = {
        "passed": True,
        "scope": "fixed_content_young_x_SO3_multiplicity_count_with_natural_input_parity",
        "content_rank": len(spec.content),
        "input_Ls": l_in,
        "natural_product_parity": natural,
        "target_L": L,
        "target_permutation": spec.target_permutation,
        "target_partition": partition,
        "carrier": spec.carrier,
        "label_kind": "compact",
        "label_count": len(labels),
        "count": len(labels),
        "fixed_content_validation": fixed,
        "basis_mode": "exact",
        "valid_labels_from": "ye3t.fixed_content.FixedContentDecomposition.compact_labels_by_target",
        "carrier_validation": carrier_validation,
    }
    provenance = {
        "api": "ye3t.couplings.count",
        "lower_level_api": "ye3t.fixed_content.FixedContentModule",
        "fixed_content_multiplicity_source": "YE3TBasisLabeler",
        "rank_product_rule": ("LR/induction for rank-additive products; Kronecker for same-rank products "
                              "in lower-level coupler plans"),
        "ace_density_young_sector": "globally trivial lambda=(N)",
        "carrier_validation_source": "ye3t.couplings",
    }
    payload = {"spec": spec.to_dict(), "input_Ls": l_in, "target": target,
               "backend": backend_plan.selected_backend, "labels": [lab.payload() for lab in labels]}
    return MultiplicityReport(
        spec=spec, counts_by_target={L: len(labels)}, labels_by_target={L: labels}, content=tuple(spec.content),
        carrier=spec.carrier, target=target, backend=backend_plan.selected_backend,
        convention_hash=_convention_hash(payload), validation_report=validation_report, provenance=provenance)


def plan(request=None, *, input_Ls=None, **kwargs):
    """Backend plan with the count's provenance (reference ``:2967-3077``, ACE_density branch).

    ``request`` is a :class:`MultiplicityReport`, or anything :func:`count`
    accepts.  The hash payload is ``{report: report.to_dict(), backend_plan:
    {requested, selected, fast_path_policy}}``.
    """
    if isinstance(request, MultiplicityReport):
        report = request
    else:
        report = count(request, input_Ls=input_Ls, **kwargs)
    spec = report.spec
    backend_plan = plan_backend(spec, input_Ls=_input_Ls_from_spec(spec, input_Ls=input_Ls))
    validation_report = {**dict(report.validation_report),
                         "backend_plan_selected": backend_plan.selected_backend,
                         "backend_plan_reason": backend_plan.reason}
    provenance = {**dict(report.provenance), "api": "ye3t.couplings.plan",
                  "backend_planner": "ye3t.global_coupler.plan_ye3t_backend"}
    payload = {"report": report.to_dict(),
               "backend_plan": {"requested": backend_plan.requested_backend,
                                "selected": backend_plan.selected_backend,
                                "fast_path_policy": backend_plan.fast_path_policy}}
    return CouplerPlan(spec=spec, report=report, backend_plan=backend_plan, content=report.content,
                       carrier=report.carrier, target=report.target, backend=backend_plan.selected_backend,
                       convention_hash=_convention_hash(payload), validation_report=validation_report,
                       provenance=provenance)
