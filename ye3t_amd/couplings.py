"""Public compiler facade for the ACE_density (globally trivial) sector.

Mirrors the reference entry points used on the hot path:

* ``compile_ace_factorized_schedules_by_L`` / ``ACEFactorizedScheduleReport``
  (reference ``ye3t/couplings/__init__.py:2565-2706``), including the
  ``convention_hash`` payload (``:242-252, 2685-2697``);
* ``count`` / ``plan`` for ``carrier="ACE_density"`` (``:2709-3077``), reduced to
  the fixed-content label path; their hash payloads embed the reference's full
  spec serialisation, which this package does not carry, so those two hashes
  are this package's own (documented as not reproducing the reference string).
"""

import hashlib
import json
from dataclasses import dataclass, field

from ye3t_amd.core import basis as _basis
from ye3t_amd.core import couplings as core_couplings


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
    """Labels and counts of one fixed-content ACE_density request."""

    content: tuple
    input_Ls: tuple
    counts_by_target: dict
    labels_by_target: dict
    carrier: str
    target: dict
    backend: str
    convention_hash: str
    validation_report: dict
    provenance: dict = field(default_factory=dict)

    def labels_for_target(self, target_L):
        return tuple(self.labels_by_target.get(int(target_L), ()))

    def require_label(self, label, *, target_L):
        if tuple(label) not in set(self.labels_for_target(target_L)):
            raise ValueError(f"Label {label!r} is not valid for target_L={target_L}.")
        return tuple(label)


@dataclass(frozen=True, eq=False)
class CouplerPlan:
    report: MultiplicityReport
    backend: str
    convention_hash: str
    validation_report: dict
    provenance: dict = field(default_factory=dict)


def count(request=None, *, content=None, input_Ls=None, target_L=None, target_permutation=None,
          carrier=None, tree_schedule=None, **_unused):
    """Valid compact labels of a fixed-content ACE_density request (reference ``:2709-2965``)."""
    if request is not None:
        raise ValueError("Only keyword fixed-content ACE_density requests are supported.")
    carrier = "ACE_density" if carrier is None else str(carrier)
    if carrier != "ACE_density":
        raise ValueError("This backend supports only carrier='ACE_density'.")
    if target_permutation not in (None, "trivial", "symmetric"):
        raise ValueError("ACE_density supports only the globally trivial Young sector.")
    n_in = tuple(int(v) for v in content)
    l_in = tuple(int(v) for v in input_Ls)
    tree_type = _basis.validate_tree_type(tree_schedule)
    target_L = 0 if target_L is None else int(target_L)
    labels = tuple(_basis.compact_labels_by_L(n_in, l_in, tree_type).get(target_L, ()))
    target = {"permutation": "trivial", "rotation": {"L_R": target_L}}
    validation = {
        "passed": True, "carrier": carrier, "target_L": target_L, "label_kind": "compact",
        "label_count": len(labels), "count": len(labels),
        "valid_labels_from": "ye3t.fixed_content.FixedContentDecomposition.compact_labels_by_target",
        "fixed_content_validation": {"passed": True},
    }
    payload = {"content": n_in, "input_Ls": l_in, "target": target, "backend": "symmetric_power_fast_path",
               "labels": [list(map(_json_ready, lab)) for lab in labels]}
    return MultiplicityReport(
        content=n_in, input_Ls=l_in, counts_by_target={target_L: len(labels)},
        labels_by_target={target_L: labels}, carrier=carrier, target=target,
        backend="symmetric_power_fast_path", convention_hash=_convention_hash(payload),
        validation_report=validation, provenance={"api": "ye3t_amd.couplings.count"})


def _json_ready(value):
    if isinstance(value, tuple):
        return [_json_ready(v) for v in value]
    return value


def plan(report):
    """Backend plan: ACE_density always takes the symmetric-power fast path (``global_coupler.py:4679-4686``)."""
    validation = {"passed": True, "selected_backend": "symmetric_power_fast_path",
                  "report_hash": report.convention_hash}
    return CouplerPlan(report=report, backend="symmetric_power_fast_path",
                       convention_hash=_convention_hash(validation), validation_report=validation,
                       provenance={"api": "ye3t_amd.couplings.plan"})
