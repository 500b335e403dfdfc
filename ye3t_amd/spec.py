"""Request records of the coupling facade: the mathematical request, its
rotation and readout targets, and the resolved backend choice.

These mirror the reference's shared specification records
(``ye3t/spec.py:327-980``: ``YE3TRotationTarget``, ``YE3TReadoutSpec``,
``YE3TSpec``, ``YE3TBackendPlan``) field for field, because their ``to_dict``
payloads enter the ``count`` / ``plan`` convention hashes verbatim.  Only what
the ACE_density request path reads is carried: no A_s role contracts, no file
I/O and no message-state specs.
"""

from collections.abc import Mapping
from dataclasses import dataclass, field

STRICT_RUNTIME_STATUSES = frozenset({
    "implemented_and_validated", "implemented_under_validation", "internal_only",
    "legacy_scalar_readout", "inventory_only", "planned_not_public",
})
TREE_SCHEDULES = frozenset({"balanced", "left", "right", "explicit"})
COEFFICIENT_BACKENDS = frozenset({
    "global_coupler", "symmetric_power_fast_path", "exterior_power_fast_path",
    "schur_weyl_tree_backend", "reference_dense", "certified_intertwiner", "ace_trivial_fast_path",
    "ace_symmetric_power_kernel_inventory", "exact_block_first_young_subgroup",
    "young_orthogonal_subduction_inventory", "A_s_slot_specht_central_projector_norms",
    "filtered_density_antisymmetric_wedge_norm", "filtered_density_trivial_slot_fast_path",
    "finite_permutation_orbitals", "explicit_phi_motif_reference", "linear_lifted_cauchy_scalar",
    "linear_tagged_cauchy_image",
})
VALIDATION_SCOPES = frozenset({"counts", "projectors", "intertwiners", "runtime_equivariance", "forces", "full"})
TASKS = frozenset({"atomic_scalar", "atomic_covariant", "fermion_scalar", "fermion_covariant",
                   "operator_learning", "descriptor_only"})
CARRIERS = frozenset({"ACE_density", "A_s", "Phi", "orbital", "message_state", "external_tensor"})
ROTATION_GROUPS = frozenset({"SO3", "O3", "E3_site"})
READOUT_AGGREGATIONS = frozenset({"none", "site_sum", "site_mean", "global_sum", "global_mean",
                                  "operator_matrix_element", "pair_tensor", "external"})


def _listed(names):
    return ", ".join(sorted(names))


def validate_runtime_status(status):
    status = str(status)
    if status not in STRICT_RUNTIME_STATUSES:
        raise ValueError(f"runtime_status must be one of {_listed(STRICT_RUNTIME_STATUSES)}; got {status!r}.")
    return status


def validate_tree_schedule(tree_schedule):
    tree_schedule = str(tree_schedule)
    if tree_schedule not in TREE_SCHEDULES:
        raise ValueError(f"tree_schedule must be one of {_listed(TREE_SCHEDULES)}.")
    return tree_schedule


def validate_coefficient_backend(backend):
    backend = str(backend)
    if backend not in COEFFICIENT_BACKENDS:
        raise ValueError(f"coefficient_backend must be recognized; got {backend!r}.")
    return backend


def validate_fast_path_policy(policy):
    """``auto | explain | disable | force | force:<known backend>``."""
    policy = str(policy)
    if policy in {"auto", "explain", "disable", "force"}:
        return policy
    choices = "fast_path_policy must be 'auto', 'explain', 'disable', 'force', or 'force:<backend>'."
    if policy.startswith("force:"):
        backend = policy.split(":", 1)[1]
        if not backend:
            raise ValueError(choices)
        if backend not in COEFFICIENT_BACKENDS:
            raise ValueError("fast_path_policy force:<backend> must name a known coefficient backend; "
                             f"{_listed(COEFFICIENT_BACKENDS)}; got {backend!r}.")
        return policy
    raise ValueError(choices)


def target_partition(target, rank=None):
    """Young partition of a requested permutation sector at the content's rank."""
    text = str(target).strip().lower()
    if rank is not None:
        rank = int(rank)
        if rank <= 0:
            raise ValueError("target_permutation requires a positive content rank.")
    if text in {"trivial", "symmetric", "antisymmetric", "sign"}:
        if rank is None:
            raise ValueError("target_permutation requires a content rank.")
        parts = (rank,) if text in {"trivial", "symmetric"} else (1,) * rank
    elif text.startswith("young:"):
        body = text.split(":", 1)[1].strip()
        if body.startswith("(") and body.endswith(")"):
            body = body[1:-1].strip()
        if body == "n":
            if rank is None:
                raise ValueError("young:(N) requires a content rank.")
            parts = (rank,)
        else:
            try:
                parts = tuple(int(p.strip()) for p in body.split(","))
            except ValueError as exc:
                raise ValueError(f"target_permutation={target!r} is not a Young partition.") from exc
    else:
        raise ValueError("target_permutation must be 'trivial', 'antisymmetric', or 'young:<partition>'; "
                         f"got {target!r}.")
    if not parts or any(p <= 0 for p in parts) or tuple(sorted(parts, reverse=True)) != parts:
        raise ValueError(f"target_permutation={target!r} must be a nonincreasing positive partition.")
    if rank is not None and sum(parts) != rank:
        raise ValueError(f"target_permutation={target!r} has size {sum(parts)}, but content rank is {rank}.")
    return parts


def _as_tuple(value):
    if value is None:
        return ()
    if isinstance(value, (tuple, list)):
        return tuple(value)
    return (value,)


@dataclass(frozen=True)
class YE3TRotationTarget:
    """Rotation / parity target of a sector (reference ``spec.py:327-375``)."""

    L_R: int = 0
    M_R: tuple = None
    parity: str = None
    group: str = "SO3"

    def __post_init__(self):
        if int(self.L_R) < 0:
            raise ValueError("L_R must be nonnegative.")
        if self.M_R is not None:
            m = tuple(int(v) for v in self.M_R)
            if any(abs(v) > int(self.L_R) for v in m):
                raise ValueError("M_R values must satisfy -L_R <= M_R <= L_R.")
            object.__setattr__(self, "M_R", m)
        if str(self.group) not in ROTATION_GROUPS:
            raise ValueError(f"rotation group must be one of {_listed(ROTATION_GROUPS)}.")
        object.__setattr__(self, "group", str(self.group))
        if self.parity is not None:
            if str(self.parity) not in {"even", "odd", "natural", "none"}:
                raise ValueError("parity must be 'even', 'odd', 'natural', 'none', or None.")
            object.__setattr__(self, "parity", str(self.parity))
        object.__setattr__(self, "L_R", int(self.L_R))

    def to_dict(self):
        return {"L_R": int(self.L_R), "M_R": None if self.M_R is None else [int(v) for v in self.M_R],
                "parity": self.parity, "group": str(self.group)}

    @classmethod
    def from_dict(cls, payload):
        payload = {} if payload is None else dict(payload)
        m = payload.get("M_R", payload.get("M_R_values", None))
        return cls(L_R=int(payload.get("L_R", 0)), M_R=None if m is None else tuple(int(v) for v in m),
                   parity=payload.get("parity", None), group=str(payload.get("group", "SO3")))


@dataclass(frozen=True)
class YE3TReadoutSpec:
    """Final readout target and aggregation (reference ``spec.py:378-410``)."""

    permutation: str = "trivial"
    rotation: YE3TRotationTarget = field(default_factory=YE3TRotationTarget)
    aggregation: str = "none"

    def __post_init__(self):
        if not isinstance(self.rotation, YE3TRotationTarget):
            object.__setattr__(self, "rotation", YE3TRotationTarget.from_dict(self.rotation))
        if str(self.aggregation) not in READOUT_AGGREGATIONS:
            raise ValueError(f"readout aggregation must be one of {_listed(READOUT_AGGREGATIONS)}.")
        object.__setattr__(self, "permutation", str(self.permutation))
        object.__setattr__(self, "aggregation", str(self.aggregation))

    def to_dict(self):
        return {"permutation": str(self.permutation), "rotation": self.rotation.to_dict(),
                "aggregation": str(self.aggregation)}

    @classmethod
    def from_dict(cls, payload):
        payload = {} if payload is None else dict(payload)
        return cls(permutation=str(payload.get("permutation", "trivial")),
                   rotation=YE3TRotationTarget.from_dict(payload.get("rotation", {})),
                   aggregation=str(payload.get("aggregation", "none")))


@dataclass(frozen=True)
class YE3TSpec:
    """Serializable coupling request (reference ``spec.py:416-470, 662-700``)."""

    content: tuple = ()
    slot_roles: tuple = ()
    target_permutation: str = "trivial"
    block_permutation: tuple = ()
    target_rotation: YE3TRotationTarget = field(default_factory=YE3TRotationTarget)
    carrier: str = "ACE_density"
    carrier_options: dict = field(default_factory=dict)
    task: str = "descriptor_only"
    readout: YE3TReadoutSpec = field(default_factory=YE3TReadoutSpec)
    radial_filters: dict = field(default_factory=dict)
    tree_schedule: str = "balanced"
    coefficient_backend: str = "global_coupler"
    fast_path_policy: str = "auto"
    validation_scope: str = "counts"
    runtime_status: str = "planned_not_public"
    metadata: dict = field(default_factory=dict)

    def __post_init__(self):
        if not isinstance(self.target_rotation, YE3TRotationTarget):
            object.__setattr__(self, "target_rotation", YE3TRotationTarget.from_dict(self.target_rotation))
        if not isinstance(self.readout, YE3TReadoutSpec):
            object.__setattr__(self, "readout", YE3TReadoutSpec.from_dict(self.readout))
        if str(self.carrier) not in CARRIERS:
            raise ValueError(f"carrier must be one of {_listed(CARRIERS)}.")
        if str(self.task) not in TASKS:
            raise ValueError(f"task must be one of {_listed(TASKS)}.")
        if str(self.validation_scope) not in VALIDATION_SCOPES:
            raise ValueError(f"validation_scope must be one of {_listed(VALIDATION_SCOPES)}.")
        set_ = lambda k, v: object.__setattr__(self, k, v)  # noqa: E731
        set_("content", _as_tuple(self.content))
        set_("slot_roles", _as_tuple(self.slot_roles))
        set_("target_permutation", str(self.target_permutation))
        set_("block_permutation", tuple(tuple(i) if isinstance(i, list) else i
                                        for i in _as_tuple(self.block_permutation)))
        set_("carrier", str(self.carrier))
        set_("carrier_options", dict(self.carrier_options))
        set_("task", str(self.task))
        set_("radial_filters", dict(self.radial_filters))
        set_("tree_schedule", validate_tree_schedule(self.tree_schedule))
        set_("coefficient_backend", validate_coefficient_backend(self.coefficient_backend))
        set_("fast_path_policy", validate_fast_path_policy(self.fast_path_policy))
        set_("validation_scope", str(self.validation_scope))
        set_("runtime_status", validate_runtime_status(self.runtime_status))
        set_("metadata", dict(self.metadata))

    def to_dict(self):
        return {
            "content": list(self.content), "slot_roles": list(self.slot_roles),
            "target_permutation": str(self.target_permutation),
            "block_permutation": list(self.block_permutation),
            "target_rotation": self.target_rotation.to_dict(), "carrier": str(self.carrier),
            "carrier_options": dict(self.carrier_options), "task": str(self.task),
            "readout": self.readout.to_dict(), "radial_filters": dict(self.radial_filters),
            "tree_schedule": str(self.tree_schedule), "coefficient_backend": str(self.coefficient_backend),
            "fast_path_policy": str(self.fast_path_policy), "validation_scope": str(self.validation_scope),
            "runtime_status": str(self.runtime_status), "metadata": dict(self.metadata),
        }

    @classmethod
    def from_dict(cls, payload):
        payload = {} if payload is None else dict(payload)
        if "target_rotation" in payload:
            rotation = payload.get("target_rotation", {})
        else:
            rotation = {
                "L_R": payload.get("target_L_R", payload.get("L_R", 0)),
                "M_R": payload.get("target_M_R", payload.get("target_M_R_values", payload.get("M_R_values", None))),
                "parity": payload.get("target_parity", payload.get("parity", None)),
                "group": payload.get("target_rotation_group", payload.get("rotation_group",
                                                                          payload.get("group", "SO3"))),
            }
        return cls(
            content=tuple(payload.get("content", ())), slot_roles=tuple(payload.get("slot_roles", ())),
            target_permutation=str(payload.get("target_permutation", "trivial")),
            block_permutation=tuple(payload.get("block_permutation", ())),
            target_rotation=YE3TRotationTarget.from_dict(rotation),
            carrier=str(payload.get("carrier", "ACE_density")),
            carrier_options=dict(payload.get("carrier_options",
                                             payload.get("carrier_config", payload.get("carrier_settings", {})))),
            task=str(payload.get("task", "descriptor_only")),
            readout=YE3TReadoutSpec.from_dict(payload.get("readout", {})),
            radial_filters=dict(payload.get("radial_filters", {})),
            tree_schedule=str(payload.get("tree_schedule", "balanced")),
            coefficient_backend=str(payload.get("coefficient_backend", "global_coupler")),
            fast_path_policy=str(payload.get("fast_path_policy", "auto")),
            validation_scope=str(payload.get("validation_scope", "counts")),
            runtime_status=str(payload.get("runtime_status", "planned_not_public")),
            metadata=dict(payload.get("metadata", {})),
        )


@dataclass(frozen=True)
class YE3TBackendPlan:
    """Resolved backend choice for a request (reference ``spec.py:870-935``)."""

    requested_backend: str = "global_coupler"
    selected_backend: str = "global_coupler"
    fast_path_policy: str = "auto"
    reason: str = ""
    runtime_status: str = "planned_not_public"

    def __post_init__(self):
        object.__setattr__(self, "requested_backend", validate_coefficient_backend(self.requested_backend))
        object.__setattr__(self, "selected_backend", validate_coefficient_backend(self.selected_backend))
        object.__setattr__(self, "fast_path_policy", validate_fast_path_policy(self.fast_path_policy))
        object.__setattr__(self, "reason", str(self.reason))
        object.__setattr__(self, "runtime_status", validate_runtime_status(self.runtime_status))

    @property
    def fast_path_policy_mode(self):
        return "force" if self.fast_path_policy.startswith("force:") else str(self.fast_path_policy)

    @property
    def forced_backend(self):
        return self.fast_path_policy.split(":", 1)[1] if self.fast_path_policy.startswith("force:") else None

    @property
    def legacy_force_policy(self):
        return self.fast_path_policy == "force"

    @property
    def recommended_force_policy(self):
        return f"force:{self.requested_backend}" if self.legacy_force_policy else None

    def to_dict(self):
        return {
            "requested_backend": str(self.requested_backend), "selected_backend": str(self.selected_backend),
            "fast_path_policy": str(self.fast_path_policy), "fast_path_policy_mode": self.fast_path_policy_mode,
            "forced_backend": self.forced_backend, "legacy_force_policy": bool(self.legacy_force_policy),
            "recommended_force_policy": self.recommended_force_policy, "reason": str(self.reason),
            "runtime_status": str(self.runtime_status),
        }


def plan_backend(spec, *, input_Ls=None):
    """Resolve the exact backend of a request without building coefficients.

    The decision table of ``plan_ye3t_backend`` (``ye3t/global_coupler.py:4582-4700``):
    a disabled policy selects ``global_coupler``; ``force:<backend>`` and the
    legacy ``force`` select the named backend when it is a compiler-dispatch
    backend valid for the request; an explicit fast-path request is honoured
    when valid; otherwise ACE_density in the trivial sector takes the
    symmetric-power fast path and a sign sector the exterior fast path.
    """
    spec = spec if isinstance(spec, YE3TSpec) else YE3TSpec.from_dict(spec)
    policy, requested, rank = str(spec.fast_path_policy), str(spec.coefficient_backend), len(spec.content)
    partition = target_partition(spec.target_permutation, rank) if rank else None
    trivial = partition == (rank,) if rank else spec.target_permutation == "trivial"
    sign = partition == (1,) * rank if rank else spec.target_permutation == "antisymmetric"
    angular = tuple(int(v) for v in (spec.metadata.get("input_Ls", ()) if input_Ls is None else input_Ls))
    dispatchable = {"global_coupler", "symmetric_power_fast_path", "exterior_power_fast_path"}
    status = spec.runtime_status

    def fast_path_error(backend):
        if backend == "symmetric_power_fast_path" and not (spec.carrier == "ACE_density" and trivial):
            return "symmetric_power_fast_path requires ACE_density with trivial global permutation."
        if backend == "exterior_power_fast_path" and not sign:
            return "exterior_power_fast_path requires target_permutation='antisymmetric'."
        return None

    def dispatch_error(backend):
        if backend not in dispatchable:
            return (f"{backend!r} is not an executable backend for CompileYE3TCouplers; "
                    "use 'global_coupler', 'symmetric_power_fast_path', or 'exterior_power_fast_path'.")
        return fast_path_error(backend)

    def make(selected, reason):
        return YE3TBackendPlan(requested_backend=requested, selected_backend=selected,
                               fast_path_policy=policy, reason=reason, runtime_status=status)

    fast = {"symmetric_power_fast_path", "exterior_power_fast_path"}
    if spec.carrier != "ACE_density" and any(angular):
        if requested in fast or (policy.startswith("force:") and policy.split(":", 1)[1] in fast):
            raise ValueError("External angular factors use the complete typed factorized compiler; "
                             "the ACE/exterior execution-plan backends are separate carrier paths.")
        return make("global_coupler", "complete typed factorization for ordered angular factors")
    if policy == "disable":
        return make("global_coupler", "fast paths disabled by request")
    if policy.startswith("force:") or policy == "force":
        selected = policy.split(":", 1)[1] if policy.startswith("force:") else requested
        error = dispatch_error(selected)
        if error is not None:
            raise ValueError(f"force:{error}")
        return make(selected, "backend forced by fast_path_policy" if policy != "force"
                    else "requested backend forced by legacy force policy")
    if requested in fast:
        error = fast_path_error(requested)
        if error is not None:
            raise ValueError(f"coefficient_backend={requested!r} is invalid for this YE3TSpec: {error}")
        return make(requested, "explicit coefficient_backend requests an exact fast path")
    if spec.carrier == "ACE_density" and trivial:
        return make("symmetric_power_fast_path",
                    "ACE_density with global lambda=(N) admits the symmetric-power fast path")
    if sign:
        return make("exterior_power_fast_path",
                    "global lambda=(1^N) admits the exterior/sign fast path when carrier realization supports it")
    return make("global_coupler", "no exact fast path selected for this representation request")


def coerce_spec(request=None, *, content=None, input_Ls=None, target_L=None, target_permutation=None,
                carrier=None, carrier_options=None, tree_schedule=None, coefficient_backend=None,
                fast_path_policy=None, validation_scope=None, runtime_status=None, metadata=None):
    """Merge a request (spec, mapping or None) with keyword overrides (reference ``couplings/__init__.py:333-405``)."""
    if isinstance(request, YE3TSpec):
        base = request.to_dict()
    elif isinstance(request, Mapping):
        base = dict(request)
    elif request is None:
        base = {}
    else:
        raise TypeError("request must be a YE3TSpec, mapping, or None.")
    merged = dict(base.get("metadata", {}))
    if metadata is not None:
        merged.update(dict(metadata))
    if input_Ls is not None:
        merged["input_Ls"] = tuple(int(v) for v in input_Ls)
    if content is not None:
        base["content"] = tuple(content)
    if target_L is not None:
        base["target_rotation"] = {**dict(base.get("target_rotation", {})), "L_R": int(target_L)}
    for key, value in (("target_permutation", target_permutation), ("carrier", carrier),
                       ("tree_schedule", tree_schedule), ("coefficient_backend", coefficient_backend),
                       ("fast_path_policy", fast_path_policy), ("validation_scope", validation_scope),
                       ("runtime_status", runtime_status)):
        if value is not None:
            base[key] = str(value)
    if carrier_options is not None:
        base["carrier_options"] = dict(carrier_options)
    base["metadata"] = merged
    return YE3TSpec.from_dict(base)
