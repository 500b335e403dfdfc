"""``ye3t.runtime`` counterpart for the ACE hot path on MI355X.

Same function names and argument meaning as the reference's Python dispatch
(``ye3t/runtime/execution_plan.py``); device tensors run the HIP library
(``libye3t_hip.so``).  This package is the device branch only: CPU tensors are
rejected (the reference's own CPU runtime serves them), and a missing library
is an error, never a silent fallback.
"""

import os

from ye3t_amd.runtime import native

_NATIVE_EXECUTION_PLAN_ABI = 42
HIP_OPERATIONS = (
    "cheb_exp_cos_radial_table_with_derivative",
    "spherical_harmonics_table_with_derivative",
    "density_accumulate",
    "density_accumulate_adjoint",
    "ace_density_forward",
    "symmetric_power_monomial",
    "evaluate_factorized_schedule",
    "ace_product_forward",
    "factorized_angular_linear",
    "factorized_angular_adjoint",
    "neighbor_list",
)


def _require_device(t, name):
    if not t.is_cuda:
        raise NotImplementedError(
            f"{name}: ye3t_amd implements the HIP device branch; CPU tensors are served by the reference CPU runtime")


def _backend(backend, allowed):
    backend = str(backend)
    if backend not in allowed:
        raise ValueError(f"backend must be one of {sorted(allowed)}")
    return backend


def cheb_exp_cos_radial_table_with_derivative(radii, cutoffs, lambdas, maximum_radial_index, backend="auto"):
    """ChebExpCos radial table and derivative (reference ``execution_plan.py:7298-7379``)."""
    _backend(backend, {"auto", "native"})
    maximum_radial_index = int(maximum_radial_index)
    if maximum_radial_index < 0:
        raise ValueError("maximum_radial_index must be non-negative")
    _require_device(radii, "cheb_exp_cos_radial_table_with_derivative")
    return native.radial_table(radii.contiguous(), cutoffs.contiguous(), lambdas.contiguous(),
                               maximum_radial_index)


def spherical_harmonics_table_with_derivative(edge_vectors, maximum_angular_momentum, *, real_output=False,
                                              epsilon=1.0e-12, backend="auto"):
    """Packed real SH table and Cartesian gradient (reference ``execution_plan.py:7479-7580``).

    Only ``real_output=True`` is provided: the ACE path of this backend works
    in the real basis and converts with an explicit unitary where needed.
    """
    _backend(backend, {"auto", "native"})
    if not real_output:
        raise NotImplementedError("only real_output=True is implemented by the HIP backend")
    maximum_angular_momentum = int(maximum_angular_momentum)
    if maximum_angular_momentum < 0:
        raise ValueError("maximum_angular_momentum must be non-negative")
    _require_device(edge_vectors, "spherical_harmonics_table_with_derivative")
    return native.real_sph_table(edge_vectors.contiguous(), maximum_angular_momentum, epsilon)


def density_accumulate(edge_values, centers, atom_count, *, backend="auto"):
    """Per-centre sums of edge rows (reference ``execution_plan.py:7913-7984``).

    Deterministic segment reduction: centres are sorted stably (a no-op for
    centre-sorted CSR input) and each atom's row is reduced by one thread.
    """
    import torch

    _backend(backend, {"auto", "native", "deterministic"})
    _require_device(edge_values, "density_accumulate")
    if edge_values.ndim != 2 or centers.ndim != 1 or centers.shape[0] != edge_values.shape[0]:
        raise ValueError("edge_values must be [E, C] and centers [E]")
    atom_count = int(atom_count)
    centers = centers.to(torch.int64)
    if centers.numel():
        lo, hi = int(centers.min()), int(centers.max())
        if lo < 0 or hi >= atom_count:
            raise RuntimeError("density_accumulate center index out of range")
    ordered = bool(centers.numel() < 2 or bool((centers[1:] >= centers[:-1]).all()))
    values = edge_values.contiguous()
    if not ordered:
        perm = torch.sort(centers, stable=True).indices
        centers = centers[perm]
        values = values[perm].contiguous()
    counts = torch.bincount(centers, minlength=atom_count)
    offsets = torch.zeros(atom_count + 1, dtype=torch.int64, device=values.device)
    offsets[1:] = torch.cumsum(counts, 0)
    return native.density_accumulate_csr(values, offsets, atom_count)


def density_accumulate_adjoint(atomic_adjoint, centers, *, backend="auto"):
    """Gather centre-row adjoints to edge rows (reference ``execution_plan.py:7987-8049``).

    ``edge_adjoint[e] = atomic_adjoint[centers[e]]``; the adjoint of
    :func:`density_accumulate`.  Any edge order; deterministic (a copy).
    """
    import torch

    _backend(backend, {"auto", "native", "deterministic"})
    atomic_adjoint = torch.as_tensor(atomic_adjoint)
    _require_device(atomic_adjoint, "density_accumulate_adjoint")
    centers = torch.as_tensor(centers, dtype=torch.int64, device=atomic_adjoint.device)
    if atomic_adjoint.ndim != 2 or centers.ndim != 1:
        raise ValueError("atomic_adjoint must be [N, C] and centers [E]")
    if centers.numel():
        lo, hi = int(centers.min()), int(centers.max())
        if lo < 0 or hi >= int(atomic_adjoint.shape[0]):
            raise RuntimeError("density_accumulate_adjoint center index out of range")
    return native.density_accumulate_adjoint(atomic_adjoint.contiguous(), centers.contiguous())


def neighbor_list(positions, cutoff, *, backend="auto"):
    """Neighbour CSR built on the device (open boundaries).

    Row i holds the j != i with ``|r_j - r_i| < cutoff`` (fp64 test, each
    operation rounded on its own), j ascending: the (target, source) order
    that ``prepare_carrier_scatter_segments`` (reference
    ``execution_plan.py:9316-9434``) gives, so its ``edge_order`` of this
    output is the identity.  Returns ``target_offsets [N+1]``,
    ``edge_targets`` (centres), ``edge_sources`` (neighbours) and
    ``edge_vectors = r_j - r_i`` in the positions' dtype -- the CSR, centres
    and vectors the density ops take.  The reference has no builder.
    """
    import torch

    _backend(backend, {"auto", "native"})
    positions = torch.as_tensor(positions)
    _require_device(positions, "neighbor_list")
    return native.neighbor_list(positions.contiguous(), float(cutoff))


def symmetric_power_monomial_contraction(input, monomial_counts, output_offsets, monomial_values, *,
                                         backend="auto"):
    """Symmetric-power monomial table contraction (reference ``ye3t_runtime_core.cpp:5279-5315``)."""
    _backend(backend, {"auto", "native"})
    _require_device(input, "symmetric_power_monomial_contraction")
    return native.symmetric_power_monomial(input.contiguous(), monomial_counts, output_offsets, monomial_values)


def native_execution_plan_capabilities():
    """Capability report (reference ``execution_plan.py:6118-6850``) with the HIP capability."""
    import torch

    available = native.available()
    has_hip = bool(available and torch.version.hip is not None and torch.cuda.is_available())
    report = {
        "schema": "ye3t_execution_plan_v1",
        "torch_independent_core_source": True,
        "prebuilt_extension": available,
        "cpu": False,
        "cuda": False,
        "cuda_operations": (),
        "hip": has_hip,
        "hip_operations": HIP_OPERATIONS if available else (),
        "hip_arch": "gfx950",
        "core_abi_version": native.ABI_VERSION if available else None,
        "minimum_core_abi_version": _NATIVE_EXECUTION_PLAN_ABI,
        "dtypes": ("float32", "float64"),
        "analysis_orientation": "conjugate_transpose",
        "density_reduction": "csr_segment_deterministic",
        "triton_available": False,
        "library_path": native.library_path(),
    }
    if has_hip:
        caps = native.device_caps(torch.cuda.current_device())
        report["hip_device"] = caps
    return report


def require_native():
    """Fail loudly unless the HIP library loads (``YE3T_REQUIRE_NATIVE`` semantics)."""
    native.lib()
    return True


if os.environ.get("YE3T_REQUIRE_NATIVE", "").strip().lower() in {"1", "true", "yes", "on"}:
    require_native()
