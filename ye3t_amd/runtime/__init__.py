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

# Operations this library runs on the device, under the reference's operation
# names (the ``operations`` tuple of ``native_execution_plan_capabilities``,
# reference ``execution_plan.py:6662-6850``), then this backend's fused ops.
REFERENCE_OPERATIONS = (
    "cheb_exp_cos_radial_with_derivative",
    "cheb_exp_cos_radial_table_with_derivative",
    "complex_spherical_harmonics_with_derivative",
    "real_spherical_harmonics_with_derivative",
    "complex_spherical_harmonics_table_with_derivative",
    "real_spherical_harmonics_table_with_derivative",
    "scheduled_radial_angular_channels_with_derivative",
    "density_accumulate",
    "density_accumulate_adjoint",
    "symmetric_power_monomial",
    "symmetric_power_monomial_adjoint",
    "symmetric_power_shared_monomial",
    "symmetric_power_shared_monomial_adjoint",
    "symmetric_power_shared_sparse_monomial",
    "symmetric_power_shared_sparse_monomial_adjoint",
    "symmetric_power_shared_sparse_monomial_double_backward",
    "factorized_angular",
    "factorized_angular_adjoint",
    "factorized_angular_linear",
    "factorized_angular_linear_adjoint",
    "factorized_angular_heterogeneous",
    "factorized_angular_heterogeneous_adjoint",
    "factorized_angular_segmented",
    "factorized_angular_segmented_adjoint",
)
FUSED_OPERATIONS = (
    "ace_density_forward",
    "ace_density_edge_gradient",
    "ace_product_forward",
    "ace_product_adjoint",
    "ace_product_linear",
    "evaluate_factorized_schedule",
    "neighbor_list",
)
HIP_OPERATIONS = REFERENCE_OPERATIONS + FUSED_OPERATIONS


def _require_device(t, name):
    if not t.is_cuda:
        raise NotImplementedError(
            f"{name}: ye3t_amd implements the HIP device branch; CPU tensors are served by the reference CPU runtime")


def _backend(backend, allowed):
    """Validate a reference ``backend=`` argument.  ``"reference"`` (the
    reference's pure-Torch implementation) is a known value that this device
    branch does not carry: it raises ``NotImplementedError`` naming the
    reference's own runtime instead of running anything else."""
    backend = str(backend)
    if backend == "reference":
        raise NotImplementedError("backend='reference' selects the reference's Torch implementation "
                                  "(ye3t.runtime); ye3t_amd runs the native HIP branch only")
    if backend not in allowed:
        raise ValueError(f"backend must be one of {sorted(allowed | {'reference'})}")
    return backend


def _radial_operands(radii, cutoffs, lambdas, name):
    """Radii as a tensor, with cutoffs and lambdas in its dtype and device,
    broadcast to its shape (scalars or one value per radius), as the
    reference prepares them (``execution_plan.py:7245-7275``)."""
    import torch

    radii = torch.as_tensor(radii)
    _require_device(radii, name)
    cutoffs = torch.as_tensor(cutoffs, dtype=radii.dtype, device=radii.device).expand_as(radii).contiguous()
    lambdas = torch.as_tensor(lambdas, dtype=radii.dtype, device=radii.device).expand_as(radii).contiguous()
    return radii.contiguous(), cutoffs, lambdas


def cheb_exp_cos_radial_table_with_derivative(radii, cutoffs, lambdas, maximum_radial_index, backend="auto"):
    """ChebExpCos radial table and derivative (reference ``execution_plan.py:7298-7379``):
    ``radii [E]`` to values and ``d/dr`` ``[E, maximum_radial_index + 1]``."""
    _backend(backend, {"auto", "native"})
    maximum_radial_index = int(maximum_radial_index)
    if maximum_radial_index < 0:
        raise ValueError("maximum_radial_index must be non-negative")
    radii, cutoffs, lambdas = _radial_operands(radii, cutoffs, lambdas, "cheb_exp_cos_radial_table_with_derivative")
    return native.radial_table(radii, cutoffs, lambdas, maximum_radial_index)


def cheb_exp_cos_radial_with_derivative(radii, cutoffs, lambdas, radial_index, backend="auto"):
    """One ChebExpCos radial function and its ``d/dr`` (reference
    ``execution_plan.py:7220-7295``), elementwise over ``radii`` of any shape:
    column ``radial_index`` of the HIP radial table."""
    _backend(backend, {"auto", "native"})
    radial_index = int(radial_index)
    if radial_index < 0:
        raise ValueError("radial_index must be non-negative")
    radii, cutoffs, lambdas = _radial_operands(radii, cutoffs, lambdas, "cheb_exp_cos_radial_with_derivative")
    v, d = native.radial_table(radii.reshape(-1), cutoffs.reshape(-1), lambdas.reshape(-1), radial_index)
    return v[:, radial_index].reshape(radii.shape), d[:, radial_index].reshape(radii.shape)


def _complex_rows(l_max):
    """Per packed complex column ``(l, m)``: the real columns and weights with
    ``Y_lm = wr * R[re] + i * wi * R[im]``.

    The reference forms its real rows from the complex ones
    (``execution_plan.py:6943-6963``): ``R_l0 = Re Y_l0``, and for ``m > 0``
    ``R_lm = sqrt2 (-1)^m Re Y_lm``, ``R_l,-m = -sqrt2 (-1)^m Im Y_lm``.  With
    ``Y_l,-m = (-1)^m conj(Y_lm)`` (``core/spherical.py:183-187``) this inverts
    to ``Y_lm = (-1)^m (R_lm - i R_l,-m) / sqrt2`` and
    ``Y_l,-m = (R_lm + i R_l,-m) / sqrt2``.
    """
    h = 0.5 ** 0.5
    re, im, wr, wi = [], [], [], []
    for l in range(l_max + 1):
        base = l * l + l
        for m in range(-l, l + 1):
            a = abs(m)
            re.append(base + a)
            im.append(base - a)
            if m == 0:
                wr.append(1.0)
                wi.append(0.0)
            elif m > 0:
                s = -1.0 if m % 2 else 1.0
                wr.append(s * h)
                wi.append(-s * h)
            else:
                wr.append(h)
                wi.append(h)
    return re, im, wr, wi


_COMPLEX_ROWS = {}


def _complex_tables(values, maximum_angular_momentum):
    """The columns and weights of :func:`_complex_rows` as tensors on
    ``values``'s device and dtype, built once per (l_max, device, dtype)."""
    import torch

    key = (int(maximum_angular_momentum), values.device, values.dtype)
    tables = _COMPLEX_ROWS.get(key)
    if tables is None:
        re, im, wr, wi = _complex_rows(key[0])
        tables = (torch.tensor(re, dtype=torch.int64, device=key[1]), torch.tensor(im, dtype=torch.int64, device=key[1]),
                  torch.tensor(wr, dtype=key[2], device=key[1]), torch.tensor(wi, dtype=key[2], device=key[1]))
        _COMPLEX_ROWS[key] = tables
    return tables


def complex_from_real_table(values, derivative, maximum_angular_momentum):
    """The reference's complex SH table and its Cartesian gradient from the
    packed real table ``values [E, W]`` and gradient ``derivative [E, W, 3]``.

    A fixed unitary per ``l`` (see :func:`_complex_rows`), applied on the
    tensors' own device.  The gradient is ``d Re Y + i d Im Y`` per
    component, as the reference's autograd rows (``execution_plan.py:7547-7578``).
    """
    import torch

    re, im, wr, wi = _complex_tables(values, maximum_angular_momentum)
    y = torch.complex(values[:, re] * wr, values[:, im] * wi)
    g = torch.complex(derivative[:, re, :] * wr[:, None], derivative[:, im, :] * wi[:, None])
    return y, g


def spherical_harmonics_table_with_derivative(edge_vectors, maximum_angular_momentum, *, real_output=False,
                                              epsilon=1.0e-12, backend="auto"):
    """Packed SH table and Cartesian gradient (reference ``execution_plan.py:7479-7580``).

    ``real_output=True``: the real tesseral table ``[E, (L+1)^2]`` and gradient
    ``[E, (L+1)^2, 3]`` from the HIP kernel.  ``real_output=False`` (the
    reference's default): the complex table and gradient (complex64 for
    float32 input, complex128 for float64), formed on the device from the
    HIP real table by :func:`complex_from_real_table`.
    """
    _backend(backend, {"auto", "native"})
    maximum_angular_momentum = int(maximum_angular_momentum)
    if maximum_angular_momentum < 0:
        raise ValueError("maximum_angular_momentum must be non-negative")
    _require_device(edge_vectors, "spherical_harmonics_table_with_derivative")
    v, g = native.real_sph_table(edge_vectors.contiguous(), maximum_angular_momentum, epsilon)
    if real_output:
        return v, g
    return complex_from_real_table(v, g, maximum_angular_momentum)


def spherical_harmonics_with_derivative(edge_vectors, angular_momentum, *, real_output=False, epsilon=1.0e-12,
                                        backend="auto"):
    """Harmonics of one ``l`` and their Cartesian gradient (reference
    ``execution_plan.py:7381-7476``): ``[E, 2l + 1]`` and ``[E, 2l + 1, 3]``,
    real or complex as in :func:`spherical_harmonics_table_with_derivative`,
    whose columns ``l^2 .. (l + 1)^2 - 1`` they are."""
    import torch

    angular_momentum = int(angular_momentum)
    if angular_momentum < 0:
        raise ValueError("angular_momentum must be non-negative")
    v, g = spherical_harmonics_table_with_derivative(torch.as_tensor(edge_vectors), angular_momentum,
                                                     real_output=real_output, epsilon=epsilon, backend=backend)
    lo = angular_momentum * angular_momentum
    return v[:, lo:].contiguous(), g[:, lo:].contiguous()


def scheduled_radial_angular_channels_with_derivative(radial_values, radial_derivatives, angular_values,
                                                      angular_derivatives, radial_directions, edge_types,
                                                      channel_radial_indices, channel_angular_indices,
                                                      channel_types, channel_scales, backend="auto"):
    """Scheduled radial-angular edge channels and their Cartesian derivatives
    (reference ``execution_plan.py:7675-7787``; CPU core
    ``ye3t_runtime_core.cpp:1550-1604``): ``(edge_values [E, K],
    edge_derivatives [E, K, 3])`` from the radial and angular tables, each
    channel ``k`` taking radial column ``channel_radial_indices[k]``, angular
    column ``channel_angular_indices[k]``, edges of type ``channel_types[k]``
    (all edges for -1) and the factor ``channel_scales[k]``.  Bit-identical to
    the reference core.  Data arguments are converted to ``radial_values``'s
    dtype and device and the index arguments to int64, as the reference does."""
    import torch

    _backend(backend, {"auto", "native"})
    radial_values = torch.as_tensor(radial_values)
    _require_device(radial_values, "scheduled_radial_angular_channels_with_derivative")
    dev, dt = radial_values.device, radial_values.dtype
    (radial_derivatives, angular_values, angular_derivatives, radial_directions, channel_scales) = (
        torch.as_tensor(t, dtype=dt, device=dev) for t in (radial_derivatives, angular_values, angular_derivatives,
                                                           radial_directions, channel_scales))
    (edge_types, channel_radial_indices, channel_angular_indices, channel_types) = (
        torch.as_tensor(t, dtype=torch.int64, device=dev) for t in (edge_types, channel_radial_indices,
                                                                    channel_angular_indices, channel_types))
    return native.scheduled_radial_angular_channels(radial_values, radial_derivatives, angular_values,
                                                    angular_derivatives, radial_directions, edge_types,
                                                    channel_radial_indices, channel_angular_indices, channel_types,
                                                    channel_scales)


def validate_density_csr(row_offsets, neighbors, atom_count, edge_count, *, species=None, species_count=None):
    """Host-side range checks of the fused density's index inputs (any device).

    ``row_offsets`` must be int64 ``[N+1]``, start at 0, be non-decreasing and
    end at ``edge_count``; ``neighbors`` int64 ``[E]`` in ``[0, N)``;
    ``species`` int32 ``[N]`` in ``[0, species_count)``.  The kernels gather
    through these indices without bounds checks, as the reference's do after
    its own ``TORCH_CHECK`` guards (``execution_plan_cuda.cu:37-197``), so bad
    indices raise here before any launch.  Each check reduces on the tensor's
    device and reads one scalar back.
    """
    import torch

    atom_count, edge_count = int(atom_count), int(edge_count)
    if row_offsets.dtype != torch.int64 or tuple(row_offsets.shape) != (atom_count + 1,):
        raise ValueError(f"row_offsets must be int64 [{atom_count + 1}]")
    first, last = int(row_offsets[0]), int(row_offsets[-1])
    if first != 0 or last != edge_count:
        raise ValueError(f"row_offsets must run from 0 to the edge count {edge_count} (got {first} .. {last})")
    if atom_count > 0 and bool((row_offsets[1:] < row_offsets[:-1]).any()):
        raise ValueError("row_offsets must be non-decreasing (edges sorted by centre)")
    if neighbors is not None:
        if neighbors.dtype != torch.int64 or tuple(neighbors.shape) != (edge_count,):
            raise ValueError(f"neighbors must be int64 [{edge_count}]")
        if edge_count and (int(neighbors.min()) < 0 or int(neighbors.max()) >= atom_count):
            raise ValueError(f"neighbor index out of range [0, {atom_count})")
    if species is not None:
        if species.dtype != torch.int32 or tuple(species.shape) != (atom_count,):
            raise ValueError(f"species must be int32 [{atom_count}]")
        if atom_count and (int(species.min()) < 0 or int(species.max()) >= int(species_count)):
            raise ValueError(f"species index out of range [0, {int(species_count)})")
    return True


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


def _density_function():
    import torch

    class _Density(torch.autograd.Function):
        @staticmethod
        def forward(ctx, edge_vectors, row_offsets, neighbors, kw):
            ctx.save_for_backward(edge_vectors, row_offsets, *(() if neighbors is None else (neighbors,)))
            ctx.kw = kw
            ctx.has_neighbors = neighbors is not None
            return native.ace_density_forward(edge_vectors, row_offsets, neighbors, **kw)

        @staticmethod
        def backward(ctx, grad):
            saved = ctx.saved_tensors
            vec, offsets = saved[0], saved[1]
            nbr = saved[2] if ctx.has_neighbors else None
            kw = {k: v for k, v in ctx.kw.items() if k not in ("out_dtype", "accumulate_dtype", "out")}
            g = grad.to(torch.float64 if grad.dtype == torch.float64 or vec.dtype == torch.float64 else grad.dtype)
            return native.ace_density_edge_gradient(g, vec, offsets, nbr, validate=False, **kw), None, None, None

    return _Density


_DENSITY_FN = None


def ace_density(edge_vectors, row_offsets, neighbors, *, atom_count, channel_count, n_max, l_max, cutoff, lam,
                epsilon=1e-12, species=None, node_features=None, radial_mix=None, out_dtype=None,
                accumulate_dtype=None):
    """Fused stage 1 ``A[N, C, R, (l_max+1)^2]`` (``ye3t_hip_ace_density_forward``),
    differentiable in ``edge_vectors``: the backward is the fused edge-vector
    gradient (``ye3t_hip_ace_density_edge_gradient``), the force path of the
    reference's chain (``scheduled_radial_angular_channels_with_derivative``,
    ``execution_plan.py:7675``, then ``density_accumulate_adjoint``).
    ``node_features`` and ``radial_mix`` are constants here (no gradient)."""
    global _DENSITY_FN
    _require_device(edge_vectors, "ace_density")
    for t, n in ((node_features, "node_features"), (radial_mix, "radial_mix")):
        if t is not None and t.requires_grad:
            raise NotImplementedError(f"ace_density: no gradient with respect to {n}")
    if _DENSITY_FN is None:
        _DENSITY_FN = _density_function()
    kw = dict(atom_count=int(atom_count), channel_count=int(channel_count), n_max=int(n_max), l_max=int(l_max),
              cutoff=float(cutoff), lam=float(lam), epsilon=float(epsilon), species=species,
              node_features=node_features, radial_mix=radial_mix, out_dtype=out_dtype,
              accumulate_dtype=accumulate_dtype)
    return _DENSITY_FN.apply(edge_vectors, row_offsets, neighbors, kw)


def ace_density_edge_gradient(density_adjoint, edge_vectors, row_offsets, neighbors, **kw):
    """Edge-vector gradient ``[E, 3]`` of ``<density_adjoint, A>`` for the fused
    stage 1 (arguments as :func:`ace_density`)."""
    _require_device(edge_vectors, "ace_density_edge_gradient")
    return native.ace_density_edge_gradient(density_adjoint, edge_vectors, row_offsets, neighbors, **kw)


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


def _monomial_functions():
    import torch

    class _Grouped(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, counts, offsets, indices, values):
            ctx.save_for_backward(x)
            ctx.table = (counts, offsets, indices, values)
            return native.symmetric_power_monomial(x, counts, offsets, values, output_indices=indices)

        @staticmethod
        def backward(ctx, g):
            (x,) = ctx.saved_tensors
            counts, offsets, indices, values = ctx.table
            return native.symmetric_power_monomial_adjoint(g.contiguous(), x, counts, indices, values,
                                                           offsets), None, None, None, None

    class _Shared(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, counts, offsets, terms, outputs, values):
            ctx.save_for_backward(x)
            ctx.table = (counts, offsets, terms, outputs, values)
            return native.symmetric_power_shared_monomial(x, counts, offsets, terms, outputs, values)

        @staticmethod
        def backward(ctx, g):
            (x,) = ctx.saved_tensors
            return (native.symmetric_power_shared_monomial_adjoint(g.contiguous(), x, *ctx.table),
                    None, None, None, None, None)

    class _Sparse(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, *tables):
            ctx.save_for_backward(x)
            ctx.table = tables
            return native.symmetric_power_shared_sparse_monomial(x, *tables)

        @staticmethod
        def backward(ctx, g):
            (x,) = ctx.saved_tensors
            return (native.symmetric_power_shared_sparse_monomial_adjoint(g.contiguous(), x, *ctx.table),) + \
                (None,) * len(ctx.table)

    return _Grouped, _Shared, _Sparse


_MONOMIAL_FNS = None


def _monomials():
    global _MONOMIAL_FNS
    if _MONOMIAL_FNS is None:
        _MONOMIAL_FNS = _monomial_functions()
    return _MONOMIAL_FNS


def _feature_rows(input, name):
    if input.ndim < 1:
        raise ValueError("symmetric-power input requires a feature axis")
    _require_device(input, name)
    return input.reshape(-1, int(input.shape[-1])).contiguous()


def symmetric_power_monomial_contraction(input, monomial_counts, output_offsets, output_indices, monomial_values, *,
                                         backend="auto"):
    """Compiler-grouped symmetric-power table contraction (reference
    ``execution_plan.py:11998-12095``; core ``ye3t_runtime_core.cpp:5279-5315``).

    ``S[..., o] = sum_{t in [output_offsets[o], output_offsets[o+1])} v_t prod_c input[..., c]^counts[t, c]``;
    ``output_indices[t]`` names the output of term t.  Differentiable: the
    backward is the library's monomial adjoint (``ye3t_runtime_core.cpp:5318-5389``).
    """
    _backend(backend, {"auto", "native"})
    flat = _feature_rows(input, "symmetric_power_monomial_contraction")
    out = _monomials()[0].apply(flat, monomial_counts, output_offsets, output_indices, monomial_values)
    return out.reshape(tuple(input.shape[:-1]) + (int(out.shape[-1]),))


def symmetric_power_shared_monomial_contraction(input, monomial_counts, output_offsets, coefficient_terms,
                                                coefficient_outputs, coefficient_values, *, backend="auto"):
    """Shared-monomial symmetric-power contraction (reference
    ``execution_plan.py:12502-12600``; core ``ye3t_runtime_core.cpp:5392-5440``):
    outputs are sparse combinations of unique monomials.  Differentiable
    (adjoint ``ye3t_runtime_core.cpp:5442-5540``)."""
    _backend(backend, {"auto", "native"})
    flat = _feature_rows(input, "symmetric_power_shared_monomial_contraction")
    out = _monomials()[1].apply(flat, monomial_counts, output_offsets, coefficient_terms, coefficient_outputs,
                                coefficient_values)
    return out.reshape(tuple(input.shape[:-1]) + (int(out.shape[-1]),))


def symmetric_power_shared_sparse_monomial_contraction(input, term_offsets, term_components, term_exponents,
                                                       output_offsets, coefficient_terms, coefficient_outputs,
                                                       coefficient_values, *, backend="auto"):
    """Shared-monomial contraction with sparse monomial supports: monomial t is
    ``prod_{q in [term_offsets[t], term_offsets[t+1])} input[..., term_components[q]]^term_exponents[q]``
    and outputs are sparse combinations of monomials (the reference's
    ``ye3t_runtime::symmetric_power_shared_sparse_monomial``,
    ``execution_plan_cuda.cu:5720-5755, 11012-11104``).  Differentiable; the
    backward is the sparse adjoint (``:5757-5813``)."""
    _backend(backend, {"auto", "native"})
    flat = _feature_rows(input, "symmetric_power_shared_sparse_monomial_contraction")
    out = _monomials()[2].apply(flat, term_offsets, term_components, term_exponents, output_offsets,
                                coefficient_terms, coefficient_outputs, coefficient_values)
    return out.reshape(tuple(input.shape[:-1]) + (int(out.shape[-1]),))


# Thresholds and constants of the reference report (execution_plan.py:27-35,
# 6536-6640) that keep their values here.  The symmetric-power CPU thresholds
# steer the reference's CPU dispatch (symmetric_power.py:1131-1150), which
# reads them whenever ``prebuilt_extension`` is true; CPU tensors are served by
# the reference's own CPU runtime, so they are carried unchanged.
_SYMMETRIC_POWER_CPU_AUTO_MAX_BATCH = 32
_SYMMETRIC_POWER_CPU_AUTO_MIN_POWER = 6
_SYMMETRIC_POWER_SHARED_CPU_MIN_REUSE = 3.0
_SYMMETRIC_POWER_SHARED_CPU_MIN_BATCH = 8
_SYMMETRIC_POWER_SHARED_GPU_MIN_REUSE = 8.0
_SYMMETRIC_POWER_SHARED_GPU_GRAD_MIN_BATCH = 256
_SYMMETRIC_POWER_SHARED_GPU_FORWARD_MIN_BATCH = 1024
_COMPACT_EXTERIOR_POWER_MAX_NATIVE_ORDER = 8
_REAL_TESSERAL_CONVENTION = "real_tesseral_from_complex_condon_shortley_young_orthogonal_v1"
_TRITON_OPERATIONS = ("dense_source_analysis_C_dagger_L_v", "dense_source_analysis_channel_mixing",
                      "packed_joint_young_angular_bilinear", "packed_joint_young_angular_channel_mixing")


def _cpu_kernels_registered():
    """True when the ``ye3t_runtime`` operators have CPU kernels in this process
    (the reference's extension loaded beside this library)."""
    try:
        import torch

        return bool(torch._C._dispatch_has_kernel_for_dispatch_key("ye3t_runtime::density_accumulate", "CPU"))
    except Exception:
        return False


def native_execution_plan_capabilities():
    """Capability report (reference ``execution_plan.py:6118-6850``) with the HIP capability.

    Every key of the reference report is present with the reference's
    meaning, read for this library:

    * ``cuda`` / ``cuda_operations``: native kernels for tensors whose device
      type is ``"cuda"``, which on PyTorch-ROCm is the HIP device.  The
      reference's consumers pick the native GPU path by testing an operation's
      name in ``cuda_operations`` (``symmetric_power.py:1131-1137``), so it
      lists the ``ye3t_runtime`` operator names this library gives a device
      kernel (:mod:`ye3t_amd.runtime.torch_ops`).  ``hip`` / ``hip_operations``
      say the same under the new capability's own name; ``hip_device`` adds
      the device (arch, CU count, LDS, HBM peak).
    * Capability flags of operator families this library does not build
      (carrier scatters, role densities, source arenas, double backward of
      the dense monomials and of the factorized-angular operators) are False,
      and the thresholds that only those families read are None, as the
      reference reports them when it lacks them.
    * ``cpu``: CPU kernels of the ``ye3t_runtime`` operators are registered in
      this process (the reference's own CPU runtime); this library has none.
    * ``cmake_core_target``: the name of the native library that holds the
      Torch-independent core (``libye3t_hip.so``, built by
      ``ye3t_amd._build``; there is no CMake project).
    """
    import torch

    available = native.available()
    has_hip = bool(available and torch.version.hip is not None and torch.cuda.is_available()
                   and native.has_hip())
    abi = native.ABI_VERSION if available else None
    ops = HIP_OPERATIONS if available else ()
    cuda_ops = ()
    if has_hip:
        from ye3t_amd.runtime import torch_ops

        cuda_ops = tuple(torch_ops.KERNELS)
    sparse = bool(has_hip and {"symmetric_power_shared_sparse_monomial",
                               "symmetric_power_shared_sparse_monomial_adjoint",
                               "symmetric_power_shared_sparse_monomial_double_backward"} <= set(cuda_ops))
    cpu = _cpu_kernels_registered()
    report = {
        "schema": "ye3t_execution_plan_v1",
        "torch_independent_core_source": True,
        "cmake_core_target": "ye3t_hip",
        "prebuilt_extension": available,
        "cpu": cpu,
        "cuda": has_hip,
        "cuda_operations": cuda_ops,
        # the HIP density reduction is a deterministic CSR segment sum at any size
        "cuda_density_auto_min_work_items": 0 if has_hip else None,
        "cuda_edge_outer_auto_min_work_items": None,
        "cpu_edge_outer_auto_min_work_items": None,
        "cpu_carrier_gated_scatter_auto_min_work_items": None,
        "cuda_carrier_gated_scatter_auto_min_work_items": None,
        "real_control_carrier_gates": False,
        "residual_carrier_gated_scatter": False,
        "segmented_carrier_gated_scatter": False,
        "segmented_factorized_angular": bool(available),
        "source_arena_gather": False,
        "source_arena_channel_transform": False,
        "carrier_channel_transform": False,
        "carrier_role_channel_map_adjoint": False,
        "cuda_segmented_carrier_scatter_min_node_feature_work": None,
        "real_control_carrier_channel_update": False,
        "scheduled_softmax_gaussian_role_density": False,
        "symmetric_power_monomial_double_backward": False,
        "symmetric_power_shared_monomial_double_backward": False,
        "symmetric_power_shared_monomial_factored_double_backward": False,
        "symmetric_power_shared_double_backward_default_algorithm": "auto",
        "symmetric_power_shared_sparse_monomial": sparse,
        "cpu_carrier_channel_update_auto_max_work_items": None,
        "cuda_carrier_channel_update_auto_max_work_items": None,
        "cuda_carrier_channel_update_auto_min_work_items": None,
        "symmetric_power_cpu_auto_max_batch": _SYMMETRIC_POWER_CPU_AUTO_MAX_BATCH if available else None,
        "symmetric_power_cpu_auto_min_power": _SYMMETRIC_POWER_CPU_AUTO_MIN_POWER if available else None,
        "symmetric_power_shared_cpu_min_reuse": _SYMMETRIC_POWER_SHARED_CPU_MIN_REUSE if available else None,
        "symmetric_power_shared_cpu_min_batch": _SYMMETRIC_POWER_SHARED_CPU_MIN_BATCH if available else None,
        "symmetric_power_shared_cuda_min_reuse": _SYMMETRIC_POWER_SHARED_GPU_MIN_REUSE if has_hip else None,
        "symmetric_power_shared_cuda_grad_min_batch": _SYMMETRIC_POWER_SHARED_GPU_GRAD_MIN_BATCH if has_hip else None,
        "symmetric_power_shared_cuda_forward_min_batch": (_SYMMETRIC_POWER_SHARED_GPU_FORWARD_MIN_BATCH
                                                          if has_hip else None),
        "triton_available": False,
        "triton_cuda_available": False,
        "triton_real_convention_id": _REAL_TESSERAL_CONVENTION,
        "triton_operations": _TRITON_OPERATIONS,
        "core_abi_version": abi,
        "factorized_workspace_metadata": "compiler_host_scalar_no_device_read",
        "heterogeneous_factorized_roots": bool(available),
        # needs the heterogeneous reverse-with-workspace and its double backward
        "cached_heterogeneous_factorized_reverse": False,
        "dtypes": ("float32", "float64", "complex64", "complex128"),
        "analysis_orientation": "conjugate_transpose",
        "operations": ops,
        "compact_exterior_power_max_native_order": _COMPACT_EXTERIOR_POWER_MAX_NATIVE_ORDER,
        # this backend's own keys
        "hip": has_hip,
        "hip_operations": ops if has_hip else (),
        "hip_arch": "gfx950",
        "hip_density_reduction": "csr_segment_deterministic",
        "minimum_core_abi_version": _NATIVE_EXECUTION_PLAN_ABI,
        "density_reduction": "csr_segment_deterministic",
        "library_path": native.library_path(),
    }
    if has_hip:
        report["hip_device"] = native.device_caps(torch.cuda.current_device())
    return report


def __getattr__(name):
    # the factorized-angular op and module load torch, so they are imported on first use
    if name in ("factorized_angular", "factorized_angular_linear", "factorized_angular_segmented",
                "YE3TFactorizedAngularModule", "YE3TSegmentedFactorizedAngularModuleGroup"):
        import importlib

        return getattr(importlib.import_module("ye3t_amd.runtime.dag"), name)
    if name in ("ExecutionPlan", "YE3TExecutionPlan"):
        from ye3t_amd.runtime.execution_plan import ExecutionPlan

        return ExecutionPlan
    if name in ("YE3THierarchicalRepeatedBlockModule", "YE3THierarchicalRepeatedBlockModuleGroup",
                "symmetric_power_product_plan_contraction", "symmetric_power_product_plan_table_report"):
        import importlib

        return getattr(importlib.import_module("ye3t_amd.runtime.hierarchical"), name)
    raise AttributeError(name)


def require_native():
    """Fail loudly unless the HIP library loads (``YE3T_REQUIRE_NATIVE`` semantics)."""
    native.lib()
    return True


if os.environ.get("YE3T_REQUIRE_NATIVE", "").strip().lower() in {"1", "true", "yes", "on"}:
    require_native()
