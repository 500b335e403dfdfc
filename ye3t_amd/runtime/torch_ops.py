"""Torch operator shim: the reference's ``ye3t_runtime`` operators on the HIP library.

The reference registers its native runtime as Torch operators in the
``ye3t_runtime`` namespace (schemas ``execution_plan_torch.cpp:7228-7730``,
``TORCH_LIBRARY_IMPL(ye3t_runtime, CPU/CUDA, ...)``) with fake (meta)
implementations and autograd formulas registered from Python
(``execution_plan.py:392-2360, 2936-4100``).  Its callers reach the native code
through ``torch.ops.ye3t_runtime.<op>``.  :func:`register` gives those
operators a device kernel here: on ROCm the ``CUDA`` dispatch key is the HIP
device, so a call with device tensors runs this library's kernels.

* Where the reference's extension is already loaded (its schemas defined),
  only the device kernels are added; otherwise the schemas are defined here,
  with the reference's exact signatures, together with fake implementations
  and the first-order autograd formulas of the forward operators (backward =
  the reference's adjoint operator; for the radial and harmonic operators,
  the saved derivative output contracted with the incoming gradient, and for
  a second derivative autograd through a differentiable Torch expression of
  the basis, as the reference does without its native double backward).
* Operators covered: the radial function and table, the harmonics of one
  ``l`` and the harmonic table (real and complex output), the scheduled
  radial-angular edge channels, density accumulation and its adjoint, the symmetric-power monomial and
  shared-monomial contractions and adjoints, the sparse shared-monomial
  contraction with its adjoint and double backward, and the factorized-angular
  forward / adjoint / linear readout / heterogeneous / segmented operators.
  The sparse shared-monomial adjoint is differentiable through its double
  backward, as in the reference; the other adjoint operators are not
  (differentiating one raises Torch's "no autograd" error).
* CPU tensors are not served: the reference's CPU kernels serve them (a call
  with CPU tensors and no reference extension raises Torch's dispatch error).
"""

import threading

import numpy as np

from ye3t_amd.runtime import native

NAMESPACE = "ye3t_runtime"

# name -> schema (the reference's, execution_plan_torch.cpp line cited per entry)
SCHEMAS = {
    # :7235
    "cheb_exp_cos_radial_with_derivative":
        "(Tensor radii, Tensor cutoffs, Tensor lambdas, int radial_index) -> (Tensor, Tensor)",
    # :7238
    "cheb_exp_cos_radial_table_with_derivative":
        "(Tensor radii, Tensor cutoffs, Tensor lambdas, int maximum_radial_index) -> (Tensor, Tensor)",
    # :7247
    "spherical_harmonics_with_derivative":
        "(Tensor edge_vectors, int angular_momentum, bool real_output, float epsilon) -> (Tensor, Tensor)",
    # :7251
    "spherical_harmonics_table_with_derivative":
        "(Tensor edge_vectors, int maximum_angular_momentum, bool real_output, float epsilon) -> (Tensor, Tensor)",
    # :7268
    "scheduled_radial_angular_channels_with_derivative":
        "(Tensor radial_values, Tensor radial_derivatives, Tensor angular_values, Tensor angular_derivatives, "
        "Tensor radial_directions, Tensor edge_types, Tensor channel_radial_indices, "
        "Tensor channel_angular_indices, Tensor channel_types, Tensor channel_scales) -> (Tensor, Tensor)",
    # :7285, :7288
    "density_accumulate": "(Tensor edge_values, Tensor centers, int atom_count) -> Tensor",
    "density_accumulate_adjoint": "(Tensor atomic_adjoint, Tensor centers) -> Tensor",
    # :7528, :7532
    "symmetric_power_monomial":
        "(Tensor input, Tensor monomial_counts, Tensor output_offsets, Tensor output_indices, "
        "Tensor monomial_values) -> Tensor",
    "symmetric_power_monomial_adjoint":
        "(Tensor output_adjoint, Tensor input, Tensor monomial_counts, Tensor output_offsets, "
        "Tensor output_indices, Tensor monomial_values) -> Tensor",
    # :7541, :7546
    "symmetric_power_shared_monomial":
        "(Tensor input, Tensor monomial_counts, Tensor output_offsets, Tensor coefficient_terms, "
        "Tensor coefficient_outputs, Tensor coefficient_values) -> Tensor",
    "symmetric_power_shared_monomial_adjoint":
        "(Tensor output_adjoint, Tensor input, Tensor monomial_counts, Tensor output_offsets, "
        "Tensor coefficient_terms, Tensor coefficient_outputs, Tensor coefficient_values) -> Tensor",
    # :7563, :7569, :7575
    "symmetric_power_shared_sparse_monomial":
        "(Tensor input, Tensor term_offsets, Tensor term_components, Tensor term_exponents, "
        "Tensor output_offsets, Tensor coefficient_terms, Tensor coefficient_outputs, "
        "Tensor coefficient_values) -> Tensor",
    "symmetric_power_shared_sparse_monomial_adjoint":
        "(Tensor output_adjoint, Tensor input, Tensor term_offsets, Tensor term_components, "
        "Tensor term_exponents, Tensor output_offsets, Tensor coefficient_terms, "
        "Tensor coefficient_outputs, Tensor coefficient_values) -> Tensor",
    "symmetric_power_shared_sparse_monomial_double_backward":
        "(Tensor input_adjoint_tangent, Tensor output_adjoint, Tensor input, Tensor term_offsets, "
        "Tensor term_components, Tensor term_exponents, Tensor output_offsets, Tensor coefficient_terms, "
        "Tensor coefficient_outputs, Tensor coefficient_values) -> (Tensor, Tensor)",
    # :7587, :7596
    "factorized_angular":
        "(Tensor packed_slots, Tensor node_offsets, Tensor node_dimensions, Tensor node_leaf_offsets, "
        "Tensor node_left, Tensor node_right, Tensor node_coefficient_offsets, Tensor coefficient_rows, "
        "Tensor coefficient_columns, Tensor coefficient_values, Tensor root_nodes, Tensor projection_values, "
        "int source_dimension, int workspace_dimension, int output_dimension) -> Tensor",
    "factorized_angular_adjoint":
        "(Tensor output_adjoint, Tensor packed_slots, Tensor node_offsets, Tensor node_dimensions, "
        "Tensor node_leaf_offsets, Tensor node_left, Tensor node_right, Tensor node_coefficient_offsets, "
        "Tensor coefficient_rows, Tensor coefficient_columns, Tensor coefficient_values, Tensor root_nodes, "
        "Tensor projection_values, int source_dimension, int workspace_dimension) -> Tensor",
    # :7613, :7623
    "factorized_angular_heterogeneous":
        "(Tensor packed_slots, Tensor node_offsets, Tensor node_dimensions, Tensor node_leaf_offsets, "
        "Tensor node_left, Tensor node_right, Tensor node_coefficient_offsets, Tensor coefficient_rows, "
        "Tensor coefficient_columns, Tensor coefficient_values, Tensor root_nodes, Tensor root_projection_starts, "
        "Tensor root_projection_dimensions, Tensor root_output_offsets, Tensor projection_values, "
        "int source_dimension, int workspace_dimension, int output_dimension) -> Tensor",
    "factorized_angular_heterogeneous_adjoint":
        "(Tensor output_adjoint, Tensor packed_slots, Tensor node_offsets, Tensor node_dimensions, "
        "Tensor node_leaf_offsets, Tensor node_left, Tensor node_right, Tensor node_coefficient_offsets, "
        "Tensor coefficient_rows, Tensor coefficient_columns, Tensor coefficient_values, Tensor root_nodes, "
        "Tensor root_projection_starts, Tensor root_projection_dimensions, Tensor root_output_offsets, "
        "Tensor projection_values, int source_dimension, int workspace_dimension) -> Tensor",
    # :7666, :7682
    "factorized_angular_segmented":
        "(Tensor packed_slots, Tensor segment_source_offsets, Tensor segment_input_offsets, "
        "Tensor segment_input_dimensions, Tensor segment_workspace_offsets, Tensor segment_workspace_dimensions, "
        "Tensor segment_node_offsets, Tensor segment_root_offsets, Tensor segment_projection_offsets, "
        "Tensor segment_projection_dimensions, Tensor segment_output_offsets, Tensor node_offsets, "
        "Tensor node_dimensions, Tensor node_leaf_offsets, Tensor node_left, Tensor node_right, "
        "Tensor node_coefficient_offsets, Tensor coefficient_rows, Tensor coefficient_columns, "
        "Tensor coefficient_values, Tensor root_nodes, Tensor root_projection_starts, "
        "Tensor root_projection_dimensions, Tensor root_output_offsets, Tensor projection_values, "
        "int total_source_count, int workspace_dimension, int output_dimension) -> Tensor",
    "factorized_angular_segmented_adjoint":
        "(Tensor output_adjoint, Tensor packed_slots, Tensor segment_source_offsets, "
        "Tensor segment_input_offsets, Tensor segment_input_dimensions, Tensor segment_workspace_offsets, "
        "Tensor segment_workspace_dimensions, Tensor segment_node_offsets, Tensor segment_root_offsets, "
        "Tensor segment_projection_offsets, Tensor segment_projection_dimensions, Tensor segment_output_offsets, "
        "Tensor node_offsets, Tensor node_dimensions, Tensor node_leaf_offsets, Tensor node_left, "
        "Tensor node_right, Tensor node_coefficient_offsets, Tensor coefficient_rows, "
        "Tensor coefficient_columns, Tensor coefficient_values, Tensor root_nodes, Tensor root_projection_starts, "
        "Tensor root_projection_dimensions, Tensor root_output_offsets, Tensor projection_values, "
        "int total_source_count, int workspace_dimension) -> Tensor",
    # :7713, :7722
    "factorized_angular_linear":
        "(Tensor packed_slots, Tensor node_offsets, Tensor node_dimensions, Tensor node_leaf_offsets, "
        "Tensor node_left, Tensor node_right, Tensor node_coefficient_offsets, Tensor coefficient_rows, "
        "Tensor coefficient_columns, Tensor coefficient_values, Tensor root_nodes, Tensor projection_values, "
        "int source_dimension, int workspace_dimension, Tensor weight, Tensor bias) -> Tensor",
    "factorized_angular_linear_adjoint":
        "(Tensor output_adjoint, Tensor packed_slots, Tensor node_offsets, Tensor node_dimensions, "
        "Tensor node_leaf_offsets, Tensor node_left, Tensor node_right, Tensor node_coefficient_offsets, "
        "Tensor coefficient_rows, Tensor coefficient_columns, Tensor coefficient_values, Tensor root_nodes, "
        "Tensor projection_values, int source_dimension, int workspace_dimension, Tensor weight) "
        "-> (Tensor, Tensor, Tensor)",
}

_LOCK = threading.Lock()
_STATE = {"registered": False, "defined": (), "libs": []}


def _ops():
    import torch

    return getattr(torch.ops, NAMESPACE)


# ---- device kernels ----------------------------------------------------------------------------------------

def _fa_tables(args):
    return dict(zip(native.FA_TABLE_NAMES, args))


def _fa_plan(packed, tables, source_dimension, workspace_dimension, output_dimension):
    from ye3t_amd.runtime.dag import plan_for

    S = int(source_dimension)
    if S <= 0 or packed.ndim != 2 or int(packed.shape[1]) % S:
        raise RuntimeError("packed_slots width must be divisible by source_dimension")
    return plan_for(tables, S, int(packed.shape[1]) // S, workspace_dimension, output_dimension, packed.dtype,
                    packed.device)


def _hetero_tables(node_tables, root_projection_starts, root_projection_dimensions, root_output_offsets,
                   projection_values, source_dimension, input_dimension, workspace_dimension, output_dimension):
    """One DAG with explicit root metadata as a one-segment segmented table set."""
    S, D, W, F = (int(v) for v in (source_dimension, input_dimension, workspace_dimension, output_dimension))
    n = int(node_tables["node_offsets"].numel())
    r = int(node_tables["root_nodes"].numel())
    proj = projection_values.detach().cpu().numpy().reshape(-1)
    if S <= 0 or proj.size % S:
        raise RuntimeError("projection weights must be nonempty and divisible by source_dimension")
    one = {
        "segment_source_offsets": [0, S], "segment_input_offsets": [0], "segment_input_dimensions": [D],
        "segment_workspace_offsets": [0], "segment_workspace_dimensions": [W], "segment_node_offsets": [0, n],
        "segment_root_offsets": [0, r], "segment_projection_offsets": [0],
        "segment_projection_dimensions": [proj.size // S], "segment_output_offsets": [0, F],
    }
    tables = {k: np.asarray(v, dtype=np.int64) for k, v in one.items()}
    for k in ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
              "node_coefficient_offsets", "coefficient_rows", "coefficient_columns", "coefficient_values",
              "root_nodes"):
        tables[k] = node_tables[k]
    tables["root_projection_starts"] = root_projection_starts
    tables["root_projection_dimensions"] = root_projection_dimensions
    tables["root_output_offsets"] = root_output_offsets
    tables["projection_values"] = projection_values
    return tables, (S * D, S, S * W, F)


def _hetero_plan(packed, node_args, roots_meta, projection_values, source_dimension, workspace_dimension,
                 output_dimension):
    from ye3t_amd.runtime.dag import segmented_plan_for

    S = int(source_dimension)
    if S <= 0 or packed.ndim != 2 or int(packed.shape[1]) % S:
        raise RuntimeError("packed_slots width must be divisible by source_dimension")
    names = ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
             "node_coefficient_offsets", "coefficient_rows", "coefficient_columns", "coefficient_values",
             "root_nodes")
    tables, dims = _hetero_tables(dict(zip(names, node_args)), *roots_meta, projection_values, S,
                                  int(packed.shape[1]) // S, workspace_dimension, output_dimension)
    return segmented_plan_for(tables, *dims, packed.dtype, packed.device)


def _seg_plan(packed, tables_args, total_source_count, workspace_dimension, output_dimension):
    from ye3t_amd.runtime.dag import segmented_plan_for

    if packed.ndim != 2:
        raise RuntimeError("packed_slots must be [batch, packed width]")
    tables = dict(zip(native.SEGMENT_TABLE_NAMES, tables_args))
    return segmented_plan_for(tables, int(packed.shape[1]), total_source_count, workspace_dimension,
                              output_dimension, packed.dtype, packed.device)


def _k_radial(radii, cutoffs, lambdas, maximum_radial_index):
    v, d = native.radial_table(radii.contiguous(), cutoffs.contiguous(), lambdas.contiguous(),
                               int(maximum_radial_index))
    return v, d


def _k_radial_one(radii, cutoffs, lambdas, radial_index):
    from ye3t_amd import runtime

    return runtime.cheb_exp_cos_radial_with_derivative(radii, cutoffs, lambdas, int(radial_index))


def _k_sph_one(edge_vectors, angular_momentum, real_output, epsilon):
    from ye3t_amd import runtime

    return runtime.spherical_harmonics_with_derivative(edge_vectors, angular_momentum,
                                                       real_output=bool(real_output), epsilon=float(epsilon))


def _k_scheduled(*args):
    return native.scheduled_radial_angular_channels(*args)


def _k_sph(edge_vectors, maximum_angular_momentum, real_output, epsilon):
    from ye3t_amd import runtime

    return runtime.spherical_harmonics_table_with_derivative(edge_vectors, maximum_angular_momentum,
                                                             real_output=bool(real_output),
                                                             epsilon=float(epsilon))


def _k_density(edge_values, centers, atom_count):
    from ye3t_amd import runtime

    return runtime.density_accumulate(edge_values, centers, atom_count)


def _k_density_adjoint(atomic_adjoint, centers):
    from ye3t_amd import runtime

    return runtime.density_accumulate_adjoint(atomic_adjoint, centers)


def _rows(x):
    return x.reshape(-1, int(x.shape[-1])).contiguous()


def _k_monomial(input, monomial_counts, output_offsets, output_indices, monomial_values):
    out = native.symmetric_power_monomial(_rows(input), monomial_counts, output_offsets, monomial_values,
                                          output_indices=output_indices)
    return out.reshape(tuple(input.shape[:-1]) + (int(out.shape[-1]),))


def _k_monomial_adjoint(output_adjoint, input, monomial_counts, output_offsets, output_indices, monomial_values):
    g = native.symmetric_power_monomial_adjoint(_rows(output_adjoint), _rows(input), monomial_counts,
                                                output_indices, monomial_values, output_offsets)
    return g.reshape(input.shape)


def _k_shared(input, monomial_counts, output_offsets, coefficient_terms, coefficient_outputs, coefficient_values):
    out = native.symmetric_power_shared_monomial(_rows(input), monomial_counts, output_offsets, coefficient_terms,
                                                 coefficient_outputs, coefficient_values)
    return out.reshape(tuple(input.shape[:-1]) + (int(out.shape[-1]),))


def _k_shared_adjoint(output_adjoint, input, monomial_counts, output_offsets, coefficient_terms,
                      coefficient_outputs, coefficient_values):
    g = native.symmetric_power_shared_monomial_adjoint(_rows(output_adjoint), _rows(input), monomial_counts,
                                                       output_offsets, coefficient_terms, coefficient_outputs,
                                                       coefficient_values)
    return g.reshape(input.shape)


def _k_sparse(input, *tables):
    out = native.symmetric_power_shared_sparse_monomial(_rows(input), *tables)
    return out.reshape(tuple(input.shape[:-1]) + (int(out.shape[-1]),))


def _k_sparse_adjoint(output_adjoint, input, *tables):
    g = native.symmetric_power_shared_sparse_monomial_adjoint(_rows(output_adjoint), _rows(input), *tables)
    return g.reshape(input.shape)


def _k_sparse_double_backward(input_adjoint_tangent, output_adjoint, input, *tables):
    ot, it = native.symmetric_power_shared_sparse_monomial_double_backward(
        _rows(input_adjoint_tangent), _rows(output_adjoint), _rows(input), *tables)
    return ot.reshape(output_adjoint.shape), it.reshape(input.shape)


def _k_fa(packed_slots, *rest):
    tables, (S, W, F) = _fa_tables(rest[:11]), rest[11:]
    return _fa_plan(packed_slots, tables, S, W, F).forward(packed_slots.contiguous())


def _k_fa_adjoint(output_adjoint, packed_slots, *rest):
    tables, (S, W) = _fa_tables(rest[:11]), rest[11:]
    return _fa_plan(packed_slots, tables, S, W, int(output_adjoint.shape[1])).adjoint(
        output_adjoint.contiguous(), packed_slots.contiguous())


def _k_fa_linear(packed_slots, *rest):
    tables, (S, W, weight, bias) = _fa_tables(rest[:11]), rest[11:]
    plan = _fa_plan(packed_slots, tables, S, W, int(weight.numel()))
    return plan.linear(packed_slots.contiguous(), weight, bias.reshape(()).item())


def _k_fa_linear_adjoint(output_adjoint, packed_slots, *rest):
    tables, (S, W, weight) = _fa_tables(rest[:11]), rest[11:]
    plan = _fa_plan(packed_slots, tables, S, W, int(weight.numel()))
    gx, gw, gb = plan.linear_adjoint(output_adjoint.contiguous(), packed_slots.contiguous(), weight)
    return gx, gw, gb


def _k_hetero(packed_slots, *rest):
    node_args, meta, proj, (S, W, F) = rest[:10], rest[10:13], rest[13], rest[14:]
    return _hetero_plan(packed_slots, node_args, meta, proj, S, W, F).forward(packed_slots.contiguous())


def _k_hetero_adjoint(output_adjoint, packed_slots, *rest):
    node_args, meta, proj, (S, W) = rest[:10], rest[10:13], rest[13], rest[14:]
    return _hetero_plan(packed_slots, node_args, meta, proj, S, W, int(output_adjoint.shape[1])).adjoint(
        output_adjoint.contiguous(), packed_slots.contiguous())


def _k_seg(packed_slots, *rest):
    tables_args, (total, W, F) = rest[:24], rest[24:]
    return _seg_plan(packed_slots, tables_args, total, W, F).forward(packed_slots.contiguous())


def _k_seg_adjoint(output_adjoint, packed_slots, *rest):
    tables_args, (total, W) = rest[:24], rest[24:]
    return _seg_plan(packed_slots, tables_args, total, W, int(output_adjoint.shape[1])).adjoint(
        output_adjoint.contiguous(), packed_slots.contiguous())


KERNELS = {
    "cheb_exp_cos_radial_table_with_derivative": _k_radial,
    "spherical_harmonics_table_with_derivative": _k_sph,
    "cheb_exp_cos_radial_with_derivative": _k_radial_one,
    "spherical_harmonics_with_derivative": _k_sph_one,
    "scheduled_radial_angular_channels_with_derivative": _k_scheduled,
    "density_accumulate": _k_density,
    "density_accumulate_adjoint": _k_density_adjoint,
    "symmetric_power_monomial": _k_monomial,
    "symmetric_power_monomial_adjoint": _k_monomial_adjoint,
    "symmetric_power_shared_monomial": _k_shared,
    "symmetric_power_shared_monomial_adjoint": _k_shared_adjoint,
    "symmetric_power_shared_sparse_monomial": _k_sparse,
    "symmetric_power_shared_sparse_monomial_adjoint": _k_sparse_adjoint,
    "symmetric_power_shared_sparse_monomial_double_backward": _k_sparse_double_backward,
    "factorized_angular": _k_fa,
    "factorized_angular_adjoint": _k_fa_adjoint,
    "factorized_angular_heterogeneous": _k_hetero,
    "factorized_angular_heterogeneous_adjoint": _k_hetero_adjoint,
    "factorized_angular_segmented": _k_seg,
    "factorized_angular_segmented_adjoint": _k_seg_adjoint,
    "factorized_angular_linear": _k_fa_linear,
    "factorized_angular_linear_adjoint": _k_fa_linear_adjoint,
}


# ---- fake (meta) implementations: output shapes and dtypes (reference execution_plan.py:392-2360) ------------

def _f_radial(radii, cutoffs, lambdas, maximum_radial_index):
    shape = (radii.shape[0], int(maximum_radial_index) + 1)
    return radii.new_empty(shape), radii.new_empty(shape)


def _f_radial_one(radii, cutoffs, lambdas, radial_index):
    return radii.new_empty(radii.shape), radii.new_empty(radii.shape)


def _f_sph_one(edge_vectors, angular_momentum, real_output, epsilon):
    import torch

    width = 2 * int(angular_momentum) + 1
    dt = edge_vectors.dtype if real_output else (torch.complex64 if edge_vectors.dtype == torch.float32
                                                 else torch.complex128)
    values = edge_vectors.new_empty((edge_vectors.shape[0], width), dtype=dt)
    return values, values.new_empty((edge_vectors.shape[0], width, 3))


def _f_scheduled(radial_values, radial_derivatives, angular_values, angular_derivatives, radial_directions,
                 edge_types, channel_radial_indices, channel_angular_indices, channel_types, channel_scales):
    E, K = radial_values.shape[0], channel_scales.numel()
    return radial_values.new_empty((E, K)), radial_values.new_empty((E, K, 3))


def _f_sph(edge_vectors, maximum_angular_momentum, real_output, epsilon):
    import torch

    width = (int(maximum_angular_momentum) + 1) ** 2
    dt = edge_vectors.dtype if real_output else (torch.complex64 if edge_vectors.dtype == torch.float32
                                                 else torch.complex128)
    values = edge_vectors.new_empty((edge_vectors.shape[0], width), dtype=dt)
    return values, values.new_empty((edge_vectors.shape[0], width, 3))


def _f_density(edge_values, centers, atom_count):
    return edge_values.new_empty((int(atom_count), edge_values.shape[1]))


def _f_density_adjoint(atomic_adjoint, centers):
    return atomic_adjoint.new_empty((centers.shape[0], atomic_adjoint.shape[1]))


def _f_monomial(input, monomial_counts, output_offsets, *rest):
    return input.new_empty(tuple(input.shape[:-1]) + (output_offsets.shape[0] - 1,))


def _f_like_input(output_adjoint, input, *rest):
    return input.new_empty(input.shape)


def _f_sparse(input, term_offsets, term_components, term_exponents, output_offsets, *rest):
    return input.new_empty(tuple(input.shape[:-1]) + (output_offsets.shape[0] - 1,))


def _f_sparse_double_backward(input_adjoint_tangent, output_adjoint, input, *rest):
    return output_adjoint.new_empty(output_adjoint.shape), input.new_empty(input.shape)


def _f_fa(packed_slots, *rest):
    return packed_slots.new_empty((packed_slots.shape[0], int(rest[-1])))


def _f_fa_adjoint(output_adjoint, packed_slots, *rest):
    return packed_slots.new_empty(packed_slots.shape)


def _f_fa_linear(packed_slots, *rest):
    return packed_slots.new_empty((packed_slots.shape[0],))


def _f_fa_linear_adjoint(output_adjoint, packed_slots, *rest):
    weight = rest[-1]
    return packed_slots.new_empty(packed_slots.shape), weight.new_empty(weight.shape), weight.new_empty(())


FAKES = {
    "cheb_exp_cos_radial_table_with_derivative": _f_radial,
    "spherical_harmonics_table_with_derivative": _f_sph,
    "cheb_exp_cos_radial_with_derivative": _f_radial_one,
    "spherical_harmonics_with_derivative": _f_sph_one,
    "scheduled_radial_angular_channels_with_derivative": _f_scheduled,
    "density_accumulate": _f_density,
    "density_accumulate_adjoint": _f_density_adjoint,
    "symmetric_power_monomial": _f_monomial,
    "symmetric_power_monomial_adjoint": _f_like_input,
    "symmetric_power_shared_monomial": _f_monomial,
    "symmetric_power_shared_monomial_adjoint": _f_like_input,
    "symmetric_power_shared_sparse_monomial": _f_sparse,
    "symmetric_power_shared_sparse_monomial_adjoint": _f_like_input,
    "symmetric_power_shared_sparse_monomial_double_backward": _f_sparse_double_backward,
    "factorized_angular": _f_fa,
    "factorized_angular_adjoint": _f_fa_adjoint,
    "factorized_angular_heterogeneous": _f_fa,
    "factorized_angular_heterogeneous_adjoint": _f_fa_adjoint,
    "factorized_angular_segmented": _f_fa,
    "factorized_angular_segmented_adjoint": _f_fa_adjoint,
    "factorized_angular_linear": _f_fa_linear,
    "factorized_angular_linear_adjoint": _f_fa_linear_adjoint,
}


# ---- first-order autograd of the forward operators (backward = the adjoint operator) ------------------------

def _setup_saving_inputs(ctx, inputs, output):
    import torch

    ctx.save_for_backward(*(x for x in inputs if isinstance(x, torch.Tensor)))
    ctx.is_tensor = tuple(isinstance(x, torch.Tensor) for x in inputs)
    ctx.scalars = tuple(None if isinstance(x, torch.Tensor) else x for x in inputs)


def _inputs(ctx):
    tensors = iter(ctx.saved_tensors)
    return tuple(next(tensors) if t else s for t, s in zip(ctx.is_tensor, ctx.scalars))


def _bw_density(ctx, grad):
    edge_values, centers, _ = _inputs(ctx)
    return _ops().density_accumulate_adjoint(grad.contiguous(), centers), None, None


def _bw_density_adjoint(ctx, grad):
    atomic_adjoint, centers = _inputs(ctx)
    return _ops().density_accumulate(grad.contiguous(), centers, int(atomic_adjoint.shape[0])), None


def _bw_monomial(ctx, grad):
    x, counts, offsets, indices, values = _inputs(ctx)
    return (_ops().symmetric_power_monomial_adjoint(grad.contiguous(), x, counts, offsets, indices, values),
            None, None, None, None)


def _bw_shared(ctx, grad):
    x, counts, offsets, terms, outputs, values = _inputs(ctx)
    return (_ops().symmetric_power_shared_monomial_adjoint(grad.contiguous(), x, counts, offsets, terms, outputs,
                                                           values),) + (None,) * 5


def _bw_sparse(ctx, grad):
    x, *tables = _inputs(ctx)
    return (_ops().symmetric_power_shared_sparse_monomial_adjoint(grad.contiguous(), x, *tables),) + (None,) * 7


def _bw_sparse_adjoint(ctx, grad):
    """Backward of the adjoint operator: its double backward gives the
    cotangents of the output adjoint and of the input (execution_plan.py:5289-5340)."""
    g, x, *tables = _inputs(ctx)
    ot, it = _ops().symmetric_power_shared_sparse_monomial_double_backward(grad.contiguous(), g.contiguous(),
                                                                           x.contiguous(), *tables)
    return (ot, it) + (None,) * 7


def _bw_fa(ctx, grad):
    packed, *rest = _inputs(ctx)
    gx = _ops().factorized_angular_adjoint(grad.contiguous(), packed, *rest[:11], rest[11], rest[12])
    return (gx,) + (None,) * 14


def _bw_hetero(ctx, grad):
    packed, *rest = _inputs(ctx)
    gx = _ops().factorized_angular_heterogeneous_adjoint(grad.contiguous(), packed, *rest[:14], rest[14], rest[15])
    return (gx,) + (None,) * 17


def _bw_seg(ctx, grad):
    packed, *rest = _inputs(ctx)
    gx = _ops().factorized_angular_segmented_adjoint(grad.contiguous(), packed, *rest[:24], rest[24], rest[25])
    return (gx,) + (None,) * 27


def _bw_fa_linear(ctx, grad):
    packed, *rest = _inputs(ctx)
    weight, bias = rest[13], rest[14]
    gx, gw, gb = _ops().factorized_angular_linear_adjoint(grad.contiguous(), packed, *rest[:11], rest[11], rest[12],
                                                          weight)
    return (gx,) + (None,) * 13 + (gw, gb.reshape(bias.shape))


def _setup_scheduled(ctx, inputs, output):
    _setup_saving_inputs(ctx, inputs, output)
    ctx.mark_non_differentiable(output[1])


def _bw_scheduled(ctx, values_adjoint, derivatives_adjoint):
    """Gradients of the channel values in the radial table, the angular table
    and the channel scales (the derivative output is not differentiable), as
    the reference's formula (``execution_plan.py:3054-3151``) gives them."""
    import torch

    (radial_values, _, angular_values, _, _, edge_types, channel_radial_indices, channel_angular_indices,
     channel_types, channel_scales) = _inputs(ctx)
    if values_adjoint is None:
        return (None,) * 10
    active = ((channel_types < 0).unsqueeze(0)
              | (edge_types.unsqueeze(1) == channel_types.unsqueeze(0))).to(radial_values.dtype)
    weighted = values_adjoint * active
    radial = radial_values.index_select(1, channel_radial_indices)
    angular = angular_values.index_select(1, channel_angular_indices)
    g_radial = g_angular = g_scales = None
    if ctx.needs_input_grad[0]:
        g_radial = torch.zeros_like(radial_values).index_add_(1, channel_radial_indices,
                                                              weighted * angular * channel_scales)
    if ctx.needs_input_grad[2]:
        g_angular = torch.zeros_like(angular_values).index_add_(1, channel_angular_indices,
                                                                weighted * radial * channel_scales)
    if ctx.needs_input_grad[9]:
        g_scales = (weighted * radial * angular).sum(0)
    return g_radial, None, g_angular, None, None, None, None, None, None, g_scales


def _setup_basis(ctx, inputs, output):
    """Radial and harmonic operators: keep the inputs and the derivative output
    (which is not differentiable)."""
    import torch

    ctx.save_for_backward(*(x for x in inputs if isinstance(x, torch.Tensor)), output[1])
    ctx.scalars = tuple(x for x in inputs if not isinstance(x, torch.Tensor))
    ctx.mark_non_differentiable(output[1])


def _bw_radial(ctx, values_adjoint, derivatives_adjoint):
    """``d loss / d radii``: the saved ``d/dr`` output contracted with the
    incoming gradient, as the reference's first-order formula
    (``execution_plan.py:2534-2670``).  When the backward is itself
    differentiated (``create_graph``), autograd through the differentiable
    Torch expression of the basis (:mod:`ye3t_amd.runtime.basis_torch`)
    instead, as the reference does without its native double backward.
    Gradients in the cutoffs or lambdas are not provided."""
    import torch

    radii, cutoffs, lambdas, derivative = ctx.saved_tensors
    if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
        raise NotImplementedError("cheb_exp_cos_radial: gradients with respect to cutoffs or lambdas are not "
                                  "provided by the HIP backend")
    if values_adjoint is None or not ctx.needs_input_grad[0]:
        return None, None, None, None
    table = derivative.ndim == radii.ndim + 1
    if torch.is_grad_enabled():
        from ye3t_amd.runtime import basis_torch

        (index,) = ctx.scalars
        values = basis_torch.cheb_exp_cos_radial(radii, cutoffs, lambdas, int(index))
        if not table:
            values = values[..., int(index)]
        if not values.requires_grad:  # index 0: a constant
            return torch.zeros_like(radii), None, None, None
        (grad,) = torch.autograd.grad(values, radii, values_adjoint, create_graph=True)
        return grad, None, None, None
    grad = values_adjoint * derivative
    if table:  # the table: sum over the radial index
        grad = grad.sum(-1)
    return grad, None, None, None


def _bw_sph(ctx, values_adjoint, derivatives_adjoint):
    """``d loss / d edge_vectors``: ``sum_lm g[e, lm] dY[e, lm, :]`` from the
    saved Cartesian gradient output, with ``Re(conj(g) dY)`` for complex
    output (Torch's convention for a real input of a complex function), as the
    reference's first-order formulas (``execution_plan.py:2845-2935``).  When
    the backward is itself differentiated, autograd through the differentiable
    Torch expression of the harmonics (:mod:`ye3t_amd.runtime.basis_torch`)."""
    import torch

    edge_vectors, derivative = ctx.saved_tensors
    if values_adjoint is None or not ctx.needs_input_grad[0]:
        return None, None, None, None
    if torch.is_grad_enabled():
        from ye3t_amd import runtime
        from ye3t_amd.runtime import basis_torch

        l, real_output, epsilon = ctx.scalars
        l = int(l)
        values = basis_torch.real_harmonics(edge_vectors, l, float(epsilon))
        if not real_output:
            re, im, wr, wi = runtime._complex_tables(values, l)
            values = torch.complex(values[:, re] * wr, values[:, im] * wi)
        if derivative.shape[1] != values.shape[1]:  # one l: its columns of the table
            values = values[:, l * l:]
        if not values.requires_grad:  # l = 0: a constant
            return torch.zeros_like(edge_vectors), None, None, None
        (grad,) = torch.autograd.grad(values, edge_vectors, values_adjoint, create_graph=True)
        return grad, None, None, None
    if derivative.is_complex():
        grad = (values_adjoint.conj().unsqueeze(-1) * derivative).real.sum(1)
    else:
        grad = (values_adjoint.unsqueeze(-1) * derivative).sum(1)
    return grad.to(edge_vectors.dtype), None, None, None


SETUPS = {
    "scheduled_radial_angular_channels_with_derivative": _setup_scheduled,
    "cheb_exp_cos_radial_with_derivative": _setup_basis,
    "cheb_exp_cos_radial_table_with_derivative": _setup_basis,
    "spherical_harmonics_with_derivative": _setup_basis,
    "spherical_harmonics_table_with_derivative": _setup_basis,
}

BACKWARDS = {
    "cheb_exp_cos_radial_with_derivative": _bw_radial,
    "cheb_exp_cos_radial_table_with_derivative": _bw_radial,
    "spherical_harmonics_with_derivative": _bw_sph,
    "spherical_harmonics_table_with_derivative": _bw_sph,
    "scheduled_radial_angular_channels_with_derivative": _bw_scheduled,
    "density_accumulate": _bw_density,
    "density_accumulate_adjoint": _bw_density_adjoint,
    "symmetric_power_monomial": _bw_monomial,
    "symmetric_power_shared_monomial": _bw_shared,
    "symmetric_power_shared_sparse_monomial": _bw_sparse,
    "symmetric_power_shared_sparse_monomial_adjoint": _bw_sparse_adjoint,
    "factorized_angular": _bw_fa,
    "factorized_angular_heterogeneous": _bw_hetero,
    "factorized_angular_segmented": _bw_seg,
    "factorized_angular_linear": _bw_fa_linear,
}


def register():
    """Give the ``ye3t_runtime`` operators HIP kernels (idempotent).

    Returns the names whose schemas this call defined (empty where the
    reference's extension had defined them)."""
    import torch

    with _LOCK:
        if _STATE["registered"]:
            return _STATE["defined"]
        defined = []
        lib_def = torch.library.Library(NAMESPACE, "FRAGMENT")
        _STATE["libs"].append(lib_def)
        for name, schema in SCHEMAS.items():
            if not hasattr(_ops(), name):
                lib_def.define(name + schema)
                defined.append(name)
        lib_impl = torch.library.Library(NAMESPACE, "IMPL")
        _STATE["libs"].append(lib_impl)
        for name, kernel in KERNELS.items():
            lib_impl.impl(name, kernel, "CUDA")
        for name in defined:
            torch.library.register_fake(f"{NAMESPACE}::{name}", FAKES[name], lib=lib_def)
            if name in BACKWARDS:
                torch.library.register_autograd(f"{NAMESPACE}::{name}", BACKWARDS[name],
                                                setup_context=SETUPS.get(name, _setup_saving_inputs), lib=lib_def)
        _STATE["registered"] = True
        _STATE["defined"] = tuple(defined)
        return _STATE["defined"]
