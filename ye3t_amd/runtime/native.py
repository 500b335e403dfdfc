"""ctypes binding of the in-tree HIP library ``libye3t_hip.so`` (C ABI: ``include/ye3t_hip.h``).

Torch provides device memory and the current stream; every entry point takes
raw device pointers.  There is no CPU fallback here: if the library is missing
or a call fails, a ``RuntimeError`` carrying the library's message is raised.
"""

import ctypes
import os

import numpy as np

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "libye3t_hip.so")
ABI_VERSION = 61
_LIB = None

F32, F64 = 0, 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64


class DensityArgs(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("atom_count", _i64), ("edge_count", _i64),
                ("row_offsets", _vp), ("neighbors", _vp), ("edge_vectors", _vp), ("species", _vp),
                ("node_features", _vp), ("radial_mix", _vp), ("channel_count", _i64),
                ("max_radial_index", _i64), ("max_angular", _i64), ("cutoff", ctypes.c_double),
                ("lambda_", ctypes.c_double), ("epsilon", ctypes.c_double), ("out_dtype", ctypes.c_int),
                ("accumulate_dtype", ctypes.c_int)]


class ProductPlanDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("a_width", _i64), ("feature_count", _i64), ("chunk_count", _i64),
                ("workspace_slots", _i64), ("chunk_word_offsets", _vp), ("chunk_coeff_offsets", _vp),
                ("chunk_out_offsets", _vp), ("chunk_first_column", _vp), ("words", _vp), ("word_count", _i64),
                ("coeffs", _vp), ("coeff_count", _i64), ("out_slots", _vp), ("out_slot_count", _i64),
                ("out_dtype", ctypes.c_int), ("in_dtype", ctypes.c_int)]


class FactorizedAngularDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("node_count", _i64), ("node_offsets", _vp), ("node_dimensions", _vp),
                ("node_leaf_offsets", _vp), ("node_left", _vp), ("node_right", _vp),
                ("node_coefficient_offsets", _vp), ("coefficient_count", _i64), ("coefficient_rows", _vp),
                ("coefficient_columns", _vp), ("coefficient_values", _vp), ("root_count", _i64),
                ("root_nodes", _vp), ("projection_count", _i64), ("projection_values", _vp),
                ("source_dimension", _i64), ("input_dimension", _i64), ("workspace_dimension", _i64),
                ("output_dimension", _i64)]


SEGMENT_TABLE_NAMES = ("segment_source_offsets", "segment_input_offsets", "segment_input_dimensions",
                       "segment_workspace_offsets", "segment_workspace_dimensions", "segment_node_offsets",
                       "segment_root_offsets", "segment_projection_offsets", "segment_projection_dimensions",
                       "segment_output_offsets", "node_offsets", "node_dimensions", "node_leaf_offsets", "node_left",
                       "node_right", "node_coefficient_offsets", "coefficient_rows", "coefficient_columns",
                       "coefficient_values", "root_nodes", "root_projection_starts", "root_projection_dimensions",
                       "root_output_offsets", "projection_values")


class FactorizedAngularSegmentedDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("segment_count", _i64)] + \
        [(n, _vp) for n in SEGMENT_TABLE_NAMES[:10]] + \
        [("node_count", _i64)] + [(n, _vp) for n in SEGMENT_TABLE_NAMES[10:16]] + \
        [("coefficient_count", _i64), ("coefficient_rows", _vp), ("coefficient_columns", _vp),
         ("coefficient_values", _vp), ("root_count", _i64), ("root_nodes", _vp), ("root_projection_starts", _vp),
         ("root_projection_dimensions", _vp), ("root_output_offsets", _vp), ("projection_count", _i64),
         ("projection_values", _vp), ("packed_input_dimension", _i64), ("total_source_count", _i64),
         ("workspace_dimension", _i64), ("output_dimension", _i64)]


class CellGrid(ctypes.Structure):
    _fields_ = [("origin", ctypes.c_double * 3), ("cell_edge", ctypes.c_double), ("dims", _i64 * 3)]


class Caps(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_char * 64), ("device", ctypes.c_int), ("cu_count", ctypes.c_int),
                ("wavefront_size", ctypes.c_int), ("lds_bytes_per_block", ctypes.c_int),
                ("clock_khz", ctypes.c_int), ("hbm_bytes", _i64), ("hbm_peak_gbs", ctypes.c_double)]


def library_path():
    return LIB_PATH


def available():
    return os.path.exists(LIB_PATH)


def lib():
    """Load the HIP library; raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"ye3t_amd HIP library not built: {LIB_PATH} is missing (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    L.ye3t_hip_abi_version.restype = ctypes.c_int
    L.ye3t_hip_has_hip.restype = ctypes.c_int
    L.ye3t_hip_has_cpu.restype = ctypes.c_int
    L.ye3t_hip_last_error.restype = ctypes.c_char_p
    L.ye3t_hip_last_density_kernel.restype = ctypes.c_char_p
    L.ye3t_hip_device_caps.argtypes = [ctypes.c_int, ctypes.POINTER(Caps)]
    L.ye3t_hip_radial_table.argtypes = [ctypes.c_int, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp]
    L.ye3t_hip_real_sph_table.argtypes = [ctypes.c_int, _vp, _i64, _i64, ctypes.c_double, _vp, _vp, _vp]
    L.ye3t_hip_scheduled_radial_angular_channels.argtypes = [ctypes.c_int, _i64, _i64, _i64, _i64] + [_vp] * 13
    L.ye3t_hip_density_accumulate_csr.argtypes = [ctypes.c_int, _vp, _vp, _i64, _i64, _vp, _vp]
    L.ye3t_hip_density_accumulate_adjoint.argtypes = [ctypes.c_int, _vp, _vp, _i64, _i64, _i64, _vp, _vp]
    L.ye3t_hip_ace_density_forward.argtypes = [ctypes.POINTER(DensityArgs), _vp, _vp]
    L.ye3t_hip_ace_density_edge_gradient.argtypes = [ctypes.POINTER(DensityArgs), ctypes.c_int, _vp, _vp, _vp]
    L.ye3t_hip_symmetric_power_monomial.argtypes = [ctypes.c_int, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64,
                                                    _vp, _vp]
    L.ye3t_hip_symmetric_power_monomial_adjoint.argtypes = [ctypes.c_int, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64,
                                                            _i64, _vp, _vp]
    L.ye3t_hip_symmetric_power_shared_monomial.argtypes = [ctypes.c_int, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp,
                                                           _i64, _i64, _vp, _vp]
    L.ye3t_hip_symmetric_power_shared_monomial_adjoint.argtypes = [ctypes.c_int, _vp, _vp, _i64, _i64, _vp, _i64, _vp,
                                                                   _vp, _vp, _i64, _i64, _vp, _vp]
    L.ye3t_hip_symmetric_power_shared_sparse_monomial.argtypes = [ctypes.c_int, _vp, _i64, _i64, _vp, _vp, _vp, _i64,
                                                                  _i64, _vp, _vp, _vp, _i64, _i64, _vp, _vp]
    L.ye3t_hip_symmetric_power_shared_sparse_monomial_adjoint.argtypes = [ctypes.c_int, _vp, _vp, _i64, _i64, _vp,
                                                                          _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64,
                                                                          _i64, _vp, _vp]
    L.ye3t_hip_symmetric_power_shared_sparse_monomial_double_backward.argtypes = [
        ctypes.c_int, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp]
    L.ye3t_hip_code_object_kernel_info.argtypes = [ctypes.c_char_p, _i64, ctypes.c_char_p, ctypes.POINTER(_i64),
                                                   ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_int)]
    L.ye3t_hip_part_private_limit.restype = _i64
    L.ye3t_hip_evaluate_factorized_schedule.argtypes = [ctypes.c_int, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp,
                                                        _vp, _i64, _vp, _vp]
    L.ye3t_hip_product_plan_create.argtypes = [ctypes.POINTER(ProductPlanDesc), ctypes.POINTER(_vp)]
    L.ye3t_hip_product_plan_destroy.argtypes = [_vp]
    L.ye3t_hip_product_plan_destroy.restype = None
    L.ye3t_hip_product_forward.argtypes = [_vp, _vp, _i64, _vp, _vp]
    L.ye3t_hip_product_launch_info.argtypes = [_vp, _i64, ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                                               ctypes.POINTER(_i64)]
    L.ye3t_hip_rtc_fingerprint.argtypes = [ctypes.c_char_p, _i64]
    L.ye3t_hip_rtc_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_vp),
                                       ctypes.POINTER(_i64)]
    L.ye3t_hip_free.argtypes = [_vp]
    L.ye3t_hip_free.restype = None
    L.ye3t_hip_product_plan_attach_generated.argtypes = [_vp, _vp, _i64, ctypes.c_char_p, _i64, _i64, ctypes.c_int,
                                                         ctypes.c_int]
    L.ye3t_hip_product_plan_select.argtypes = [_vp, ctypes.c_int]
    L.ye3t_hip_product_plan_attach_generated_parts.argtypes = [_vp, _i64, ctypes.POINTER(_vp), ctypes.POINTER(_i64),
                                                               ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i64)]
    L.ye3t_hip_product_plan_attach_adjoint_parts.argtypes = [_vp, _i64, ctypes.POINTER(_vp), ctypes.POINTER(_i64),
                                                             ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i64),
                                                             _i64, _vp, _vp]
    L.ye3t_hip_product_adjoint_parts_workspace_bytes.argtypes = [_vp, _i64]
    L.ye3t_hip_product_adjoint_parts_workspace_bytes.restype = _i64
    L.ye3t_hip_product_adjoint_parts.argtypes = [_vp, _vp, _i64, ctypes.c_int, _vp, _i64, _vp, _i64, _vp, _vp]
    L.ye3t_hip_product_plan_attach_readout_parts.argtypes = [_vp, _i64, ctypes.POINTER(_vp), ctypes.POINTER(_i64),
                                                             ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i64)]
    L.ye3t_hip_product_linear_parts_workspace_bytes.argtypes = [_vp, _i64]
    L.ye3t_hip_product_linear_parts_workspace_bytes.restype = _i64
    L.ye3t_hip_product_linear_forward_parts.argtypes = [_vp, _vp, _i64, ctypes.c_int, _i64, _vp, ctypes.c_double,
                                                        _vp, _i64, _vp, _vp]
    L.ye3t_hip_product_plan_attach_readout.argtypes = [_vp, _vp, _i64, ctypes.c_char_p, ctypes.c_int]
    L.ye3t_hip_product_linear_forward.argtypes = [_vp, _vp, _i64, _vp, ctypes.c_double, _vp, _vp]
    L.ye3t_hip_rows_dot.argtypes = [ctypes.c_int, _vp, _i64, _i64, _vp, ctypes.c_double, _vp, _vp]
    L.ye3t_hip_product_plan_attach_adjoint.argtypes = [_vp, _vp, _i64, ctypes.c_char_p, ctypes.c_int]
    L.ye3t_hip_product_adjoint.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp]
    L.ye3t_hip_transpose.argtypes = [ctypes.c_int, _vp, _i64, _i64, _vp, _i64, _vp]
    L.ye3t_hip_product_forward_columns.argtypes = [_vp, _vp, _i64, _i64, _vp, _vp]
    L.ye3t_hip_product_plan_uses_stream.argtypes = [_vp]
    L.ye3t_hip_product_stream_encode.argtypes = [ctypes.POINTER(ProductPlanDesc), _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    L.ye3t_hip_product_adjoint_workspace_bytes.argtypes = [_vp, _i64]
    L.ye3t_hip_product_adjoint_workspace_bytes.restype = _i64
    L.ye3t_hip_product_adjoint_stream.argtypes = [_vp, _vp, _i64, ctypes.c_int, _vp, _i64, _vp, _i64, _vp, _vp]
    L.ye3t_hip_product_adjoint_stream_noalloc.argtypes = [_vp, _vp, _i64, ctypes.c_int, _vp, _i64, _vp, _vp]
    L.ye3t_hip_factorized_angular_plan_create.argtypes = [ctypes.POINTER(FactorizedAngularDesc), ctypes.POINTER(_vp)]
    L.ye3t_hip_factorized_angular_plan_destroy.argtypes = [_vp]
    L.ye3t_hip_factorized_angular_plan_destroy.restype = None
    L.ye3t_hip_factorized_angular_plan_info.argtypes = [_vp, _vp]
    L.ye3t_hip_factorized_angular_forward.argtypes = [_vp, _vp, _i64, _vp, _vp]
    L.ye3t_hip_factorized_angular_adjoint.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp]
    L.ye3t_hip_factorized_angular_linear_forward.argtypes = [_vp, _vp, _i64, _vp, _vp, _vp, _vp]
    L.ye3t_hip_factorized_angular_linear_adjoint.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp]
    L.ye3t_hip_factorized_angular_segmented_plan_create.argtypes = [ctypes.POINTER(FactorizedAngularSegmentedDesc),
                                                                    ctypes.POINTER(_vp)]
    L.ye3t_hip_factorized_angular_segmented_plan_destroy.argtypes = [_vp]
    L.ye3t_hip_factorized_angular_segmented_plan_destroy.restype = None
    L.ye3t_hip_factorized_angular_segmented_plan_info.argtypes = [_vp, _vp]
    L.ye3t_hip_factorized_angular_segmented_forward.argtypes = [_vp, _vp, _i64, _vp, _vp]
    L.ye3t_hip_factorized_angular_segmented_adjoint.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp]
    L.ye3t_hip_neighbor_workspace_bytes.argtypes = [_i64, ctypes.POINTER(CellGrid)]
    L.ye3t_hip_neighbor_workspace_bytes.restype = _i64
    L.ye3t_hip_neighbor_count.argtypes = [ctypes.c_int, _vp, _i64, ctypes.POINTER(CellGrid), ctypes.c_double, _vp,
                                          _i64, _vp, _vp]
    L.ye3t_hip_neighbor_fill.argtypes = [ctypes.c_int, _i64, ctypes.POINTER(CellGrid), ctypes.c_double, _vp, _i64,
                                         _vp, _i64, _vp, _vp, _vp, _vp]
    version = L.ye3t_hip_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"ye3t_hip ABI {version} does not match the bindings ({ABI_VERSION})")
    _LIB = L
    return L


EXPORTED_SYMBOLS = (
    "ye3t_hip_abi_version", "ye3t_hip_has_hip", "ye3t_hip_has_cpu", "ye3t_hip_last_error", "ye3t_hip_device_caps", "ye3t_hip_radial_table",
    "ye3t_hip_real_sph_table", "ye3t_hip_scheduled_radial_angular_channels", "ye3t_hip_density_accumulate_csr", "ye3t_hip_ace_density_forward",
    "ye3t_hip_symmetric_power_monomial", "ye3t_hip_evaluate_factorized_schedule",
    "ye3t_hip_product_plan_create", "ye3t_hip_product_plan_destroy", "ye3t_hip_product_forward",
    "ye3t_hip_product_launch_info", "ye3t_hip_rtc_compile", "ye3t_hip_rtc_fingerprint", "ye3t_hip_free",
    "ye3t_hip_product_plan_attach_generated", "ye3t_hip_product_plan_select", "ye3t_hip_last_density_kernel",
    "ye3t_hip_product_plan_attach_generated_parts",
    "ye3t_hip_product_plan_attach_adjoint_parts", "ye3t_hip_product_adjoint_parts_workspace_bytes",
    "ye3t_hip_product_adjoint_parts", "ye3t_hip_product_plan_attach_readout_parts",
    "ye3t_hip_product_linear_parts_workspace_bytes", "ye3t_hip_product_linear_forward_parts",
    "ye3t_hip_density_accumulate_adjoint", "ye3t_hip_product_plan_attach_readout", "ye3t_hip_product_linear_forward",
    "ye3t_hip_rows_dot", "ye3t_hip_product_plan_attach_adjoint", "ye3t_hip_product_adjoint",
    "ye3t_hip_neighbor_workspace_bytes", "ye3t_hip_neighbor_count", "ye3t_hip_neighbor_fill",
    "ye3t_hip_transpose", "ye3t_hip_product_forward_columns", "ye3t_hip_product_plan_uses_stream",
    "ye3t_hip_product_adjoint_workspace_bytes", "ye3t_hip_product_adjoint_stream", "ye3t_hip_product_stream_encode",
    "ye3t_hip_product_adjoint_stream_noalloc", "ye3t_hip_factorized_angular_plan_create",
    "ye3t_hip_factorized_angular_plan_destroy", "ye3t_hip_factorized_angular_plan_info",
    "ye3t_hip_factorized_angular_forward", "ye3t_hip_factorized_angular_adjoint",
    "ye3t_hip_factorized_angular_linear_forward", "ye3t_hip_factorized_angular_linear_adjoint",
    "ye3t_hip_symmetric_power_monomial_adjoint", "ye3t_hip_symmetric_power_shared_monomial",
    "ye3t_hip_symmetric_power_shared_monomial_adjoint", "ye3t_hip_factorized_angular_segmented_plan_create",
    "ye3t_hip_factorized_angular_segmented_plan_destroy", "ye3t_hip_factorized_angular_segmented_plan_info",
    "ye3t_hip_factorized_angular_segmented_forward", "ye3t_hip_factorized_angular_segmented_adjoint",
    "ye3t_hip_ace_density_edge_gradient", "ye3t_hip_symmetric_power_shared_sparse_monomial",
    "ye3t_hip_symmetric_power_shared_sparse_monomial_adjoint",
    "ye3t_hip_symmetric_power_shared_sparse_monomial_double_backward", "ye3t_hip_code_object_kernel_info",
    "ye3t_hip_part_private_limit",
)


def _check(rc, what):
    if rc != 0:
        msg = lib().ye3t_hip_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


C64, C128 = 2, 3


def _dtype_code(t):
    import torch

    if t.dtype == torch.float64:
        return F64
    if t.dtype == torch.float32:
        return F32
    raise TypeError(f"unsupported dtype {t.dtype}; expected float32 or float64")


def _any_dtype_code(dtype):
    """ABI code of a real or complex torch dtype."""
    import torch

    codes = {torch.float32: F32, torch.float64: F64, torch.complex64: C64, torch.complex128: C128}
    if dtype not in codes:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float64, complex64 or complex128")
    return codes[dtype]


def _stream():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(t, name):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def _opt(t, name):
    return None if t is None else _dev(t, name)


def has_hip():
    """The library's ``ye3t_hip_has_hip()``: a HIP device is visible."""
    return bool(lib().ye3t_hip_has_hip())


def device_caps(device=0):
    caps = Caps()
    _check(lib().ye3t_hip_device_caps(int(device), ctypes.byref(caps)), "ye3t_hip_device_caps")
    return {"arch": caps.arch.decode(), "device": caps.device, "cu_count": caps.cu_count,
            "wavefront_size": caps.wavefront_size, "lds_bytes_per_block": caps.lds_bytes_per_block,
            "clock_khz": caps.clock_khz, "hbm_bytes": int(caps.hbm_bytes), "hbm_peak_gbs": caps.hbm_peak_gbs}


def radial_table(radii, cutoffs, lambdas, n_max, with_derivative=True):
    import torch

    E = int(radii.shape[0])
    for t, n in ((radii, "radii"), (cutoffs, "cutoffs"), (lambdas, "lambdas")):
        if t.shape != (E,) or t.dtype != radii.dtype:
            raise ValueError(f"{n} must be a [{E}] tensor of dtype {radii.dtype}")
    values = torch.empty((E, n_max + 1), dtype=radii.dtype, device=radii.device)
    derivs = torch.empty_like(values) if with_derivative else None
    _check(lib().ye3t_hip_radial_table(_dtype_code(radii), _dev(radii, "radii"), _dev(cutoffs, "cutoffs"),
                                       _dev(lambdas, "lambdas"), E, int(n_max), _dev(values, "values"),
                                       _opt(derivs, "derivatives"), _stream()), "ye3t_hip_radial_table")
    return values, derivs


def scheduled_radial_angular_channels(radial_values, radial_derivatives, angular_values, angular_derivatives,
                                      radial_directions, edge_types, channel_radial_indices,
                                      channel_angular_indices, channel_types, channel_scales):
    """``ye3t_hip_scheduled_radial_angular_channels`` with the reference's
    argument checks and messages (``execution_plan_torch.cpp:1241-1305``);
    the index ranges are checked by one device reduction each.  Returns
    ``(edge_values [E, K], edge_derivatives [E, K, 3])``."""
    import torch

    data = (radial_values, radial_derivatives, angular_values, angular_derivatives, radial_directions,
            channel_scales)
    dtype = radial_values.dtype
    if dtype not in (torch.float32, torch.float64):
        raise ValueError("scheduled radial-angular channels require float32 or float64")
    if any(t.dtype != dtype for t in data):
        raise ValueError("scheduled radial-angular data tensors must share one dtype")
    idx = (edge_types, channel_radial_indices, channel_angular_indices, channel_types)
    if any(t.dtype != torch.int64 or t.ndim != 1 for t in idx):
        raise ValueError("edge_types and the channel schedule arrays must be int64 vectors")
    if radial_values.ndim != 2 or angular_values.ndim != 2 or channel_scales.ndim != 1:
        raise ValueError("radial_values and angular_values must be [edge_count, width], channel_scales a vector")
    E, NR = (int(v) for v in radial_values.shape)
    NA, K = int(angular_values.shape[1]), int(channel_scales.numel())
    if tuple(radial_derivatives.shape) != (E, NR):
        raise ValueError("radial derivatives must match radial values")
    if tuple(angular_derivatives.shape) != (E, NA, 3):
        raise ValueError("angular derivatives must have shape [edge_count, angular_width, 3]")
    if int(angular_values.shape[0]) != E:
        raise ValueError("radial and angular tables must share one edge axis")
    if tuple(radial_directions.shape) != (E, 3):
        raise ValueError("radial directions must have shape [edge_count, 3]")
    if int(edge_types.numel()) != E:
        raise ValueError("edge_types must have length edge_count")
    if not (channel_radial_indices.numel() == channel_angular_indices.numel() == channel_types.numel() == K):
        raise ValueError("channel schedule arrays must have length channel_count")
    if K > 0:
        if int(channel_radial_indices.min()) < 0 or int(channel_radial_indices.max()) >= NR:
            raise ValueError("channel radial indices must lie in the radial table")
        if int(channel_angular_indices.min()) < 0 or int(channel_angular_indices.max()) >= NA:
            raise ValueError("channel angular indices must lie in the angular table")
        if int(channel_types.min()) < -1:
            raise ValueError("channel types must be -1 or a nonnegative edge type")
    values = torch.empty((E, K), dtype=dtype, device=radial_values.device)
    derivs = torch.empty((E, K, 3), dtype=dtype, device=radial_values.device)
    inputs = [t.contiguous() for t in (radial_values, radial_derivatives, angular_values, angular_derivatives,
                                        radial_directions, edge_types, channel_radial_indices,
                                        channel_angular_indices, channel_types, channel_scales)]
    args = [_dev(t, n) for t, n in zip(inputs, (
        "radial_values", "radial_derivatives", "angular_values", "angular_derivatives", "radial_directions",
        "edge_types", "channel_radial_indices", "channel_angular_indices", "channel_types", "channel_scales"))]
    _check(lib().ye3t_hip_scheduled_radial_angular_channels(_dtype_code(radial_values), E, NR, NA, K, *args,
                                                            _dev(values, "edge_values"),
                                                            _dev(derivs, "edge_derivatives"), _stream()),
           "ye3t_hip_scheduled_radial_angular_channels")
    return values, derivs


def real_sph_table(vectors, l_max, epsilon=1e-12, with_gradient=True):
    import torch

    if vectors.ndim != 2 or vectors.shape[1] != 3:
        raise ValueError("edge_vectors must have shape [E, 3]")
    E = int(vectors.shape[0])
    width = (l_max + 1) ** 2
    values = torch.empty((E, width), dtype=vectors.dtype, device=vectors.device)
    grads = torch.empty((E, width, 3), dtype=vectors.dtype, device=vectors.device) if with_gradient else None
    _check(lib().ye3t_hip_real_sph_table(_dtype_code(vectors), _dev(vectors, "edge_vectors"), E, int(l_max),
                                         float(epsilon), _dev(values, "values"), _opt(grads, "gradients"),
                                         _stream()), "ye3t_hip_real_sph_table")
    return values, grads


def density_accumulate_csr(edge_values, row_offsets, atom_count):
    import torch

    if edge_values.ndim != 2:
        raise ValueError("edge_values must be [E, C]")
    if row_offsets.dtype != torch.int64 or row_offsets.shape != (atom_count + 1,):
        raise ValueError("row_offsets must be int64 [N+1]")
    C = int(edge_values.shape[1])
    out = torch.empty((atom_count, C), dtype=edge_values.dtype, device=edge_values.device)
    _check(lib().ye3t_hip_density_accumulate_csr(_dtype_code(edge_values), _dev(edge_values, "edge_values"),
                                                 _dev(row_offsets, "row_offsets"), int(atom_count), C,
                                                 _dev(out, "out"), _stream()), "ye3t_hip_density_accumulate_csr")
    return out


def density_accumulate_adjoint(atomic_adjoint, centers):
    """``edge_adjoint[e] = atomic_adjoint[centers[e]]``; centres must lie in ``[0, N)``."""
    import torch

    if atomic_adjoint.ndim != 2 or centers.ndim != 1 or centers.dtype != torch.int64:
        raise ValueError("atomic_adjoint must be [N, C] and centers int64 [E]")
    N, C = (int(x) for x in atomic_adjoint.shape)
    E = int(centers.shape[0])
    out = torch.empty((E, C), dtype=atomic_adjoint.dtype, device=atomic_adjoint.device)
    _check(lib().ye3t_hip_density_accumulate_adjoint(_dtype_code(atomic_adjoint), _dev(atomic_adjoint, "atomic_adjoint"),
                                                     _dev(centers, "centers"), E, C, N, _dev(out, "out"), _stream()),
           "ye3t_hip_density_accumulate_adjoint")
    return out


def ace_density_forward(edge_vectors, row_offsets, neighbors, *, atom_count, channel_count, n_max, l_max, cutoff,
                        lam, epsilon=1e-12, species=None, node_features=None, radial_mix=None, out=None,
                        out_dtype=None, accumulate_dtype=None, validate=True):
    """Fused stage 1; returns ``A[N, C, R, (l_max+1)^2]``.

    ``out_dtype`` (a torch dtype, default: that of the inputs) is the type of
    ``A``; float64 with float32 inputs gives an fp64 density of fp32 data.
    ``accumulate_dtype`` (default: ``out_dtype``) is the type of the
    accumulation: float64 with a float32 ``A`` accumulates in fp64 and rounds
    each density value once to fp32.  ``validate`` range-checks the CSR
    offsets, neighbour and species indices first (one device reduction and a
    scalar read-back each); a caller that has already validated these inputs
    may skip it.
    """
    import torch

    rows = 1 if radial_mix is not None else n_max + 1
    shape = (atom_count, channel_count, rows, (l_max + 1) ** 2)
    a_dtype = edge_vectors.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty(shape, dtype=a_dtype, device=edge_vectors.device)
    elif tuple(out.shape) != shape or out.dtype != a_dtype:
        raise ValueError(f"out must be {shape} of dtype {a_dtype}")
    if row_offsets.dtype != torch.int64 or row_offsets.shape != (atom_count + 1,):
        raise ValueError("row_offsets must be int64 [N+1]")
    if neighbors is not None and neighbors.dtype != torch.int64:
        raise ValueError("neighbors must be int64")
    if species is not None and species.dtype != torch.int32:
        raise ValueError("species must be int32")
    if edge_vectors.ndim != 2 or edge_vectors.shape[1] != 3:
        raise ValueError("edge_vectors must be [E, 3]")
    if validate:
        from ye3t_amd.runtime import validate_density_csr

        validate_density_csr(row_offsets, neighbors, atom_count, int(edge_vectors.shape[0]), species=species,
                             species_count=channel_count)
    if node_features is not None and tuple(node_features.shape) != (atom_count, channel_count):
        raise ValueError(f"node_features must be [{atom_count}, {channel_count}]")
    if radial_mix is not None and tuple(radial_mix.shape) != (channel_count, n_max + 1):
        raise ValueError(f"radial_mix must be [{channel_count}, {n_max + 1}]")
    for t, n in ((node_features, "node_features"), (radial_mix, "radial_mix")):
        if t is not None and t.dtype != edge_vectors.dtype:
            raise ValueError(f"{n} must have dtype {edge_vectors.dtype}")
    args = DensityArgs(
        dtype=_dtype_code(edge_vectors), atom_count=int(atom_count), edge_count=int(edge_vectors.shape[0]),
        row_offsets=_dev(row_offsets, "row_offsets"), neighbors=_opt(neighbors, "neighbors"),
        edge_vectors=_dev(edge_vectors, "edge_vectors"), species=_opt(species, "species"),
        node_features=_opt(node_features, "node_features"), radial_mix=_opt(radial_mix, "radial_mix"),
        channel_count=int(channel_count), max_radial_index=int(n_max), max_angular=int(l_max),
        cutoff=float(cutoff), lambda_=float(lam), epsilon=float(epsilon), out_dtype=_dtype_code(out),
        accumulate_dtype=-1 if accumulate_dtype is None else (F64 if accumulate_dtype == torch.float64 else F32))
    _check(lib().ye3t_hip_ace_density_forward(ctypes.byref(args), _dev(out, "A"), _stream()),
           "ye3t_hip_ace_density_forward")
    return out


def ace_density_edge_gradient(density_adjoint, edge_vectors, row_offsets, neighbors, *, atom_count, channel_count,
                              n_max, l_max, cutoff, lam, epsilon=1e-12, species=None, node_features=None,
                              radial_mix=None, validate=True):
    """Edge-vector gradient ``[E, 3]`` of ``<density_adjoint, A(edge_vectors)>``
    for the fused stage 1 with the same arguments as :func:`ace_density_forward`
    (``ye3t_hip_ace_density_edge_gradient``).  ``density_adjoint`` has A's
    shape; float64, or float32/float64 with float32 edge vectors.  The result
    has the edge vectors' dtype."""
    import torch

    rows = 1 if radial_mix is not None else n_max + 1
    shape = (atom_count, channel_count, rows, (l_max + 1) ** 2)
    if tuple(density_adjoint.shape) != shape:
        raise ValueError(f"density_adjoint must be {shape}")
    if density_adjoint.dtype not in (torch.float32, torch.float64) or \
            (density_adjoint.dtype == torch.float32 and edge_vectors.dtype == torch.float64):
        raise ValueError("density_adjoint must be float64, or float32 with float32 edge vectors")
    if row_offsets.dtype != torch.int64 or row_offsets.shape != (atom_count + 1,):
        raise ValueError("row_offsets must be int64 [N+1]")
    if edge_vectors.ndim != 2 or edge_vectors.shape[1] != 3:
        raise ValueError("edge_vectors must be [E, 3]")
    if neighbors is not None and neighbors.dtype != torch.int64:
        raise ValueError("neighbors must be int64")
    if species is not None and species.dtype != torch.int32:
        raise ValueError("species must be int32")
    if validate:
        from ye3t_amd.runtime import validate_density_csr

        validate_density_csr(row_offsets, neighbors, atom_count, int(edge_vectors.shape[0]), species=species,
                             species_count=channel_count)
    if node_features is not None and tuple(node_features.shape) != (atom_count, channel_count):
        raise ValueError(f"node_features must be [{atom_count}, {channel_count}]")
    if radial_mix is not None and tuple(radial_mix.shape) != (channel_count, n_max + 1):
        raise ValueError(f"radial_mix must be [{channel_count}, {n_max + 1}]")
    for t, n in ((node_features, "node_features"), (radial_mix, "radial_mix")):
        if t is not None and t.dtype != edge_vectors.dtype:
            raise ValueError(f"{n} must have dtype {edge_vectors.dtype}")
    g = density_adjoint.contiguous()
    vec = edge_vectors.contiguous()
    out = torch.empty((int(vec.shape[0]), 3), dtype=vec.dtype, device=vec.device)
    args = DensityArgs(
        dtype=_dtype_code(edge_vectors), atom_count=int(atom_count), edge_count=int(edge_vectors.shape[0]),
        row_offsets=_dev(row_offsets, "row_offsets"), neighbors=_opt(neighbors, "neighbors"),
        edge_vectors=_dev(vec, "edge_vectors"), species=_opt(species, "species"),
        node_features=_opt(node_features, "node_features"), radial_mix=_opt(radial_mix, "radial_mix"),
        channel_count=int(channel_count), max_radial_index=int(n_max), max_angular=int(l_max),
        cutoff=float(cutoff), lambda_=float(lam), epsilon=float(epsilon), out_dtype=-1, accumulate_dtype=-1)
    _check(lib().ye3t_hip_ace_density_edge_gradient(ctypes.byref(args), _dtype_code(g), _dev(g, "density_adjoint"),
                                                    _dev(out, "edge_gradient"), _stream()),
           "ye3t_hip_ace_density_edge_gradient")
    return out


def last_density_kernel():
    """Kernel launched by the last ``ace_density_forward`` call on this thread."""
    return lib().ye3t_hip_last_density_kernel().decode()


def _host_i64(a):
    return np.ascontiguousarray(np.asarray(a.detach().cpu() if hasattr(a, "detach") else a), dtype=np.int64)


def _host_real(a):
    return np.asarray(a.detach().cpu() if hasattr(a, "detach") else a)


def check_monomial_table(D, monomial_counts, output_offsets, output_indices, monomial_values):
    """Host checks of a grouped monomial table (the reference op's and core's
    contract, execution_plan.py:11894-11940, execution_plan_torch.cpp): returns
    the int64 host arrays."""
    counts = _host_i64(monomial_counts)
    offs = _host_i64(output_offsets).reshape(-1)
    idx = _host_i64(output_indices).reshape(-1)
    T = int(np.asarray(_host_real(monomial_values)).reshape(-1).shape[0])
    if counts.ndim != 2 or int(counts.shape[1]) != int(D):
        raise ValueError("monomial_counts must have shape [term, input_dimension]")
    if int(idx.size) != int(counts.shape[0]):
        raise ValueError("output_indices length must match the term count")
    if T != int(counts.shape[0]):
        raise ValueError("monomial_values length must match the term count")
    if offs.size < 1:
        raise ValueError("output_offsets must contain at least one entry")
    O = int(offs.size) - 1
    if offs[0] != 0 or offs[-1] != T or np.any(np.diff(offs) < 0):
        raise ValueError("output_offsets must be a nondecreasing CSR over the terms")
    if T and np.any(np.repeat(np.arange(O), np.diff(offs)) != idx):
        raise ValueError("output_indices must agree with output_offsets")
    if np.any(counts < 0):
        raise ValueError("monomial_counts must be nonnegative")
    return counts, offs, idx


def check_shared_table(D, monomial_counts, output_offsets, coefficient_terms, coefficient_outputs,
                       coefficient_values):
    """Host checks of a shared monomial table (execution_plan.py:12100-12160,
    execution_plan_torch.cpp:5820-5860); returns the int64 host arrays."""
    counts = _host_i64(monomial_counts)
    offs = _host_i64(output_offsets).reshape(-1)
    terms = _host_i64(coefficient_terms).reshape(-1)
    outs = _host_i64(coefficient_outputs).reshape(-1)
    C = int(np.asarray(_host_real(coefficient_values)).reshape(-1).shape[0])
    if counts.ndim != 2 or int(counts.shape[1]) != int(D):
        raise ValueError("monomial_counts must have shape [monomial, input_dimension]")
    if int(outs.size) != int(terms.size):
        raise ValueError("coefficient_outputs length must match coefficient_terms")
    if C != int(terms.size):
        raise ValueError("coefficient_values length must match coefficient_terms")
    if offs.size < 1:
        raise ValueError("output_offsets must contain at least one entry")
    O = int(offs.size) - 1
    if offs[0] != 0 or offs[-1] != C or np.any(np.diff(offs) < 0):
        raise ValueError("output_offsets must span the coefficient table")
    if C and (terms.min() < 0 or terms.max() >= counts.shape[0]):
        raise ValueError("coefficient_terms contains an invalid monomial")
    if C and np.any(np.repeat(np.arange(O), np.diff(offs)) != outs):
        raise ValueError("coefficient_outputs must agree with output_offsets")
    if np.any(counts < 0):
        raise ValueError("monomial_counts must be nonnegative")
    return counts, offs, terms, outs


def _dev_i64(a, device):
    import torch

    return torch.as_tensor(a, dtype=torch.int64, device=device).contiguous()


def symmetric_power_monomial(x, monomial_counts, output_offsets, monomial_values, output_indices=None):
    """Grouped monomial table on the device (``output_indices`` defaults to the
    offsets' own term-to-output map)."""
    import torch

    B, D = (int(s) for s in x.shape)
    if output_indices is None:
        offs = _host_i64(output_offsets).reshape(-1)
        output_indices = np.repeat(np.arange(offs.size - 1), np.diff(offs))
    counts, offs, idx = check_monomial_table(D, monomial_counts, output_offsets, output_indices, monomial_values)
    T, O = int(counts.shape[0]), int(offs.size - 1)
    out = torch.empty((B, O), dtype=x.dtype, device=x.device)
    dv = torch.as_tensor(_host_real(monomial_values), device=x.device).to(x.dtype).contiguous()
    dc, do, di = _dev_i64(counts, x.device), _dev_i64(offs, x.device), _dev_i64(idx, x.device)
    _check(lib().ye3t_hip_symmetric_power_monomial(_dtype_code(x), _dev(x, "input"), B, D, _dev(dc, "counts"),
                                                   _dev(do, "offsets"), _dev(di, "indices"), _dev(dv, "values"), T, O,
                                                   _dev(out, "out"), _stream()), "ye3t_hip_symmetric_power_monomial")
    return out


def symmetric_power_monomial_adjoint(output_adjoint, x, monomial_counts, output_indices, monomial_values,
                                     output_offsets):
    import torch

    B, D = (int(s) for s in x.shape)
    counts, offs, idx = check_monomial_table(D, monomial_counts, output_offsets, output_indices, monomial_values)
    T, O = int(counts.shape[0]), int(offs.size - 1)
    g = output_adjoint.to(x.dtype).contiguous()
    if tuple(g.shape) != (B, O):
        raise ValueError(f"output_adjoint must be [{B}, {O}]")
    out = torch.empty_like(x)
    dv = torch.as_tensor(_host_real(monomial_values), device=x.device).to(x.dtype).contiguous()
    dc, di = _dev_i64(counts, x.device), _dev_i64(idx, x.device)
    _check(lib().ye3t_hip_symmetric_power_monomial_adjoint(_dtype_code(x), _dev(g, "output_adjoint"),
                                                           _dev(x, "input"), B, D, _dev(dc, "counts"),
                                                           _dev(di, "indices"), _dev(dv, "values"), T, O,
                                                           _dev(out, "input_adjoint"), _stream()),
           "ye3t_hip_symmetric_power_monomial_adjoint")
    return out


def symmetric_power_shared_monomial(x, monomial_counts, output_offsets, coefficient_terms, coefficient_outputs,
                                    coefficient_values):
    import torch

    B, D = (int(s) for s in x.shape)
    counts, offs, terms, _ = check_shared_table(D, monomial_counts, output_offsets, coefficient_terms,
                                                coefficient_outputs, coefficient_values)
    M, C, O = int(counts.shape[0]), int(terms.size), int(offs.size - 1)
    out = torch.empty((B, O), dtype=x.dtype, device=x.device)
    dv = torch.as_tensor(_host_real(coefficient_values), device=x.device).to(x.dtype).contiguous()
    dc, do, dt = _dev_i64(counts, x.device), _dev_i64(offs, x.device), _dev_i64(terms, x.device)
    _check(lib().ye3t_hip_symmetric_power_shared_monomial(_dtype_code(x), _dev(x, "input"), B, D,
                                                          _dev(dc, "counts") if M else None, M, _dev(do, "offsets"),
                                                          _dev(dt, "terms") if C else None,
                                                          _dev(dv, "values") if C else None, C, O, _dev(out, "out"),
                                                          _stream()), "ye3t_hip_symmetric_power_shared_monomial")
    return out


def symmetric_power_shared_monomial_adjoint(output_adjoint, x, monomial_counts, output_offsets, coefficient_terms,
                                            coefficient_outputs, coefficient_values):
    import torch

    B, D = (int(s) for s in x.shape)
    counts, offs, terms, _ = check_shared_table(D, monomial_counts, output_offsets, coefficient_terms,
                                                coefficient_outputs, coefficient_values)
    M, C, O = int(counts.shape[0]), int(terms.size), int(offs.size - 1)
    g = output_adjoint.to(x.dtype).contiguous()
    if tuple(g.shape) != (B, O):
        raise ValueError(f"output_adjoint must be [{B}, {O}]")
    out = torch.empty_like(x)
    dv = torch.as_tensor(_host_real(coefficient_values), device=x.device).to(x.dtype).contiguous()
    dc, do, dt = _dev_i64(counts, x.device), _dev_i64(offs, x.device), _dev_i64(terms, x.device)
    _check(lib().ye3t_hip_symmetric_power_shared_monomial_adjoint(
        _dtype_code(x), _dev(g, "output_adjoint"), _dev(x, "input"), B, D, _dev(dc, "counts") if M else None, M,
        _dev(do, "offsets"), _dev(dt, "terms") if C else None, _dev(dv, "values") if C else None, C, O,
        _dev(out, "input_adjoint"), _stream()), "ye3t_hip_symmetric_power_shared_monomial_adjoint")
    return out


def check_sparse_table(D, term_offsets, term_components, term_exponents, output_offsets, coefficient_terms,
                       coefficient_outputs, coefficient_values):
    """Host checks of a sparse shared monomial table: the reference's host checks
    (execution_plan_cuda.cu:11012-11060) plus every index its kernels assert
    (:5723-5755, 5962-6030); returns the int64 host arrays."""
    toff = _host_i64(term_offsets).reshape(-1)
    comp = _host_i64(term_components).reshape(-1)
    ex = _host_i64(term_exponents).reshape(-1)
    offs = _host_i64(output_offsets).reshape(-1)
    terms = _host_i64(coefficient_terms).reshape(-1)
    outs = _host_i64(coefficient_outputs).reshape(-1)
    C = int(np.asarray(_host_real(coefficient_values)).reshape(-1).shape[0])
    if toff.size < 1:
        raise ValueError("term_offsets must contain at least one entry")
    if comp.size != ex.size:
        raise ValueError("sparse support component and exponent arrays must have equal length")
    if outs.size != terms.size or C != terms.size:
        raise ValueError("shared symmetric-power coefficient arrays must have equal length")
    if offs.size < 1:
        raise ValueError("output_offsets must contain at least one entry")
    M, S, O = int(toff.size) - 1, int(comp.size), int(offs.size) - 1
    if toff[0] != 0 or toff[-1] != S or np.any(np.diff(toff) < 0):
        raise ValueError("term_offsets must span the support arrays")
    if S and (comp.min() < 0 or comp.max() >= int(D)):
        raise ValueError("term_components contains an invalid input component")
    if S and ex.min() <= 0:
        raise ValueError("term_exponents must be positive")
    if offs[0] != 0 or offs[-1] != C or np.any(np.diff(offs) < 0):
        raise ValueError("output_offsets must span the coefficient table")
    if C and (terms.min() < 0 or terms.max() >= M):
        raise ValueError("coefficient_terms contains an invalid monomial")
    if C and np.any(np.repeat(np.arange(O), np.diff(offs)) != outs):
        raise ValueError("coefficient_outputs must agree with output_offsets")
    return toff, comp, ex, offs, terms


def _sparse_call(fn_name, x, tables, *tensors_before, outputs):
    toff, comp, ex, offs, terms, values = tables
    M, S, C, O = int(toff.size - 1), int(comp.size), int(terms.size), int(offs.size - 1)
    import torch

    dv = torch.as_tensor(_host_real(values), device=x.device).to(x.dtype).contiguous()
    dt, dc, de = _dev_i64(toff, x.device), _dev_i64(comp, x.device), _dev_i64(ex, x.device)
    do, dk = _dev_i64(offs, x.device), _dev_i64(terms, x.device)
    B, D = (int(s) for s in x.shape)
    args = [_any_dtype_code(x.dtype), *[_dev(t, "tensor") for t in tensors_before], _dev(x, "input"), B, D,
            _dev(dt, "term_offsets"), _dev(dc, "term_components") if S else None,
            _dev(de, "term_exponents") if S else None, M, S, _dev(do, "output_offsets"),
            _dev(dk, "coefficient_terms") if C else None, _dev(dv, "coefficient_values") if C else None, C, O,
            *[_dev(t, "output") if t.numel() else None for t in outputs], _stream()]
    _check(getattr(lib(), fn_name)(*args), fn_name)


class SparseMonomialTable:
    """A sparse shared monomial table validated once (``check_sparse_table``)
    and resident on one device in one dtype (real or complex), for callers
    that apply it many times (the hierarchical runtime's block powers)."""

    def __init__(self, D, term_offsets, term_components, term_exponents, output_offsets, coefficient_terms,
                 coefficient_outputs, coefficient_values, device, dtype):
        import torch

        toff, comp, ex, offs, terms = check_sparse_table(D, term_offsets, term_components, term_exponents,
                                                         output_offsets, coefficient_terms, coefficient_outputs,
                                                         coefficient_values)
        self.D = int(D)
        self.M, self.S, self.C, self.O = int(toff.size - 1), int(comp.size), int(terms.size), int(offs.size - 1)
        self.dtype = dtype
        self.code = _any_dtype_code(dtype)
        self.term_offsets = _dev_i64(toff, device)
        self.term_components = _dev_i64(comp, device)
        self.term_exponents = _dev_i64(ex, device)
        self.output_offsets = _dev_i64(offs, device)
        self.coefficient_terms = _dev_i64(terms, device)
        self.coefficient_values = torch.as_tensor(_host_real(coefficient_values)).to(device=device,
                                                                                     dtype=dtype).contiguous()

    def _args(self):
        return (_dev(self.term_offsets, "term_offsets"),
                _dev(self.term_components, "term_components") if self.S else None,
                _dev(self.term_exponents, "term_exponents") if self.S else None, self.M, self.S,
                _dev(self.output_offsets, "output_offsets"),
                _dev(self.coefficient_terms, "coefficient_terms") if self.C else None,
                _dev(self.coefficient_values, "coefficient_values") if self.C else None, self.C, self.O)

    def _rows(self, x):
        if x.dtype != self.dtype or x.ndim != 2 or int(x.shape[1]) != self.D:
            raise ValueError(f"input must be [batch, {self.D}] of {self.dtype}")
        return int(x.shape[0])

    def forward(self, x):
        import torch

        B = self._rows(x)
        out = torch.empty((B, self.O), dtype=self.dtype, device=x.device)
        if B * self.O:
            _check(lib().ye3t_hip_symmetric_power_shared_sparse_monomial(
                self.code, _dev(x, "input"), B, self.D, *self._args(), _dev(out, "output"), _stream()),
                "ye3t_hip_symmetric_power_shared_sparse_monomial")
        return out

    def adjoint(self, g, x):
        import torch

        B = self._rows(x)
        if g.dtype != self.dtype or tuple(g.shape) != (B, self.O):
            raise ValueError("output_adjoint must match the table's outputs and dtype")
        out = torch.empty_like(x)
        if B * self.D:
            _check(lib().ye3t_hip_symmetric_power_shared_sparse_monomial_adjoint(
                self.code, _dev(g, "output_adjoint") if self.O else None, _dev(x, "input"), B, self.D,
                *self._args(), _dev(out, "input_adjoint"), _stream()),
                "ye3t_hip_symmetric_power_shared_sparse_monomial_adjoint")
        return out

    def double_backward(self, v, g, x):
        import torch

        B = self._rows(x)
        if v.dtype != self.dtype or tuple(v.shape) != (B, self.D):
            raise ValueError("input_adjoint_tangent must match the input")
        if g.dtype != self.dtype or tuple(g.shape) != (B, self.O):
            raise ValueError("output_adjoint must match the table's outputs and dtype")
        out_t, in_t = torch.empty_like(g), torch.empty_like(x)
        if B:
            _check(lib().ye3t_hip_symmetric_power_shared_sparse_monomial_double_backward(
                self.code, _dev(v, "input_adjoint_tangent") if self.D else None,
                _dev(g, "output_adjoint") if self.O else None, _dev(x, "input"), B, self.D, *self._args(),
                _dev(out_t, "output_tangent") if self.O else None, _dev(in_t, "input_tangent") if self.D else None,
                _stream()), "ye3t_hip_symmetric_power_shared_sparse_monomial_double_backward")
        return out_t, in_t


def _sparse_tables(D, term_offsets, term_components, term_exponents, output_offsets, coefficient_terms,
                   coefficient_outputs, coefficient_values):
    toff, comp, ex, offs, terms = check_sparse_table(D, term_offsets, term_components, term_exponents,
                                                     output_offsets, coefficient_terms, coefficient_outputs,
                                                     coefficient_values)
    return toff, comp, ex, offs, terms, coefficient_values


def symmetric_power_shared_sparse_monomial(x, term_offsets, term_components, term_exponents, output_offsets,
                                           coefficient_terms, coefficient_outputs, coefficient_values):
    import torch

    B, D = (int(s) for s in x.shape)
    tables = _sparse_tables(D, term_offsets, term_components, term_exponents, output_offsets, coefficient_terms,
                            coefficient_outputs, coefficient_values)
    out = torch.empty((B, int(tables[3].size - 1)), dtype=x.dtype, device=x.device)
    _sparse_call("ye3t_hip_symmetric_power_shared_sparse_monomial", x, tables, outputs=(out,))
    return out


def symmetric_power_shared_sparse_monomial_adjoint(output_adjoint, x, term_offsets, term_components, term_exponents,
                                                   output_offsets, coefficient_terms, coefficient_outputs,
                                                   coefficient_values):
    import torch

    B, D = (int(s) for s in x.shape)
    tables = _sparse_tables(D, term_offsets, term_components, term_exponents, output_offsets, coefficient_terms,
                            coefficient_outputs, coefficient_values)
    g = output_adjoint.to(x.dtype).contiguous()
    if tuple(g.shape) != (B, int(tables[3].size - 1)):
        raise ValueError("output_adjoint dtype and batch must match input")
    out = torch.empty_like(x)
    _sparse_call("ye3t_hip_symmetric_power_shared_sparse_monomial_adjoint", x, tables, g, outputs=(out,))
    return out


def symmetric_power_shared_sparse_monomial_double_backward(input_adjoint_tangent, output_adjoint, x, term_offsets,
                                                           term_components, term_exponents, output_offsets,
                                                           coefficient_terms, coefficient_outputs,
                                                           coefficient_values):
    import torch

    B, D = (int(s) for s in x.shape)
    tables = _sparse_tables(D, term_offsets, term_components, term_exponents, output_offsets, coefficient_terms,
                            coefficient_outputs, coefficient_values)
    v = input_adjoint_tangent.to(x.dtype).contiguous()
    g = output_adjoint.to(x.dtype).contiguous()
    if tuple(v.shape) != (B, D):
        raise ValueError("input_adjoint_tangent shape must match input")
    if tuple(g.shape) != (B, int(tables[3].size - 1)):
        raise ValueError("output_adjoint batch dimension must match input")
    out_t, in_t = torch.empty_like(g), torch.empty_like(x)
    _sparse_call("ye3t_hip_symmetric_power_shared_sparse_monomial_double_backward", x, tables, v, g,
                 outputs=(out_t, in_t))
    return out_t, in_t


def evaluate_factorized_schedule(block_values, schedule):
    """Device evaluation of a :class:`FactorizedCoefficientSchedule` (validated on the host)."""
    import torch

    flat = schedule.flat_arrays()
    bv = block_values.contiguous()
    B, basis, blocks, mdim = (int(s) for s in bv.shape)
    K = schedule.component_count
    offs, labels, midx = flat["component_offsets"], flat["component_label_index"], flat["block_m_indices"]
    T = int(flat["coeffs"].shape[0])
    if offs.shape != (K + 1,) or offs[0] != 0 or offs[-1] != T or np.any(np.diff(offs) < 0):
        raise ValueError("component_offsets are inconsistent")
    if labels.size and (labels.min() < 0 or labels.max() >= basis):
        raise ValueError("component_label_index out of range")
    if midx.size and (midx.min() < 0 or midx.max() >= mdim):
        raise ValueError("block_m_indices out of range")
    if midx.shape != (T, blocks):
        raise ValueError("block_m_indices shape mismatch")
    dev = bv.device
    out = torch.empty((B, K), dtype=bv.dtype, device=dev)
    t_offs = torch.as_tensor(offs, device=dev)
    t_lab = torch.as_tensor(labels, device=dev)
    t_m = torch.as_tensor(midx, device=dev).contiguous()
    t_c = torch.as_tensor(flat["coeffs"], dtype=bv.dtype, device=dev)
    _check(lib().ye3t_hip_evaluate_factorized_schedule(
        _dtype_code(bv), _dev(bv, "block_values"), B, basis, blocks, mdim, _dev(t_offs, "offsets"),
        _dev(t_lab, "labels"), _dev(t_m, "m_indices") if T else None, _dev(t_c, "coeffs") if T else None, K,
        _dev(out, "out"), _stream()), "ye3t_hip_evaluate_factorized_schedule")
    return out


def _jit_cache_dir():
    """Code objects of generated kernels, keyed by ``rtc_cache_key``: ``YE3T_AMD_JIT_CACHE``,
    else ``jit_cache/`` beside this package (built ahead with
    ``python -m ye3t_amd.ace.prebuild`` it travels with the tree), else a
    temporary directory when the package directory is read-only."""
    import tempfile

    path = os.environ.get("YE3T_AMD_JIT_CACHE")
    if not path:
        path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "jit_cache")
        try:
            os.makedirs(path, exist_ok=True)
        except OSError:
            path = os.path.join(tempfile.gettempdir(), "ye3t_amd_jit")
    os.makedirs(path, exist_ok=True)
    return path


def rtc_fingerprint():
    """hipRTC version, options and ABI version of ``ye3t_hip_rtc_compile``
    (``ye3t_hip_rtc_fingerprint``): with the source and architecture, what
    decides a generated code object."""
    buf = ctypes.create_string_buffer(512)
    _check(lib().ye3t_hip_rtc_fingerprint(buf, len(buf)), "ye3t_hip_rtc_fingerprint")
    return buf.value.decode()


def rtc_cache_key(source, arch="gfx950"):
    """Name of a code object in the JIT cache: a hash of the architecture, the
    compiler fingerprint and the source, so a different hipRTC, option set or
    ABI never reads another's code object."""
    import hashlib

    return hashlib.sha256((arch + "\0" + rtc_fingerprint() + "\0" + source).encode()).hexdigest()[:24]


def rtc_compile(source, name="ye3t_generated.hip", arch="gfx950"):
    """Compile HIP source with hipRTC (cached on disk under ``rtc_cache_key``); returns the code object bytes."""
    key = rtc_cache_key(source, arch)
    path = os.path.join(_jit_cache_dir(), key + ".co")
    if os.path.exists(path):
        with open(path, "rb") as fh:
            return fh.read()
    code, size = _vp(), _i64()
    _check(lib().ye3t_hip_rtc_compile(source.encode(), name.encode(), arch.encode(), ctypes.byref(code),
                                      ctypes.byref(size)), "ye3t_hip_rtc_compile")
    try:
        blob = ctypes.string_at(code, size.value)
    finally:
        lib().ye3t_hip_free(code)
    tmp = path + f".{os.getpid()}.tmp"
    with open(tmp, "wb") as fh:
        fh.write(blob)
    os.replace(tmp, path)
    return blob


def code_object_kernel_info(code, kernel_name):
    """``{"private_segment_bytes", "group_segment_bytes", "uses_dynamic_stack"}``
    of a kernel in a gfx950 code object, read on the host from its kernel
    descriptor (``ye3t_hip_code_object_kernel_info``)."""
    priv, group, dyn = _i64(), _i64(), ctypes.c_int()
    _check(lib().ye3t_hip_code_object_kernel_info(bytes(code), len(code), kernel_name.encode(), ctypes.byref(priv),
                                                  ctypes.byref(group), ctypes.byref(dyn)),
           "ye3t_hip_code_object_kernel_info")
    return {"private_segment_bytes": priv.value, "group_segment_bytes": group.value,
            "uses_dynamic_stack": bool(dyn.value)}


def part_private_limit():
    """Bytes of scratch per lane above which the parts attach entry points refuse a kernel."""
    return int(lib().ye3t_hip_part_private_limit())


def _plan_desc(program, out_dtype, in_dtype=None):
    """``ye3t_product_plan_desc`` of a compiled program and the arrays it points into."""
    keep = {k: np.ascontiguousarray(v) for k, v in program.items() if isinstance(v, np.ndarray)}

    def ptr(name):
        return ctypes.c_void_p(keep[name].ctypes.data) if keep[name].size else None

    desc = ProductPlanDesc(
        dtype=F64 if program["dtype"] == "f64" else F32, a_width=program["a_width"],
        feature_count=program["feature_count"], chunk_count=program["chunk_count"],
        workspace_slots=program["workspace_slots"], chunk_word_offsets=ptr("chunk_word_offsets"),
        chunk_coeff_offsets=ptr("chunk_coeff_offsets"), chunk_out_offsets=ptr("chunk_out_offsets"),
        chunk_first_column=ptr("chunk_first_column"), words=ptr("words"), word_count=int(keep["words"].size),
        coeffs=ptr("coeffs"), coeff_count=int(keep["coeffs"].size), out_slots=ptr("out_slots"),
        out_slot_count=int(keep["out_slots"].size), out_dtype=F64 if out_dtype == "f64" else F32,
        in_dtype=-1 if in_dtype is None else (F64 if in_dtype == "f64" else F32))
    return desc, keep


def stream_encode(program):
    """The term stream the device interpreter would run for ``program`` (host
    only): dict of records ``[R, 4]`` uint32, flags ``[R]``, rec_off, loads
    ``[L, 2]``, load_off and layout; ``None`` when the plan gets no term stream."""
    L = lib()
    desc, keep = _plan_desc(program, program["dtype"])
    counts = np.zeros(3, dtype=np.int64)
    vp = ctypes.c_void_p
    _check(L.ye3t_hip_product_stream_encode(ctypes.byref(desc), vp(counts.ctypes.data), None, None, None, None,
                                            None, None), "ye3t_hip_product_stream_encode")
    nrec, nload, chunks = (int(x) for x in counts)
    if chunks == 0:
        return None
    recs = np.zeros((nrec, 4), dtype=np.uint32)
    flags = np.zeros(nrec, dtype=np.uint32)
    rec_off = np.zeros(chunks + 1, dtype=np.int64)
    loads = np.zeros((nload, 2), dtype=np.uint32)
    load_off = np.zeros(chunks + 1, dtype=np.int64)
    layout = np.zeros(8, dtype=np.int64)
    _check(L.ye3t_hip_product_stream_encode(ctypes.byref(desc), vp(counts.ctypes.data), vp(recs.ctypes.data),
                                            vp(flags.ctypes.data), vp(rec_off.ctypes.data), vp(loads.ctypes.data),
                                            vp(load_off.ctypes.data), vp(layout.ctypes.data)),
           "ye3t_hip_product_stream_encode")
    del keep
    names = ("ws_bytes", "rec_at", "flag_at", "load_at", "out_at", "one_off", "lds_bytes", "group")
    return {"records": recs, "flags": flags, "rec_off": rec_off, "loads": loads, "load_off": load_off,
            "layout": dict(zip(names, (int(x) for x in layout)))}


class ProductPlanHandle:
    """Device-resident compiled product program (owns a ``ye3t_hip_product_plan``).

    The arithmetic uses the program's dtype; ``out_dtype`` ("f32" or "f64",
    default: the same) is the type of the B-features and ``in_dtype`` (default:
    the program's dtype) that of the density rows.  An "f32" density with an
    "f64" program runs on attached generated kernels only.
    """

    def __init__(self, program, out_dtype=None, in_dtype=None):
        self.program = program
        self.dtype = program["dtype"]
        self.out_dtype = out_dtype or self.dtype
        self.in_dtype = in_dtype or self.dtype
        if self.out_dtype not in ("f32", "f64") or (self.dtype == "f32" and self.out_dtype == "f64"):
            raise ValueError(f"unsupported output dtype {self.out_dtype!r} for a {self.dtype} plan")
        if self.in_dtype not in ("f32", "f64") or (self.dtype == "f32" and self.in_dtype == "f64"):
            raise ValueError(f"unsupported density dtype {self.in_dtype!r} for a {self.dtype} plan")
        desc, self._keep = _plan_desc(program, self.out_dtype, self.in_dtype)
        handle = ctypes.c_void_p()
        _check(lib().ye3t_hip_product_plan_create(ctypes.byref(desc), ctypes.byref(handle)),
               "ye3t_hip_product_plan_create")
        self._handle = handle

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h is not None and h.value and _LIB is not None:
            _LIB.ye3t_hip_product_plan_destroy(h)
            self._handle = None

    @property
    def feature_count(self):
        return int(self.program["feature_count"])

    def attach_generated(self, source, meta):
        """Compile and attach a plan-specialised kernel (``ye3t_amd.ace.codegen``)."""
        if meta["feature_count"] != self.feature_count or meta["a_width"] != self.program["a_width"]:
            raise ValueError("generated kernel does not match this plan")
        if meta["dtype"] != self.dtype or meta.get("out_dtype", meta["dtype"]) != self.out_dtype or \
                meta.get("in_dtype", meta["dtype"]) != self.in_dtype:
            raise ValueError("generated kernel dtypes do not match this plan")
        blob = rtc_compile(source)
        self._code = ctypes.create_string_buffer(blob, len(blob))
        _check(lib().ye3t_hip_product_plan_attach_generated(self._handle, self._code, len(blob),
                                                            meta["kernel"].encode(), int(meta["chunks"]),
                                                            int(meta.get("rows", 64)),
                                                            1 if meta.get("persistent") else 0,
                                                            int(meta.get("threads", 64))),
               "ye3t_hip_product_plan_attach_generated")
        self.generated = meta

    def attach_generated_parts(self, parts, workers=None):
        """Compile (hipRTC, in parallel threads, cached on disk) and attach a
        plan-specialised kernel in parts (``ye3t_amd.ace.codegen.generate_parts``)."""
        from concurrent.futures import ThreadPoolExecutor

        first = 0
        for _source, meta in parts:
            if meta["feature_count"] != self.feature_count or meta["a_width"] != self.program["a_width"]:
                raise ValueError("generated part does not match this plan")
            if meta["dtype"] != self.dtype or meta.get("out_dtype", meta["dtype"]) != self.out_dtype or \
                    meta.get("in_dtype", meta["dtype"]) != self.in_dtype:
                raise ValueError("generated part dtypes do not match this plan")
            if meta["first_output"] != first:
                raise ValueError("generated parts must cover the outputs in order")
            first = meta["last_output"]
        if first != self.feature_count:
            raise ValueError("generated parts do not cover every output")
        workers = workers or min(16, os.cpu_count() or 1)
        with ThreadPoolExecutor(max(1, workers)) as pool:
            blobs = list(pool.map(lambda part: rtc_compile(part[0]), parts))
        n = len(parts)
        self._part_code = [ctypes.create_string_buffer(b, len(b)) for b in blobs]
        codes = (_vp * n)(*[ctypes.cast(c, _vp) for c in self._part_code])
        sizes = (_i64 * n)(*[len(b) for b in blobs])
        names = (ctypes.c_char_p * n)(*[m["kernel"].encode() for _, m in parts])
        chunks = (_i64 * n)(*[int(m["chunks"]) for _, m in parts])
        _check(lib().ye3t_hip_product_plan_attach_generated_parts(self._handle, n, codes, sizes, names, chunks),
               "ye3t_hip_product_plan_attach_generated_parts")
        self.generated_parts = [m for _, m in parts]

    def attach_adjoint_parts(self, parts, reduction, workers=None):
        """Compile and attach the reverse mode in parts
        (``ye3t_amd.ace.codegen.generate_adjoint_parts``)."""
        from concurrent.futures import ThreadPoolExecutor

        for _source, meta in parts:
            if meta["feature_count"] != self.feature_count or meta["a_width"] != self.program["a_width"]:
                raise ValueError("adjoint part does not match this plan")
            if meta["dtype"] != self.dtype or meta["grad_dtype"] != self.out_dtype or meta["in_dtype"] != self.in_dtype:
                raise ValueError("adjoint part dtypes do not match this plan")
        workers = workers or min(16, os.cpu_count() or 1)
        with ThreadPoolExecutor(max(1, workers)) as pool:
            blobs = list(pool.map(lambda part: rtc_compile(part[0]), parts))
        n = len(parts)
        self._adjoint_part_code = [ctypes.create_string_buffer(b, len(b)) for b in blobs]
        codes = (_vp * n)(*[ctypes.cast(c, _vp) for c in self._adjoint_part_code])
        sizes = (_i64 * n)(*[len(b) for b in blobs])
        names = (ctypes.c_char_p * n)(*[m["kernel"].encode() for _, m in parts])
        chunks = (_i64 * n)(*[int(m["chunks"]) for _, m in parts])
        col_off = np.ascontiguousarray(reduction["col_off"], dtype=np.int64)
        rows = np.ascontiguousarray(reduction["rows"], dtype=np.int64)
        _check(lib().ye3t_hip_product_plan_attach_adjoint_parts(
            self._handle, n, codes, sizes, names, chunks, int(reduction["partial_rows"]),
            col_off.ctypes.data, rows.ctypes.data if rows.size else None),
            "ye3t_hip_product_plan_attach_adjoint_parts")
        self.adjoint_part_meta = [m for _, m in parts]

    def attach_readout_parts(self, parts, workers=None):
        """Compile and attach the fused linear readout in parts
        (``ye3t_amd.ace.codegen.generate_readout_parts``)."""
        from concurrent.futures import ThreadPoolExecutor

        for _source, meta in parts:
            if meta["feature_count"] != self.feature_count or meta["a_width"] != self.program["a_width"]:
                raise ValueError("readout part does not match this plan")
            if meta["dtype"] != self.dtype or meta["in_dtype"] != self.in_dtype:
                raise ValueError("readout part dtypes do not match this plan")
        workers = workers or min(16, os.cpu_count() or 1)
        with ThreadPoolExecutor(max(1, workers)) as pool:
            blobs = list(pool.map(lambda part: rtc_compile(part[0]), parts))
        n = len(parts)
        self._readout_part_code = [ctypes.create_string_buffer(b, len(b)) for b in blobs]
        codes = (_vp * n)(*[ctypes.cast(c, _vp) for c in self._readout_part_code])
        sizes = (_i64 * n)(*[len(b) for b in blobs])
        names = (ctypes.c_char_p * n)(*[m["kernel"].encode() for _, m in parts])
        chunks = (_i64 * n)(*[int(m["chunks"]) for _, m in parts])
        _check(lib().ye3t_hip_product_plan_attach_readout_parts(self._handle, n, codes, sizes, names, chunks),
               "ye3t_hip_product_plan_attach_readout_parts")
        self.readout_part_meta = [m for _, m in parts]

    def linear_parts(self, A, weight, bias, samples=None, columns=False, out=None):
        """``out[s] = bias + sum_k B[s, k] weight[k]`` on the attached readout
        parts (B never stored): ``A`` row-major or, with ``columns``, a
        column-major view ``[a_width, >= samples]``; ``weight`` in the plan's
        dtype; ``out`` in its out_dtype."""
        import torch

        want = torch.float64 if self.in_dtype == "f64" else torch.float32
        w_t = torch.float64 if self.dtype == "f64" else torch.float32
        o_t = torch.float64 if self.out_dtype == "f64" else torch.float32
        W = int(self.program["a_width"])
        if A.dtype != want or A.ndim != 2:
            raise ValueError(f"A must be a 2-d {want} tensor")
        if columns:
            if int(A.shape[0]) != W or (A.stride(1) != 1 and int(A.shape[1]) > 1) or int(A.shape[1]) < int(samples):
                raise ValueError(f"A must be a column-major [{W}, >= samples] view")
            S, lda = int(samples), int(A.stride(0))
        else:
            if int(A.shape[1]) != W or not A.is_contiguous():
                raise ValueError(f"A must be contiguous [samples, {W}]")
            S, lda = int(A.shape[0]), W
        if weight.dtype != w_t or tuple(weight.shape) != (self.feature_count,) or not weight.is_contiguous():
            raise ValueError(f"weight must be a contiguous {w_t} vector of {self.feature_count}")
        if out is None:
            out = torch.empty((S,), dtype=o_t, device=A.device)
        elif tuple(out.shape) != (S,) or out.dtype != o_t or not out.is_contiguous():
            raise ValueError("out has the wrong shape or dtype")
        L = lib()
        nbytes = int(L.ye3t_hip_product_linear_parts_workspace_bytes(self._handle, S))
        if nbytes < 0:
            _check(-1, "ye3t_hip_product_linear_parts_workspace_bytes")
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=A.device)
        if not A.is_cuda:
            raise ValueError("A must be a GPU tensor")
        _check(L.ye3t_hip_product_linear_forward_parts(self._handle, ctypes.c_void_p(A.data_ptr()), lda,
                                                       1 if columns else 0, S, _dev(weight, "weight"), float(bias),
                                                       _dev(ws, "workspace"), nbytes, _dev(out, "out"), _stream()),
               "ye3t_hip_product_linear_forward_parts")
        return out

    def adjoint_parts(self, A, gB, samples=None, columns=False, out=None):
        """``gA[s] = J(A[s])^T gB[s]`` on the attached adjoint parts: ``A``
        row-major ``[samples, a_width]`` or, with ``columns``, column-major
        ``[a_width, ld]``; returns row-major ``gA`` in the density's type."""
        import torch

        want = torch.float64 if self.in_dtype == "f64" else torch.float32
        g_t = torch.float64 if self.out_dtype == "f64" else torch.float32
        W = int(self.program["a_width"])
        if A.dtype != want:
            raise ValueError(f"A must be {want} for this plan")
        if columns:
            # a column-major view [a_width, >= samples] with unit sample stride (a slice of the
            # copy ``transpose`` writes serves a block of samples)
            if A.ndim != 2 or int(A.shape[0]) != W or (A.stride(1) != 1 and int(A.shape[1]) > 1):
                raise ValueError(f"A must be a column-major [{W}, ld] view")
            S, lda = int(samples), int(A.stride(0))
            if int(A.shape[1]) < S:
                raise ValueError("A has fewer columns than samples")
        else:
            if A.ndim != 2 or int(A.shape[1]) != W or not A.is_contiguous():
                raise ValueError(f"A must be contiguous [samples, {W}]")
            S, lda = int(A.shape[0]), W
        if gB.dtype != g_t or tuple(gB.shape) != (S, self.feature_count) or not gB.is_contiguous():
            raise ValueError(f"gB must be contiguous {g_t} [{S}, {self.feature_count}]")
        if out is None:
            out = torch.empty((S, W), dtype=want, device=A.device)
        elif tuple(out.shape) != (S, W) or out.dtype != want or not out.is_contiguous():
            raise ValueError("out has the wrong shape or dtype")
        L = lib()
        nbytes = int(L.ye3t_hip_product_adjoint_parts_workspace_bytes(self._handle, S))
        if nbytes < 0:
            _check(-1, "ye3t_hip_product_adjoint_parts_workspace_bytes")
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=A.device)
        if not A.is_cuda:
            raise ValueError("A must be a GPU tensor")
        a_ptr = ctypes.c_void_p(A.data_ptr())  # strides checked above (a column view may start past 0)
        _check(L.ye3t_hip_product_adjoint_parts(self._handle, a_ptr, lda, 1 if columns else 0,
                                                _dev(gB, "gB"), S, _dev(ws, "workspace"), nbytes, _dev(out, "gA"),
                                                _stream()), "ye3t_hip_product_adjoint_parts")
        return out

    def select(self, use_interpreter):
        _check(lib().ye3t_hip_product_plan_select(self._handle, 1 if use_interpreter else 0),
               "ye3t_hip_product_plan_select")

    def launch_info(self, samples):
        g, b, l = _i64(), _i64(), _i64()
        _check(lib().ye3t_hip_product_launch_info(self._handle, int(samples), ctypes.byref(g), ctypes.byref(b),
                                                  ctypes.byref(l)), "ye3t_hip_product_launch_info")
        return {"grid": g.value, "block": b.value, "lds_bytes": l.value}

    def forward(self, A, out=None):
        import torch

        if A.ndim != 2 or int(A.shape[1]) != int(self.program["a_width"]):
            raise ValueError(f"A must be [samples, {self.program['a_width']}]")
        want = torch.float64 if self.in_dtype == "f64" else torch.float32
        if A.dtype != want:
            raise ValueError(f"A must be {want} for this plan")
        out_t = torch.float64 if self.out_dtype == "f64" else torch.float32
        S = int(A.shape[0])
        if out is None:
            out = torch.empty((S, self.feature_count), dtype=out_t, device=A.device)
        elif tuple(out.shape) != (S, self.feature_count) or out.dtype != out_t:
            raise ValueError("out has the wrong shape or dtype")
        _check(lib().ye3t_hip_product_forward(self._handle, _dev(A, "A"), S, _dev(out, "B"), _stream()),
               "ye3t_hip_product_forward")
        return out

    @property
    def uses_stream(self):
        """True when the plan's interpreter is the term stream (see ``forward_columns``)."""
        return bool(lib().ye3t_hip_product_plan_uses_stream(self._handle))

    def forward_columns(self, At, samples, out=None):
        """The product on a column-major density ``At [a_width, ld]`` (``ld`` a
        multiple of 64 covering ``samples``), as :func:`transpose` writes it."""
        import torch

        if At.ndim != 2 or int(At.shape[0]) != int(self.program["a_width"]):
            raise ValueError(f"At must be [{self.program['a_width']}, ld]")
        want = torch.float64 if self.in_dtype == "f64" else torch.float32
        if At.dtype != want:
            raise ValueError(f"At must be {want} for this plan")
        S, ld = int(samples), int(At.shape[1])
        out_t = torch.float64 if self.out_dtype == "f64" else torch.float32
        if out is None:
            out = torch.empty((S, self.feature_count), dtype=out_t, device=At.device)
        elif tuple(out.shape) != (S, self.feature_count) or out.dtype != out_t:
            raise ValueError("out has the wrong shape or dtype")
        _check(lib().ye3t_hip_product_forward_columns(self._handle, _dev(At, "At"), ld, S, _dev(out, "B"),
                                                      _stream()), "ye3t_hip_product_forward_columns")
        return out

    def adjoint_stream(self, A, gB, samples=None, columns=False, out=None):
        """``gA[s] = J(A[s])^T gB[s]`` by the term-stream interpreter's reverse mode:
        ``A`` row-major ``[samples, a_width]`` or, with ``columns``, column-major
        ``[a_width, ld]``; returns row-major ``gA`` in the plan's dtype."""
        import torch

        want = torch.float64 if self.dtype == "f64" else torch.float32
        g_t = torch.float64 if self.out_dtype == "f64" else torch.float32
        W = int(self.program["a_width"])
        if A.dtype != want:
            raise ValueError(f"A must be {want} for this plan")
        if columns:
            if A.ndim != 2 or int(A.shape[0]) != W:
                raise ValueError(f"A must be [{W}, ld]")
            S, lda = int(samples), int(A.shape[1])
        else:
            if A.ndim != 2 or int(A.shape[1]) != W:
                raise ValueError(f"A must be [samples, {W}]")
            S, lda = int(A.shape[0]), W
        if gB.dtype != g_t or tuple(gB.shape) != (S, self.feature_count):
            raise ValueError(f"gB must be {g_t} [{S}, {self.feature_count}]")
        if out is None:
            out = torch.empty((S, W), dtype=want, device=A.device)
        elif tuple(out.shape) != (S, W) or out.dtype != want:
            raise ValueError("out has the wrong shape or dtype")
        L = lib()
        nbytes = int(L.ye3t_hip_product_adjoint_workspace_bytes(self._handle, S))
        if nbytes < 0:
            _check(-1, "ye3t_hip_product_adjoint_workspace_bytes")
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=A.device)
        _check(L.ye3t_hip_product_adjoint_stream(self._handle, _dev(A, "A"), lda, 1 if columns else 0,
                                                 _dev(gB, "gB"), S, _dev(ws, "workspace"), nbytes, _dev(out, "gA"),
                                                 _stream()), "ye3t_hip_product_adjoint_stream")
        return out

    def adjoint_stream_noalloc(self, A, gB, out, samples=None, columns=False):
        """:meth:`adjoint_stream` through the library's allocation-free entry
        point (partial gradients in its static device scratch; ``out`` must be
        given).  Calls on one device are serialised by the library (an eager
        call on another stream waits for the previous call's kernels); a call
        captured into a graph records its kernels only, so a replay must not
        overlap other users of the scratch on that device."""
        import torch

        want = torch.float64 if self.dtype == "f64" else torch.float32
        g_t = torch.float64 if self.out_dtype == "f64" else torch.float32
        W = int(self.program["a_width"])
        if A.dtype != want:
            raise ValueError(f"A must be {want} for this plan")
        if columns:
            if A.ndim != 2 or int(A.shape[0]) != W:
                raise ValueError(f"A must be [{W}, ld]")
            S, lda = int(samples), int(A.shape[1])
        else:
            if A.ndim != 2 or int(A.shape[1]) != W:
                raise ValueError(f"A must be [samples, {W}]")
            S, lda = int(A.shape[0]), W
        if gB.dtype != g_t or tuple(gB.shape) != (S, self.feature_count):
            raise ValueError(f"gB must be {g_t} [{S}, {self.feature_count}]")
        if tuple(out.shape) != (S, W) or out.dtype != want:
            raise ValueError("out has the wrong shape or dtype")
        _check(lib().ye3t_hip_product_adjoint_stream_noalloc(self._handle, _dev(A, "A"), lda, 1 if columns else 0,
                                                             _dev(gB, "gB"), S, _dev(out, "gA"), _stream()),
               "ye3t_hip_product_adjoint_stream_noalloc")
        return out

    def attach_readout(self, source, meta):
        """Compile and attach a fused linear readout kernel (``codegen.generate_readout``)."""
        if meta["feature_count"] != self.feature_count or meta["a_width"] != self.program["a_width"]:
            raise ValueError("readout kernel does not match this plan")
        if meta["dtype"] != self.dtype or meta.get("out_dtype", meta["dtype"]) != self.out_dtype or \
                meta.get("in_dtype", meta["dtype"]) != self.in_dtype:
            raise ValueError("readout kernel dtypes do not match this plan")
        blob = rtc_compile(source)
        self._readout_code = ctypes.create_string_buffer(blob, len(blob))
        _check(lib().ye3t_hip_product_plan_attach_readout(self._handle, self._readout_code, len(blob),
                                                          meta["kernel"].encode(), int(meta["threads"])),
               "ye3t_hip_product_plan_attach_readout")
        self.readout = meta

    def attach_adjoint(self, source, meta):
        """Compile and attach a plan-specialised adjoint kernel (``codegen.generate_adjoint``)."""
        if meta["feature_count"] != self.feature_count or meta["a_width"] != self.program["a_width"]:
            raise ValueError("adjoint kernel does not match this plan")
        if meta["dtype"] != self.dtype or meta.get("grad_dtype", meta["dtype"]) != self.out_dtype or \
                meta.get("in_dtype", meta["dtype"]) != self.in_dtype:
            raise ValueError("adjoint kernel dtypes do not match this plan")
        blob = rtc_compile(source)
        self._adjoint_code = ctypes.create_string_buffer(blob, len(blob))
        _check(lib().ye3t_hip_product_plan_attach_adjoint(self._handle, self._adjoint_code, len(blob),
                                                          meta["kernel"].encode(), int(meta["threads"])),
               "ye3t_hip_product_plan_attach_adjoint")
        self.adjoint_kernel = meta

    def adjoint(self, A, gB, out=None):
        """``gA[s] = J(A[s])^T gB[s]`` with the attached adjoint kernel (forward values recomputed)."""
        import torch

        W = int(self.program["a_width"])
        a_t = torch.float64 if self.in_dtype == "f64" else torch.float32
        g_t = torch.float64 if self.out_dtype == "f64" else torch.float32
        if A.ndim != 2 or int(A.shape[1]) != W or A.dtype != a_t:
            raise ValueError(f"A must be [samples, {W}] of {a_t}")
        S = int(A.shape[0])
        if tuple(gB.shape) != (S, self.feature_count) or gB.dtype != g_t:
            raise ValueError(f"gB must be [{S}, {self.feature_count}] of {g_t}")
        if out is None:
            out = torch.empty((S, W), dtype=a_t, device=A.device)
        elif tuple(out.shape) != (S, W) or out.dtype != a_t:
            raise ValueError("out has the wrong shape or dtype")
        _check(lib().ye3t_hip_product_adjoint(self._handle, _dev(A, "A"), _dev(gB.contiguous(), "gB"), S,
                                              _dev(out, "gA"), _stream()), "ye3t_hip_product_adjoint")
        return out

    def linear(self, A, weight, bias, out=None):
        """``out[s] = bias + sum_k B[s, k] weight[k]`` with the attached fused kernel (B never stored)."""
        import torch

        if A.ndim != 2 or int(A.shape[1]) != int(self.program["a_width"]):
            raise ValueError(f"A must be [samples, {self.program['a_width']}]")
        want = torch.float64 if self.dtype == "f64" else torch.float32
        a_t = torch.float64 if self.in_dtype == "f64" else torch.float32
        if A.dtype != a_t or weight.dtype != want or tuple(weight.shape) != (self.feature_count,):
            raise ValueError(f"A must be {a_t} and weight [{self.feature_count}] {want} for this plan")
        out_t = torch.float64 if self.out_dtype == "f64" else torch.float32
        S = int(A.shape[0])
        if out is None:
            out = torch.empty((S,), dtype=out_t, device=A.device)
        elif tuple(out.shape) != (S,) or out.dtype != out_t:
            raise ValueError("out has the wrong shape or dtype")
        _check(lib().ye3t_hip_product_linear_forward(self._handle, _dev(A, "A"), S, _dev(weight, "weight"),
                                                     float(bias), _dev(out, "out"), _stream()),
               "ye3t_hip_product_linear_forward")
        return out


def rows_dot(B, weight, bias, out=None):
    """``out[s] = bias + sum_k B[s, k] weight[k]`` over a materialised B (fp64 sums, fixed order)."""
    import torch

    if B.ndim != 2 or weight.ndim != 1 or int(weight.shape[0]) != int(B.shape[1]) or weight.dtype != B.dtype:
        raise ValueError("B must be [S, F] and weight [F] of the same dtype")
    S, F = (int(x) for x in B.shape)
    if out is None:
        out = torch.empty((S,), dtype=B.dtype, device=B.device)
    elif tuple(out.shape) != (S,) or out.dtype != B.dtype:
        raise ValueError("out has the wrong shape or dtype")
    _check(lib().ye3t_hip_rows_dot(_dtype_code(B), _dev(B, "B"), S, F, _dev(weight, "weight"), float(bias),
                                   _dev(out, "out"), _stream()), "ye3t_hip_rows_dot")
    return out


MAX_GRID_DIM = 1 << 24


def cell_grid(lower, upper, cutoff, atom_count):
    """Cell grid covering the box ``[lower, upper]`` with cells a little wider
    than ``cutoff`` (the builder requires ``cell_edge >= cutoff (1 + 1e-9)``),
    widened further so that there are at most ``max(4 N, 64)`` cells."""
    import math

    cutoff = float(cutoff)
    if not (cutoff > 0.0 and math.isfinite(cutoff)):
        raise ValueError("cutoff must be positive and finite")
    lower = [float(x) for x in lower]
    upper = [float(x) for x in upper]
    if not all(math.isfinite(x) for x in lower + upper):
        raise ValueError("positions must be finite")
    span = [max(hi - lo, 0.0) for lo, hi in zip(lower, upper)]
    edge = cutoff * (1.0 + 1e-6)
    limit = max(4 * int(atom_count), 64)
    while True:
        dims = [min(MAX_GRID_DIM, int(s / edge) + 1) for s in span]
        if dims[0] * dims[1] * dims[2] <= limit:
            break
        edge *= max(1.05, (dims[0] * dims[1] * dims[2] / limit) ** (1.0 / 3.0))
    grid = CellGrid()
    for a in range(3):
        grid.origin[a] = lower[a]
        grid.dims[a] = dims[a]
    grid.cell_edge = edge
    return grid


def neighbor_list(positions, cutoff, grid=None):
    """Neighbour CSR of ``positions [N, 3]`` (open boundaries): row i holds the
    j != i with ``|r_j - r_i| < cutoff`` in ascending j.  Two passes with one
    host synchronisation between them (the edge count sizes the outputs)."""
    import torch

    if positions.ndim != 2 or positions.shape[1] != 3:
        raise ValueError("positions must be [N, 3]")
    N = int(positions.shape[0])
    dev = positions.device
    if grid is None:
        if N:
            lo, hi = torch.aminmax(positions, dim=0)
            lo, hi = lo.double().cpu().tolist(), hi.double().cpu().tolist()
        else:
            lo = hi = [0.0, 0.0, 0.0]
        grid = cell_grid(lo, hi, cutoff, N)
    L = lib()
    ws_bytes = int(L.ye3t_hip_neighbor_workspace_bytes(N, ctypes.byref(grid)))
    if ws_bytes < 0:
        _check(-1, "ye3t_hip_neighbor_workspace_bytes")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    offsets = torch.empty(N + 1, dtype=torch.int64, device=dev)
    code = _dtype_code(positions)
    pos = _dev(positions, "positions")
    _check(L.ye3t_hip_neighbor_count(code, pos, N, ctypes.byref(grid), float(cutoff), _dev(ws, "workspace"),
                                     ws_bytes, _dev(offsets, "row_offsets"), _stream()), "ye3t_hip_neighbor_count")
    E = int(offsets[N])
    centers = torch.empty(E, dtype=torch.int64, device=dev)
    nbrs = torch.empty(E, dtype=torch.int64, device=dev)
    vecs = torch.empty((E, 3), dtype=positions.dtype, device=dev)
    if E:
        _check(L.ye3t_hip_neighbor_fill(code, N, ctypes.byref(grid), float(cutoff), _dev(ws, "workspace"),
                                        ws_bytes, _dev(offsets, "row_offsets"), E, _dev(centers, "centers"),
                                        _dev(nbrs, "neighbors"), _dev(vecs, "edge_vectors"), _stream()),
               "ye3t_hip_neighbor_fill")
    return {"schema": "ye3t_amd_neighbor_csr_v1", "target_offsets": offsets, "edge_targets": centers,
            "edge_sources": nbrs, "edge_vectors": vecs, "node_count": N, "cutoff": float(cutoff)}


def transpose(A, out=None, ld=None):
    """Column-major copy ``At [cols, ld]`` of ``A [rows, cols]`` (``ld`` defaults to
    ``rows`` rounded up to 64; the rows past ``rows`` are zero)."""
    import torch

    if A.ndim != 2:
        raise ValueError("A must be 2-D")
    rows, cols = (int(x) for x in A.shape)
    ld = int(ld) if ld is not None else (rows + 63) // 64 * 64
    if out is None:
        out = torch.empty((cols, ld), dtype=A.dtype, device=A.device)
    elif tuple(out.shape) != (cols, ld) or out.dtype != A.dtype:
        raise ValueError("out has the wrong shape or dtype")
    _check(lib().ye3t_hip_transpose(_dtype_code(A), _dev(A, "A"), rows, cols, _dev(out, "At"), ld, _stream()),
           "ye3t_hip_transpose")
    return out


FA_TABLE_NAMES = ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
                  "node_coefficient_offsets", "coefficient_rows", "coefficient_columns", "coefficient_values",
                  "root_nodes", "projection_values")


class FactorizedAngularPlanHandle:
    """A validated, device-resident factorized-angular DAG
    (``ye3t_hip_factorized_angular_plan``): the reference op's tables
    (``execution_plan_torch.cpp:7586-7594``) in ``dtype`` (a torch real or
    complex dtype)."""

    def __init__(self, tables, source_dimension, input_dimension, workspace_dimension, output_dimension, dtype):
        import torch

        self.dtype = dtype
        np_t = {torch.float32: np.float32, torch.float64: np.float64, torch.complex64: np.complex64,
                torch.complex128: np.complex128}[dtype]
        keep = {}
        for name in FA_TABLE_NAMES[:8] + ("root_nodes",):
            v = tables[name]
            v = v.detach().cpu().numpy() if hasattr(v, "detach") else np.asarray(v)
            keep[name] = np.ascontiguousarray(v.reshape(-1), dtype=np.int64)
        for name in ("coefficient_values", "projection_values"):
            v = tables[name]
            v = v.detach().cpu().numpy() if hasattr(v, "detach") else np.asarray(v)
            keep[name] = np.ascontiguousarray(v.reshape(-1).astype(np_t))
        self._keep = keep

        def ptr(name):
            a = keep[name]
            return ctypes.c_void_p(a.ctypes.data) if a.size else None

        desc = FactorizedAngularDesc(
            dtype=_any_dtype_code(dtype), node_count=int(keep["node_offsets"].size),
            node_offsets=ptr("node_offsets"), node_dimensions=ptr("node_dimensions"),
            node_leaf_offsets=ptr("node_leaf_offsets"), node_left=ptr("node_left"), node_right=ptr("node_right"),
            node_coefficient_offsets=ptr("node_coefficient_offsets"),
            coefficient_count=int(keep["coefficient_rows"].size), coefficient_rows=ptr("coefficient_rows"),
            coefficient_columns=ptr("coefficient_columns"), coefficient_values=ptr("coefficient_values"),
            root_count=int(keep["root_nodes"].size), root_nodes=ptr("root_nodes"),
            projection_count=int(keep["projection_values"].size), projection_values=ptr("projection_values"),
            source_dimension=int(source_dimension), input_dimension=int(input_dimension),
            workspace_dimension=int(workspace_dimension), output_dimension=int(output_dimension))
        if int(keep["coefficient_values"].size) != desc.coefficient_count or \
                int(keep["coefficient_columns"].size) != desc.coefficient_count:
            raise RuntimeError("factorized coefficient arrays must have equal length")
        n = desc.node_count
        for name in ("node_dimensions", "node_leaf_offsets", "node_left", "node_right"):
            if int(keep[name].size) != n:
                raise RuntimeError("factorized node arrays must have equal length")
        if int(keep["node_coefficient_offsets"].size) != n + 1:
            raise RuntimeError("node_coefficient_offsets must have node_count + 1 entries")
        handle = ctypes.c_void_p()
        _check(lib().ye3t_hip_factorized_angular_plan_create(ctypes.byref(desc), ctypes.byref(handle)),
               "ye3t_hip_factorized_angular_plan_create")
        self._handle = handle
        self.source_dimension = int(source_dimension)
        self.input_dimension = int(input_dimension)
        self.workspace_dimension = int(workspace_dimension)
        self.output_dimension = int(output_dimension)

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h is not None and h.value and _LIB is not None:
            _LIB.ye3t_hip_factorized_angular_plan_destroy(h)
            self._handle = None

    def _packed(self, packed):
        if not packed.is_cuda or packed.dtype != self.dtype or packed.ndim != 2 or \
                int(packed.shape[1]) != self.source_dimension * self.input_dimension:
            raise ValueError(f"packed_slots must be a {self.dtype} GPU tensor "
                             f"[batch, {self.source_dimension * self.input_dimension}]")
        return packed.contiguous()

    def forward(self, packed):
        import torch

        packed = self._packed(packed)
        B = int(packed.shape[0])
        out = torch.empty((B, self.output_dimension), dtype=self.dtype, device=packed.device)
        _check(lib().ye3t_hip_factorized_angular_forward(self._handle, _dev(packed, "packed_slots"), B,
                                                         _dev(out, "output"), _stream()),
               "ye3t_hip_factorized_angular_forward")
        return out

    def adjoint(self, output_adjoint, packed):
        import torch

        packed = self._packed(packed)
        B = int(packed.shape[0])
        g = output_adjoint.to(self.dtype).contiguous()
        if tuple(g.shape) != (B, self.output_dimension):
            raise ValueError(f"output_adjoint must be [{B}, {self.output_dimension}]")
        out = torch.empty_like(packed)
        _check(lib().ye3t_hip_factorized_angular_adjoint(self._handle, _dev(g, "output_adjoint"),
                                                         _dev(packed, "packed_slots"), B, _dev(out, "adjoint"),
                                                         _stream()), "ye3t_hip_factorized_angular_adjoint")
        return out

    def _bias(self, bias):
        if self.dtype.is_complex:
            b = complex(bias)
            dt = np.complex64 if self.dtype == __import__("torch").complex64 else np.complex128
        else:
            b = float(bias)
            dt = np.float32 if self.dtype == __import__("torch").float32 else np.float64
        return np.array([b], dtype=dt)

    def linear(self, packed, weight, bias):
        import torch

        packed = self._packed(packed)
        B = int(packed.shape[0])
        w = weight.to(device=packed.device, dtype=self.dtype).contiguous()
        if tuple(w.shape) != (self.output_dimension,):
            raise ValueError("weight must be a vector matching factorized output dimension")
        b = self._bias(bias)
        out = torch.empty((B,), dtype=self.dtype, device=packed.device)
        _check(lib().ye3t_hip_factorized_angular_linear_forward(self._handle, _dev(packed, "packed_slots"), B,
                                                                _dev(w, "weight"), ctypes.c_void_p(b.ctypes.data),
                                                                _dev(out, "output"), _stream()),
               "ye3t_hip_factorized_angular_linear_forward")
        return out

    def linear_adjoint(self, output_adjoint, packed, weight):
        import torch

        packed = self._packed(packed)
        B = int(packed.shape[0])
        g = output_adjoint.to(self.dtype).contiguous()
        w = weight.to(device=packed.device, dtype=self.dtype).contiguous()
        if tuple(g.shape) != (B,) or tuple(w.shape) != (self.output_dimension,):
            raise ValueError("output_adjoint must be [batch] and weight [output_dimension]")
        feats = torch.empty((B, self.output_dimension), dtype=self.dtype, device=packed.device)
        gx = torch.empty_like(packed)
        gw = torch.empty_like(w)
        gb = torch.empty((), dtype=self.dtype, device=packed.device)
        _check(lib().ye3t_hip_factorized_angular_linear_adjoint(
            self._handle, _dev(g, "output_adjoint"), _dev(packed, "packed_slots"), B, _dev(w, "weight"),
            _dev(feats, "features"), _dev(gx, "packed_adjoint"), _dev(gw, "weight_adjoint"),
            ctypes.c_void_p(gb.data_ptr()), _stream()), "ye3t_hip_factorized_angular_linear_adjoint")
        return gx, gw, gb


class FactorizedAngularSegmentedPlanHandle:
    """A validated, device-resident segmented factorized-angular plan
    (``ye3t_hip_factorized_angular_segmented_plan``): the reference op's
    segment, node, coefficient, root and projection tables
    (``execution_plan_torch.cpp:7666-7679``) in ``dtype``."""

    def __init__(self, tables, packed_input_dimension, total_source_count, workspace_dimension, output_dimension,
                 dtype):
        import torch

        self.dtype = dtype
        np_t = {torch.float32: np.float32, torch.float64: np.float64, torch.complex64: np.complex64,
                torch.complex128: np.complex128}[dtype]
        keep = {}
        for name in SEGMENT_TABLE_NAMES:
            v = tables[name]
            v = v.detach().cpu().numpy() if hasattr(v, "detach") else np.asarray(v)
            if name in ("coefficient_values", "projection_values"):
                if np.iscomplexobj(v) and not np.iscomplexobj(np.empty(0, np_t)):
                    v = v.real
                keep[name] = np.ascontiguousarray(v.reshape(-1).astype(np_t))
            else:
                keep[name] = np.ascontiguousarray(v.reshape(-1), dtype=np.int64)
        self._keep = keep
        K = int(keep["segment_input_offsets"].size)
        counts = {"segment_source_offsets": K + 1, "segment_node_offsets": K + 1, "segment_root_offsets": K + 1,
                  "segment_output_offsets": K + 1}
        for name in SEGMENT_TABLE_NAMES[:10]:
            if int(keep[name].size) != counts.get(name, K):
                raise RuntimeError("segmented boundary offsets must contain segment_count + 1 entries"
                                   if name in counts else "segmented per-plan metadata must match segment count")
        n = int(keep["node_offsets"].size)
        for name in ("node_dimensions", "node_leaf_offsets", "node_left", "node_right"):
            if int(keep[name].size) != n:
                raise RuntimeError("segmented node metadata has inconsistent lengths")
        if int(keep["node_coefficient_offsets"].size) != n + 1:
            raise RuntimeError("segmented node metadata has inconsistent lengths")
        e = int(keep["coefficient_rows"].size)
        if int(keep["coefficient_columns"].size) != e or int(keep["coefficient_values"].size) != e:
            raise RuntimeError("segmented coefficient arrays must have equal length")
        r = int(keep["root_nodes"].size)
        for name in ("root_projection_starts", "root_projection_dimensions", "root_output_offsets"):
            if int(keep[name].size) != r:
                raise RuntimeError("segmented root metadata has inconsistent lengths")

        def ptr(name):
            a = keep[name]
            return ctypes.c_void_p(a.ctypes.data) if a.size else None

        desc = FactorizedAngularSegmentedDesc(
            dtype=_any_dtype_code(dtype), segment_count=K, node_count=n, coefficient_count=e, root_count=r,
            projection_count=int(keep["projection_values"].size), packed_input_dimension=int(packed_input_dimension),
            total_source_count=int(total_source_count), workspace_dimension=int(workspace_dimension),
            output_dimension=int(output_dimension), **{name: ptr(name) for name in SEGMENT_TABLE_NAMES})
        handle = ctypes.c_void_p()
        _check(lib().ye3t_hip_factorized_angular_segmented_plan_create(ctypes.byref(desc), ctypes.byref(handle)),
               "ye3t_hip_factorized_angular_segmented_plan_create")
        self._handle = handle
        self.packed_input_dimension = int(packed_input_dimension)
        self.output_dimension = int(output_dimension)

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h is not None and h.value and _LIB is not None:
            _LIB.ye3t_hip_factorized_angular_segmented_plan_destroy(h)
            self._handle = None

    def _packed(self, packed):
        if not packed.is_cuda or packed.dtype != self.dtype or packed.ndim != 2 or \
                int(packed.shape[1]) != self.packed_input_dimension:
            raise ValueError(f"packed_slots must be a {self.dtype} GPU tensor [batch, {self.packed_input_dimension}]")
        return packed.contiguous()

    def forward(self, packed):
        import torch

        packed = self._packed(packed)
        B = int(packed.shape[0])
        out = torch.empty((B, self.output_dimension), dtype=self.dtype, device=packed.device)
        _check(lib().ye3t_hip_factorized_angular_segmented_forward(self._handle, _dev(packed, "packed_slots"), B,
                                                                   _dev(out, "output"), _stream()),
               "ye3t_hip_factorized_angular_segmented_forward")
        return out

    def adjoint(self, output_adjoint, packed):
        import torch

        packed = self._packed(packed)
        B = int(packed.shape[0])
        g = output_adjoint.to(self.dtype).contiguous()
        if tuple(g.shape) != (B, self.output_dimension):
            raise ValueError(f"output_adjoint must be [{B}, {self.output_dimension}]")
        out = torch.empty_like(packed)
        _check(lib().ye3t_hip_factorized_angular_segmented_adjoint(self._handle, _dev(g, "output_adjoint"),
                                                                   _dev(packed, "packed_slots"), B,
                                                                   _dev(out, "adjoint"), _stream()),
               "ye3t_hip_factorized_angular_segmented_adjoint")
        return out
