"""Host-side behaviour of the ``ye3t.runtime`` mirror (no GPU work).

* the capability report keeps the reference's keys and reports operations
  under the reference's names (``execution_plan.py:6118-6850``);
* index inputs of the fused density are range-checked before any launch;
* ``backend="reference"`` is a known value that this device branch refuses
  explicitly.
"""

import pytest
import torch

from ye3t_amd import runtime
from ye3t_amd.runtime import native

# every key of the reference report, in its order (execution_plan.py:6316-6849)
REFERENCE_KEYS = (
    "schema", "torch_independent_core_source", "cmake_core_target", "prebuilt_extension", "cpu", "cuda",
    "cuda_operations", "cuda_density_auto_min_work_items", "cuda_edge_outer_auto_min_work_items",
    "cpu_edge_outer_auto_min_work_items", "cpu_carrier_gated_scatter_auto_min_work_items",
    "cuda_carrier_gated_scatter_auto_min_work_items", "real_control_carrier_gates", "residual_carrier_gated_scatter",
    "segmented_carrier_gated_scatter", "segmented_factorized_angular", "source_arena_gather",
    "source_arena_channel_transform", "carrier_channel_transform", "carrier_role_channel_map_adjoint",
    "cuda_segmented_carrier_scatter_min_node_feature_work", "real_control_carrier_channel_update",
    "scheduled_softmax_gaussian_role_density", "symmetric_power_monomial_double_backward",
    "symmetric_power_shared_monomial_double_backward", "symmetric_power_shared_monomial_factored_double_backward",
    "symmetric_power_shared_double_backward_default_algorithm", "symmetric_power_shared_sparse_monomial",
    "cpu_carrier_channel_update_auto_max_work_items", "cuda_carrier_channel_update_auto_max_work_items",
    "cuda_carrier_channel_update_auto_min_work_items", "symmetric_power_cpu_auto_max_batch",
    "symmetric_power_cpu_auto_min_power", "symmetric_power_shared_cpu_min_reuse",
    "symmetric_power_shared_cpu_min_batch", "symmetric_power_shared_cuda_min_reuse",
    "symmetric_power_shared_cuda_grad_min_batch", "symmetric_power_shared_cuda_forward_min_batch",
    "triton_available", "triton_cuda_available", "triton_real_convention_id", "triton_operations",
    "core_abi_version", "factorized_workspace_metadata", "heterogeneous_factorized_roots",
    "cached_heterogeneous_factorized_reverse", "dtypes", "analysis_orientation", "operations",
    "compact_exterior_power_max_native_order",
)

# operation names of the reference report's ``operations`` tuple for the ops
# this backend implements (execution_plan.py:6662-6850)
REFERENCE_NAMES = {"cheb_exp_cos_radial_table_with_derivative", "real_spherical_harmonics_table_with_derivative",
                   "density_accumulate", "density_accumulate_adjoint", "symmetric_power_monomial"}


def test_capability_report_keys_and_names():
    report = runtime.native_execution_plan_capabilities()
    assert len(REFERENCE_KEYS) == len(set(REFERENCE_KEYS)) == 50
    assert [k for k in report if k in REFERENCE_KEYS] == list(REFERENCE_KEYS)
    assert report["schema"] == "ye3t_execution_plan_v1"
    # the reference's own assertions on its report (tests/test_execution_plan_native.py:569-585)
    assert report["symmetric_power_cpu_auto_max_batch"] == 32
    assert report["symmetric_power_cpu_auto_min_power"] == 6
    assert report["symmetric_power_shared_cpu_min_reuse"] == 3.0
    assert report["symmetric_power_shared_cpu_min_batch"] == 8
    assert report["triton_real_convention_id"] == "real_tesseral_from_complex_condon_shortley_young_orthogonal_v1"
    assert "dense_source_analysis_C_dagger_L_v" in report["triton_operations"]
    assert report["compact_exterior_power_max_native_order"] == 8
    assert report["cpu"] is False  # no reference extension in this process
    assert report["core_abi_version"] == native.ABI_VERSION >= report["minimum_core_abi_version"] == 42
    assert report["analysis_orientation"] == "conjugate_transpose"
    assert REFERENCE_NAMES <= set(report["operations"])
    # the reference names its SH table op with the real_ prefix
    assert "spherical_harmonics_table_with_derivative" not in report["operations"]
    assert len(set(report["operations"])) == len(report["operations"])
    # no GPU in this environment: the HIP capability is off and lists nothing
    if not torch.cuda.is_available():
        assert report["hip"] is False and report["hip_operations"] == ()
        assert report["cuda"] is False and report["cuda_operations"] == ()
        assert report["symmetric_power_shared_cuda_min_reuse"] is None
        assert "hip_device" not in report


def test_symmetric_power_auto_dispatch_reads_the_report():
    """The reference's one in-library consumer of the report
    (``runtime/symmetric_power.py:1131-1150``), restated: on a device tensor it
    picks the native kernel when ``cuda_operations`` names it; on the CPU it
    reads the two CPU thresholds, which must be integers whenever
    ``prebuilt_extension`` is true."""
    report = runtime.native_execution_plan_capabilities()
    if report["prebuilt_extension"]:
        assert int(report["symmetric_power_cpu_auto_max_batch"]) == 32
        assert int(report["symmetric_power_cpu_auto_min_power"]) == 6
    assert ("symmetric_power_monomial" in report["cuda_operations"]) == report["cuda"]


def test_has_hip_and_has_cpu_are_exported():
    lib = native.lib()
    assert lib.ye3t_hip_has_cpu() == 0
    assert hasattr(lib, "ye3t_hip_has_hip")


def _csr(N=5, K=3):
    offs = torch.arange(N + 1, dtype=torch.int64) * K
    nbr = (torch.arange(N * K, dtype=torch.int64) * 7) % N
    return offs, nbr


def test_density_csr_validation_accepts_good_input():
    offs, nbr = _csr()
    species = torch.tensor([0, 1, 2, 3, 1], dtype=torch.int32)
    assert runtime.validate_density_csr(offs, nbr, 5, 15, species=species, species_count=4)
    # atoms without edges and an empty edge list are fine
    assert runtime.validate_density_csr(torch.zeros(4, dtype=torch.int64), None, 3, 0)


@pytest.mark.parametrize("case", ["first", "last", "decreasing", "nbr_high", "nbr_negative", "species_high",
                                  "species_dtype", "offsets_dtype", "offsets_shape"])
def test_density_csr_validation_rejects_bad_input(case):
    offs, nbr = _csr()
    species = torch.tensor([0, 1, 2, 3, 1], dtype=torch.int32)
    N, E = 5, 15
    if case == "first":
        offs = offs + 1
    elif case == "last":
        offs = offs.clone()
        offs[-1] = E - 1
    elif case == "decreasing":
        offs = offs.clone()
        offs[2] = offs[3] + 1
    elif case == "nbr_high":
        nbr = nbr.clone()
        nbr[4] = N
    elif case == "nbr_negative":
        nbr = nbr.clone()
        nbr[0] = -1
    elif case == "species_high":
        species = species.clone()
        species[2] = 4
    elif case == "species_dtype":
        species = species.to(torch.int64)
    elif case == "offsets_dtype":
        offs = offs.to(torch.int32)
    elif case == "offsets_shape":
        offs = offs[:-1]
    with pytest.raises(ValueError):
        runtime.validate_density_csr(offs, nbr, N, E, species=species, species_count=4)


def test_backend_reference_is_refused_explicitly():
    x = torch.zeros(3, dtype=torch.float64)
    with pytest.raises(NotImplementedError, match="reference"):
        runtime.cheb_exp_cos_radial_table_with_derivative(x, x, x, 2, backend="reference")
    with pytest.raises(ValueError, match="backend"):
        runtime.cheb_exp_cos_radial_table_with_derivative(x, x, x, 2, backend="triton")


def test_monomial_table_checks():
    import numpy as np

    counts = np.array([[2, 0], [1, 1], [0, 2]])
    offs = np.array([0, 1, 3])
    idx = np.array([0, 1, 1])
    vals = np.array([1.0, 2.0, 3.0])
    native.check_monomial_table(2, counts, offs, idx, vals)
    for bad in ({"idx": np.array([0, 0, 1])}, {"offs": np.array([0, 2, 2])}, {"counts": counts[:, :1]},
                {"vals": vals[:2]}, {"counts": -counts}):
        kw = {"counts": counts, "offs": offs, "idx": idx, "vals": vals, **bad}
        with pytest.raises(ValueError):
            native.check_monomial_table(2, kw["counts"], kw["offs"], kw["idx"], kw["vals"])
    native.check_shared_table(2, counts, offs, np.array([0, 1, 2]), idx, vals)
    with pytest.raises(ValueError, match="coefficient_terms"):
        native.check_shared_table(2, counts, offs, np.array([0, 1, 3]), idx, vals)
    with pytest.raises(ValueError, match="coefficient_outputs"):
        native.check_shared_table(2, counts, offs, np.array([0, 1, 2]), np.array([1, 1, 1]), vals)


REF_EXECUTION_PLAN = "/root/reference/ye3t/runtime/execution_plan.py"


@pytest.mark.skipif(not __import__("os").path.exists(REF_EXECUTION_PLAN), reason="reference tree not present")
def test_reference_operation_names_are_the_reference_report_names():
    """Every name this backend reports under the reference's names appears,
    quoted, among the operation names of the reference's capability report
    (``cuda_operations`` and ``operations``, ``execution_plan.py:6118-6850``;
    adjacent string literals joined), and each has a runtime function or an
    operator (the ``real_`` / ``complex_`` harmonic names are the
    ``spherical_harmonics_*`` functions with ``real_output`` set)."""
    import re

    with open(REF_EXECUTION_PLAN) as fh:
        text = fh.read()
    start = text.index("def native_execution_plan_capabilities")
    names = set()
    for key in ('"cuda_operations": (', '"operations": ('):
        i = text.index(key, start) + len(key) - 1
        depth, j = 0, i
        while True:  # the tuple's extent, by matching parentheses
            depth += {"(": 1, ")": -1}.get(text[j], 0)
            if depth == 0:
                break
            j += 1
        names |= set(re.findall(r'"([a-z_0-9]+)"', re.sub(r'"\s*\n\s*"', "", text[i:j + 1])))
    assert "density_accumulate" in names and "scheduled_radial_angular_channels_with_derivative" in names
    for name in runtime.REFERENCE_OPERATIONS:
        assert name in names, name
        base = re.sub(r"^(real|complex)_(?=spherical)", "", name)
        assert hasattr(runtime, base) or hasattr(runtime, base + "_contraction") or base.startswith(
            ("factorized_angular", "symmetric_power")), name
