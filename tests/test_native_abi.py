"""The C-ABI library loads here (no GPU) and exports every declared symbol."""

import ctypes
import os
import re

import pytest

from ye3t_amd.runtime import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "ye3t_hip.h")).read()
    return sorted(set(re.findall(r"\b(ye3t_hip_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    if not native.available():
        pytest.fail("libye3t_hip.so is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(native.library_path())
    declared = _declared()
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(native.EXPORTED_SYMBOLS) == declared


def test_abi_version_and_error_channel():
    lib = native.lib()
    assert lib.ye3t_hip_abi_version() == native.ABI_VERSION >= 42
    assert lib.ye3t_hip_last_error() is not None


def test_invalid_arguments_are_rejected_without_gpu_work():
    lib = native.lib()
    # negative sizes and out-of-range degrees fail on the host before any launch
    assert lib.ye3t_hip_radial_table(0, None, None, None, -1, 3, None, None, None) == -1
    assert lib.ye3t_hip_real_sph_table(0, None, 5, 40, 1e-12, None, None, None) == -1
    assert b"maximum_angular_momentum" in lib.ye3t_hip_last_error()
    assert lib.ye3t_hip_radial_table(7, None, None, None, 0, 3, None, None, None) == 0  # empty is a no-op


def test_plan_validation_rejects_bad_program():
    import numpy as np

    from ye3t_amd.ace.plan import ACEFeatureSpec, ProductPlan
    from ye3t_amd.ace.program import compile_program

    prog = compile_program(ProductPlan(ACEFeatureSpec(channel_count=1, l_max=1, nu_max=2, targets=(0,))), "f32")
    bad = dict(prog)
    bad["words"] = prog["words"].copy()
    # corrupt the first operand slot beyond the workspace
    for i, w in enumerate(bad["words"]):
        if (int(w) >> 28) == 3:
            bad["words"][i + 2] = np.uint32(0xFFFF)
            break
    with pytest.raises(RuntimeError, match="bad operand"):
        native.ProductPlanHandle(bad)


def test_neighbor_list_arguments_are_checked_on_the_host():
    L = native.lib()
    grid = native.cell_grid([0.0, 0.0, 0.0], [10.0, 10.0, 10.0], 2.0, 100)
    need = L.ye3t_hip_neighbor_workspace_bytes(100, ctypes.byref(grid))
    assert need > 0
    # a cutoff above the cell edge, a short workspace and a bad dtype fail before any launch
    assert L.ye3t_hip_neighbor_count(1, None, 100, ctypes.byref(grid), 2.5, None, need, None, None) == -1
    assert b"cutoff" in L.ye3t_hip_last_error()
    assert L.ye3t_hip_neighbor_count(1, None, 100, ctypes.byref(grid), 2.0, ctypes.c_void_p(256), need - 1,
                                     ctypes.c_void_p(256), None) == -1
    assert b"workspace" in L.ye3t_hip_last_error()
    assert L.ye3t_hip_neighbor_count(9, ctypes.c_void_p(256), 100, ctypes.byref(grid), 2.0, ctypes.c_void_p(256),
                                     need, ctypes.c_void_p(256), None) == -3
    bad = native.CellGrid()
    bad.cell_edge = 1.0
    bad.dims[0], bad.dims[1], bad.dims[2] = 1, 0, 1
    assert L.ye3t_hip_neighbor_workspace_bytes(10, ctypes.byref(bad)) == -1


def test_cell_grid_sizes():
    g = native.cell_grid([0.0, 0.0, 0.0], [100.0, 100.0, 100.0], 5.0, 50000)
    assert list(g.dims) == [20, 20, 20] and g.cell_edge >= 5.0 * (1 + 1e-9)
    # sparse atoms far apart: the grid is widened to at most max(4 N, 64) cells
    g = native.cell_grid([0.0, 0.0, 0.0], [1e6, 1.0, 1.0], 5.0, 10)
    assert g.dims[0] * g.dims[1] * g.dims[2] <= 64 and g.dims[0] * g.cell_edge > 1e6
    g = native.cell_grid([0.0] * 3, [0.0] * 3, 1.0, 0)
    assert list(g.dims) == [1, 1, 1]
    with pytest.raises(ValueError):
        native.cell_grid([0.0, float("nan"), 0.0], [1.0, 1.0, 1.0], 1.0, 4)
    with pytest.raises(ValueError):
        native.cell_grid([0.0] * 3, [1.0] * 3, 0.0, 4)
