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
