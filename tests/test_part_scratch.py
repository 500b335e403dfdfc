"""Scratch bound of generated parts, checked on the host.

Config 5 in 550-value chunks (kernels with 2 052 and 1 260 bytes of scratch
per lane) ended in a memory aperture violation on the GPU; 400-value chunks
(772 bytes) ran clean.  The library reads each part's kernel descriptor from
its code object before loading it and refuses parts above 1 024 bytes per lane
or with a dynamic stack.  These tests compile small kernels with hipRTC (no
GPU needed) and check:

* the descriptor reader against kernels of known scratch (a 300-double local
  array indexed at run time, and none) and against malformed input;
* that the default chunk sizes of config 2 (forward, reverse mode and readout
  parts) stay within the bound;
* that the chunk-size knobs refuse values above 400;
* that parts above the bound are regenerated in smaller chunks.
"""

import pytest

from ye3t_amd.runtime import native

BIG = '''extern "C" __global__ void probe(double* out, int k) {
  volatile double a[300];
  for (int i = 0; i < 300; ++i) a[i] = out[i] * i;
  out[threadIdx.x] = a[k];
}'''
SMALL = '''extern "C" __global__ void probe(double* out, int k) { out[threadIdx.x] = out[k] * 2.0; }'''


def test_descriptor_reader_on_kernels_of_known_scratch():
    big = native.code_object_kernel_info(native.rtc_compile(BIG, name="probe.hip"), "probe")
    small = native.code_object_kernel_info(native.rtc_compile(SMALL, name="probe.hip"), "probe")
    assert big["private_segment_bytes"] >= 300 * 8 > native.part_private_limit()
    assert small["private_segment_bytes"] == 0
    assert not big["uses_dynamic_stack"] and not small["uses_dynamic_stack"]
    assert native.part_private_limit() == 1024


def test_descriptor_reader_refuses_malformed_input():
    blob = native.rtc_compile(SMALL, name="probe.hip")
    with pytest.raises(RuntimeError, match="not found"):
        native.code_object_kernel_info(blob, "no_such_kernel")
    with pytest.raises(RuntimeError, match="ELF"):
        native.code_object_kernel_info(b"\0" * 128, "probe")
    with pytest.raises(RuntimeError):
        native.code_object_kernel_info(blob[:200], "probe")


def test_default_parts_of_config2_stay_within_the_bound():
    from ye3t_amd.ace import workloads as W
    from ye3t_amd.ace.codegen import generate_adjoint_parts, generate_parts, generate_readout_parts
    from ye3t_amd.ace.pipeline import ADJOINT_PART_CHUNKS, ADJOINT_PART_MAX_LIVE
    from ye3t_amd.ace.plan import ProductPlan

    plan = ProductPlan(W.config(2).feature_spec)
    parts = generate_parts(plan, "f64", out_dtype="f64", in_dtype="f64")
    adjoint, _ = generate_adjoint_parts(plan, "f64", max_live=ADJOINT_PART_MAX_LIVE,
                                        chunks_per_part=ADJOINT_PART_CHUNKS, grad_dtype="f64", in_dtype="f64")
    readout, _ = generate_readout_parts(plan, "f64", in_dtype="f64")
    for source, meta in parts + adjoint + readout:
        info = native.code_object_kernel_info(native.rtc_compile(source), meta["kernel"])
        assert info["private_segment_bytes"] <= native.part_private_limit(), (meta["kernel"], info)
        assert not info["uses_dynamic_stack"]


@pytest.mark.parametrize("knob", ["YE3T_PARTS_MAX_LIVE", "YE3T_ADJOINT_PARTS_MAX_LIVE"])
def test_chunk_size_knobs_are_bounded(monkeypatch, knob):
    """Both knobs refuse chunks above 400 values before any part is generated."""
    from ye3t_amd.ace import workloads as W
    from ye3t_amd.ace.pipeline import ACEPipeline
    from ye3t_amd.ace.plan import ProductPlan

    pipe = ACEPipeline.__new__(ACEPipeline)  # the knobs need only the plan and the arithmetic type
    pipe.plan, pipe.accumulate = ProductPlan(W.config(4).feature_spec), "f64"
    read = pipe._parts_max_live if knob == "YE3T_PARTS_MAX_LIVE" else pipe._adjoint_parts_max_live
    monkeypatch.setenv(knob, "400")
    assert read() == 400
    for bad in ("550", "0"):
        monkeypatch.setenv(knob, bad)
        with pytest.raises(ValueError, match="must be in"):
            read()


@pytest.mark.gpu
def test_attach_refuses_a_part_above_the_bound(gpu):
    """The C ABI's parts attach reads the descriptor before loading anything
    and returns an error naming the scratch; the plan keeps working."""
    import ctypes

    import torch

    from ye3t_amd.ace import workloads as W
    from ye3t_amd.ace.pipeline import ACEPipeline
    from tests._util import flush

    flush("parts attach refuses a kernel with 2.4 KB of scratch per lane")
    pipe = ACEPipeline(W.config(4).feature_spec, "f32", accumulate="f64", density="f32")
    blob = native.rtc_compile(BIG, name="probe.hip")
    buf = ctypes.create_string_buffer(blob, len(blob))
    codes = (ctypes.c_void_p * 1)(ctypes.cast(buf, ctypes.c_void_p))
    sizes = (ctypes.c_int64 * 1)(len(blob))
    names = (ctypes.c_char_p * 1)(b"probe")
    chunks = (ctypes.c_int64 * 1)(1)
    lib = native.lib()
    for fn in (lib.ye3t_hip_product_plan_attach_generated_parts, lib.ye3t_hip_product_plan_attach_readout_parts):
        rc = fn(pipe.handle._handle, 1, codes, sizes, names, chunks)
        assert rc != 0
        assert b"scratch per lane" in lib.ye3t_hip_last_error()
    A = torch.zeros((64, pipe.plan.a_width), dtype=torch.float32, device=gpu)
    assert torch.equal(pipe.product(A), torch.zeros((64, pipe.feature_count), dtype=torch.float32, device=gpu))


def test_parts_above_the_bound_are_regenerated_in_smaller_chunks():
    """``fit_parts_to_scratch`` steps the node-value budget down until every
    compiled part is within the bound: here a real kernel of known scratch
    stands for the parts made at 300 values, a scratch-free one for 250 and
    below, so the fit settles on 250."""
    from ye3t_amd.ace.pipeline import PART_LIVE_STEP, fit_parts_to_scratch

    asked = []

    def make(n):
        asked.append(n)
        return [(SMALL, {}), (BIG if n > 250 else SMALL, {})]

    parts = fit_parts_to_scratch(make, 300, "probe")
    assert asked == [300, 300 - PART_LIVE_STEP] and PART_LIVE_STEP == 50
    assert [src for src, _ in parts] == [SMALL, SMALL]
    # a budget that cannot get smaller is returned as it is (the attach entry points then refuse it)
    assert [src for src, _ in fit_parts_to_scratch(lambda n: [(BIG, {})], PART_LIVE_STEP, "probe")] == [BIG]
