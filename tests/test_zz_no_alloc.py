"""The allocation-free stream adjoint (``ye3t_hip_product_adjoint_stream_noalloc``).

Its partial gradients live in the library's static device scratch instead of a
workspace argument.  Checked through the C ABI against the workspace entry
point (``ye3t_hip_product_adjoint_stream``) and the oracle's reverse mode, on
two calls in a row with the second smaller (the scratch keeps the first call's
contents, which the call must clear), and a size beyond the scratch is refused
on the host.
"""

import numpy as np
import pytest

import oracle
from tests._util import TOL, column_rel_error, flush
from ye3t_amd.ace import workloads as W
from ye3t_amd.ace.pipeline import ACEPipeline

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cid,dtype", [(2, "f64"), (2, "f32")])
def test_noalloc_stream_adjoint_matches_workspace_entry_point(gpu, cid, dtype):
    import torch

    pipe = ACEPipeline(W.config(cid).feature_spec, dtype, kernel="interpreter")
    handle = pipe.handle
    assert handle.uses_stream
    real = torch.float64 if dtype == "f64" else torch.float32
    rng = np.random.default_rng(61)
    for samples in (777, 130):  # two calls in a row, the second smaller
        flush(f"noalloc stream adjoint config {cid} {dtype} samples {samples}")
        A = torch.as_tensor(rng.normal(size=(samples, pipe.plan.a_width)), dtype=real, device=gpu)
        gB = torch.as_tensor(rng.normal(size=(samples, pipe.feature_count)), dtype=real, device=gpu)
        want = handle.adjoint_stream(A, gB)
        got = torch.full_like(want, float("nan"))
        handle.adjoint_stream_noalloc(A, gB, got)
        torch.cuda.synchronize()
        err = column_rel_error(got.cpu().double().numpy(), want.cpu().double().numpy())
        ref = oracle.ace_product_flat_adjoint(A.double().cpu().numpy(), gB.double().cpu().numpy(),
                                              pipe.plan.flat_arrays())
        err_ref = column_rel_error(got.cpu().double().numpy(), ref)
        flush(f"  vs workspace entry point {err:.3e}, vs oracle {err_ref:.3e}")
        assert err < TOL[dtype]
        assert err_ref < TOL[dtype]
        # the column-major density gives the same bits as the row-major one
        got_cols = torch.full_like(want, float("nan"))
        from ye3t_amd.runtime import native

        At = native.transpose(A)
        handle.adjoint_stream_noalloc(At, gB, got_cols, samples=samples, columns=True)
        assert torch.equal(got_cols, got)


def test_noalloc_stream_adjoint_refuses_sizes_beyond_the_scratch(gpu):
    import torch

    pipe = ACEPipeline(W.config(2).feature_spec, "f64", kernel="interpreter")
    W_ = pipe.plan.a_width
    samples = (64 << 20) // (W_ * 8) + 64  # one group's partial gradients exceed 64 MiB
    A = torch.zeros((samples, W_), dtype=torch.float64, device=gpu)
    gB = torch.zeros((samples, pipe.feature_count), dtype=torch.float64, device=gpu)
    out = torch.empty_like(A)
    with pytest.raises(RuntimeError, match="static scratch"):
        pipe.handle.adjoint_stream_noalloc(A, gB, out)


def _inputs(rng, pipe, samples, real, gpu):
    import torch

    A = torch.as_tensor(rng.normal(size=(samples, pipe.plan.a_width)), dtype=real, device=gpu)
    gB = torch.as_tensor(rng.normal(size=(samples, pipe.feature_count)), dtype=real, device=gpu)
    return A, gB


def test_noalloc_calls_on_two_streams_are_ordered(gpu):
    """Back-to-back calls on two streams share the scratch: the second waits
    for the first's kernels, so each equals the same call made alone."""
    import torch

    pipe = ACEPipeline(W.config(2).feature_spec, "f64", kernel="interpreter")
    handle = pipe.handle
    rng = np.random.default_rng(62)
    A1, gB1 = _inputs(rng, pipe, 4000, torch.float64, gpu)
    A2, gB2 = _inputs(rng, pipe, 700, torch.float64, gpu)
    alone = []
    for A, gB in ((A1, gB1), (A2, gB2)):
        out = torch.empty_like(A)
        handle.adjoint_stream_noalloc(A, gB, out)
        torch.cuda.synchronize()
        alone.append(out)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [torch.full_like(A1, float("nan")), torch.full_like(A2, float("nan")), torch.full_like(A1, float("nan"))]
    flush("noalloc: calls on streams s1, s2, s1 without host synchronisation")
    with torch.cuda.stream(s1):
        handle.adjoint_stream_noalloc(A1, gB1, outs[0])
    with torch.cuda.stream(s2):
        handle.adjoint_stream_noalloc(A2, gB2, outs[1])
    with torch.cuda.stream(s1):
        handle.adjoint_stream_noalloc(A1, gB1, outs[2])
    torch.cuda.synchronize()
    assert torch.equal(outs[0], alone[0])
    assert torch.equal(outs[1], alone[1])
    assert torch.equal(outs[2], alone[0])


def test_noalloc_call_captured_in_a_graph(gpu):
    """A captured call (its fill kernel clears the scratch: no memset node)
    replays to the eager result, with eager calls that reuse the scratch and
    host synchronisations between the replays."""
    import torch

    pipe = ACEPipeline(W.config(2).feature_spec, "f64", kernel="interpreter")
    handle = pipe.handle
    rng = np.random.default_rng(63)
    A, gB = _inputs(rng, pipe, 1500, torch.float64, gpu)
    A2, gB2 = _inputs(rng, pipe, 900, torch.float64, gpu)
    want = torch.empty_like(A)
    handle.adjoint_stream_noalloc(A, gB, want)
    want2 = torch.empty_like(A2)
    handle.adjoint_stream_noalloc(A2, gB2, want2)
    torch.cuda.synchronize()
    out = torch.empty_like(A)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        handle.adjoint_stream_noalloc(A, gB, out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    flush("noalloc: capturing the call into a graph")
    with torch.cuda.graph(graph):
        handle.adjoint_stream_noalloc(A, gB, out)
    torch.cuda.synchronize()
    for replay in range(3):
        flush(f"noalloc: replay {replay}")
        out.fill_(float("nan"))
        other = torch.full_like(A2, float("nan"))
        handle.adjoint_stream_noalloc(A2, gB2, other)  # eager use of the scratch between replays
        torch.cuda.synchronize()
        assert torch.equal(other, want2)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
