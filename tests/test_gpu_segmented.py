"""Segmented factorized-angular DAGs on the GPU (``ye3t_hip_factorized_angular_segmented_*``).

* random segmented tables (roots of any dimension projecting onto random
  projection intervals into shuffled output blocks; two to five segments with
  their own source counts) against the pinned oracle: forward and the
  autograd adjoint, f64/c128 at 1e-12 and f32/c64 at 2e-5 column-relative,
  batches that leave partial blocks, and an empty batch;
* the reference-written plans grouped by the segmented module group: every
  member's output and slot gradients against the reference branch's (1e-12).
"""

import json

import numpy as np
import pytest

import oracle
from tests._dag import SEGMENT_KEYS, random_segmented
from tests._util import TOL, column_rel_error, flush
from tests.test_execution_plan_loader import DATA, _arr

pytestmark = pytest.mark.gpu


def _err(got, ref):
    """Column-relative error; a complex column is scaled by the RMS of its
    moduli (not its real and imaginary parts apart, whose cancellations are
    not the feature's scale)."""
    g, r = np.asarray(got), np.asarray(ref)
    if not np.iscomplexobj(r):
        return column_rel_error(g, r)
    g = g.astype(np.complex128).reshape(r.shape[0], -1)
    r = r.astype(np.complex128).reshape(r.shape[0], -1)
    rms = np.sqrt(np.mean(np.abs(r) ** 2, axis=0))
    err = np.max(np.abs(g - r), axis=0) / np.where(rms > 0, rms, 1.0)
    return float(err.max()) if err.size else 0.0


@pytest.mark.parametrize("dtype", ["f64", "c128", "f32", "c64"])
@pytest.mark.parametrize("seed,batch", [(1, 1), (2, 67), (3, 300), (4, 130)])
def test_segmented_random_tables_against_oracle(gpu, seed, batch, dtype):
    flush(f"segmented random tables seed={seed} batch={batch} dtype={dtype}")
    import torch

    from ye3t_amd.runtime import factorized_angular_segmented

    cplx = dtype in ("c64", "c128")
    tdt = {"f64": torch.float64, "c128": torch.complex128, "f32": torch.float32, "c64": torch.complex64}[dtype]
    npdt = {"f64": np.float64, "c128": np.complex128, "f32": np.float32, "c64": np.complex64}[dtype]
    tables, (D, S, W, F) = random_segmented(seed, complex_data=cplx, count=2 + seed % 4)
    # the device computes from the tables and inputs rounded to its dtype
    tables = {k: (v.astype(npdt) if k in ("coefficient_values", "projection_values") else v) for k, v in tables.items()}
    rng = np.random.default_rng(seed + 100)
    x = (rng.normal(size=(batch, D)) + (1j * rng.normal(size=(batch, D)) if cplx else 0)).astype(npdt)
    g = (rng.normal(size=(batch, F)) + (1j * rng.normal(size=(batch, F)) if cplx else 0)).astype(npdt)
    args = [torch.as_tensor(tables[k], device=gpu) for k in SEGMENT_KEYS]
    xg = torch.as_tensor(x, device=gpu).requires_grad_(True)
    out = factorized_angular_segmented(xg, *args, S, W, F)
    assert out.dtype == tdt and tuple(out.shape) == (batch, F)
    tol = TOL["f64"] if dtype in ("f64", "c128") else TOL["f32"]
    wide = {k: (v.astype(np.complex128 if cplx else np.float64) if v.dtype.kind in "fc" else v)
            for k, v in tables.items()}
    ref = oracle.factorized_angular_segmented(x.astype(np.complex128 if cplx else np.float64), wide, F)
    assert _err(out.detach().cpu().numpy(), ref) < tol
    (gx,) = torch.autograd.grad(out, xg, torch.as_tensor(g, device=gpu))
    ref_adj = oracle.factorized_angular_segmented_adjoint(g.astype(ref.dtype), x.astype(ref.dtype), wide)
    assert _err(gx.cpu().numpy(), ref_adj) < tol
    empty = factorized_angular_segmented(xg[:0].detach(), *args, S, W, F)
    assert tuple(empty.shape) == (0, F)


@pytest.mark.parametrize("dtype", ["float64", "complex128"])
def test_segmented_group_of_reference_plans(gpu, dtype):
    flush(f"segmented group of the reference-written plans ({dtype})")
    import torch

    from ye3t_amd.runtime import YE3TFactorizedAngularModule, YE3TSegmentedFactorizedAngularModuleGroup

    dt = {"float64": torch.float64, "complex128": torch.complex128}[dtype]
    names = sorted(DATA["plans"])
    cases = {c["plan"]: c for c in DATA["cases"] if c["dtype"] == dtype}
    modules = [YE3TFactorizedAngularModule(json.loads(DATA["plans"][n]["plan_json"]), backend="native", dtype=dt,
                                           device=gpu) for n in names]
    group = YE3TSegmentedFactorizedAngularModuleGroup(modules)
    slots = [tuple(torch.as_tensor(_arr(s, dtype), dtype=dt, device=gpu).requires_grad_(True)
                   for s in cases[n]["slots"]) for n in names]
    outs = group(slots)
    assert len(outs) == len(names)
    report = group.runtime_report()
    assert report["member_plan_hashes"] == tuple(DATA["plans"][n]["plan_hash"] for n in names)
    assert report["native_call_count"] == 1
    cots = []
    for n, o in zip(names, outs):
        expected = torch.as_tensor(_arr(cases[n]["output"], dtype), dtype=dt)
        torch.testing.assert_close(o.detach().cpu(), expected, rtol=0.0, atol=1e-12)
        cots.append(torch.as_tensor(_arr(cases[n]["output_cotangent"], dtype), dtype=dt, device=gpu))
    flat = [s for group_slots in slots for s in group_slots]
    grads = torch.autograd.grad(outs, flat, cots)
    k = 0
    for n in names:
        for e in cases[n]["slot_adjoints"]:
            torch.testing.assert_close(grads[k].cpu(), torch.as_tensor(_arr(e, dtype), dtype=dt), rtol=0.0,
                                       atol=1e-12)
            k += 1
