"""The reference's general factorized-angular DAG op on the GPU
(``ye3t_hip_factorized_angular_*`` through the C ABI).

* the closed-form known-answer case of the reference's installed-CUDA smoke
  test (``cmake/smoke_installed_cuda.py:106-240``): forward, the autograd
  gradient, the fused linear readout and its three gradients, at the smoke
  test's own tolerance (2e-10) and at the parity bar;
* random DAGs against the pinned oracle (real, complex; fp64 at 1e-12, fp32 at
  2e-5 column-relative), forward, adjoint and linear readout with adjoint,
  including several sources, several roots, a workspace too wide for 64
  samples per wave, and an empty batch;
* the module mirror (slot packing, output shape, readout).
"""

import numpy as np
import pytest

import oracle
from tests._dag import (KAT_LINEAR_BIAS, KAT_LINEAR_WEIGHT, KAT_OUTPUT_ADJOINT, KAT_OUTPUT, KAT_PACKED,
                        KAT_SOURCES, KAT_TABLES, KAT_WORKSPACE, kat_closed_form, random_dag)
from tests._util import TOL, column_rel_error, flush

pytestmark = pytest.mark.gpu


def _args(tables, dev, dtype):
    import torch

    out = []
    for name in ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
                 "node_coefficient_offsets", "coefficient_rows", "coefficient_columns"):
        out.append(torch.as_tensor(np.asarray(tables[name]), dtype=torch.int64, device=dev))
    out.append(torch.as_tensor(np.asarray(tables["coefficient_values"]), device=dev).to(dtype))
    out.append(torch.as_tensor(np.asarray(tables["root_nodes"]), dtype=torch.int64, device=dev))
    out.append(torch.as_tensor(np.asarray(tables["projection_values"]), device=dev).to(dtype))
    return out


def _torch_kat(packed):
    import torch

    src = packed.reshape(2, 2, 6)
    c = torch.as_tensor(KAT_TABLES["coefficient_values"], device=packed.device)
    roots = (src[:, :, :3] * src[:, :, 3:] * c.conj().reshape(1, 1, 3)).sum(dim=2)
    return roots @ torch.as_tensor(KAT_TABLES["projection_values"], device=packed.device).reshape(2, 2)


def test_known_answer_forward_gradient_and_linear(gpu):
    flush("factorized_angular known-answer case (complex128)")
    import torch

    from ye3t_amd.runtime import factorized_angular, factorized_angular_linear

    dt = torch.complex128
    args = _args(KAT_TABLES, gpu, dt)
    packed = torch.as_tensor(KAT_PACKED, dtype=dt, device=gpu).requires_grad_(True)
    actual = factorized_angular(packed, *args, KAT_SOURCES, KAT_WORKSPACE, KAT_OUTPUT)
    expected = torch.as_tensor(kat_closed_form(KAT_PACKED.astype(np.complex128)), device=gpu)
    torch.testing.assert_close(actual, expected, rtol=2.0e-10, atol=2.0e-10)
    assert column_rel_error(actual.detach().cpu().numpy().view(np.float64),
                            expected.cpu().numpy().view(np.float64)) < TOL["f64"]
    g = torch.as_tensor(KAT_OUTPUT_ADJOINT, device=gpu)
    (grad,) = torch.autograd.grad(actual, packed, g)
    ref_in = torch.as_tensor(KAT_PACKED, dtype=dt).requires_grad_(True)
    (expected_grad,) = torch.autograd.grad(_torch_kat(ref_in), ref_in, g.cpu())
    torch.testing.assert_close(grad.cpu(), expected_grad, rtol=2.0e-10, atol=2.0e-10)
    # fused linear readout and its gradients in the slots, the weight and the bias
    x = torch.as_tensor(KAT_PACKED, dtype=dt, device=gpu).requires_grad_(True)
    w = torch.as_tensor(KAT_LINEAR_WEIGHT, device=gpu).requires_grad_(True)
    b = torch.tensor(KAT_LINEAR_BIAS, dtype=dt, device=gpu).requires_grad_(True)
    lin = factorized_angular_linear(x, *args, KAT_SOURCES, KAT_WORKSPACE, w, b)
    rx = torch.as_tensor(KAT_PACKED, dtype=dt).requires_grad_(True)
    rw = torch.as_tensor(KAT_LINEAR_WEIGHT).requires_grad_(True)
    rb = torch.tensor(KAT_LINEAR_BIAS, dtype=dt).requires_grad_(True)
    ref_lin = _torch_kat(rx) @ rw + rb
    torch.testing.assert_close(lin.detach().cpu(), ref_lin.detach(), rtol=2.0e-10, atol=2.0e-10)
    ga = torch.as_tensor(KAT_OUTPUT_ADJOINT[:, 0], device=gpu)
    got = torch.autograd.grad(lin, (x, w, b), ga)
    want = torch.autograd.grad(ref_lin, (rx, rw, rb), ga.cpu())
    for a, e in zip(got, want):
        torch.testing.assert_close(a.cpu(), e, rtol=2.0e-10, atol=2.0e-10)


def _cplx_err(got, ref):
    g = np.asarray(got)
    r = np.asarray(ref)
    if np.iscomplexobj(r):
        g = np.ascontiguousarray(g.astype(np.complex128)).view(np.float64)
        r = np.ascontiguousarray(r.astype(np.complex128)).view(np.float64)
    return column_rel_error(g, r)


@pytest.mark.parametrize("dtype", ["float64", "complex128", "float32", "complex64"])
@pytest.mark.parametrize("seed,B,max_nodes", [(11, 1, 9), (12, 130, 9), (13, 257, 14)])
def test_random_dags_against_the_oracle(gpu, dtype, seed, B, max_nodes):
    flush(f"factorized_angular random DAG seed {seed} batch {B} {dtype}")
    import torch

    from ye3t_amd.runtime import factorized_angular, factorized_angular_linear

    dt = getattr(torch, dtype)
    cplx = dt.is_complex
    tables, S, D = random_dag(seed, complex_data=cplx, max_nodes=max_nodes)
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(B, S * D)) + (1j * rng.normal(size=(B, S * D)) if cplx else 0)
    low = dt in (torch.float32, torch.complex64)
    # the oracle sees the values as the device holds them
    x_dev = torch.as_tensor(x, device=gpu).to(dt)
    t_dev = dict(tables)
    for k in ("coefficient_values", "projection_values"):
        t_dev[k] = torch.as_tensor(tables[k]).to(dt).numpy()
    xr = x_dev.cpu().numpy()
    tol = TOL["f32"] if low else TOL["f64"]
    args = _args(t_dev, gpu, dt)
    W = int(tables["node_offsets"][-1] + tables["node_dimensions"][-1])
    P = len(tables["projection_values"]) // S
    K = len(tables["root_nodes"]) * P * int(tables["node_dimensions"][tables["root_nodes"][0]])
    xg = x_dev.clone().requires_grad_(True)
    out = factorized_angular(xg, *args, S, W, K)
    ref = oracle.factorized_angular(xr, t_dev, S)
    err = _cplx_err(out.detach().cpu().numpy(), ref)
    g = rng.normal(size=ref.shape) + (1j * rng.normal(size=ref.shape) if cplx else 0)
    g_dev = torch.as_tensor(g, device=gpu).to(dt)
    (gx,) = torch.autograd.grad(out, xg, g_dev)
    gref = oracle.factorized_angular_adjoint(g_dev.cpu().numpy(), xr, t_dev, S)
    gerr = _cplx_err(gx.cpu().numpy(), gref)
    w = rng.normal(size=K) + (1j * rng.normal(size=K) if cplx else 0)
    w_dev = torch.as_tensor(w, device=gpu).to(dt)
    bias = complex(0.25, -0.5) if cplx else 0.25
    xl = x_dev.clone().requires_grad_(True)
    wl = w_dev.clone().requires_grad_(True)
    bl = torch.tensor(bias, dtype=dt, device=gpu).requires_grad_(True)
    lin = factorized_angular_linear(xl, *args, S, W, wl, bl)
    lref = oracle.factorized_angular_linear(xr, t_dev, S, w_dev.cpu().numpy(), bias)
    lerr = float(np.max(np.abs(lin.detach().cpu().numpy() - lref)) / np.sqrt(np.mean(np.abs(lref) ** 2)))
    ga = rng.normal(size=B) + (1j * rng.normal(size=B) if cplx else 0)
    ga_dev = torch.as_tensor(ga, device=gpu).to(dt)
    gxl, gwl, gbl = torch.autograd.grad(lin, (xl, wl, bl), ga_dev)
    rx, rw, rb = oracle.factorized_angular_linear_adjoint(ga_dev.cpu().numpy(), xr, t_dev, S, w_dev.cpu().numpy())
    rw = np.asarray(rw)
    gw_err = float(np.max(np.abs(gwl.cpu().numpy() - rw)) / np.sqrt(np.mean(np.abs(rw) ** 2)))
    lgerr = max(_cplx_err(gxl.cpu().numpy(), rx), gw_err,
                abs(complex(gbl) - complex(rb)) / max(1.0, abs(complex(rb))))
    flush(f"  forward {err:.2e} adjoint {gerr:.2e} linear {lerr:.2e} linear adjoint {lgerr:.2e}")
    assert err < tol and gerr < tol and lerr < tol and lgerr < tol


def test_wide_workspace_runs_fewer_samples_per_wave(gpu):
    """A DAG whose workspace does not fit 64 complex128 samples per wave in
    64 KB of LDS (forward: 4 KB per sample at 256 values)."""
    flush("factorized_angular wide workspace")
    import torch

    from ye3t_amd.runtime import factorized_angular

    tables, S, D = random_dag(21, complex_data=True, leaves_L=(6, 6, 5, 4, 6, 6), max_nodes=40)
    W = int(tables["node_offsets"][-1] + tables["node_dimensions"][-1])
    assert W * 16 * 64 > 64 * 1024
    B = 100
    rng = np.random.default_rng(21)
    x = rng.normal(size=(B, S * D)) + 1j * rng.normal(size=(B, S * D))
    P = len(tables["projection_values"]) // S
    K = len(tables["root_nodes"]) * P * 3
    xg = torch.as_tensor(x, device=gpu).requires_grad_(True)
    out = factorized_angular(xg, *_args(tables, gpu, torch.complex128), S, W, K)
    assert _cplx_err(out.detach().cpu().numpy(), oracle.factorized_angular(x, tables, S)) < TOL["f64"]
    g = rng.normal(size=(B, K)) + 1j * rng.normal(size=(B, K))
    (gx,) = torch.autograd.grad(out, xg, torch.as_tensor(g, device=gpu))
    assert _cplx_err(gx.cpu().numpy(), oracle.factorized_angular_adjoint(g, x, tables, S)) < TOL["f64"]


def test_module_mirror_packs_slots_and_reads_out(gpu):
    flush("YE3TFactorizedAngularModule from tables")
    import torch

    from ye3t_amd.runtime import YE3TFactorizedAngularModule

    mod = YE3TFactorizedAngularModule.from_tables(KAT_TABLES, input_Ls=(1, 1), source_dimension=2, output_L=0)
    assert mod.output_dimension == 2 and mod.workspace_dimension == KAT_WORKSPACE
    src = torch.as_tensor(KAT_PACKED, dtype=torch.complex128, device=gpu).reshape(2, 2, 6)
    out = mod((src[..., :3], src[..., 3:]))
    assert tuple(out.shape) == (2, 2, 1)
    expected = kat_closed_form(KAT_PACKED.astype(np.complex128))
    torch.testing.assert_close(out.reshape(2, 2).cpu(), torch.as_tensor(expected), rtol=1e-12, atol=1e-12)
    lin = mod.linear_readout((src[..., :3], src[..., 3:]), KAT_LINEAR_WEIGHT, KAT_LINEAR_BIAS)
    torch.testing.assert_close(lin.cpu(), torch.as_tensor(expected @ KAT_LINEAR_WEIGHT + KAT_LINEAR_BIAS),
                               rtol=1e-12, atol=1e-12)
    assert mod.last_linear_readout_backend == "native_fused_factorized_linear"
    assert mod.runtime_report()["unique_node_count"] == 3
    # an empty batch and bad slot shapes
    assert tuple(mod((src[:0, :, :3], src[:0, :, 3:])).shape) == (0, 2, 1)
    with pytest.raises(ValueError):
        mod((src[..., :2], src[..., 3:]))


def test_plan_validation_rejects_bad_tables(gpu):
    import torch

    from ye3t_amd.runtime import factorized_angular

    packed = torch.as_tensor(KAT_PACKED, dtype=torch.complex128, device=gpu)
    bad = dict(KAT_TABLES)
    bad["coefficient_rows"] = np.array([0, 4, 9])  # row 9 is past 3 x 3
    with pytest.raises(RuntimeError, match="coefficient row"):
        factorized_angular(packed, *_args(bad, gpu, torch.complex128), 2, 7, 2)
    with pytest.raises(RuntimeError, match="workspace_dimension"):
        factorized_angular(packed, *_args(KAT_TABLES, gpu, torch.complex128), 2, 8, 2)
    with pytest.raises(RuntimeError, match="output width"):
        factorized_angular(packed, *_args(KAT_TABLES, gpu, torch.complex128), 2, 7, 3)
