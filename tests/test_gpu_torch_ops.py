"""The ``ye3t_runtime`` Torch operators on the GPU through the shim.

Each covered operator, called as the reference's Python calls it
(``torch.ops.ye3t_runtime.<op>`` on device tensors), runs this library's
kernels: its results equal the direct entry points' (the same kernels) and the
oracle's, and ``torch.library.opcheck`` (schema, fake tensor, autograd
registration, AOT dispatch) passes, as the reference's own operator tests
require (``tests/test_execution_plan_native.py:6303-6350``).
"""

import numpy as np
import pytest

import oracle
from tests._dag import KAT_OUTPUT, KAT_PACKED, KAT_SOURCES, KAT_TABLES, KAT_WORKSPACE, SEGMENT_KEYS, random_segmented
from tests._util import TOL, column_rel_error, flush

pytestmark = pytest.mark.gpu


def _ops():
    import torch

    from ye3t_amd.runtime import torch_ops

    torch_ops.register()
    return torch.ops.ye3t_runtime


def _opcheck(op, args):
    import torch

    result = torch.library.opcheck(op, args, raise_exception=False)
    assert all(v == "SUCCESS" for v in result.values()), result


def _fa_args(dev, dt):
    import torch

    out = [torch.as_tensor(np.asarray(KAT_TABLES[n]), dtype=torch.int64, device=dev) for n in (
        "node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
        "node_coefficient_offsets", "coefficient_rows", "coefficient_columns")]
    out.append(torch.as_tensor(np.asarray(KAT_TABLES["coefficient_values"]), device=dev).to(dt))
    out.append(torch.as_tensor(np.asarray(KAT_TABLES["root_nodes"]), dtype=torch.int64, device=dev))
    out.append(torch.as_tensor(np.asarray(KAT_TABLES["projection_values"]), device=dev).to(dt))
    return out


def test_factorized_angular_operators(gpu):
    flush("torch ops: factorized_angular / adjoint / linear (complex128)")
    import torch

    ops = _ops()
    dt = torch.complex128
    args = _fa_args(gpu, dt)
    packed = torch.as_tensor(KAT_PACKED, dtype=dt, device=gpu)
    out = ops.factorized_angular(packed, *args, KAT_SOURCES, KAT_WORKSPACE, KAT_OUTPUT)
    ref = oracle.factorized_angular(KAT_PACKED.astype(np.complex128), KAT_TABLES, KAT_SOURCES)
    assert np.max(np.abs(out.cpu().numpy() - ref)) <= 1e-12
    _opcheck(ops.factorized_angular.default,
             (packed.clone().requires_grad_(True), *args, KAT_SOURCES, KAT_WORKSPACE, KAT_OUTPUT))
    g = torch.randn(out.shape, dtype=dt, device=gpu)
    adj = ops.factorized_angular_adjoint(g, packed, *args, KAT_SOURCES, KAT_WORKSPACE)
    assert np.max(np.abs(adj.cpu().numpy() - oracle.factorized_angular_adjoint(
        g.cpu().numpy(), KAT_PACKED.astype(np.complex128), KAT_TABLES, KAT_SOURCES))) <= 1e-12
    _opcheck(ops.factorized_angular_adjoint.default, (g, packed, *args, KAT_SOURCES, KAT_WORKSPACE))
    w = torch.randn(KAT_OUTPUT, dtype=dt, device=gpu)
    b = torch.tensor(0.25 - 0.5j, dtype=dt, device=gpu)
    lin = ops.factorized_angular_linear(packed, *args, KAT_SOURCES, KAT_WORKSPACE, w, b)
    torch.testing.assert_close(lin, out @ w + b, rtol=1e-12, atol=1e-12)
    _opcheck(ops.factorized_angular_linear.default,
             (packed.clone().requires_grad_(True), *args, KAT_SOURCES, KAT_WORKSPACE, w.clone().requires_grad_(True),
              b.clone().requires_grad_(True)))


@pytest.mark.parametrize("count", [1, 3])
def test_segmented_and_heterogeneous_operators(gpu, count):
    flush(f"torch ops: factorized_angular_segmented / heterogeneous ({count} segments)")
    import torch

    ops = _ops()
    tables, (D, S, W, F) = random_segmented(20 + count, complex_data=False, count=count)
    t = {k: torch.as_tensor(v, device=gpu) for k, v in tables.items()}
    x = torch.randn(37, D, dtype=torch.float64, device=gpu)
    seg_args = tuple(t[k] for k in SEGMENT_KEYS)
    out = ops.factorized_angular_segmented(x, *seg_args, S, W, F)
    ref = oracle.factorized_angular_segmented(x.cpu().numpy(), tables, F)
    assert column_rel_error(out.cpu().numpy(), ref) < TOL["f64"]
    _opcheck(ops.factorized_angular_segmented.default, (x.clone().requires_grad_(True), *seg_args, S, W, F))
    if count == 1:
        node = tuple(t[k] for k in ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
                                    "node_coefficient_offsets", "coefficient_rows", "coefficient_columns",
                                    "coefficient_values", "root_nodes"))
        het = node + (t["root_projection_starts"], t["root_projection_dimensions"], t["root_output_offsets"],
                      t["projection_values"])
        h = ops.factorized_angular_heterogeneous(x, *het, S, int(tables["segment_workspace_dimensions"][0]), F)
        assert torch.equal(h, out)
        _opcheck(ops.factorized_angular_heterogeneous.default,
                 (x.clone().requires_grad_(True), *het, S, int(tables["segment_workspace_dimensions"][0]), F))


def test_density_and_monomial_operators(gpu):
    flush("torch ops: density_accumulate, monomials, radial and harmonic tables")
    import torch

    from ye3t_amd import runtime

    ops = _ops()
    rng = np.random.default_rng(3)
    centers = torch.as_tensor(np.sort(rng.integers(0, 11, size=50)), device=gpu)
    vals = torch.randn(50, 6, dtype=torch.float64, device=gpu)
    acc = ops.density_accumulate(vals, centers, 11)
    assert torch.equal(acc, runtime.density_accumulate(vals, centers, 11))
    _opcheck(ops.density_accumulate.default, (vals.clone().requires_grad_(True), centers, 11))
    _opcheck(ops.density_accumulate_adjoint.default, (acc.clone().requires_grad_(True), centers))
    x = torch.randn(9, 3, dtype=torch.float64, device=gpu)
    counts = torch.tensor([[2, 0, 0], [0, 1, 1], [1, 1, 0], [0, 0, 2]], dtype=torch.int64, device=gpu)
    offsets = torch.tensor([0, 2, 4], dtype=torch.int64, device=gpu)
    indices = torch.tensor([0, 0, 1, 1], dtype=torch.int64, device=gpu)
    values = torch.tensor([0.75, -1.25, 0.5, -0.625], dtype=torch.float64, device=gpu)
    mono = ops.symmetric_power_monomial(x, counts, offsets, indices, values)
    assert torch.equal(mono, runtime.symmetric_power_monomial_contraction(x, counts, offsets, indices, values))
    _opcheck(ops.symmetric_power_monomial.default, (x.clone().requires_grad_(True), counts, offsets, indices, values))
    s_off = torch.tensor([0, 2, 4, 5], dtype=torch.int64, device=gpu)
    terms = torch.tensor([0, 1, 1, 2, 0], dtype=torch.int64, device=gpu)
    outs = torch.tensor([0, 0, 1, 1, 2], dtype=torch.int64, device=gpu)
    cvals = torch.tensor([0.75, -1.25, 0.5, -0.625, 1.5], dtype=torch.float64, device=gpu)
    shared = ops.symmetric_power_shared_monomial(x, counts, s_off, terms, outs, cvals)
    assert torch.equal(shared, runtime.symmetric_power_shared_monomial_contraction(x, counts, s_off, terms, outs,
                                                                                  cvals))
    _opcheck(ops.symmetric_power_shared_monomial.default,
             (x.clone().requires_grad_(True), counts, s_off, terms, outs, cvals))
    r = torch.rand(40, dtype=torch.float64, device=gpu) * 4.5 + 0.3
    c = torch.full_like(r, 5.0)
    lam = torch.full_like(r, 1.5)
    v, d = ops.cheb_exp_cos_radial_table_with_derivative(r, c, lam, 7)
    v2, d2 = runtime.cheb_exp_cos_radial_table_with_derivative(r, c, lam, 7)
    assert torch.equal(v, v2) and torch.equal(d, d2)
    e = torch.randn(40, 3, dtype=torch.float64, device=gpu)
    y, gy = ops.spherical_harmonics_table_with_derivative(e, 3, True, 1e-12)
    y2, gy2 = runtime.spherical_harmonics_table_with_derivative(e, 3, real_output=True)
    assert torch.equal(y, y2) and torch.equal(gy, gy2)


@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_complex_harmonic_table(gpu, dtype):
    """``real_output=False`` (the reference's default) on the device: the
    complex table and gradient from the HIP real table equal the oracle's real
    table put through the same conversion on the CPU (pinned against SciPy's
    complex harmonics in ``test_complex_sph``), to the north-star tolerance,
    through the runtime function and the Torch operator alike."""
    flush(f"complex harmonic table {dtype}")
    import torch

    from ye3t_amd import runtime

    ops = _ops()
    l_max = 5
    tdt = torch.float64 if dtype == "f64" else torch.float32
    rng = np.random.default_rng(21)
    v = rng.normal(size=(500, 3)) * rng.uniform(0.5, 3.0, size=(500, 1))
    e = torch.as_tensor(v, dtype=tdt, device=gpu)
    y, g = runtime.spherical_harmonics_table_with_derivative(e, l_max)
    assert y.dtype == (torch.complex128 if dtype == "f64" else torch.complex64) and g.shape == (500, 36, 3)
    y2, g2 = ops.spherical_harmonics_table_with_derivative(e, l_max, False, 1e-12)
    assert torch.equal(y, y2) and torch.equal(g, g2)
    rv, rg = oracle.real_sph_table(e.double().cpu().numpy(), l_max)
    ry, rgc = runtime.complex_from_real_table(torch.from_numpy(rv), torch.from_numpy(rg), l_max)
    for got, ref in ((y, ry), (g, rgc)):
        got, ref = got.cpu().to(torch.complex128).numpy(), ref.numpy()
        err = max(column_rel_error(got.real, ref.real), column_rel_error(got.imag, ref.imag))
        flush(f"  column error {err:.3e}")
        assert err <= TOL[dtype]


def test_single_index_radial_and_harmonics(gpu):
    """``cheb_exp_cos_radial_with_derivative`` (one radial index, radii of any
    shape, scalar cutoff and lambda broadcast as the reference does) and
    ``spherical_harmonics_with_derivative`` (one ``l``, real and complex): the
    oracle's radial table column (reference-core bit-exact on the CPU) to the
    north-star fp64 tolerance, and the table op's columns bit for bit, through
    the runtime functions and the Torch operators."""
    flush("single-index radial function and single-l harmonics")
    import torch

    from ye3t_amd import runtime

    ops = _ops()
    rng = np.random.default_rng(5)
    r = torch.as_tensor(rng.uniform(0.3, 5.5, size=(6, 7)), device=gpu)
    for n in (0, 1, 4, 8):
        v, d = runtime.cheb_exp_cos_radial_with_derivative(r, 5.0, 1.5, n)
        assert v.shape == r.shape and d.shape == r.shape
        rv, rd = oracle.radial_table(r.cpu().numpy().reshape(-1), np.full(42, 5.0), np.full(42, 1.5), n)
        assert column_rel_error(v.cpu().numpy().reshape(-1, 1), rv[:, n:n + 1]) <= TOL["f64"]
        assert column_rel_error(d.cpu().numpy().reshape(-1, 1), rd[:, n:n + 1]) <= TOL["f64"]
        tv, td = runtime.cheb_exp_cos_radial_table_with_derivative(r.reshape(-1), 5.0, 1.5, n)
        assert torch.equal(v.reshape(-1), tv[:, n]) and torch.equal(d.reshape(-1), td[:, n])
        v2, d2 = ops.cheb_exp_cos_radial_with_derivative(r, torch.full_like(r, 5.0), torch.full_like(r, 1.5), n)
        assert torch.equal(v, v2) and torch.equal(d, d2)
    e = torch.as_tensor(rng.normal(size=(50, 3)), device=gpu)
    for real in (True, False):
        tv, tg = runtime.spherical_harmonics_table_with_derivative(e, 4, real_output=real)
        for l in range(5):
            v, g = runtime.spherical_harmonics_with_derivative(e, l, real_output=real)
            assert v.shape == (50, 2 * l + 1) and g.shape == (50, 2 * l + 1, 3)
            assert torch.equal(v, tv[:, l * l:(l + 1) * (l + 1)]) and torch.equal(g, tg[:, l * l:(l + 1) * (l + 1)])
            v2, g2 = ops.spherical_harmonics_with_derivative(e, l, real, 1e-12)
            assert torch.equal(v, v2) and torch.equal(g, g2)


def test_radial_and_harmonic_operators_differentiate(gpu):
    """Autograd of the radial and harmonic operators: the gradient in the
    radii / edge vectors equals central differences of the operator's own
    values (fp64, real and complex harmonics, one index and the table), and
    the second derivative (the backward differentiated again) equals central
    differences of the first-order gradient."""
    flush("torch ops: radial and harmonic autograd")
    import torch

    ops = _ops()
    rng = np.random.default_rng(11)
    r = torch.as_tensor(rng.uniform(0.4, 4.5, size=30), device=gpu)
    c, lam = torch.full_like(r, 5.0), torch.full_like(r, 1.5)
    e = torch.as_tensor(rng.normal(size=(30, 3)), device=gpu)
    h = 1e-6

    def check(f, x, tol):
        xg = x.clone().requires_grad_(True)
        loss = f(xg)
        (g,) = torch.autograd.grad(loss, xg)
        fd = torch.zeros_like(x)
        flat = fd.view(-1)
        for i in range(x.numel()):
            step = torch.zeros_like(x).view(-1)
            step[i] = h
            step = step.view(x.shape)
            flat[i] = (f(x + step) - f(x - step)) / (2 * h)
        torch.testing.assert_close(g, fd, rtol=tol, atol=tol)

    w_tab = torch.as_tensor(rng.normal(size=(30, 8)), device=gpu)
    check(lambda x: (ops.cheb_exp_cos_radial_table_with_derivative(x, c, lam, 7)[0] * w_tab).sum(), r, 1e-6)
    check(lambda x: (ops.cheb_exp_cos_radial_with_derivative(x, c, lam, 5)[0] * w_tab[:, 0]).sum(), r, 1e-6)
    w_sh = torch.as_tensor(rng.normal(size=(30, 16)), device=gpu)
    w_im = torch.as_tensor(rng.normal(size=(30, 16)), device=gpu)
    check(lambda x: (ops.spherical_harmonics_table_with_derivative(x, 3, True, 1e-12)[0] * w_sh).sum(), e, 1e-6)

    def complex_loss(x):
        y = ops.spherical_harmonics_table_with_derivative(x, 3, False, 1e-12)[0]
        return (y.real * w_sh + y.imag * w_im).sum()

    check(complex_loss, e, 1e-6)
    check(lambda x: (ops.spherical_harmonics_with_derivative(x, 2, True, 1e-12)[0] * w_sh[:, :5]).sum(), e, 1e-6)
    _opcheck(ops.cheb_exp_cos_radial_table_with_derivative.default, (r.clone().requires_grad_(True), c, lam, 7))
    _opcheck(ops.spherical_harmonics_table_with_derivative.default, (e.clone().requires_grad_(True), 3, True, 1e-12))

    # second derivatives: the gradient taken with create_graph equals the
    # first-order one, and its own gradient equals central differences of the
    # first-order gradient (which the HIP derivative outputs give)
    def first(f, x):
        xg = x.clone().requires_grad_(True)
        return torch.autograd.grad(f(xg), xg)[0]

    def second(f, x, w2):
        xg = x.clone().requires_grad_(True)
        (g,) = torch.autograd.grad(f(xg), xg, create_graph=True)
        torch.testing.assert_close(g.detach(), first(f, x), rtol=1e-12, atol=1e-12)
        (h,) = torch.autograd.grad((g * w2).sum(), xg)
        fd = torch.zeros_like(x)
        for i in range(x.numel()):
            step = torch.zeros_like(x).view(-1)
            step[i] = h_step
            step = step.view(x.shape)
            fd.view(-1)[i] = ((first(f, x + step) - first(f, x - step)) * w2).sum() / (2 * h_step)
        torch.testing.assert_close(h, fd, rtol=1e-6, atol=1e-6)

    h_step = 1e-6
    second(lambda x: (ops.cheb_exp_cos_radial_table_with_derivative(x, c, lam, 7)[0] * w_tab).sum(), r,
           torch.as_tensor(rng.normal(size=30), device=gpu))
    w2 = torch.as_tensor(rng.normal(size=(30, 3)), device=gpu)
    second(lambda x: (ops.spherical_harmonics_table_with_derivative(x, 3, True, 1e-12)[0] * w_sh).sum(), e, w2)
    second(complex_loss, e, w2)
    second(lambda x: (ops.spherical_harmonics_with_derivative(x, 2, True, 1e-12)[0] * w_sh[:, :5]).sum(), e, w2)


def test_capability_report_hip_branch(gpu):
    """On the GPU the report's HIP branch is on: the ``cuda`` keys describe
    torch's ``cuda`` device type (the HIP device on ROCm), every listed
    operator has a device kernel registered, and the device facts are read
    from the library."""
    flush("capability report, HIP branch")
    import torch

    from ye3t_amd import runtime
    from ye3t_amd.runtime import native, torch_ops

    report = runtime.native_execution_plan_capabilities()
    assert report["hip"] is True and report["cuda"] is True
    assert report["hip_operations"] == report["operations"] and report["operations"]
    torch_ops.register()
    for name in report["cuda_operations"]:
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"ye3t_runtime::{name}", "CUDA"), name
    for name in ("symmetric_power_monomial", "symmetric_power_shared_monomial", "factorized_angular",
                 "density_accumulate", "symmetric_power_shared_sparse_monomial_double_backward"):
        assert name in report["cuda_operations"], name
    assert report["symmetric_power_shared_sparse_monomial"] is True
    assert report["symmetric_power_shared_cuda_min_reuse"] == 8.0
    assert report["symmetric_power_shared_cuda_grad_min_batch"] == 256
    assert report["symmetric_power_shared_cuda_forward_min_batch"] == 1024
    assert report["cuda_density_auto_min_work_items"] == 0
    dev = report["hip_device"]
    caps = native.device_caps(torch.cuda.current_device())
    assert dev == caps
    flush(f"  hip_device {dev}")
    assert "gfx950" in str(dev.get("arch", dev))
