"""HIP kernels vs the CPU oracle on identical seeded inputs (needs an MI355X)."""

import json
import os

import numpy as np
import pytest

import oracle
from tests._util import TOL, column_rel_error, flush, fp32_rounding_ratio, rounded_inputs
from ye3t_amd.ace import workloads as W
from ye3t_amd.ace.pipeline import ACEPipeline, to_device_inputs
from ye3t_amd.ace.plan import ProductPlan
from ye3t_amd.runtime import native

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _t(x, dtype, dev):
    import torch

    return torch.as_tensor(np.asarray(x), dtype=torch.float64 if dtype == "f64" else torch.float32, device=dev)


@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_radial_table(gpu, dtype):
    flush(f"radial_table {dtype}")
    rng = np.random.default_rng(10)
    E = 3001
    r = rng.uniform(0, 6, E)
    rc = rng.uniform(2, 5.5, E)
    lam = rng.uniform(0.1, 2.0, E)
    ref_in = [np.asarray(x, dtype=np.float32).astype(np.float64) if dtype == "f32" else x for x in (r, rc, lam)]
    v_ref, d_ref = oracle.radial_table(*ref_in, 12)
    v, d = native.radial_table(*(_t(x, dtype, gpu) for x in (r, rc, lam)), 12)
    v, d = v.cpu().numpy(), d.cpu().numpy()
    flush(f"  values {column_rel_error(v, v_ref):.3e} derivatives {column_rel_error(d, d_ref):.3e}")
    if dtype == "f64":
        # the reference's own bounds for this table (tests/test_execution_plan_native.py:748-759)
        np.testing.assert_allclose(v, v_ref, rtol=2e-13, atol=2e-13)
        np.testing.assert_allclose(d, d_ref, rtol=2e-12, atol=2e-12)
    else:
        assert column_rel_error(v, v_ref) < 2e-5
        assert column_rel_error(d, d_ref) < 2e-5


@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_real_sph_table(gpu, dtype):
    flush(f"real_sph_table {dtype}")
    rng = np.random.default_rng(11)
    vec = rng.normal(size=(2049, 3)) * rng.uniform(0.5, 5, (2049, 1))
    vec[5] = 0.0
    ref_vec = np.asarray(vec, dtype=np.float32).astype(np.float64) if dtype == "f32" else vec
    for lmax in (0, 3, 6, 8):
        y_ref, g_ref = oracle.real_sph_table(ref_vec, lmax)
        y, g = native.real_sph_table(_t(vec, dtype, gpu), lmax)
        tol = 1e-12 if dtype == "f64" else 2e-5
        assert column_rel_error(y.cpu().numpy(), y_ref) < tol, lmax
        assert column_rel_error(g.cpu().numpy().reshape(len(vec), -1), g_ref.reshape(len(vec), -1)) < tol * 10


def test_density_accumulate_unsorted(gpu):
    flush("density_accumulate")
    import torch

    from ye3t_amd.runtime import density_accumulate

    rng = np.random.default_rng(12)
    E, C, N = 5000, 33, 700
    ev = rng.normal(size=(E, C))
    centers = rng.integers(0, N - 50, E)  # the last atoms get no edges
    ref = oracle.density_accumulate(ev, centers, N)
    got = density_accumulate(torch.as_tensor(ev, device=gpu), torch.as_tensor(centers, device=gpu), N)
    assert column_rel_error(got.cpu().numpy(), ref) < 1e-12
    with pytest.raises(RuntimeError, match="out of range"):
        density_accumulate(torch.as_tensor(ev, device=gpu), torch.as_tensor(centers + 100, device=gpu), N)


@pytest.mark.parametrize("dtype", ["f32", "f64"])
@pytest.mark.parametrize("C", [1, 3, 16, 33])
def test_density_accumulate_adjoint(gpu, dtype, C):
    """Gather of centre-row adjoints: bit-exact copy of the oracle, transpose of density_accumulate."""
    flush(f"density_accumulate_adjoint {dtype} C={C}")
    import torch

    from ye3t_amd.runtime import density_accumulate, density_accumulate_adjoint

    rng = np.random.default_rng(100 + C)
    E, N = 5000, 700
    tdt = torch.float64 if dtype == "f64" else torch.float32
    adj = torch.as_tensor(rng.normal(size=(N, C)), dtype=tdt)
    centers = rng.integers(0, N - 50, E)  # unsorted; the last atoms own no edges
    got = density_accumulate_adjoint(adj.to(gpu), torch.as_tensor(centers, device=gpu))
    ref = oracle.density_accumulate_adjoint(adj.double().numpy(), centers)
    assert got.dtype == tdt and tuple(got.shape) == (E, C)
    assert np.array_equal(got.cpu().double().numpy(), ref)
    # <accumulate(x), y> = <x, adjoint(y)> on the device pair
    x = torch.as_tensor(rng.normal(size=(E, C)), dtype=torch.float64, device=gpu)
    y = adj.double().to(gpu)
    cen = torch.as_tensor(centers, device=gpu)
    lhs = float((density_accumulate(x, cen, N) * y).sum())
    rhs = float((x * density_accumulate_adjoint(y, cen)).sum())
    assert abs(lhs - rhs) <= 1e-10 * max(1.0, abs(lhs))
    empty = density_accumulate_adjoint(adj.to(gpu), torch.zeros(0, dtype=torch.int64, device=gpu))
    assert tuple(empty.shape) == (0, C)
    with pytest.raises(RuntimeError, match="out of range"):
        density_accumulate_adjoint(adj.to(gpu), torch.as_tensor(centers + N, device=gpu))


def _ragged_workload(dtype_mode):
    """Atoms with 0, 1, 63, 64, 65 and 130 neighbours (empty rows and multi-tile rows)."""
    rng = np.random.default_rng(13)
    counts = np.array([0, 1, 63, 64, 65, 130, 0, 7])
    N = len(counts)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    E = int(offsets[-1])
    vec = rng.normal(size=(E, 3))
    vec = vec / np.linalg.norm(vec, axis=1, keepdims=True) * rng.uniform(0.8, 5.0, (E, 1))
    inp = {"atom_count": N, "edge_count": E, "centers": np.repeat(np.arange(N), counts), "row_offsets": offsets,
           "neighbors": rng.integers(0, N, E), "edge_vectors": vec, "n_max": 8, "l_max": 4, "cutoff": 5.0,
           "lambda": W.LAMBDA, "epsilon": 1e-12, "species": None, "node_features": None, "radial_mix": None}
    if dtype_mode == "species":
        inp.update(channel_count=3, species=rng.integers(0, 3, N).astype(np.int32))
    elif dtype_mode == "features":
        inp.update(channel_count=5, node_features=rng.normal(size=(N, 5)), radial_mix=rng.normal(size=(5, 9)) / 3)
    else:
        inp.update(channel_count=1)
    return inp


@pytest.mark.parametrize("mode", ["single", "species", "features"])
@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_ace_density_ragged(gpu, mode, dtype):
    flush(f"ace_density ragged {mode} {dtype}")
    inp = _ragged_workload(mode)
    ref = oracle.ace_density(rounded_inputs(inp, dtype))
    pipe_inp = to_device_inputs(inp, dtype, gpu)
    A = native.ace_density_forward(
        pipe_inp["edge_vectors"], pipe_inp["row_offsets"], pipe_inp["neighbors"], atom_count=inp["atom_count"],
        channel_count=inp["channel_count"], n_max=inp["n_max"], l_max=inp["l_max"], cutoff=inp["cutoff"],
        lam=inp["lambda"], species=pipe_inp.get("species"), node_features=pipe_inp.get("node_features"),
        radial_mix=pipe_inp.get("radial_mix"))
    got = A.cpu().numpy()
    assert np.all(got[0] == 0) and np.all(got[6] == 0)
    assert column_rel_error(got.reshape(inp["atom_count"], -1), ref.reshape(inp["atom_count"], -1)) < TOL[dtype]


@pytest.mark.parametrize("cid,dtype", [(2, "f64"), (3, "f64"), (3, "f32"), (4, "f32"), (4, "f64"), (5, "f32")])
def test_ace_density_configs(gpu, cid, dtype):
    flush(f"ace_density config {cid} {dtype}")
    cfg = W.config(cid, atom_count=300)
    inp = cfg.density.generate()
    ref = oracle.ace_density(rounded_inputs(inp, dtype))
    dev = to_device_inputs(inp, dtype, gpu)
    A = native.ace_density_forward(
        dev["edge_vectors"], dev["row_offsets"], dev["neighbors"], atom_count=inp["atom_count"],
        channel_count=inp["channel_count"], n_max=inp["n_max"], l_max=inp["l_max"], cutoff=inp["cutoff"],
        lam=inp["lambda"], species=dev.get("species"), node_features=dev.get("node_features"),
        radial_mix=dev.get("radial_mix"))
    err = column_rel_error(A.cpu().numpy().reshape(300, -1), ref.reshape(300, -1))
    flush(f"  err {err:.3e}")
    assert err < TOL[dtype]


def test_symmetric_monomial_golden_fixture_on_gpu(gpu):
    import torch

    fx = json.load(open(os.path.join(GOLDEN, "shared_monomial_plan_v1.json")))
    D = int(fx["input_dimension"])
    mono = np.array(fx["monomial_counts"], dtype=np.int64).reshape(-1, D)
    terms = np.array(fx["coefficient_terms"], dtype=np.int64)
    x = torch.as_tensor(np.array(fx["input"]).reshape(-1, D), device=gpu)
    out = native.symmetric_power_monomial(x, mono[terms], np.array(fx["output_offsets"]),
                                          torch.as_tensor(fx["coefficient_values"], dtype=torch.float64))
    np.testing.assert_allclose(out.cpu().numpy().reshape(-1), fx["expected_output"], rtol=0, atol=5e-13)


def test_config1_schedule_evaluation(gpu):
    """Config 1: README sector on supplied factors through the compiled schedule."""
    flush("config 1 schedule evaluation")
    import torch

    from ye3t_amd.core.symmetric_power import complex_monomial_entries
    from ye3t_amd.couplings import compile_ace_factorized_schedules_by_L

    a11, a20 = W.config1_factors()
    rep = compile_ace_factorized_schedules_by_L(content=(1, 1, 2), input_Ls=(1, 1, 0))
    x = torch.as_tensor(a11.reshape(-1, 3), device=gpu)
    for L, sched in rep.schedules_by_L.items():
        spec = sched.block_specs[0][0]
        rows = complex_monomial_entries(2, 1, spec["Lambda"], 0)
        counts = np.array([r[1] for r in rows], dtype=np.int64)
        outs = np.array([r[0] for r in rows])
        order = np.argsort(outs, kind="stable")
        offs = np.searchsorted(outs[order], np.arange(2 * spec["Lambda"] + 2))
        vals = torch.as_tensor(np.array([r[2] for r in rows])[order])
        sym = native.symmetric_power_monomial(x, counts[order], offs, vals)
        sym_ref = oracle.symmetric_power_monomial(a11.reshape(-1, 3), counts[order], offs, vals.numpy())
        assert column_rel_error(sym.cpu().numpy(), sym_ref) < 1e-12
        mdim = sched.flat_arrays()["max_block_m_dim"]
        bv = torch.zeros((x.shape[0], 1, 2, mdim), dtype=torch.float64, device=gpu)
        bv[:, 0, 0, :sym.shape[1]] = sym
        bv[:, 0, 1, 0] = torch.as_tensor(a20.reshape(-1), device=gpu)
        got = rep.evaluate(bv, target_L=L).cpu().numpy()
        ref = oracle.evaluate_componentwise(bv.cpu().numpy(), sched.flat_arrays())
        assert got.shape == (32768, 2 * L + 1)
        assert column_rel_error(got, ref) < 1e-12


@pytest.mark.parametrize("content", [((1, 1, 1), (1, 2, 3)), ((1, 1, 1, 1), (2, 2, 2, 2)),
                                     ((1, 1, 2, 2), (1, 1, 2, 2))])
def test_real_tesseral_schedule_evaluation(gpu, content):
    """The real-tesseral schedule (reference ``core/couplings.py:1818-1966``) on the HIP evaluator."""
    flush(f"real tesseral schedule {content}")
    import torch

    from ye3t_amd.core.couplings import (evaluate_real_factorized_schedule_torch,
                                         generate_real_factorized_coefficient_schedule_for_labels)
    from ye3t_amd.couplings import count

    from ye3t_amd.core.couplings import generate_factorized_coefficient_schedules_by_L

    rng = np.random.default_rng(31)
    for L in sorted(generate_factorized_coefficient_schedules_by_L(*content)):
        labels = count(content=content[0], input_Ls=content[1], target_L=L).labels_for_target(L)
        sched = generate_real_factorized_coefficient_schedule_for_labels(labels)
        flat = sched.flat_arrays()
        bv = rng.normal(size=(4099, sched.basis_count, sched.block_count, flat["max_block_m_dim"]))
        got = evaluate_real_factorized_schedule_torch(torch.as_tensor(bv, device=gpu), sched)
        ref = oracle.evaluate_componentwise(bv, flat)
        assert column_rel_error(got.cpu().numpy(), ref) < 1e-12, L


def _species_rank4_spec():
    from ye3t_amd.ace.plan import ACEFeatureSpec

    # config-3 shaped (species-folded channels, l<=4, rank up to 4) at a test-sized truncation
    return ACEFeatureSpec(channel_count=44, l_max=4, nu_max=4, targets=(0,), parity="even",
                          radial_per_species=11, caps={1: (11, 0), 2: (3, 4), 3: (2, 2), 4: (1, 2)})


@pytest.mark.parametrize("cid,dtype,samples,max_slots,kernel", [
    (4, "f32", 1000, None, "interpreter"), (4, "f64", 333, None, "interpreter"), (4, "f32", 63, 250, "interpreter"),
    (4, "f32", 130, 48, "interpreter"), (2, "f64", 200, None, "interpreter"), (3, "f32", 100, None, "interpreter"),
    (3, "f64", 70, None, "interpreter"), (4, "f32", 1000, None, "generated"), (4, "f64", 333, None, "generated"),
    (4, "f32", 63, None, "generated"), (4, "f32", 65, None, "generated"), (2, "f64", 200, None, "parts"),
    (2, "f64", 65, None, "parts"), (3, "f32", 100, None, "parts"), (3, "f64", 70, None, "parts"),
    (4, "f32", 1000, None, "parts"), (4, "f64", 1, None, "parts")])
def test_product_kernel_vs_flat_oracle(gpu, cid, dtype, samples, max_slots, kernel):
    flush(f"product config {cid} {dtype} samples={samples} slots={max_slots} kernel={kernel}")
    import torch

    spec = _species_rank4_spec() if cid == 3 else W.config(cid).feature_spec
    pipe = ACEPipeline(spec, dtype, max_slots, kernel=kernel)
    assert pipe.kernel == kernel
    A = np.random.default_rng(14).normal(size=(samples, pipe.plan.a_width))
    A_dev = _t(A, dtype, gpu)
    B = pipe.product(A_dev).cpu().numpy()
    ref = oracle.ace_product_flat(A_dev.double().cpu().numpy(), pipe.plan.flat_arrays())
    err = column_rel_error(B, ref)
    flush(f"  err {err:.3e}")
    assert err < TOL[dtype]
    # determinism: bit-identical on a second run
    assert np.array_equal(B, pipe.product(A_dev).cpu().numpy())


@pytest.mark.parametrize("cid,dtype,samples,max_slots", [
    (2, "f64", 200, None), (3, "f32", 100, None), (3, "f64", 70, None), (4, "f32", 130, 48), (4, "f64", 1, None),
    (4, "f64", 129, 120)])
def test_interpreter_column_major_density(gpu, cid, dtype, samples, max_slots):
    """The term-stream interpreter on a column-major density (``transpose`` +
    ``forward_columns``) equals its row-major run bit for bit and the oracle
    within tolerance; a workspace too wide for 16-bit offsets keeps the word
    interpreter and refuses the column-major entry point."""
    flush(f"product columns config {cid} {dtype} samples={samples} slots={max_slots}")
    import torch

    spec = _species_rank4_spec() if cid == 3 else W.config(cid).feature_spec
    pipe = ACEPipeline(spec, dtype, max_slots, kernel="interpreter")
    A = np.random.default_rng(15).normal(size=(samples, pipe.plan.a_width))
    A_dev = _t(A, dtype, gpu)
    At = native.transpose(A_dev)
    assert At.shape[1] % 64 == 0 and At.shape[1] >= samples
    assert torch.equal(At[:, :samples], A_dev.t()) and bool((At[:, samples:] == 0).all())
    B_rows = pipe.product(A_dev)
    elem = 8 if dtype == "f64" else 4
    # the stream needs the workspace plus the staged density loads and output
    # slots within 64 KB of LDS: the default workspaces (48 fp64 / 96 fp32
    # slots) always take it
    if (pipe.program["workspace_slots"] + 2) * 64 * elem <= 32 * 1024:
        assert pipe.handle.uses_stream
    if not pipe.handle.uses_stream:
        with pytest.raises(RuntimeError, match="term stream"):
            pipe.handle.forward_columns(At, samples)
    else:
        B_cols = pipe.handle.forward_columns(At, samples)
        assert torch.equal(B_cols, B_rows)
    ref = oracle.ace_product_flat(A_dev.double().cpu().numpy(), pipe.plan.flat_arrays())
    err = column_rel_error(B_rows.cpu().numpy(), ref)
    flush(f"  err {err:.3e}")
    assert err < TOL[dtype]


def test_parts_and_interpreter_agree_on_config2(gpu, monkeypatch):
    """Config 2's full plan (16 810 terms) at its full 10 000 samples: the
    generated kernel in parts (the default for this plan size) against the
    term-stream interpreter, and against the flat oracle on a slice; the parts
    run in sample blocks of 512 (YE3T_PARTS_BLOCK_MB=1, 20 blocks, the last
    ragged) give the same bits as in one block."""
    flush("generated parts vs interpreter, config 2 full sample count")
    import torch

    cfg = W.config(2)
    pipe = ACEPipeline(cfg.feature_spec, "f64")
    assert pipe.kernel == "parts" and len(pipe.handle.generated_parts) > 1
    A = torch.as_tensor(np.random.default_rng(21).normal(size=(10000, pipe.plan.a_width)), device=gpu)
    B_parts = pipe.product(A)
    pipe.handle.select(use_interpreter=True)
    B_int = pipe.handle.forward(A)
    pipe.handle.select(use_interpreter=False)
    torch.cuda.synchronize()
    err = column_rel_error(B_parts.cpu().numpy(), B_int.cpu().numpy())
    flush(f"  parts vs interpreter {err:.3e}")
    assert err < TOL["f64"]
    ref = oracle.ace_product_flat(A[:96].cpu().numpy(), pipe.plan.flat_arrays())
    assert column_rel_error(B_parts[:96].cpu().numpy(), ref) < TOL["f64"]
    monkeypatch.setenv("YE3T_PARTS_BLOCK_MB", "1")
    assert torch.equal(pipe.product(A), B_parts)
    assert torch.equal(pipe.product(A[:1000]), B_parts[:1000])


def test_generated_and_interpreter_agree_on_config4(gpu):
    flush("generated vs interpreter, config 4 full sample count")
    import torch

    cfg = W.config(4)
    pipe = ACEPipeline(cfg.feature_spec, "f32", kernel="generated")
    A = torch.randn((800000, 16), dtype=torch.float32, device=gpu)
    B_gen = pipe.product(A)
    pipe.handle.select(use_interpreter=True)
    B_int = pipe.product(A)
    torch.cuda.synchronize()
    rms = B_int.double().pow(2).mean(dim=0).sqrt().clamp_min(1e-30)
    err = ((B_gen.double() - B_int.double()).abs().amax(dim=0) / rms).max().item()
    flush(f"  err {err:.3e}")
    assert err < 2e-5


@pytest.mark.parametrize("cid,dtype,atoms", [(4, "f32", 257), (2, "f64", 257), (3, "f64", 67), (3, "f32", 67),
                                              (5, "f32", 33)])
def test_end_to_end_small(gpu, cid, dtype, atoms):
    """Full feature plans of every density configuration, on a few seeded atoms."""
    flush(f"end to end config {cid} {dtype} atoms={atoms}")
    cfg = W.config(cid, atom_count=atoms)
    inp = cfg.density.generate()
    pipe = ACEPipeline(cfg.feature_spec, dtype, accumulate=cfg.accumulate if dtype == "f32" else None,
                       density=cfg.density_dtype if dtype == "f32" else None)
    flush(f"  plan built: {pipe.feature_count} features, kernel {pipe.kernel}, accumulate {pipe.accumulate}, "
          f"density {pipe.density_dtype}")
    A, B = pipe.forward(to_device_inputs(inp, dtype, gpu), channelwise=cfg.channelwise)
    A_ref = oracle.ace_density(rounded_inputs(inp, dtype))
    assert column_rel_error(A.cpu().numpy().reshape(atoms, -1), A_ref.reshape(atoms, -1)) < TOL[dtype]
    rows = A_ref.reshape(-1, pipe.plan.a_width)
    B_ref = oracle.ace_product_flat(rows, pipe.plan.flat_arrays())
    err = column_rel_error(B.cpu().numpy(), B_ref)
    flush(f"  err {err:.3e}")
    assert err < TOL[dtype]


@pytest.mark.parametrize("cid,dtype,atoms,kernel", [(4, "f32", 257, "auto"), (2, "f64", 129, "auto"),
                                                   (3, "f32", 67, "auto"), (2, "f64", 129, "interpreter")])
def test_linear_readout(gpu, cid, dtype, atoms, kernel):
    """Fused (generated plans, whole or in parts) and block-materialised
    (interpreted plans) readouts vs B_ref @ w + bias."""
    flush(f"linear readout config {cid} {dtype} atoms={atoms} kernel={kernel}")
    import torch

    cfg = W.config(cid, atom_count=atoms)
    inp = cfg.density.generate()
    f32 = dtype == "f32"
    pipe = ACEPipeline(cfg.feature_spec, dtype, kernel=kernel, accumulate=cfg.accumulate if f32 else None,
                       density=cfg.density_dtype if f32 and kernel != "interpreter" else None)
    A = pipe.density(to_device_inputs(inp, dtype, gpu))
    rows = A.reshape(-1, pipe.plan.a_width)
    F = pipe.feature_count
    rng = np.random.default_rng(40 + cid)
    w = rng.normal(size=F)
    got = pipe.linear(rows, torch.as_tensor(w, device=gpu), 0.37)
    backend = pipe.last_linear_backend
    flush(f"  backend {backend}")
    assert backend == {"generated": "fused_generated", "parts": "fused_parts"}.get(pipe.kernel, "materialized_blocks")
    A_ref = oracle.ace_density(rounded_inputs(inp, dtype)).reshape(-1, pipe.plan.a_width)
    ref = oracle.linear_readout(oracle.ace_product_flat(A_ref, pipe.plan.flat_arrays()), w, 0.37)
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(got.cpu().double().numpy() - ref))) / rms
    flush(f"  err {err:.3e}")
    assert err < TOL[dtype]
    # small sample blocks on the materialised path agree with one block
    if backend == "materialized_blocks":
        again = pipe.linear(rows, torch.as_tensor(w, device=gpu), 0.37, block_bytes=F * 8 * 37)
        assert torch.equal(again, got)
    # a one-hot weight reads one feature column exactly
    B = pipe.product(rows)
    for k in (0, F // 2, F - 1):
        e = np.zeros(F)
        e[k] = 1.0
        col = pipe.linear(rows, torch.as_tensor(e, device=gpu), 0.0)
        assert torch.equal(col, B[:, k])


@pytest.mark.parametrize("dtype,accumulate,density,tol", [
    ("f32", "f64", "f64", 1e-12), ("f64", "f64", "f64", 1e-12), ("f32", "f32", "f32", 2e-5),
    ("f32", "f64", "f32", None)])
def test_product_adjoint(gpu, dtype, accumulate, density, tol):
    """gA = J(A)^T gB from the generated adjoint kernel vs the oracle's reverse
    mode (config 4 plan).  With an fp32 density and fp64 arithmetic (tol None),
    each gA value is the oracle's rounded once to fp32."""
    flush(f"product adjoint storage {dtype} accumulate {accumulate} density {density}")
    import torch

    pipe = ACEPipeline(W.config(4).feature_spec, dtype, accumulate=accumulate, density=density)
    rng = np.random.default_rng(31)
    S = 4112  # 64 full tiles and a partial one
    a_t = torch.float64 if density == "f64" else torch.float32
    g_t = torch.float64 if dtype == "f64" else torch.float32
    A = torch.as_tensor(rng.normal(size=(S, pipe.plan.a_width)), dtype=a_t)
    gB = torch.as_tensor(rng.normal(size=(S, pipe.feature_count)), dtype=g_t)
    gA = pipe.product_adjoint(A.to(gpu), gB.to(gpu))
    assert gA.dtype == a_t and tuple(gA.shape) == (S, pipe.plan.a_width)
    ref = oracle.ace_product_flat_adjoint(A.double().numpy(), gB.double().numpy(), pipe.plan.flat_arrays())
    if tol is None:
        ratio = fp32_rounding_ratio(gA.cpu().double().numpy(), ref)
        flush(f"  error / fp32 rounding bound {ratio:.3f}")
        assert ratio <= 1.0
    else:
        err = column_rel_error(gA.cpu().double().numpy(), ref)
        flush(f"  err {err:.3e}")
        assert err < tol
    # linear in the feature gradient: doubling gB doubles every intermediate exactly
    assert torch.equal(pipe.product_adjoint(A.to(gpu), 2 * gB.to(gpu)), 2 * gA)


@pytest.mark.parametrize("cid,dtype,accumulate,samples,tol", [
    (2, "f64", "f64", 150, 1e-12), (3, "f64", "f64", 70, 1e-12), (3, "f32", "f32", 70, 2e-5),
    (4, "f32", "f64", 4112, 1e-12), (4, "f32", "f32", 1000, 2e-5)])
def test_stream_product_adjoint(gpu, cid, dtype, accumulate, samples, tol):
    """gA = J(A)^T gB by the term stream's reverse mode (interpreter plans) vs the
    oracle's reverse mode; row-major and column-major densities give the same
    bits, doubling gB doubles gA exactly, and a rerun gives the same bits."""
    flush(f"stream adjoint config {cid} storage {dtype} accumulate {accumulate} samples {samples}")
    import torch

    spec = _species_rank4_spec() if cid == 3 else W.config(cid).feature_spec
    pipe = ACEPipeline(spec, dtype, kernel="interpreter", accumulate=accumulate)
    rng = np.random.default_rng(41 + cid)
    a_t = torch.float64 if accumulate == "f64" else torch.float32
    g_t = torch.float64 if dtype == "f64" else torch.float32
    A = torch.as_tensor(rng.normal(size=(samples, pipe.plan.a_width)), dtype=a_t).to(gpu)
    gB = torch.as_tensor(rng.normal(size=(samples, pipe.feature_count)), dtype=g_t).to(gpu)
    gA = pipe.product_adjoint(A, gB)
    assert pipe.last_adjoint_backend == "stream"
    assert gA.dtype == a_t and tuple(gA.shape) == (samples, pipe.plan.a_width)
    ref = oracle.ace_product_flat_adjoint(A.double().cpu().numpy(), gB.double().cpu().numpy(),
                                          pipe.plan.flat_arrays())
    err = column_rel_error(gA.cpu().double().numpy(), ref)
    flush(f"  err {err:.3e}")
    assert err < tol
    assert torch.equal(pipe._adjoint_handle.adjoint_stream(A, gB), gA)  # row-major density
    assert torch.equal(pipe.product_adjoint(A, 2 * gB), 2 * gA)
    assert torch.equal(pipe.product_adjoint(A, gB), gA)


@pytest.mark.parametrize("cid,dtype,accumulate,samples,tol", [
    (2, "f64", "f64", 150, 1e-12), (2, "f64", "f64", 1000, 1e-12), (3, "f64", "f64", 70, 1e-12),
    (3, "f32", "f32", 70, 2e-5), (4, "f32", "f64", 4112, None), (4, "f64", "f64", 1, 1e-12)])
def test_parts_product_adjoint(gpu, cid, dtype, accumulate, samples, tol):
    """gA = J(A)^T gB by the generated reverse mode in parts (partial rows per
    chunk, fixed-order reduction) vs the oracle's reverse mode; doubling gB
    doubles gA exactly, a rerun and a run in several sample blocks give the
    same bits.  With an fp32 density (tol None) each value is the oracle's
    rounded once to fp32."""
    flush(f"parts adjoint config {cid} storage {dtype} accumulate {accumulate} samples {samples}")
    import torch

    spec = _species_rank4_spec() if cid == 3 else W.config(cid).feature_spec
    density = "f32" if tol is None else None
    pipe = ACEPipeline(spec, dtype, kernel="parts", accumulate=accumulate, density=density)
    rng = np.random.default_rng(51 + cid)
    a_t = torch.float32 if density == "f32" or accumulate == "f32" else torch.float64
    g_t = torch.float64 if dtype == "f64" else torch.float32
    A = torch.as_tensor(rng.normal(size=(samples, pipe.plan.a_width)), dtype=a_t).to(gpu)
    gB = torch.as_tensor(rng.normal(size=(samples, pipe.feature_count)), dtype=g_t).to(gpu)
    gA = pipe.product_adjoint(A, gB)
    assert pipe.last_adjoint_backend == "parts"
    assert gA.dtype == a_t and tuple(gA.shape) == (samples, pipe.plan.a_width)
    ref = oracle.ace_product_flat_adjoint(A.double().cpu().numpy(), gB.double().cpu().numpy(),
                                          pipe.plan.flat_arrays())
    if tol is None:
        ratio = fp32_rounding_ratio(gA.cpu().double().numpy(), ref)
        flush(f"  error / fp32 rounding bound {ratio:.3f}")
        assert ratio <= 1.0
    else:
        err = column_rel_error(gA.cpu().double().numpy(), ref)
        flush(f"  err {err:.3e}")
        assert err < tol
    assert torch.equal(pipe.product_adjoint(A, 2 * gB), 2 * gA)
    assert torch.equal(pipe.product_adjoint(A, gB), gA)
    blocked = pipe._adjoint_parts(A, gB, None, block_bytes=pipe._adjoint_rows * 8 * 64)
    assert torch.equal(blocked, gA)


@pytest.fixture(scope="module")
def config3_plan():
    from ye3t_amd.ace.plan import ProductPlan

    flush("building the config-3 product plan on the host (about a minute)")
    return ProductPlan(W.config(3).feature_spec)


@pytest.mark.parametrize("dtype,tol", [("f64", 1e-12), ("f32", 2e-5)])
def test_config3_adjoint_runs_in_parts(gpu, config3_plan, dtype, tol):
    """The benchmark's own config-3 plan with the kernel chosen automatically
    takes its reverse mode in parts (the default chunk sizes, precompiled),
    matches the oracle's reverse mode, and gives the same bits in small sample
    blocks."""
    import torch

    flush(f"config-3 adjoint in parts, {dtype}")
    pipe = ACEPipeline(W.config(3).feature_spec, dtype, plan=config3_plan)
    assert pipe.kernel == "parts"
    real = torch.float64 if dtype == "f64" else torch.float32
    rng = np.random.default_rng(53)
    samples = 130
    A = torch.as_tensor(rng.normal(size=(samples, pipe.plan.a_width)), dtype=real).to(gpu)
    gB = torch.as_tensor(rng.normal(size=(samples, pipe.feature_count)), dtype=real).to(gpu)
    gA = pipe.product_adjoint(A, gB)
    assert pipe.last_adjoint_backend == "parts"
    ref = oracle.ace_product_flat_adjoint(A.double().cpu().numpy(), gB.double().cpu().numpy(),
                                          pipe.plan.flat_arrays())
    err = column_rel_error(gA.cpu().double().numpy(), ref)
    flush(f"  err {err:.3e}")
    assert err < tol
    elem = 8 if dtype == "f64" else 4
    blocked = pipe._adjoint_parts(A, gB, None, block_bytes=pipe._adjoint_rows * elem * 64)
    assert torch.equal(blocked, gA)


def test_product_adjoint_needs_a_term_stream(gpu, monkeypatch):
    """A workspace too wide for the term stream has no device adjoint; one whose
    forward stream fits 64 KB of LDS but whose reverse mode (values and
    gradients) does not is refused by the library before any launch."""
    import torch

    monkeypatch.setenv("YE3T_ADJOINT_SLOTS", "130")
    pipe = ACEPipeline(W.config(4).feature_spec, "f64", 130, kernel="interpreter")
    assert not pipe.handle.uses_stream
    A = torch.zeros((3, pipe.plan.a_width), dtype=torch.float64, device=gpu)
    gB = torch.zeros((3, pipe.feature_count), dtype=torch.float64, device=gpu)
    with pytest.raises(NotImplementedError):
        pipe.product_adjoint(A, gB)
    monkeypatch.setenv("YE3T_ADJOINT_SLOTS", "120")
    pipe = ACEPipeline(W.config(4).feature_spec, "f64", 120, kernel="interpreter")
    assert pipe.handle.uses_stream  # records take no LDS: the forward stream fits
    with pytest.raises(RuntimeError, match="64 KB"):
        pipe.product_adjoint(A, gB)


@pytest.mark.parametrize("dtype", ["f32", "f64"])
def test_rows_dot(gpu, dtype):
    flush(f"rows_dot {dtype}")
    import torch

    tdt = torch.float64 if dtype == "f64" else torch.float32
    rng = np.random.default_rng(9)
    for S, F in ((1, 1), (7, 161), (1001, 3273), (5, 0)):
        B = torch.as_tensor(rng.normal(size=(S, F)), dtype=tdt)
        w = torch.as_tensor(rng.normal(size=F), dtype=tdt)
        got = native.rows_dot(B.to(gpu), w.to(gpu), -1.5).cpu().double().numpy()
        ref = oracle.linear_readout(B.double().numpy(), w.double().numpy(), -1.5)
        scale = max(1.0, float(np.sqrt(np.mean(ref * ref))))
        assert np.max(np.abs(got - ref)) / scale < (1e-13 if dtype == "f64" else 1e-6)


@pytest.mark.parametrize("kernel", ["interpreter", "generated", "parts"])
def test_fp64_plan_with_fp32_features(gpu, kernel):
    """accumulate=f64 with f32 storage: only the final store rounds."""
    flush(f"mixed precision product, kernel {kernel}")
    import torch

    pipe = ACEPipeline(W.config(4).feature_spec, "f32", kernel=kernel, accumulate="f64")
    A = np.random.default_rng(15).normal(size=(300, pipe.plan.a_width))
    B = pipe.product(torch.as_tensor(A, dtype=torch.float64, device=gpu))
    assert B.dtype == torch.float32
    ref = oracle.ace_product_flat(A, pipe.plan.flat_arrays())
    # per column, relative to the column RMS: the fp32 rounding of the result only
    err = column_rel_error(B.cpu().numpy(), ref)
    flush(f"  err {err:.3e}")
    assert err < 1e-6


@pytest.mark.parametrize("mode", ["single", "species", "features"])
def test_fp64_density_of_fp32_inputs(gpu, mode):
    """out_dtype=f64 with f32 inputs: the fp64 density of the fp32-rounded data."""
    flush(f"fp64 density of fp32 inputs, {mode}")
    import torch

    inp = _ragged_workload(mode)
    dev = to_device_inputs(inp, "f32", gpu)
    A = native.ace_density_forward(
        dev["edge_vectors"], dev["row_offsets"], dev["neighbors"], atom_count=inp["atom_count"],
        channel_count=inp["channel_count"], n_max=inp["n_max"], l_max=inp["l_max"], cutoff=inp["cutoff"],
        lam=inp["lambda"], epsilon=inp["epsilon"], species=dev.get("species"), node_features=dev.get("node_features"),
        radial_mix=dev.get("radial_mix"), out_dtype=torch.float64)
    assert A.dtype == torch.float64
    ref = oracle.ace_density(rounded_inputs(inp, "f32"))
    N = inp["atom_count"]
    err = column_rel_error(A.cpu().numpy().reshape(N, -1), ref.reshape(N, -1))
    flush(f"  err {err:.3e}")
    assert err < TOL["f64"]


def _random_csr_workload(mode, atoms, max_degree, seed, n_max=8, l_max=3, channels=16):
    """Random degrees in [0, max_degree] (empty atoms included) for the compiled fp64 MFMA shapes."""
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, max_degree + 1, atoms)
    counts[0] = 0
    counts[-1] = 0
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    E = int(offsets[-1])
    vec = rng.normal(size=(E, 3))
    vec = vec / np.linalg.norm(vec, axis=1, keepdims=True) * rng.uniform(0.8, 5.2, (E, 1))  # some beyond cutoff
    inp = {"atom_count": atoms, "edge_count": E, "centers": np.repeat(np.arange(atoms), counts),
           "row_offsets": offsets, "neighbors": rng.integers(0, atoms, E), "edge_vectors": vec, "n_max": n_max,
           "l_max": l_max, "cutoff": 5.0, "lambda": W.LAMBDA, "epsilon": 1e-12, "species": None,
           "node_features": None, "radial_mix": None}
    if mode == "features":
        inp.update(channel_count=channels, node_features=rng.normal(size=(atoms, channels)),
                   radial_mix=rng.normal(size=(channels, n_max + 1)) / 3)
    else:
        inp.update(channel_count=1)
    return inp


@pytest.mark.parametrize("storage", ["f32", "f64"])
def test_channel_density_aligned_rows_and_cutoff_ties(gpu, storage):
    """The channel kernel's unmasked form (atom ends on k-block boundaries, with
    empty atoms between some of them, which send those chunks to the masked
    form) and edges at exactly the cutoff distance and one ulp either side of it."""
    flush(f"channel density aligned rows and cutoff ties {storage}")
    inp = _random_csr_workload("features", 400, 64, 77)
    rng = np.random.default_rng(78)
    counts = 4 * rng.integers(0, 17, 400)
    counts[::7] = 24
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    E = int(offsets[-1])
    vec = rng.normal(size=(E, 3))
    vec = vec / np.linalg.norm(vec, axis=1, keepdims=True) * rng.uniform(0.8, 5.2, (E, 1))
    ft = np.float32 if storage == "f32" else np.float64
    c = ft(5.0)
    for k, v in enumerate([(c, 0, 0), (0, -c, 0), (0, 0, c), (np.nextafter(c, ft(6)), 0, 0),
                           (0, np.nextafter(c, ft(4)), 0), (0, 0, -np.nextafter(c, ft(6)))]):
        vec[k::37] = np.asarray(v, dtype=np.float64)
    inp.update(edge_count=E, row_offsets=offsets, centers=np.repeat(np.arange(400), counts),
               neighbors=rng.integers(0, 400, E), edge_vectors=vec)
    dev = to_device_inputs(inp, storage, gpu)
    ref = oracle.ace_density(rounded_inputs(inp, storage)).reshape(400, -1)
    import torch

    A = native.ace_density_forward(
        dev["edge_vectors"], dev["row_offsets"], dev["neighbors"], atom_count=400, channel_count=16, n_max=8,
        l_max=3, cutoff=5.0, lam=inp["lambda"], epsilon=inp["epsilon"], node_features=dev["node_features"],
        radial_mix=dev["radial_mix"], out_dtype=torch.float64)
    assert native.last_density_kernel() == "ace_density_channel16_kernel"
    err = column_rel_error(A.cpu().numpy().reshape(400, -1), ref)
    flush(f"  err {err:.3e}")
    assert err < TOL[storage]
    assert np.all(A.cpu().numpy()[counts == 0] == 0)


@pytest.mark.parametrize("waves", [None, "1", "5", "64"])
@pytest.mark.parametrize("mode,shape", [("features", (8, 3)), ("single", (8, 3)), ("single", (10, 4)),
                                        ("single", (12, 6))])
@pytest.mark.parametrize("storage", ["f32", "f64"])
def test_fp64_mfma_density_random_csr(gpu, monkeypatch, mode, shape, storage, waves):
    """The fp64 matrix-core density (per-atom MFMA over CSR k-blocks) on ragged CSR rows."""
    flush(f"fp64 MFMA density {mode} n_max,l_max={shape} storage {storage} waves={waves}")
    import torch

    if waves is not None:
        monkeypatch.setenv("YE3T_DENSITY_WAVES", waves)
    inp = _random_csr_workload(mode, 301, 150, 31, n_max=shape[0], l_max=shape[1])
    dev = to_device_inputs(inp, storage, gpu)
    N = inp["atom_count"]
    ref = oracle.ace_density(rounded_inputs(inp, storage)).reshape(N, -1)
    outs = {}
    # (YE3T_DENSITY_MFMA64, YE3T_DENSITY_MIX_MFMA): fp64 MFMA kernel (default) / VALU kernel
    kernels = {"mfma64": ("1", "1"), "valu": ("0", "1")}
    if mode == "features":
        kernels["mix-on-valu"] = ("1", "0")  # generic MFMA kernel with the radial mix on VALU
    for mfma, (flag64, flagmix) in kernels.items():
        monkeypatch.setenv("YE3T_DENSITY_MFMA64", flag64)
        monkeypatch.setenv("YE3T_DENSITY_MIX_MFMA", flagmix)
        A = native.ace_density_forward(
            dev["edge_vectors"], dev["row_offsets"], dev["neighbors"], atom_count=N,
            channel_count=inp["channel_count"], n_max=inp["n_max"], l_max=inp["l_max"], cutoff=inp["cutoff"],
            lam=inp["lambda"], epsilon=inp["epsilon"], node_features=dev.get("node_features"),
            radial_mix=dev.get("radial_mix"), out_dtype=torch.float64)
        outs[mfma] = A.cpu().numpy().reshape(N, -1)
        err = column_rel_error(outs[mfma], ref)
        flush(f"  mfma64={mfma} ({native.last_density_kernel()}) err {err:.3e}")
        if mfma == "mfma64":
            expect = "ace_density_channel16_kernel" if mode == "features" else "ace_density_mfma64_kernel"
            assert native.last_density_kernel() == expect
        assert err < TOL["f64"]
    # empty atoms are exact zeros
    empty = np.diff(inp["row_offsets"]) == 0
    for key in ("mfma64", "mix-on-valu"):
        if key in outs:
            assert not np.any(outs[key][empty])


@pytest.mark.parametrize("mode,shape", [("features", (8, 3)), ("single", (8, 3)), ("single", (12, 6))])
def test_fp32_density_accumulated_in_fp64(gpu, mode, shape):
    """accumulate_dtype=f64 with an fp32 A: the fp64 matrix-core accumulation
    rounded once, i.e. exactly the fp64 density's values rounded to fp32."""
    flush(f"fp32 density accumulated in fp64, {mode} n_max,l_max={shape}")
    import torch

    inp = _random_csr_workload(mode, 301, 150, 32, n_max=shape[0], l_max=shape[1])
    dev = to_device_inputs(inp, "f32", gpu)
    N = inp["atom_count"]
    kw = dict(atom_count=N, channel_count=inp["channel_count"], n_max=inp["n_max"], l_max=inp["l_max"],
              cutoff=inp["cutoff"], lam=inp["lambda"], epsilon=inp["epsilon"],
              node_features=dev.get("node_features"), radial_mix=dev.get("radial_mix"))
    A64 = native.ace_density_forward(dev["edge_vectors"], dev["row_offsets"], dev["neighbors"],
                                     out_dtype=torch.float64, **kw)
    A32 = native.ace_density_forward(dev["edge_vectors"], dev["row_offsets"], dev["neighbors"],
                                     out_dtype=torch.float32, accumulate_dtype=torch.float64, **kw)
    assert A32.dtype == torch.float32
    assert torch.equal(A32, A64.to(torch.float32))
    ref = oracle.ace_density(rounded_inputs(inp, "f32")).reshape(N, -1)
    assert column_rel_error(A32.cpu().numpy().reshape(N, -1), ref) < 1e-6


def test_fp32_density_accumulated_in_fp64_needs_an_mfma_shape(gpu):
    """A shape no fp64 matrix-core kernel covers (more than 16 species): the
    mixed precision is refused."""
    import torch

    inp = _ragged_workload("species")
    rng = np.random.default_rng(5)
    inp.update(channel_count=20, species=rng.integers(0, 20, inp["atom_count"]).astype(np.int32))
    dev = to_device_inputs(inp, "f32", gpu)
    with pytest.raises(RuntimeError, match="fp64 matrix-core shapes"):
        native.ace_density_forward(
            dev["edge_vectors"], dev["row_offsets"], dev["neighbors"], atom_count=inp["atom_count"],
            channel_count=inp["channel_count"], n_max=inp["n_max"], l_max=inp["l_max"], cutoff=inp["cutoff"],
            lam=inp["lambda"], species=dev["species"], out_dtype=torch.float32, accumulate_dtype=torch.float64)


def _species_workload(atoms, species, n_max, l_max, seed, max_degree=150):
    """Ragged rows for the species kernel: random degrees in [0, max_degree]
    (rows of more than 64 edges take several windows), a run of 40 empty atoms
    (more than one chunk's worth of them), single-edge rows, and edges beyond
    the cutoff."""
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, max_degree + 1, atoms)
    counts[:3] = 0
    counts[10:50] = 0
    counts[50:60] = 1
    counts[-1] = 0
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    E = int(offsets[-1])
    vec = rng.normal(size=(E, 3))
    vec = vec / np.linalg.norm(vec, axis=1, keepdims=True) * rng.uniform(0.8, 5.2, (E, 1))
    return {"atom_count": atoms, "edge_count": E, "centers": np.repeat(np.arange(atoms), counts),
            "row_offsets": offsets, "neighbors": rng.integers(0, atoms, E), "edge_vectors": vec, "n_max": n_max,
            "l_max": l_max, "cutoff": 5.0, "lambda": W.LAMBDA, "epsilon": 1e-12, "channel_count": species,
            "species": rng.integers(0, species, atoms).astype(np.int32), "node_features": None, "radial_mix": None}


@pytest.mark.parametrize("waves", [None, "1", "7"])
@pytest.mark.parametrize("species,shape,max_degree", [(4, (10, 4), 150), (8, (12, 6), 150), (16, (15, 8), 90),
                                                      (3, (0, 0), 70), (5, (3, 1), 20), (8, (12, 6), 48)])
@pytest.mark.parametrize("storage", ["f32", "f64"])
def test_species_density_on_the_matrix_cores(gpu, monkeypatch, species, shape, max_degree, storage, waves):
    """The species kernel (edges grouped by (atom, species), one fp64 MFMA
    product per group) against the oracle and the VALU kernel, on ragged rows
    (empty runs, windows of long rows), every CT instantiation from l_max 0 to
    8, and with the fp32 density accumulated in fp64 equal to the fp64 density
    rounded once."""
    flush(f"species density S={species} n_max,l_max={shape} deg<={max_degree} {storage} waves={waves}")
    import torch

    if waves is not None:
        monkeypatch.setenv("YE3T_DENSITY_WAVES", waves)
    inp = _species_workload(301, species, shape[0], shape[1], 40 + species, max_degree)
    dev = to_device_inputs(inp, storage, gpu)
    N = inp["atom_count"]
    kw = dict(atom_count=N, channel_count=species, n_max=shape[0], l_max=shape[1], cutoff=5.0, lam=inp["lambda"],
              epsilon=inp["epsilon"], species=dev["species"])
    ref = oracle.ace_density(rounded_inputs(inp, storage)).reshape(N, -1)
    A = native.ace_density_forward(dev["edge_vectors"], dev["row_offsets"], dev["neighbors"],
                                   out_dtype=torch.float64, **kw)
    assert native.last_density_kernel() == "ace_density_species_kernel"
    got = A.cpu().numpy().reshape(N, -1)
    err = column_rel_error(got, ref)
    monkeypatch.setenv("YE3T_DENSITY_SPECIES_MFMA", "0")
    V = native.ace_density_forward(dev["edge_vectors"], dev["row_offsets"], dev["neighbors"],
                                   out_dtype=torch.float64, **kw)
    assert native.last_density_kernel() == "ace_density_kernel"
    monkeypatch.delenv("YE3T_DENSITY_SPECIES_MFMA")
    err_valu = column_rel_error(got, V.cpu().numpy().reshape(N, -1))
    flush(f"  err {err:.3e} (vs VALU kernel {err_valu:.3e})")
    assert err < TOL["f64"] and err_valu < TOL["f64"]
    empty = np.diff(inp["row_offsets"]) == 0
    assert not np.any(got[empty])
    # a species absent from an atom's neighbours leaves an exact zero block
    blocks = got.reshape(N, species, -1)
    sp_of = inp["species"][inp["neighbors"]]
    for i in (60, 100, 200):
        present = set(sp_of[inp["row_offsets"][i]:inp["row_offsets"][i + 1]].tolist())
        for s in range(species):
            if s not in present:
                assert not np.any(blocks[i, s])
    if storage == "f32":
        A32 = native.ace_density_forward(dev["edge_vectors"], dev["row_offsets"], dev["neighbors"],
                                         out_dtype=torch.float32, accumulate_dtype=torch.float64, **kw)
        assert torch.equal(A32, A.to(torch.float32))
        A32b = native.ace_density_forward(dev["edge_vectors"], dev["row_offsets"], dev["neighbors"], **kw)
        assert A32b.dtype == torch.float32 and torch.equal(A32b, A32)


def test_density_rejects_bad_indices_before_launch(gpu):
    """Out-of-range neighbours and inconsistent CSR offsets raise on the host."""
    import torch

    inp = _random_csr_workload("features", 50, 20, 33)
    dev = to_device_inputs(inp, "f32", gpu)
    kw = dict(atom_count=50, channel_count=16, n_max=8, l_max=3, cutoff=5.0, lam=W.LAMBDA,
              node_features=dev["node_features"], radial_mix=dev["radial_mix"])
    bad = dev["neighbors"].clone()
    bad[-1] = 50
    with pytest.raises(ValueError, match="neighbor index"):
        native.ace_density_forward(dev["edge_vectors"], dev["row_offsets"], bad, **kw)
    offs = dev["row_offsets"].clone()
    offs[-1] -= 1
    with pytest.raises(ValueError, match="row_offsets"):
        native.ace_density_forward(dev["edge_vectors"], offs, dev["neighbors"], **kw)
    torch.cuda.synchronize()


@pytest.mark.parametrize("cid,dtype", [(2, "f64"), (3, "f32")])
def test_stream_multi_tile_workgroups(gpu, monkeypatch, cid, dtype):
    """Four 64-sample tiles per stream workgroup (the per-tile record re-read and
    the next-tile density prefetch), five tiles with a partial last one:
    row-major, column-major and the oracle agree, and the reverse mode matches
    the oracle's and reruns to the same bits."""
    flush(f"stream with 4 tiles per workgroup, config {cid} {dtype}")
    import torch

    monkeypatch.setenv("YE3T_STREAM_TILES", "4")
    spec = _species_rank4_spec() if cid == 3 else W.config(cid).feature_spec
    pipe = ACEPipeline(spec, dtype, kernel="interpreter")
    assert pipe.handle.uses_stream
    samples = 4 * 64 + 37
    A = _t(np.random.default_rng(17).normal(size=(samples, pipe.plan.a_width)), dtype, gpu)
    B_rows = pipe.handle.forward(A)
    B_cols = pipe.product(A)  # column-major density
    assert torch.equal(B_rows, B_cols)
    ref = oracle.ace_product_flat(A.double().cpu().numpy(), pipe.plan.flat_arrays())
    err = column_rel_error(B_rows.cpu().numpy(), ref)
    flush(f"  forward err {err:.3e}")
    assert err < TOL[dtype]
    g_t = torch.float64 if dtype == "f64" else torch.float32
    gB = torch.as_tensor(np.random.default_rng(18).normal(size=(samples, pipe.feature_count)), dtype=g_t,
                         device=gpu)
    gA = pipe.product_adjoint(A, gB)
    gref = oracle.ace_product_flat_adjoint(A.double().cpu().numpy(), gB.double().cpu().numpy(),
                                           pipe.plan.flat_arrays())
    err = column_rel_error(gA.cpu().double().numpy(), gref)
    flush(f"  adjoint err {err:.3e}")
    assert err < TOL[dtype]
    assert torch.equal(pipe.product_adjoint(A, gB), gA)


@pytest.mark.parametrize("waves", ["1", "2"])
@pytest.mark.parametrize("accumulate", ["f32", "f64"])
def test_persistent_generated_kernel_tiles_and_misaligned_output(gpu, monkeypatch, accumulate, waves):
    """Persistent plan-specialised kernel: partial last tiles, more tiles than resident
    workgroups, and an output view that is not 16-byte aligned (generic kernel runs);
    one or two waves per tile."""
    flush(f"persistent generated kernel, accumulate {accumulate}, waves {waves}")
    import torch

    monkeypatch.setenv("YE3T_PRODUCT_WAVES", waves)
    pipe = ACEPipeline(W.config(4).feature_spec, "f32", kernel="generated", accumulate=accumulate)
    assert pipe.handle.generated["threads"] == 64 * int(waves)
    assert pipe.handle.generated.get("persistent")
    real = torch.float64 if accumulate == "f64" else torch.float32
    _check_persistent_tiles(gpu, pipe, real, accumulate)


@pytest.mark.parametrize("samples", [1, 65, 4097, 200003])
def test_fp32_density_with_fp64_arithmetic(gpu, samples):
    """An fp32 density read into fp64 arithmetic by the persistent generated
    kernel (config 4's mode): equals the fp64 plan on the same fp32 values to
    the fp32 rounding of B, and the generic kernels refuse such a plan."""
    flush(f"fp32 density, fp64 arithmetic, samples {samples}")
    import torch

    spec = W.config(4).feature_spec
    mixed = ACEPipeline(spec, "f32", accumulate="f64", density="f32")
    wide = ACEPipeline(spec, "f32", accumulate="f64")
    assert mixed.kernel == "generated" and mixed.handle.generated["in_dtype"] == "f32"
    A32 = torch.as_tensor(np.random.default_rng(samples).normal(size=(samples, mixed.plan.a_width)),
                          dtype=torch.float32, device=gpu)
    B_mixed = mixed.product(A32)
    B_wide = wide.product(A32.double())
    assert torch.equal(B_mixed, B_wide)  # same fp64 arithmetic on the same values
    if samples <= 4097:
        ref = oracle.ace_product_flat(A32.double().cpu().numpy(), mixed.plan.flat_arrays())
        assert column_rel_error(B_mixed.cpu().numpy(), ref) < 1e-5
    # the word and stream interpreters read densities of the plan's dtype only
    mixed.handle.select(use_interpreter=True)
    with pytest.raises(RuntimeError, match="generated kernel only"):
        mixed.product(A32)
    mixed.handle.select(use_interpreter=False)
    flat = torch.empty(samples * mixed.feature_count + 1, dtype=torch.float32, device=gpu)
    with pytest.raises(RuntimeError, match="generated kernel only"):
        mixed.product(A32, out=flat[1:].view(samples, mixed.feature_count))  # misaligned B: no persistent kernel


def _check_persistent_tiles(gpu, pipe, real, accumulate):
    import torch

    for samples in (1, 64, 65, 4097, 200003):
        A = torch.as_tensor(np.random.default_rng(samples).normal(size=(samples, pipe.plan.a_width)), dtype=real,
                            device=gpu)
        ref = oracle.ace_product_flat(A.double().cpu().numpy(), pipe.plan.flat_arrays()) if samples <= 4097 else None
        B = pipe.product(A)
        flat = torch.empty(samples * pipe.feature_count + 1, dtype=torch.float32, device=gpu)
        B_mis = flat[1:].view(samples, pipe.feature_count)
        pipe.product(A, out=B_mis)
        torch.cuda.synchronize()
        got, got_mis = B.cpu().numpy(), B_mis.cpu().numpy()
        if ref is not None:
            err = column_rel_error(got, ref)
            flush(f"  samples={samples} err {err:.3e}")
            # fp64 arithmetic: only the fp32 rounding of each value, up to ~20x the column RMS
            assert err < (1e-5 if accumulate == "f64" else TOL["f32"])
        # the generic kernel on the misaligned view agrees with the persistent kernel
        assert column_rel_error(got_mis, got.astype(np.float64)) < (1e-6 if accumulate == "f64" else 1e-5)


@pytest.mark.parametrize("cid,dtype,samples", [(4, "f32", 300), (2, "f64", 150)])
def test_pipeline_from_a_saved_plan(gpu, tmp_path, cid, dtype, samples):
    """A plan written to disk and loaded back runs to the same bits (generated
    kernel for config 4, term-stream interpreter for config 2)."""
    flush(f"saved plan config {cid} {dtype}")
    import torch

    from ye3t_amd.ace import plan_io

    spec = W.config(cid).feature_spec
    pipe = ACEPipeline(spec, dtype)
    path = tmp_path / "plan.json"
    plan_io.save_plan(pipe.plan, path)
    loaded = ACEPipeline(spec, dtype, plan=plan_io.load_plan(path))
    assert loaded.kernel == pipe.kernel
    A = _t(np.random.default_rng(16).normal(size=(samples, pipe.plan.a_width)), dtype, gpu)
    assert torch.equal(loaded.product(A), pipe.product(A))
