"""Config 4 at its full benchmark size (50 000 nodes x 16 channels = 800 000 samples).

* parity: the fp32-storage HIP pipeline (fp64 density and products, the
  configuration's precision) against the fp64 oracle on the same fp32-rounded
  inputs, per feature column (max |diff| / column RMS <= 2e-5);
* size-independent property: rotating every neighbour vector by R maps each
  L-block of B to ``D^L(R)`` times the unrotated block (invariance for L = 0),
  checked in fp64 over all 800 000 samples.  ``D^L`` is fitted from the oracle's
  real spherical harmonics, so the check is independent of the plan compiler.
"""

import numpy as np
import pytest

import oracle
from tests._util import TOL, column_rel_error, flush, fp32_rounding_ratio, rotation, rounded_inputs, wigner_real
from ye3t_amd.ace import workloads as W
from ye3t_amd.ace.pipeline import ACEPipeline, to_device_inputs

pytestmark = pytest.mark.gpu


def test_config4_full_size_fp32_parity(gpu):
    """fp32 inputs, density and features with the configuration's fp64
    arithmetic (the density is accumulated in fp64 and rounded once)."""
    flush("config 4 full size, fp32 storage vs fp64 oracle")
    cfg = W.config(4)
    inp = cfg.density.generate()
    pipe = ACEPipeline(cfg.feature_spec, "f32", accumulate=cfg.accumulate, density=cfg.density_dtype)
    A, B = pipe.forward(to_device_inputs(inp, "f32", gpu), channelwise=True)
    A_ref = oracle.ace_density(rounded_inputs(inp, "f32"))
    N = cfg.density.atom_count
    errA = column_rel_error(A.cpu().numpy().reshape(N, -1), A_ref.reshape(N, -1))
    B_ref = oracle.ace_product_flat(A_ref.reshape(-1, pipe.plan.a_width), pipe.plan.flat_arrays())
    errB = column_rel_error(B.cpu().numpy(), B_ref)
    flush(f"  A err {errA:.3e}  B err {errB:.3e}  ({B_ref.shape[0]} samples x {B_ref.shape[1]} features)")
    assert errA < TOL["f32"]
    assert errB < TOL["f32"]


def test_config4_full_size_fused_linear_readout(gpu):
    """The fused readout over all 800 000 samples against B_ref @ w + bias."""
    flush("config 4 full size, fused linear readout")
    import torch

    cfg = W.config(4)
    inp = cfg.density.generate()
    pipe = ACEPipeline(cfg.feature_spec, "f32", accumulate=cfg.accumulate, density=cfg.density_dtype)
    A = pipe.density(to_device_inputs(inp, "f32", gpu))
    w = np.random.default_rng(77).normal(size=pipe.feature_count)
    got = pipe.linear(A.reshape(-1, pipe.plan.a_width), torch.as_tensor(w, device=gpu), -2.0)
    assert pipe.last_linear_backend == "fused_generated"
    A_ref = oracle.ace_density(rounded_inputs(inp, "f32")).reshape(-1, pipe.plan.a_width)
    ref = oracle.linear_readout(oracle.ace_product_flat(A_ref, pipe.plan.flat_arrays()), w, -2.0)
    err = float(np.max(np.abs(got.cpu().double().numpy() - ref))) / float(np.sqrt(np.mean(ref * ref)))
    flush(f"  err {err:.3e}")
    assert err < TOL["f32"]


def test_config4_full_size_product_adjoint(gpu):
    """dL/dA over all 800 000 samples of the benchmark density against the oracle's reverse mode."""
    flush("config 4 full size, product adjoint")
    import torch

    cfg = W.config(4)
    pipe = ACEPipeline(cfg.feature_spec, "f32", accumulate=cfg.accumulate, density=cfg.density_dtype)
    A = pipe.density(to_device_inputs(cfg.density.generate(), "f32", gpu)).reshape(-1, pipe.plan.a_width)
    gB = torch.as_tensor(np.random.default_rng(78).normal(size=(A.shape[0], pipe.feature_count)),
                         dtype=torch.float32, device=gpu)
    gA = pipe.product_adjoint(A, gB)
    ref = oracle.ace_product_flat_adjoint(A.cpu().double().numpy(), gB.cpu().double().numpy(),
                                          pipe.plan.flat_arrays())
    got = gA.cpu().double().numpy()
    if pipe.density_dtype == "f64":
        err = column_rel_error(got, ref)
        flush(f"  err {err:.3e}")
        assert err < 1e-12
    else:
        # fp64 arithmetic, gA stored in the density's fp32: each value is the
        # oracle's rounded once (within half an fp32 ulp, 2^-24 relative)
        ratio = fp32_rounding_ratio(got, ref)
        flush(f"  error / fp32 rounding bound {ratio:.3f}")
        assert ratio <= 1.0


def test_config4_full_size_rotation_covariance_fp64(gpu):
    flush("config 4 full size, rotation covariance of every L block (fp64)")
    import torch

    cfg = W.config(4)
    inp = cfg.density.generate()
    R = rotation(21)
    rot = dict(inp)
    rot["edge_vectors"] = inp["edge_vectors"] @ R.T
    pipe = ACEPipeline(cfg.feature_spec, "f64")
    _, B0 = pipe.forward(to_device_inputs(inp, "f64", gpu), channelwise=True)
    B0 = B0.cpu().numpy()
    _, B1 = pipe.forward(to_device_inputs(rot, "f64", gpu), channelwise=True)
    B1 = B1.cpu().numpy()
    torch.cuda.synchronize()
    expected = np.empty_like(B0)
    for L, _ci, _lab, first in pipe.plan.label_records:
        D = wigner_real(R, L)
        cols = slice(first, first + 2 * L + 1)
        expected[:, cols] = B0[:, cols] @ D.T
    err = column_rel_error(B1, expected)
    flush(f"  covariance err {err:.3e}")
    assert err < 1e-10  # fitted D^L carries ~1e-13 of least-squares error


@pytest.mark.parametrize("dtype", ["f32", "f64"])
def test_config4_full_size_neighbor_list(gpu, dtype):
    """50 000 uniform random atoms at config 4's cutoff (about 24 neighbours
    each): the device list equals the brute-force oracle bit for bit, and is
    symmetric (j in row i iff i in row j) with antisymmetric vectors."""
    flush(f"config 4 full size neighbour list {dtype}")
    import torch

    from ye3t_amd.runtime import neighbor_list

    d = W.config(4).density
    N, cutoff = d.atom_count, float(d.radius)
    box = (N / 0.05) ** (1.0 / 3.0)
    pos = np.random.default_rng(5).uniform(0.0, box, size=(N, 3)).astype(np.float64 if dtype == "f64" else
                                                                          np.float32)
    got = neighbor_list(torch.as_tensor(pos, device=gpu), cutoff)
    ref = oracle.neighbor_list(pos, cutoff)
    E = len(ref["edge_sources"])
    flush(f"  {E} edges ({E / N:.1f} per atom)")
    assert E > 20 * N
    for key in ("target_offsets", "edge_targets", "edge_sources", "edge_vectors"):
        assert np.array_equal(got[key].cpu().numpy(), ref[key]), key
    tgt, src = ref["edge_targets"], ref["edge_sources"]
    fwd = tgt * N + src
    rev = src * N + tgt
    pos_of = np.searchsorted(fwd, rev)
    assert np.array_equal(fwd[pos_of], rev)
    assert np.array_equal(ref["edge_vectors"][pos_of], -ref["edge_vectors"])


def test_neighbor_list_three_level_scans(gpu):
    """4.3 M atoms on about 9 M cells: both device scans (cell starts and row
    offsets) take three levels.  Row lengths equal those of an independent k-d
    tree, rows are ascending, and sampled rows equal the tree's sets."""
    flush("neighbour list, 4.3 M atoms (three-level scans)")
    import torch
    from scipy.spatial import cKDTree

    from ye3t_amd.runtime import native, neighbor_list

    N, cutoff = 4_300_000, 1.0
    box = (N / (2.0 / (4.0 / 3.0 * np.pi))) ** (1.0 / 3.0)  # about 2 neighbours per atom
    pos = np.random.default_rng(13).uniform(0.0, box, size=(N, 3))
    grid = native.cell_grid(pos.min(0), pos.max(0), cutoff, N)
    cells = grid.dims[0] * grid.dims[1] * grid.dims[2]
    assert cells > 2048 * 2048 and N > 2048 * 2048
    got = neighbor_list(torch.as_tensor(pos, device=gpu), cutoff)
    offs = got["target_offsets"].cpu().numpy()
    src = got["edge_sources"].cpu().numpy()
    pairs = cKDTree(pos).query_pairs(cutoff, output_type="ndarray")
    counts = np.bincount(pairs.ravel(), minlength=N)
    flush(f"  {cells} cells, {len(src)} edges")
    assert np.array_equal(np.diff(offs), counts) and offs[0] == 0
    tgt = np.repeat(np.arange(N), counts)
    assert np.array_equal(got["edge_targets"].cpu().numpy(), tgt)
    same_row = tgt[1:] == tgt[:-1]
    assert np.all(src[1:][same_row] > src[:-1][same_row])
    tree = cKDTree(pos)
    for i in np.random.default_rng(14).integers(0, N, 200):
        want = sorted(j for j in tree.query_ball_point(pos[i], cutoff) if j != i)
        assert src[offs[i]:offs[i + 1]].tolist() == want
