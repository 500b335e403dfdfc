"""Edge-vector gradient of the fused stage 1 (forces) on the GPU.

``ye3t_hip_ace_density_edge_gradient`` against the pinned oracle
(``oracle.ace_density_edge_gradient``) on the same seeded, dtype-rounded
inputs: one-hot species, node features with a radial mix, one channel; every
l_max the kernel is built for (0..8); ragged CSR rows with empty atoms, edges
beyond the cutoff and near zero length; fp64 (1e-12) and fp32 edge vectors with
fp32 or fp64 adjoints (2e-5), column-relative over the three components;
config 4's 16-channel mix shape (its own kernel path) in the three dtype pairs.
Autograd through ``runtime.ace_density`` gives the same gradient, and an
fp64 config-sized case is checked at full size.
"""

import numpy as np
import pytest

import oracle
from tests._util import TOL, column_rel_error, flush, rounded_inputs
from ye3t_amd.ace import workloads as W

pytestmark = pytest.mark.gpu


def _workload(mode, atoms, max_degree, seed, n_max, l_max, channels=6):
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, max_degree + 1, atoms)
    counts[0] = 0
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    E = int(offsets[-1])
    vec = rng.normal(size=(E, 3))
    vec = vec / np.linalg.norm(vec, axis=1, keepdims=True) * rng.uniform(0.05, 5.3, (E, 1))
    vec[:3] *= 1e-14  # below epsilon: the harmonics' direction is v / epsilon
    inp = {"atom_count": atoms, "edge_count": E, "centers": np.repeat(np.arange(atoms), counts),
           "row_offsets": offsets, "neighbors": rng.integers(0, atoms, E), "edge_vectors": vec, "n_max": n_max,
           "l_max": l_max, "cutoff": 5.0, "lambda": W.LAMBDA, "epsilon": 1e-12, "species": None,
           "node_features": None, "radial_mix": None, "channel_count": 1}
    if mode == "species":
        inp.update(channel_count=channels, species=rng.integers(0, channels, atoms).astype(np.int32))
    elif mode == "features":
        inp.update(channel_count=channels, node_features=rng.normal(size=(atoms, channels)),
                   radial_mix=rng.normal(size=(channels, n_max + 1)) / 3)
    elif mode == "features_nomix":
        inp.update(channel_count=channels, node_features=rng.normal(size=(atoms, channels)))
    return inp


def _device(inp, dtype, gpu):
    import torch

    real = torch.float64 if dtype == "f64" else torch.float32
    d = {"row_offsets": torch.as_tensor(inp["row_offsets"], device=gpu),
         "neighbors": torch.as_tensor(inp["neighbors"], dtype=torch.int64, device=gpu),
         "edge_vectors": torch.as_tensor(inp["edge_vectors"], dtype=real, device=gpu)}
    kw = dict(atom_count=inp["atom_count"], channel_count=inp["channel_count"], n_max=inp["n_max"],
              l_max=inp["l_max"], cutoff=inp["cutoff"], lam=inp["lambda"], epsilon=inp["epsilon"])
    if inp["species"] is not None:
        kw["species"] = torch.as_tensor(inp["species"], dtype=torch.int32, device=gpu)
    for k in ("node_features", "radial_mix"):
        if inp[k] is not None:
            kw[k] = torch.as_tensor(inp[k], dtype=real, device=gpu)
    return d, kw


@pytest.mark.parametrize("mode", ["species", "features", "features_nomix", "single"])
@pytest.mark.parametrize("dtype,adjoint", [("f64", "f64"), ("f32", "f32"), ("f32", "f64")])
@pytest.mark.parametrize("l_max", [0, 3, 6])
def test_edge_gradient_against_oracle(gpu, mode, dtype, adjoint, l_max):
    flush(f"density edge gradient mode={mode} dtype={dtype} adjoint={adjoint} l_max={l_max}")
    import torch

    from ye3t_amd.runtime import native

    inp = _workload(mode, 120, 40, 11 + l_max, n_max=7, l_max=l_max)
    d, kw = _device(inp, dtype, gpu)
    rows = 1 if inp["radial_mix"] is not None else inp["n_max"] + 1
    shape = (inp["atom_count"], inp["channel_count"], rows, (l_max + 1) ** 2)
    gA = np.random.default_rng(3).normal(size=shape)
    adt = torch.float64 if adjoint == "f64" else torch.float32
    gA_dev = torch.as_tensor(gA, dtype=adt, device=gpu)
    got = native.ace_density_edge_gradient(gA_dev, d["edge_vectors"], d["row_offsets"], d["neighbors"], **kw)
    assert got.dtype == d["edge_vectors"].dtype and tuple(got.shape) == (inp["edge_count"], 3)
    ref_inp = rounded_inputs(inp, dtype)
    ref = oracle.ace_density_edge_gradient(ref_inp, gA_dev.double().cpu().numpy())
    err = column_rel_error(got.cpu().numpy(), ref)
    assert err < TOL["f64" if dtype == "f64" else "f32"], err


@pytest.mark.parametrize("l_max", [1, 2, 4, 5, 7, 8])
def test_edge_gradient_every_built_l_max(gpu, l_max):
    flush(f"density edge gradient l_max={l_max} (f64, species)")
    import torch

    from ye3t_amd.runtime import native

    inp = _workload("species", 40, 20, 100 + l_max, n_max=4, l_max=l_max, channels=3)
    d, kw = _device(inp, "f64", gpu)
    shape = (inp["atom_count"], 3, 5, (l_max + 1) ** 2)
    gA = torch.as_tensor(np.random.default_rng(l_max).normal(size=shape), device=gpu)
    got = native.ace_density_edge_gradient(gA, d["edge_vectors"], d["row_offsets"], d["neighbors"], **kw)
    ref = oracle.ace_density_edge_gradient(inp, gA.cpu().numpy())
    assert column_rel_error(got.cpu().numpy(), ref) < TOL["f64"]


def test_autograd_through_the_fused_density(gpu):
    flush("density edge gradient through autograd (config-4 shapes, 2000 atoms, f64)")
    import torch

    from ye3t_amd import runtime

    cfg = W.config(4, atom_count=2000)
    inp = cfg.density.generate()
    d, kw = _device({**inp, "species": inp.get("species")}, "f64", gpu)
    vec = d["edge_vectors"].clone().requires_grad_(True)
    A = runtime.ace_density(vec, d["row_offsets"], d["neighbors"], **kw)
    gA = torch.randn_like(A)
    (g,) = torch.autograd.grad(A, vec, gA)
    ref = oracle.ace_density_edge_gradient(inp, gA.cpu().numpy())
    assert column_rel_error(g.cpu().numpy(), ref) < TOL["f64"]
    direct = runtime.ace_density_edge_gradient(gA, d["edge_vectors"], d["row_offsets"], d["neighbors"], **kw)
    assert torch.equal(direct, g)


def test_edge_gradient_empty_and_errors(gpu):
    import torch

    from ye3t_amd.runtime import native

    inp = _workload("single", 5, 3, 1, n_max=3, l_max=2)
    d, kw = _device(inp, "f64", gpu)
    empty = native.ace_density_edge_gradient(
        torch.zeros((5, 1, 4, 9), dtype=torch.float64, device=gpu), d["edge_vectors"][:0],
        torch.zeros(6, dtype=torch.int64, device=gpu), d["neighbors"][:0], **kw)
    assert tuple(empty.shape) == (0, 3)
    with pytest.raises(ValueError, match="density_adjoint"):
        native.ace_density_edge_gradient(torch.zeros((5, 1, 4, 8), dtype=torch.float64, device=gpu),
                                         d["edge_vectors"], d["row_offsets"], d["neighbors"], **kw)
    kw9 = dict(kw, l_max=9)
    with pytest.raises(RuntimeError, match="l_max"):
        native.ace_density_edge_gradient(torch.zeros((5, 1, 4, 100), dtype=torch.float64, device=gpu),
                                         d["edge_vectors"], d["row_offsets"], d["neighbors"], **kw9)


@pytest.mark.parametrize("dtype,adjoint", [("f64", "f64"), ("f32", "f32"), ("f32", "f64")])
def test_edge_gradient_sixteen_channel_mix(gpu, dtype, adjoint):
    """Config 4's shape (16 feature channels with a radial mix, n_max 8,
    l_max 3), which runs the kernel's unrolled-row path: the neighbour's
    feature row read once, each channel's adjoint row one channel ahead."""
    flush(f"density edge gradient, 16 channels with a mix, dtype={dtype} adjoint={adjoint}")
    import torch

    from ye3t_amd.runtime import native

    cfg = W.config(4, atom_count=700)
    inp = cfg.density.generate()
    assert inp["channel_count"] == 16 and inp["n_max"] == 8 and inp["l_max"] == 3
    d, kw = _device({**inp, "species": inp.get("species")}, dtype, gpu)
    shape = (inp["atom_count"], 16, 1, 16)
    adt = torch.float64 if adjoint == "f64" else torch.float32
    gA = torch.as_tensor(np.random.default_rng(41).normal(size=shape), dtype=adt, device=gpu)
    got = native.ace_density_edge_gradient(gA, d["edge_vectors"], d["row_offsets"], d["neighbors"], **kw)
    ref = oracle.ace_density_edge_gradient(rounded_inputs(inp, dtype), gA.double().cpu().numpy())
    err = column_rel_error(got.cpu().numpy(), ref)
    flush(f"  err {err:.3e}")
    assert err < TOL["f64" if dtype == "f64" else "f32"], err
