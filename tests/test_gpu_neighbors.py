"""On-device neighbour list vs the brute-force oracle: bit-exact CSR, edge
order and edge vectors (needs an MI355X)."""

import ctypes

import numpy as np
import pytest

import oracle
from tests._util import column_rel_error, flush
from ye3t_amd.runtime import native

pytestmark = pytest.mark.gpu


def _lattice(n, spacing=1.0):
    g = np.arange(n, dtype=np.float64) * spacing
    return np.stack(np.meshgrid(g, g, g, indexing="ij"), -1).reshape(-1, 3)


def _case(name, rng):
    """(positions float64 [N, 3], cutoff)"""
    if name == "uniform":
        return rng.uniform(-3.0, 22.0, size=(4000, 3)), 3.0
    if name == "lattice_tie":  # every bond exactly at the cutoff: no edges
        return _lattice(8), 1.0
    if name == "lattice_axis":
        return _lattice(8), 1.0 + 1e-12
    if name == "lattice_face":
        return _lattice(8), 1.42
    if name == "clustered":  # one cell holds 600 atoms: rows of ~600 entries
        ball = rng.normal(size=(600, 3)) * 0.2 + 10.0
        return np.concatenate([rng.uniform(0.0, 30.0, size=(2000, 3)), ball]), 2.5
    if name == "coincident":
        return np.full((300, 3), 1.25), 0.5
    if name == "one_cell":  # cutoff wider than the box
        return rng.uniform(0.0, 1.0, size=(200, 3)), 5.0
    if name == "single":
        return np.array([[0.5, -1.0, 2.0]]), 1.0
    if name == "empty":
        return np.zeros((0, 3)), 1.0
    raise KeyError(name)


CASES = ["uniform", "lattice_tie", "lattice_axis", "lattice_face", "clustered", "coincident", "one_cell", "single",
         "empty"]


def _check(got, ref, dtype):
    for key in ("target_offsets", "edge_targets", "edge_sources"):
        assert np.array_equal(got[key].cpu().numpy(), ref[key]), key
    vec = got["edge_vectors"]
    assert vec.dtype == dtype
    assert np.array_equal(vec.cpu().numpy(), ref["edge_vectors"])


@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("case", CASES)
def test_neighbor_list_matches_oracle(gpu, dtype, case):
    flush(f"neighbor_list {dtype} {case}")
    import torch

    from ye3t_amd.runtime import neighbor_list

    pos, cutoff = _case(case, np.random.default_rng(7))
    npdt, tdt = (np.float64, torch.float64) if dtype == "f64" else (np.float32, torch.float32)
    pos = pos.astype(npdt)
    ref = oracle.neighbor_list(pos, cutoff)
    got = neighbor_list(torch.as_tensor(pos, device=gpu), cutoff)
    _check(got, ref, tdt)
    if case == "uniform":
        assert len(ref["edge_sources"]) > 20 * len(pos)
        again = neighbor_list(torch.as_tensor(pos, device=gpu), cutoff)
        for key in ("target_offsets", "edge_sources", "edge_vectors"):
            assert torch.equal(again[key], got[key])


def test_neighbor_list_grid_not_covering_the_atoms(gpu):
    """Atoms outside the grid are clamped into its border cells: same list."""
    flush("neighbor_list outside grid")
    import torch

    rng = np.random.default_rng(8)
    pos = rng.uniform(-10.0, 10.0, size=(1500, 3))
    ref = oracle.neighbor_list(pos, 2.0)
    grid = native.cell_grid([-2.0, -2.0, -2.0], [2.0, 2.0, 2.0], 2.0, len(pos))
    got = native.neighbor_list(torch.as_tensor(pos, device=gpu), 2.0, grid=grid)
    _check(got, ref, torch.float64)


@pytest.mark.parametrize("rows", ["short", "long"])
def test_neighbor_fill_respects_edge_capacity(gpu, rows):
    """Edges at or beyond edge_capacity are not written; the row cut by it
    holds its smallest neighbours (rows built in LDS, and rows longer than the
    LDS buffer built in global memory)."""
    flush(f"neighbor_list capacity {rows} rows")
    import torch

    rng = np.random.default_rng(9)
    if rows == "short":
        pos_np = rng.uniform(0.0, 12.0, size=(800, 3))
    else:  # 700 atoms within 0.1 of each other: rows of 699 entries
        pos_np = 5.0 + rng.uniform(-0.05, 0.05, size=(700, 3))
    ref = oracle.neighbor_list(pos_np, 2.0)
    E = len(ref["edge_sources"])
    offs_ref = ref["target_offsets"]
    row = int(np.searchsorted(offs_ref, E // 2, side="right")) - 1
    while offs_ref[row + 1] - offs_ref[row] < 2:
        row += 1
    cap = int(offs_ref[row] + (offs_ref[row + 1] - offs_ref[row]) // 2)  # inside a row
    assert offs_ref[row] < cap < offs_ref[row + 1]
    pos = torch.as_tensor(pos_np, device=gpu)
    grid = native.cell_grid(pos_np.min(0), pos_np.max(0), 2.0, len(pos_np))
    L = native.lib()
    ws_bytes = L.ye3t_hip_neighbor_workspace_bytes(len(pos_np), ctypes.byref(grid))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
    offs = torch.empty(len(pos_np) + 1, dtype=torch.int64, device=gpu)
    stream = native._stream()
    assert L.ye3t_hip_neighbor_count(native.F64, pos.data_ptr(), len(pos_np), ctypes.byref(grid), 2.0,
                                     ws.data_ptr(), ws_bytes, offs.data_ptr(), stream) == 0
    assert np.array_equal(offs.cpu().numpy(), ref["target_offsets"])
    sentinel = -7
    cen = torch.full((E,), sentinel, dtype=torch.int64, device=gpu)
    nbr = torch.full((E,), sentinel, dtype=torch.int64, device=gpu)
    vec = torch.full((E, 3), float(sentinel), dtype=torch.float64, device=gpu)
    assert L.ye3t_hip_neighbor_fill(native.F64, len(pos_np), ctypes.byref(grid), 2.0, ws.data_ptr(), ws_bytes,
                                    offs.data_ptr(), cap, cen.data_ptr(), nbr.data_ptr(), vec.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert np.array_equal(cen[:cap].cpu().numpy(), ref["edge_targets"][:cap])
    assert np.array_equal(nbr[:cap].cpu().numpy(), ref["edge_sources"][:cap])
    assert np.array_equal(vec[:cap].cpu().numpy(), ref["edge_vectors"][:cap])
    assert bool((cen[cap:] == sentinel).all()) and bool((nbr[cap:] == sentinel).all())
    assert bool((vec[cap:] == sentinel).all())


def test_neighbor_list_feeds_the_density(gpu):
    """positions -> neighbour CSR -> fused stage 1 equals the oracle chain on the oracle's CSR."""
    flush("neighbor_list -> ace_density")
    import torch

    rng = np.random.default_rng(12)
    pos = rng.uniform(0.0, 14.0, size=(900, 3))
    species = rng.integers(0, 3, len(pos)).astype(np.int32)
    cutoff, n_max, l_max, lam = 3.2, 6, 3, 1.1
    nl = native.neighbor_list(torch.as_tensor(pos, device=gpu), cutoff)
    A = native.ace_density_forward(nl["edge_vectors"], nl["target_offsets"], nl["edge_sources"],
                                   atom_count=len(pos), channel_count=3, n_max=n_max, l_max=l_max, cutoff=cutoff,
                                   lam=lam, species=torch.as_tensor(species, device=gpu))
    ref = oracle.neighbor_list(pos, cutoff)
    A_ref = oracle.ace_density({"atom_count": len(pos), "edge_count": len(ref["edge_sources"]),
                                "centers": ref["edge_targets"], "neighbors": ref["edge_sources"],
                                "edge_vectors": ref["edge_vectors"], "species": species, "channel_count": 3,
                                "n_max": n_max, "l_max": l_max, "cutoff": cutoff, "lambda": lam})
    assert len(ref["edge_sources"]) > 10 * len(pos)
    assert column_rel_error(A.cpu().numpy(), A_ref) <= 1e-12
