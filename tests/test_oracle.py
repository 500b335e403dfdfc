"""Pin the CPU oracle before trusting it.

Each oracle function is checked against something other than its own formula:
the reference's golden vectors, the reference's own compiled CPU core
(``oracle/_ref``, where built), closed forms, independent libraries (SciPy's
complex spherical harmonics), quadrature identities and brute force.
"""

import json
import math
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _ref_or_skip():
    lib = oracle.ref_lib()
    if lib is None:
        pytest.skip("reference CPU core not built (oracle/_ref, needs /root/reference)")
    return lib


# ----------------------------------------------------------------- radial
def test_radial_golden_vector_from_reference_fixture():
    # tests/cpp/test_runtime_core_standalone.cpp:608-660: r=1.37, rc=4, lambda=0.5723.
    # PACE column 0 is ChebExpCos n=1 and column 2 is n=2 inside the outer switch.
    v, d = oracle.radial_table([1.37], [4.0], [0.5723], 2)
    assert abs(v[0, 1] - 0.7374281949352972) < 1e-15
    assert abs(v[0, 2] - 0.7127134551156157) < 1e-15
    assert abs(d[0, 1] - (-0.3456000490756779)) < 1e-15
    assert abs(d[0, 2] - (-0.18827917863553195)) < 1e-15


def test_radial_closed_forms_and_cutoff():
    r = np.array([0.0, 0.3, 1.7, 2.9, 3.0, 3.5])
    rc, lam = 3.0, 0.8
    v, d = oracle.radial_table(r, np.full(6, rc), np.full(6, lam), 6)
    s = r / rc
    env = 1 + np.cos(np.pi * s)
    x = 1 - 2 * np.expm1(-lam * (s - 1)) / np.expm1(lam)
    inside = s <= 1
    assert np.all(v[inside, 0] == 1.0)
    np.testing.assert_allclose(v[inside, 1], 0.5 * env[inside], rtol=0, atol=1e-15)
    for n in range(2, 7):
        cheb = np.cos(n * np.arccos(np.clip(x, -1, 1)))  # T_n by its trigonometric definition
        np.testing.assert_allclose(v[inside, n], 0.25 * (1 - cheb[inside]) * env[inside], atol=1e-13)
    assert np.all(v[~inside] == 0.0) and np.all(d[~inside] == 0.0)
    # derivative by central differences
    h = 1e-6
    rr = np.array([0.4, 1.1, 2.2])
    vp, _ = oracle.radial_table(rr + h, np.full(3, rc), np.full(3, lam), 6)
    vm, _ = oracle.radial_table(rr - h, np.full(3, rc), np.full(3, lam), 6)
    _, dd = oracle.radial_table(rr, np.full(3, rc), np.full(3, lam), 6)
    np.testing.assert_allclose(dd, (vp - vm) / (2 * h), atol=2e-8)


def test_radial_matches_reference_core_bitwise():
    _ref_or_skip()
    rng = np.random.default_rng(1)
    r = rng.uniform(0, 6, 500)
    rc = rng.uniform(2, 5.5, 500)
    lam = rng.uniform(0.1, 2.0, 500)
    a = oracle.radial_table(r, rc, lam, 12)
    b = oracle.radial_table(r, rc, lam, 12, use_reference=True)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


# -------------------------------------------------------------------- SH
def _unitary(l):
    from ye3t_amd.core.cg import real_to_complex_unitary

    return real_to_complex_unitary(l)


def test_real_sh_against_scipy_complex_harmonics():
    sp = pytest.importorskip("scipy.special")
    rng = np.random.default_rng(2)
    vec = rng.normal(size=(40, 3)) * rng.uniform(0.5, 3, (40, 1))
    Y, _ = oracle.real_sph_table(vec, 8)
    u = vec / np.linalg.norm(vec, axis=1, keepdims=True)
    th, ph = np.arccos(u[:, 2]), np.arctan2(u[:, 1], u[:, 0])
    for l in range(9):
        yc = np.stack([sp.sph_harm_y(l, m, th, ph) for m in range(-l, l + 1)], axis=1)
        W = _unitary(l)
        np.testing.assert_allclose(yc, Y[:, l * l:(l + 1) ** 2] @ W.T, atol=1e-12)


def test_real_sh_y00_orthonormality_and_gradient():
    Y, G = oracle.real_sph_table(np.array([[0.3, -1.2, 0.7]]), 4)
    assert abs(Y[0, 0] - 0.5 / math.sqrt(math.pi)) < 1e-15
    # Gauss-Legendre x uniform-phi quadrature is exact for these polynomials
    zs, wz = np.polynomial.legendre.leggauss(16)
    phis = np.arange(32) * 2 * np.pi / 32
    Z, P = np.meshgrid(zs, phis, indexing="ij")
    s = np.sqrt(1 - Z ** 2)
    pts = np.stack([s * np.cos(P), s * np.sin(P), Z], axis=-1).reshape(-1, 3)
    w = (wz[:, None] * np.full((1, 32), 2 * np.pi / 32)).reshape(-1)
    Yq, _ = oracle.real_sph_table(pts, 6)
    gram = (Yq * w[:, None]).T @ Yq
    np.testing.assert_allclose(gram, np.eye(49), atol=1e-12)
    # gradient by central differences
    v0 = np.array([[0.8, -0.4, 1.3]])
    _, g0 = oracle.real_sph_table(v0, 5)
    h = 1e-6
    for a in range(3):
        dv = np.zeros((1, 3))
        dv[0, a] = h
        yp, _ = oracle.real_sph_table(v0 + dv, 5)
        ym, _ = oracle.real_sph_table(v0 - dv, 5)
        np.testing.assert_allclose(g0[0, :, a], (yp - ym)[0] / (2 * h), atol=1e-8)


def test_real_sh_matches_reference_core_bitwise():
    _ref_or_skip()
    rng = np.random.default_rng(3)
    vec = rng.normal(size=(300, 3))
    vec[0] = 0.0  # zero vector goes through the epsilon branch
    a = oracle.real_sph_table(vec, 8)
    b = oracle.real_sph_table(vec, 8, use_reference=True)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


# --------------------------------------------------------------- density
def test_density_against_index_add_and_reference():
    rng = np.random.default_rng(4)
    E, C, N = 300, 7, 40
    ev = rng.normal(size=(E, C))
    centers = rng.integers(0, N, E)
    out = oracle.density_accumulate(ev, centers, N)
    brute = np.zeros((N, C))
    np.add.at(brute, centers, ev)
    np.testing.assert_allclose(out, brute, atol=1e-13)
    if oracle.ref_lib() is not None:
        assert np.array_equal(out, oracle.density_accumulate(ev, centers, N, use_reference=True))


def test_density_adjoint_is_the_gather_and_the_transpose():
    rng = np.random.default_rng(5)
    E, C, N = 400, 9, 50
    adj = rng.normal(size=(N, C))
    centers = rng.integers(0, N, E)
    out = oracle.density_accumulate_adjoint(adj, centers)
    assert np.array_equal(out, adj[centers])
    # <accumulate(x), y> = <x, adjoint(y)>: the gather is the transpose of the scatter-add
    x = rng.normal(size=(E, C))
    lhs = np.sum(oracle.density_accumulate(x, centers, N) * adj)
    rhs = np.sum(x * out)
    assert abs(lhs - rhs) <= 1e-12 * max(1.0, abs(lhs))
    assert oracle.density_accumulate_adjoint(adj, np.zeros(0, dtype=np.int64)).shape == (0, C)
    with pytest.raises(ValueError):
        oracle.density_accumulate_adjoint(adj, centers + N)
    ref = oracle.ref_lib()
    if ref is not None and hasattr(ref, "ref_density_accumulate_adjoint"):
        assert np.array_equal(out, oracle.density_accumulate_adjoint(adj, centers, use_reference=True))


def test_ace_density_is_the_reference_chain_and_rotation_covariant():
    from ye3t_amd.ace import workloads as W

    inp = W.config(4, atom_count=30).density.generate()
    A = oracle.ace_density(inp)
    # same chain from the individual oracle pieces (radial mix, feature weights)
    r = np.linalg.norm(inp["edge_vectors"], axis=1)
    R, _ = oracle.radial_table(r, np.full_like(r, inp["cutoff"]), np.full_like(r, inp["lambda"]), inp["n_max"])
    Y, _ = oracle.real_sph_table(inp["edge_vectors"], inp["l_max"])
    Rc = R @ inp["radial_mix"].T
    w = inp["node_features"][inp["neighbors"]]
    edge = (w * Rc)[:, :, None] * Y[:, None, :]
    ref = oracle.density_accumulate(edge.reshape(len(r), -1), inp["centers"], inp["atom_count"])
    np.testing.assert_allclose(A.reshape(inp["atom_count"], -1), ref, rtol=0, atol=1e-12)
    # the l=0 block is rotation invariant
    th = 0.7
    Rot = np.array([[np.cos(th), -np.sin(th), 0], [np.sin(th), np.cos(th), 0], [0, 0, 1]])
    rot = dict(inp, edge_vectors=inp["edge_vectors"] @ Rot.T)
    A2 = oracle.ace_density(rot)
    np.testing.assert_allclose(A2[..., 0], A[..., 0], atol=1e-12)


# ------------------------------------------------ symmetric-power monomials
def test_symmetric_monomial_golden_fixture():
    fx = json.load(open(os.path.join(GOLDEN, "shared_monomial_plan_v1.json")))
    D = int(fx["input_dimension"])
    mono = np.array(fx["monomial_counts"], dtype=np.int64).reshape(-1, D)
    offsets = np.array(fx["output_offsets"], dtype=np.int64)
    terms = np.array(fx["coefficient_terms"], dtype=np.int64)
    values = np.array(fx["coefficient_values"])
    x = np.array(fx["input"]).reshape(int(fx["batch_size"]), D)
    out = oracle.symmetric_power_monomial(x, mono[terms], offsets, values)
    np.testing.assert_allclose(out.reshape(-1), fx["expected_output"], rtol=0, atol=5e-13)
    if oracle.ref_lib() is not None:
        ref = oracle.symmetric_power_monomial(x, mono[terms], offsets, values, use_reference=True)
        assert np.array_equal(out, ref)


# -------------------------------------------------------- schedule evaluation
def test_evaluate_componentwise_brute_force():
    rng = np.random.default_rng(5)
    B, basis, blocks, mdim, K = 5, 3, 3, 5, 7
    bv = rng.normal(size=(B, basis, blocks, mdim))
    counts = rng.integers(0, 4, K)
    offs = np.concatenate([[0], np.cumsum(counts)])
    T = int(offs[-1])
    flat = {"component_offsets": offs, "component_label_index": rng.integers(0, basis, K),
            "block_m_indices": rng.integers(0, mdim, (T, blocks)), "coeffs": rng.normal(size=T)}
    out = oracle.evaluate_componentwise(bv, flat)
    brute = np.zeros((B, K))
    for b in range(B):
        for k in range(K):
            for t in range(offs[k], offs[k + 1]):
                v = flat["coeffs"][t]
                for blk in range(blocks):
                    v *= bv[b, flat["component_label_index"][k], blk, flat["block_m_indices"][t, blk]]
                brute[b, k] += v
    np.testing.assert_allclose(out, brute, atol=1e-13)


def test_config4_features_rotate_by_wigner_d():
    """Oracle density -> plan product: every L block of B rotates by D^L(R) (L = 0 invariant)."""
    from tests._util import rotation, wigner_real
    from ye3t_amd.ace import workloads as W
    from ye3t_amd.ace.plan import ProductPlan

    cfg = W.config(4, atom_count=40)
    inp = cfg.density.generate()
    plan = ProductPlan(cfg.feature_spec)
    R = rotation(5)
    rot = dict(inp)
    rot["edge_vectors"] = inp["edge_vectors"] @ R.T
    B0 = oracle.ace_product_flat(oracle.ace_density(inp).reshape(-1, plan.a_width), plan.flat_arrays())
    B1 = oracle.ace_product_flat(oracle.ace_density(rot).reshape(-1, plan.a_width), plan.flat_arrays())
    for L, _ci, _lab, first in plan.label_records:
        cols = slice(first, first + 2 * L + 1)
        np.testing.assert_allclose(B1[:, cols], B0[:, cols] @ wigner_real(R, L).T, rtol=1e-9,
                                   atol=1e-9 * np.abs(B0[:, cols]).max())


def test_linear_readout_selects_columns_and_is_linear():
    rng = np.random.default_rng(8)
    B = rng.normal(size=(50, 7))
    for k in range(7):
        e = np.zeros(7)
        e[k] = 1.0
        assert np.array_equal(oracle.linear_readout(B, e, 0.0), B[:, k])
    w1, w2 = rng.normal(size=7), rng.normal(size=7)
    lhs = oracle.linear_readout(B, w1 + w2, 0.5)
    rhs = oracle.linear_readout(B, w1, 0.25) + oracle.linear_readout(B, w2, 0.25)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-13, atol=1e-13)


def test_product_adjoint_matches_the_exact_directional_derivative():
    """<gB, f'(A) d> = <f'(A)^T gB, d>, with f'(A) d taken from five forward
    evaluations: B(A + t d) is a polynomial of degree <= 4 in t, for which the
    central stencil (f(-2) - 8 f(-1) + 8 f(1) - f(2)) / 12 is exact."""
    from ye3t_amd.ace import workloads as W
    from ye3t_amd.ace.plan import ProductPlan

    rng = np.random.default_rng(21)
    for cid in (4, 2):
        plan = ProductPlan(W.config(cid).feature_spec)
        arrays = plan.flat_arrays()
        A = rng.normal(size=(6, plan.a_width))
        d = rng.normal(size=A.shape)
        gB = rng.normal(size=(6, plan.feature_count))
        f = {t: oracle.ace_product_flat(A + t * d, arrays) for t in (-2, -1, 1, 2)}
        jd = (f[-2] - 8 * f[-1] + 8 * f[1] - f[2]) / 12.0
        gA = oracle.ace_product_flat_adjoint(A, gB, arrays)
        lhs = np.sum(gB * jd, axis=1)
        rhs = np.sum(gA * d, axis=1)
        np.testing.assert_allclose(lhs, rhs, rtol=1e-9, atol=1e-9 * np.max(np.abs(lhs)))
        # columns of A no feature depends on have zero gradient
        used = np.zeros(plan.a_width, dtype=bool)
        vf = np.asarray(arrays["value_factors"])
        used[vf[vf >= 0]] = True
        assert not np.any(gA[:, ~used])


def _reference_segment_order(targets, sources, node_count):
    """numpy restatement of the edge order of prepare_carrier_scatter_segments
    (execution_plan.py:9316-9434): stable argsort of target * N + source."""
    return np.argsort(targets * node_count + sources, kind="stable")


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_neighbor_list_against_kdtree_and_the_segment_convention(dtype):
    from scipy.spatial import cKDTree

    rng = np.random.default_rng(11)
    pos = rng.uniform(-7.0, 13.0, size=(1500, 3)).astype(dtype)
    cutoff = 2.7
    nl = oracle.neighbor_list(pos, cutoff)
    offs, tgt, src, vec = nl["target_offsets"], nl["edge_targets"], nl["edge_sources"], nl["edge_vectors"]
    # the pair set of an independent implementation (both directions)
    pairs = cKDTree(pos.astype(np.float64)).query_pairs(cutoff, output_type="ndarray")
    both = np.concatenate([pairs, pairs[:, ::-1]])
    assert len(tgt) == len(both) > 0
    order = _reference_segment_order(both[:, 0], both[:, 1], len(pos))
    np.testing.assert_array_equal(tgt, both[order, 0])
    np.testing.assert_array_equal(src, both[order, 1])
    # already in the reference's order: its stable argsort is the identity
    np.testing.assert_array_equal(_reference_segment_order(tgt, src, len(pos)), np.arange(len(tgt)))
    np.testing.assert_array_equal(offs, np.concatenate([[0], np.cumsum(np.bincount(tgt, minlength=len(pos)))]))
    # r_j - r_i, one rounding in the positions' type
    np.testing.assert_array_equal(vec, pos[src] - pos[tgt])
    assert vec.dtype == dtype


def test_neighbor_list_lattice_closed_forms_and_strict_cutoff():
    n = 6
    g = np.arange(n, dtype=np.float64)
    pos = np.stack(np.meshgrid(g, g, g, indexing="ij"), -1).reshape(-1, 3)
    # spacing 1 exactly: r < 1 excludes every lattice bond, r < 1.5 keeps the
    # 3 n^2 (n-1) axis bonds, r < 1.45 vs 1.42 brackets the face diagonals sqrt(2)
    assert oracle.neighbor_list(pos, 1.0)["target_offsets"][-1] == 0
    axis = 2 * 3 * n * n * (n - 1)
    assert oracle.neighbor_list(pos, 1.0 + 1e-12)["target_offsets"][-1] == axis
    assert oracle.neighbor_list(pos, 1.41)["target_offsets"][-1] == axis
    face = 2 * 3 * 2 * n * (n - 1) ** 2
    nl = oracle.neighbor_list(pos, 1.42)
    assert nl["target_offsets"][-1] == axis + face
    # an interior site has 6 + 12 neighbours
    centre = (2 * n + 2) * n + 2
    assert np.diff(nl["target_offsets"])[centre] == 18
    # coincident atoms are neighbours of each other (distance 0 < cutoff)
    same = np.zeros((5, 3))
    nl = oracle.neighbor_list(same, 0.5)
    assert nl["target_offsets"].tolist() == [0, 4, 8, 12, 16, 20]
    assert nl["edge_sources"][:4].tolist() == [1, 2, 3, 4]
    empty = oracle.neighbor_list(np.zeros((0, 3)), 1.0)
    assert empty["target_offsets"].tolist() == [0] and len(empty["edge_sources"]) == 0
