"""Host compiler: labels, factorized schedules, symmetric blocks, real lowering.

Pins: independent multiplicity counts (brute-force weight enumeration),
SymPy's CG and nullspace/srepr machinery (the library the reference uses for
these objects), rotation invariance of evaluated schedules on complex
spherical-harmonic inputs from SciPy, and the reference's own facade tests
(README quick start, ``tests/test_couplings_namespace.py``).
"""

import itertools
from collections import Counter

import numpy as np
import pytest

from ye3t_amd.core import basis
from ye3t_amd.core import symmetric_power as SP
from ye3t_amd.core.cg import cg_float, cg_matrix, real_cg_tensor, real_to_complex_unitary
from ye3t_amd.core.couplings import generate_factorized_coefficient_schedules_by_L
from ye3t_amd.couplings import compile_ace_factorized_schedules_by_L, count, plan


# ------------------------------------------------------------------ facade
def test_readme_quickstart():
    report = count(content=(1, 1, 2), input_Ls=(1, 1, 0), target_L=0)
    labels = report.labels_for_target(0)
    assert len(labels) == 1
    report.require_label(labels[0], target_L=0)
    assert plan(report).validation_report["passed"]
    compiled = compile_ace_factorized_schedules_by_L(content=report.content, input_Ls=(1, 1, 0))
    assert compiled.validation_report["passed"]
    assert compiled.schedules_by_L[0].basis_count == len(labels)
    assert len(compiled.convention_hash) == 16


def test_facade_counts_like_reference_namespace_test():
    report = compile_ace_factorized_schedules_by_L(content=(1, 1, 1), input_Ls=(1, 1, 1),
                                                   constructor_backend="python", cache_policy="clear_before")
    assert report.backend == "ace_factorized_coefficient_schedule"
    assert report.validation_report["cache_policy"] == "clear_before"
    payload = report.to_dict()
    assert payload["schedule_summary"][1]["basis_count"] == 1
    assert payload["schedule_summary"][3]["basis_count"] == 1
    for L, s in report.schedules_by_target.items():
        assert s.basis_count == count(content=(1, 1, 1), input_Ls=(1, 1, 1), target_L=L).counts_by_target[L]


# -------------------------------------------------------------- multiplicity
def _brute_weight_counts(blocks):
    """Weight multiplicities of (x)_b Sym^{k_b}(V_{l_b}) by enumerating multisets."""
    total = Counter({0: 1})
    for n, l, k in blocks:
        w = Counter(sum(ms) for ms in itertools.combinations_with_replacement(range(-l, l + 1), k))
        nxt = Counter()
        for a, ca in total.items():
            for b, cb in w.items():
                nxt[a + b] += ca * cb
        total = nxt
    return total


@pytest.mark.parametrize("ls", [(1, 1, 1), (1, 2, 3), (2, 2, 2), (3, 3, 3), (0, 1, 1), (2, 3, 3), (1, 1, 2, 2),
                                (3, 3, 3, 3), (2, 2, 2, 1), (1, 1, 1, 1)])
def test_label_counts_match_brute_force_weights(ls):
    ns = tuple(1 for _ in ls)
    n_c, l_c = basis.canonicalize_leaf_quantum_numbers(ns, ls)
    weights = _brute_weight_counts(basis.young_blocks(n_c, l_c))
    labels = basis.compact_labels_by_L(ns, ls)
    for L in range(0, sum(ls) + 1):
        expected = weights.get(L, 0) - weights.get(L + 1, 0)
        assert len(labels.get(L, [])) == expected, (ls, L)
        # compact labels are unique and sorted
        assert labels.get(L, []) == sorted(set(labels.get(L, [])))


def test_canonical_order_is_l_first():
    assert basis.canonicalize_leaf_quantum_numbers((2, 1, 3), (0, 1, 1)) == ((1, 3, 2), (1, 1, 0))
    assert basis.canonicalize_leaf_quantum_numbers((1, 1, 2), (1, 1, 0)) == ((1, 1, 2), (1, 1, 0))


# ---------------------------------------------------------------------- CG
def test_cg_against_sympy():
    cgmod = pytest.importorskip("sympy.physics.quantum.cg")
    for l1, l2 in [(1, 1), (2, 1), (3, 2), (3, 3), (4, 2)]:
        for L in range(abs(l1 - l2), l1 + l2 + 1):
            for m1 in range(-l1, l1 + 1):
                for m2 in range(-l2, l2 + 1):
                    if abs(m1 + m2) > L:
                        continue
                    ref = float(cgmod.CG(l1, m1, l2, m2, L, m1 + m2).doit())
                    assert abs(cg_float(l1, m1, l2, m2, L, m1 + m2) - ref) < 2e-16 * max(1, abs(ref)) * 4


def test_real_cg_tensor_is_orthogonal_coupling():
    for l1, l2 in [(1, 1), (2, 3), (3, 3), (4, 2)]:
        rows = []
        for L in range(abs(l1 - l2), l1 + l2 + 1):
            T = real_cg_tensor(l1, l2, L)
            rows.append(T.reshape(-1, 2 * L + 1).T)
        M = np.concatenate(rows, axis=0)
        np.testing.assert_allclose(M @ M.T, np.eye(M.shape[0]), atol=1e-13)


# ------------------------------------------------------- symmetric blocks
def _sympy_highest_weights(l, k, Lam):
    """The reference procedure (``homogeneous.py:99-160, 411-434``) run in SymPy."""
    sp = pytest.importorskip("sympy")
    bas = SP.occupancy_basis_by_weight(l, k)
    wb, tgt = bas.get(Lam, ()), bas.get(Lam + 1, ())
    idx = {a: i for i, a in enumerate(tgt)}
    if not tgt:
        kern = [sp.eye(len(wb))[:, i] for i in range(len(wb))]
    else:
        J = sp.zeros(len(tgt), len(wb))
        for col, a in enumerate(wb):
            for i in range(2 * l):
                if a[i]:
                    m = i - l
                    new = list(a)
                    new[i] -= 1
                    new[i + 1] += 1
                    J[idx[tuple(new)], col] += sp.sqrt(sp.Integer(a[i] * (a[i + 1] + 1) * (l - m) * (l + m + 1)))
        kern = list(J.nullspace())

    def key(v):
        e = [sp.simplify(x) for x in v]
        p = next(i for i, x in enumerate(e) if x != 0)
        return p, tuple(sp.srepr(sp.simplify(x / e[p])) for x in e)

    out = []
    for v in sorted(kern, key=key):
        e = [sp.simplify(x) for x in v]
        p = next(i for i, x in enumerate(e) if x != 0)
        out.append([float(sp.simplify(x / e[p])) for x in e])
    return out


@pytest.mark.parametrize("l,k", [(1, 2), (1, 3), (2, 2), (2, 3), (3, 3), (2, 4), (1, 4)])
def test_symmetric_block_basis_matches_sympy_procedure(l, k):
    for Lam, mult in basis.symmetric_power_irrep_multiplicities(l, k).items():
        ref = _sympy_highest_weights(l, k, Lam)
        wb, mine = SP.highest_weight_vectors(l, k, Lam)
        assert len(ref) == len(mine) == mult
        for rv, (u, p) in zip(ref, mine):
            d2 = [SP._d_squared(l, a) for a in wb]
            got = [float(c) * float(r) ** 0.5 for c, r in (SP._radical(u[j], d2[j] / d2[p]) for j in range(len(wb)))]
            np.testing.assert_allclose(got, rv, atol=1e-13)


def test_symmetric_block_lowering_is_an_irrep():
    # lowered states of Sym^k(V_l)->V_Lam satisfy J_+ v_M = sqrt((Lam-M)(Lam+M+1)) v_{M+1}
    for l, k in [(2, 2), (3, 3), (2, 4)]:
        for Lam, mult in basis.symmetric_power_irrep_multiplicities(l, k).items():
            for c in range(mult):
                exp = SP.occupancy_expansion(l, k, Lam, c)
                bas = SP.occupancy_basis_by_weight(l, k)

                def vec(M):
                    return np.array([float(exp[M].get(a, (0, 1))[0]) * float(exp[M].get(a, (0, 1))[1]) ** 0.5
                                     for a in bas[M]])

                for M in range(-Lam, Lam):
                    Jp = np.zeros((len(bas[M + 1]), len(bas[M])))
                    index = {a: i for i, a in enumerate(bas[M + 1])}
                    for col, a in enumerate(bas[M]):
                        for i in range(2 * l):
                            if a[i]:
                                m = i - l
                                new = list(a)
                                new[i] -= 1
                                new[i + 1] += 1
                                Jp[index[tuple(new)], col] += np.sqrt(a[i] * (a[i + 1] + 1) * (l - m) * (l + m + 1))
                    np.testing.assert_allclose(Jp @ vec(M), np.sqrt((Lam - M) * (Lam + M + 1)) * vec(M + 1),
                                               atol=1e-12)


# ------------------------------------------- evaluated schedules are invariant
def _complex_multiplets(vectors, l):
    sp = pytest.importorskip("scipy.special")
    u = vectors / np.linalg.norm(vectors, axis=-1, keepdims=True)
    th, ph = np.arccos(u[..., 2]), np.arctan2(u[..., 1], u[..., 0])
    return np.stack([sp.sph_harm_y(l, m, th, ph) for m in range(-l, l + 1)], axis=-1)


def _densities(vectors, ls, weights):
    """Complex CS density multiplets A_(n,l) = sum_j w_nj Y_l(r_j) for each channel."""
    return {(n, l): (weights[n][:, None] * _complex_multiplets(vectors, l)).sum(axis=0)
            for n in weights for l in ls}


def _evaluate_complex(schedule, dens):
    """Reference evaluation: block values (leaf or complex sym monomials), then the schedule."""
    flat = schedule.flat_arrays()
    mdim = flat["max_block_m_dim"]
    bv = np.zeros((1, schedule.basis_count, schedule.block_count, mdim), dtype=np.complex128)
    for li, specs in enumerate(schedule.block_specs):
        for bi, s in enumerate(specs):
            a = dens[(s["n"], s["l"])]
            if s["kind"] == "leaf":
                vals = a
            else:
                vals = np.zeros(2 * s["Lambda"] + 1, dtype=np.complex128)
                for out_c, alpha, value in SP.complex_monomial_entries(s["k_b"], s["l"], s["Lambda"],
                                                                       s["multiplicity_index"]):
                    vals[out_c] += value * np.prod([a[m] ** e for m, e in enumerate(alpha)])
            bv[0, li, bi, :len(vals)] = vals
    out = np.zeros(schedule.component_count, dtype=np.complex128)
    for k in range(schedule.component_count):
        lab = flat["component_label_index"][k]
        for t in range(flat["component_offsets"][k], flat["component_offsets"][k + 1]):
            v = flat["coeffs"][t]
            for blk in range(schedule.block_count):
                v = v * bv[0, lab, blk, flat["block_m_indices"][t, blk]]
            out[k] += v
    return out


def _rotation(seed):
    q = np.random.default_rng(seed).normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array([[a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)],
                     [2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)],
                     [2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d]])


@pytest.mark.parametrize("ns,ls", [((1, 1, 2), (1, 1, 0)), ((1, 1, 1), (1, 2, 3)), ((1, 1, 1), (2, 2, 2)),
                                   ((1, 2, 2), (2, 1, 1)), ((1, 1, 1), (3, 3, 3)), ((1, 1, 2, 2), (1, 1, 2, 2)),
                                   ((1, 1, 1, 1), (2, 2, 2, 2)), ((1, 2), (2, 3))])
def test_complex_schedules_give_rotation_invariant_norms(ns, ls):
    rng = np.random.default_rng(7)
    vec = rng.normal(size=(12, 3))
    weights = {n: rng.normal(size=12) for n in set(ns)}
    R = _rotation(11)
    d0 = _densities(vec, set(ls), weights)
    d1 = _densities(vec @ R.T, set(ls), weights)
    for L, sched in generate_factorized_coefficient_schedules_by_L(ns, ls).items():
        b0 = _evaluate_complex(sched, d0).reshape(sched.basis_count, 2 * L + 1)
        b1 = _evaluate_complex(sched, d1).reshape(sched.basis_count, 2 * L + 1)
        np.testing.assert_allclose(np.sum(np.abs(b0) ** 2, axis=1), np.sum(np.abs(b1) ** 2, axis=1),
                                   rtol=1e-10, atol=1e-10)
        if L == 0:
            np.testing.assert_allclose(b0, b1, rtol=1e-10, atol=1e-10)


def test_rank_two_schedule_coefficients_are_cg_values():
    sched = generate_factorized_coefficient_schedules_by_L((1, 2), (2, 3))[3]
    C = cg_matrix(2, 3, 3)
    for k in range(sched.component_count):
        M = int(sched.component_M_R[k])
        tuples, coeffs = sched.component_terms(k)
        expected = [(m1, M - m1) for m1 in range(-2, 3) if abs(M - m1) <= 3 and C[m1 + 2, M - m1 + 3] != 0]
        assert [tuple(map(int, t)) for t in tuples] == expected
        assert np.array_equal(coeffs.real, [C[a + 2, b + 3] for a, b in expected])


# ------------------------------------------------------------ real lowering
@pytest.mark.parametrize("ns,ls", [((1, 1, 1), (1, 2, 3)), ((1, 1, 1), (2, 2, 2)), ((1, 1, 1), (3, 3, 3)),
                                   ((1, 1, 1), (1, 1, 2)), ((1, 1, 1), (0, 1, 1)), ((1, 1, 1, 1), (2, 2, 2, 2)),
                                   ((1, 1, 1), (1, 1, 1))])
def test_real_plan_equals_unitary_transform_of_complex_schedule(ns, ls):
    """B^r = phase * W_L^dagger B^c(W A^r): the real plan is the reference schedule in real coordinates."""
    from ye3t_amd.ace.plan import ACEFeatureSpec, ProductPlan, _label_phase_odd
    from ye3t_amd.core.cg import parity_phase
    import oracle

    l_max = max(ls)
    spec = ACEFeatureSpec(channel_count=max(ns), l_max=l_max, nu_max=len(ls), nu_min=len(ls),
                          targets=tuple(range(0, sum(ls) + 1)))
    spec_contents = [(basis.canonicalize_leaf_quantum_numbers(ns, ls))]
    spec.contents = lambda: iter(spec_contents)
    plan_ = ProductPlan(spec)
    rng = np.random.default_rng(9)
    A = rng.normal(size=(3, plan_.a_width))
    B = oracle.ace_product_flat(A, plan_.flat_arrays())
    scheds = generate_factorized_coefficient_schedules_by_L(*spec_contents[0])
    for s in range(3):
        dens = {}
        for n in set(ns):
            for l in set(ls):
                off = spec.leaf_offset(n, l)
                dens[(n, l)] = real_to_complex_unitary(l) @ A[s, off:off + 2 * l + 1]
        for L, ci, lab, first in plan_.label_records:
            sched = scheds[L]
            li = list(sched.structured_labels).index(lab)
            bc = _evaluate_complex(sched, dens).reshape(sched.basis_count, 2 * L + 1)[li]
            odd = _label_phase_odd(lab)
            expected = (parity_phase(1) ** odd) * (np.conj(real_to_complex_unitary(L)).T @ bc)
            np.testing.assert_allclose(expected.imag, 0, atol=1e-10)
            np.testing.assert_allclose(B[s, first:first + 2 * L + 1], expected.real, rtol=1e-10, atol=1e-10)
