"""The schedule compiler pinned against what the reference itself holds.

* ``factorized_runtime.cpp`` -- the reference's C++ schedule assembler and CPU
  evaluator -- compiled from its source into ``oracle/_ref`` (``make -C oracle
  ref``): the builder's complex schedules must equal its output (offsets,
  labels and block m-tuples exactly, coefficients to a few ulps) and the
  oracle's evaluator must agree with its evaluator.  Skipped where the module
  is not built (the GPU box never holds it).
* label payloads the reference's tests freeze
  (``tests/test_scalar_ace_coordinate.py:233-278``,
  ``tests/test_basis_labels.py:128-166``) appear in ``count()``'s labels;
* the real-tesseral schedule obeys the reference's own relation to the complex
  schedule (``tests/test_numeric_structured_expansion.py:411-480``) with the
  tesseral map its test writes out (``:495-540``);
* the ACE plans' real basis (the spherical-harmonic tables' ordering) is the
  tesseral ordering reversed, component by component, and with that reversal
  the builder's Sym^2(V_1) table is the reference fixture's
  (``tests/fixtures/shared_monomial_plan_v1.txt``).
"""

import json
import os

import numpy as np
import pytest

from ye3t_amd.core import basis as B
from ye3t_amd.core import couplings as C
from ye3t_amd.core import symmetric_power as SP
from ye3t_amd.core.cg import real_to_complex_unitary, tesseral_unitary
from ye3t_amd.couplings import count

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SO = os.path.join(HERE, "..", "oracle", "_ref", "ye3t_factorized_ref.so")


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_SO):
        pytest.skip("reference factorized_runtime module not built (make -C oracle ref)")
    import importlib.util

    import torch  # noqa: F401  (the module links against libtorch)

    spec = importlib.util.spec_from_file_location("ye3t_factorized_ref", REF_SO)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _contents(config_id, limit, seed):
    """(n, l) contents of a benchmark configuration (a seeded sample of at most ``limit``)."""
    from ye3t_amd.ace import workloads as W

    if config_id == 1:
        return [((1, 1, 2), (1, 1, 0))]
    contents = [c for c in W.config(config_id).feature_spec.contents() if len(c[0]) >= 2]
    if len(contents) > limit:
        rng = np.random.default_rng(seed)
        contents = [contents[i] for i in sorted(rng.choice(len(contents), limit, replace=False))]
    return contents


def _ulp_bound(rank):
    """A product of ``rank - 1`` CG values, each rounded within about 2 ulps on
    either side: the two fp64 routes may differ by that many ulps per factor."""
    return 2.0 * max(1, rank - 1) + 1.0


def _ulps(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if not a.size:
        return 0.0
    return float(np.max(np.abs(a - b) / np.spacing(np.maximum(np.abs(a), np.abs(b)))))


# ---------------------------------------------------------- reference assembler
@pytest.mark.parametrize("config_id,limit", [(1, 1), (2, 40), (3, 25), (4, 40)])
def test_complex_schedules_equal_reference_assembler(ref, config_id, limit):
    """``assemble_factorized_schedule_from_keys_cpp`` (``factorized_runtime.cpp:301-424``)
    on the builder's path keys reproduces every array of the builder's schedule."""
    checked, worst = 0, 0.0
    for n_c, l_c in _contents(config_id, limit, seed=config_id):
        for L, s in C.generate_factorized_coefficient_schedules_by_L(n_c, l_c).items():
            if not s.structured_labels or s.rank < 3:
                continue  # rank <= 2 uses the direct fast paths, not the assembler
            keys = [B.path_key(lab) for lab in s.structured_labels]
            li, cm, offs, tup, co = (t.numpy() for t in ref.assemble_factorized_schedule_from_keys_cpp(
                keys, list(range(-L, L + 1)), 1e-14))
            assert np.array_equal(li, s.component_label_index), (n_c, l_c, L)
            assert np.array_equal(cm, s.component_M_R), (n_c, l_c, L)
            assert np.array_equal(offs, s.component_offsets), (n_c, l_c, L)
            assert np.array_equal(tup, s.block_m_tuples), (n_c, l_c, L)
            worst = max(worst, _ulps(co, s.coeffs.real) / _ulp_bound(s.rank))
            checked += 1
    assert checked or config_id == 1
    # both sides round CG products in fp64 by different routes (Racah sums here,
    # log-factorials there): a few ulps, far below the 1e-12 parity bar
    assert worst <= 1.0, worst


def test_config1_rank3_schedule_equals_reference_assembler(ref):
    s = C.generate_factorized_coefficient_schedules_by_L((1, 1, 2), (1, 1, 0))[0]
    keys = [B.path_key(lab) for lab in s.structured_labels]
    li, cm, offs, tup, co = (t.numpy() for t in ref.assemble_factorized_schedule_from_keys_cpp(keys, [0], 1e-14))
    assert np.array_equal(offs, s.component_offsets) and np.array_equal(tup, s.block_m_tuples)
    assert _ulps(co, s.coeffs.real) <= _ulp_bound(3)


def test_path_expansion_equals_reference(ref):
    """``expand_block_m_path_arrays_cpp`` (``factorized_runtime.cpp:151-224``) per key."""
    for n_c, l_c in [((1, 1, 1), (1, 2, 3)), ((1, 1, 1, 1), (2, 2, 2, 2)), ((1, 2, 3, 4), (1, 2, 2, 3))]:
        for L, labs in B.structured_labels_by_L(n_c, l_c).items():
            for lab in labs[:6]:
                key = B.path_key(lab)
                rM, tup, co = (t.numpy() for t in ref.expand_block_m_path_arrays_cpp(key))
                oM, otup, oco = C.expand_path_key(key)
                assert np.array_equal(rM, oM) and np.array_equal(tup, otup)
                assert _ulps(co, oco) <= _ulp_bound(len(lab_l := B.l_sequence(lab))), lab_l


def test_oracle_evaluator_equals_reference_evaluator(ref):
    """``evaluate_factorized_schedule_cpu`` (``factorized_runtime.cpp:251-285, 426-548``)
    against the oracle's restatement on the same schedule and block values."""
    import torch

    import oracle

    rng = np.random.default_rng(5)
    for n_c, l_c in [((1, 1, 2), (1, 1, 0)), ((1, 1, 1), (1, 2, 3)), ((1, 1, 2, 2), (1, 1, 2, 2)),
                     ((1, 1, 1, 1), (2, 2, 2, 2))]:
        for L, s in C.generate_factorized_coefficient_schedules_by_L(n_c, l_c).items():
            flat = s.flat_arrays()
            bv = rng.normal(size=(7, s.basis_count, s.block_count, flat["max_block_m_dim"]))
            got = oracle.evaluate_componentwise(bv, flat)
            want = ref.evaluate_factorized_schedule_cpu(
                torch.from_numpy(bv), torch.from_numpy(flat["component_offsets"]),
                torch.from_numpy(flat["component_label_index"]), torch.from_numpy(flat["block_m_indices"]),
                torch.from_numpy(flat["coeffs"]), s.component_count, True).numpy()
            scale = max(1.0, float(np.max(np.abs(want))))
            assert np.max(np.abs(got - want)) <= 1e-13 * scale, (n_c, l_c, L)


# ------------------------------------------------------------------- labels
# (payload of test_scalar_ace_coordinate.py:233-278) -> compact label
SCALAR_ACE_PAYLOADS = [
    ({"n_tuple": [1, 1, 1, 1], "l_tuple": [1, 1, 1, 1], "internal_Ls": [0], "L_R": 0,
      "tree_type": "balanced", "basis_key": ["sym", 0, 0]}),
    ({"n_tuple": [1, 1, 1, 2], "l_tuple": [1, 1, 1, 1], "internal_Ls": [1, 0], "L_R": 0,
      "tree_type": "balanced", "basis_key": ["node", ["sym", 1, 0], []]}),
    ({"n_tuple": [1, 1, 1, 1, 2, 2, 2, 2], "l_tuple": [1] * 8, "internal_Ls": [4, 4, 0], "L_R": 0,
      "tree_type": "balanced", "basis_key": ["node", ["sym", 4, 0], ["sym", 4, 0]]}),
]


def _tup(x):
    return tuple(_tup(v) for v in x) if isinstance(x, (list, tuple)) else x


@pytest.mark.parametrize("payload", SCALAR_ACE_PAYLOADS)
def test_frozen_scalar_ace_labels_appear_in_count(payload):
    compact = (_tup(payload["n_tuple"]), _tup(payload["l_tuple"]), _tup(payload["internal_Ls"]),
               payload["tree_type"], _tup(payload["basis_key"]))
    report = count(content=compact[0], input_Ls=compact[1], target_L=payload["L_R"])
    labels = [lab.compact_label() for lab in report.labels_for_target(payload["L_R"])]
    assert compact in labels
    assert labels == sorted(labels)
    # the structured label behind it round-trips through the compact form
    lab = C.structured_label_from_compact(compact)
    assert B.compact_label(lab) == compact


def test_basis_label_fixture_heads_appear_in_count():
    """``tests/test_basis_labels.py:128-166`` hold the compact labels
    ``((1, 1), (0, 0), (0,))`` (a printer fixture: the head of the Sym^2(V_0)
    label, whose sym key ``count`` appends) and ``((2, 5), (0, 0), (0,))``."""
    (lab,) = count(content=(1, 1), input_Ls=(0, 0), target_L=0).labels_for_target(0)
    assert lab.payload() == ((1, 1), (0, 0), (0,), "balanced", ("sym", 0, 0))
    (lab,) = count(content=(2, 5), input_Ls=(0, 0), target_L=0).labels_for_target(0)
    assert lab.compact_label() == ((2, 5), (0, 0), (0,))


# ----------------------------------------------------------- real tesseral
def test_tesseral_unitary_is_the_reference_formula():
    """The map written out in ``test_numeric_structured_expansion.py:495-520``:
    cosine at ``L-m``, sine at ``L+m``."""
    for L in range(1, 5):
        values = np.linspace(-0.8, 1.1, 3 * (2 * L + 1)).reshape(3, 2 * L + 1)
        parts = []
        for m in range(L, 0, -1):
            parts.append((values[:, L - m] + 1j * values[:, L + m]) * 2 ** -0.5)
        parts.append(values[:, L].astype(np.complex128))
        for m in range(1, L + 1):
            parts.append((-1) ** m * (values[:, L - m] - 1j * values[:, L + m]) * 2 ** -0.5)
        expected = np.stack(parts, axis=-1)
        np.testing.assert_allclose(values @ tesseral_unitary(L).T, expected, rtol=0, atol=2e-15)
        # the spherical-harmonic tables' ordering is the same map with the index reversed
        np.testing.assert_array_equal(real_to_complex_unitary(L)[:, ::-1], tesseral_unitary(L))


def _complex_blocks(real_blocks, block_L):
    out = np.zeros(real_blocks.shape, dtype=np.complex128)
    for li in range(block_L.shape[0]):
        for bi in range(block_L.shape[1]):
            L = int(block_L[li, bi])
            w = 2 * L + 1
            out[:, li, bi, :w] = real_blocks[:, li, bi, :w] @ tesseral_unitary(L).T
    return out


def _eval(bv, flat):
    out = np.zeros((bv.shape[0], flat["component_offsets"].shape[0] - 1), dtype=bv.dtype)
    for k in range(out.shape[1]):
        lab = flat["component_label_index"][k]
        for t in range(flat["component_offsets"][k], flat["component_offsets"][k + 1]):
            v = np.full(bv.shape[0], flat["coeffs"][t], dtype=bv.dtype)
            for blk in range(bv.shape[2]):
                v = v * bv[:, lab, blk, flat["block_m_indices"][t, blk]]
            out[:, k] += v
    return out


@pytest.mark.parametrize("n_tuple,l_tuple", [((1, 1, 2, 2), (1, 1, 1, 1)), ((1, 2, 3), (1, 1, 1)),
                                             ((1, 2, 3), (1, 1, 2)), ((1, 2, 3), (1, 2, 2)),
                                             ((1, 2, 3), (2, 2, 2))])
def test_real_schedule_matches_complex_scalar_schedule(n_tuple, l_tuple):
    """Restates ``test_real_factorized_schedule_matches_complex_scalar_schedule``
    (``tests/test_numeric_structured_expansion.py:411-480``)."""
    labels = count(content=n_tuple, input_Ls=l_tuple, target_L=0).labels_for_target(0)
    assert labels
    complex_schedule = C.generate_factorized_coefficient_schedules_by_L(n_tuple, l_tuple)[0]
    real_schedule = C.generate_real_factorized_coefficient_schedule_for_labels(labels, component_indices=(0,))
    assert real_schedule.basis_convention == "real_tesseral"
    assert real_schedule.permutation_sector == "trivial"
    assert real_schedule.backend_provenance == "real_cg_direct"
    assert real_schedule.complex_term_count == complex_schedule.term_count
    flat_r, flat_c = real_schedule.flat_arrays(), complex_schedule.flat_arrays()
    rng = np.random.default_rng(2028)
    real_blocks = rng.normal(size=(5, real_schedule.basis_count, real_schedule.block_count,
                                   flat_r["max_block_m_dim"]))
    cblocks = _complex_blocks(real_blocks, real_schedule.block_L_by_label())
    real_out = _eval(real_blocks, flat_r)
    complex_out = _eval(cblocks, {**flat_c, "coeffs": complex_schedule.coeffs})
    phased = (-1j if sum(l_tuple) % 2 else 1.0) * complex_out
    np.testing.assert_allclose(real_out, phased.real, rtol=1e-10, atol=1e-10)
    assert np.max(np.abs(phased.imag)) <= 1e-10
    if sum(l_tuple) % 2:
        assert np.max(np.abs(complex_out.imag)) > 1e-3


def _odd_nodes(label):
    if label[0] != "node":
        return 0
    return (_odd_nodes(label[1]) + _odd_nodes(label[2])
            + (B.total_L(label[1]) + B.total_L(label[2]) - label[3]) % 2)


@pytest.mark.parametrize("n_tuple,l_tuple", [((1, 1, 1), (1, 2, 3)), ((1, 1, 2), (2, 2, 1)),
                                             ((1, 1, 1, 1), (2, 2, 2, 2))])
def test_real_schedule_covariant_components(n_tuple, l_tuple):
    """All ``2L+1`` components: ``real = Re(phase * W_tess,L^dagger complex)``."""
    for L, cs in C.generate_factorized_coefficient_schedules_by_L(n_tuple, l_tuple).items():
        labels = count(content=n_tuple, input_Ls=l_tuple, target_L=L).labels_for_target(L)
        rs = C.generate_real_factorized_coefficient_schedule_for_labels(labels)
        fr, fc = rs.flat_arrays(), cs.flat_arrays()
        X = np.random.default_rng(L).normal(size=(3, rs.basis_count, rs.block_count, fr["max_block_m_dim"]))
        real_out = _eval(X, fr).reshape(3, rs.basis_count, 2 * L + 1)
        cout = _eval(_complex_blocks(X, rs.block_L_by_label()), {**fc, "coeffs": cs.coeffs})
        cout = cout.reshape(3, cs.basis_count, 2 * L + 1) @ np.conj(tesseral_unitary(L))
        # each odd coupling node contributes its own factor -i
        odd = np.array([_odd_nodes(lab) for lab in rs.structured_labels])
        phased = ((-1j) ** odd)[None, :, None] * cout
        np.testing.assert_allclose(real_out, phased.real, rtol=1e-10, atol=1e-10)
        assert np.max(np.abs(phased.imag)) <= 1e-10


@pytest.mark.parametrize("ns,ls", [((1, 1, 1), (1, 2, 3)), ((1, 1, 1), (2, 2, 2)), ((1, 1, 2), (1, 1, 0)),
                                   ((1, 1, 1, 1), (2, 2, 2, 2)), ((1, 1, 2, 2), (1, 1, 2, 2))])
def test_ace_real_plan_is_reversed_tesseral_schedule(ns, ls):
    """The ACE plans' real features = the reference's real-tesseral schedule on
    the reversed multiplets, output reversed (leaves: ``A[2l-a]``; sym blocks:
    the builder's real sym block reversed)."""
    import oracle
    from ye3t_amd.ace.plan import ACEFeatureSpec, ProductPlan

    spec = ACEFeatureSpec(channel_count=max(ns), l_max=max(ls), nu_max=len(ls), nu_min=len(ls),
                          targets=tuple(range(0, sum(ls) + 1)))
    content = B.canonicalize_leaf_quantum_numbers(ns, ls)
    spec.contents = lambda: iter([content])
    plan_ = ProductPlan(spec)
    A = np.random.default_rng(9).normal(size=(2, plan_.a_width))
    Bf = oracle.ace_product_flat(A, plan_.flat_arrays())
    for L, ci, lab, first in plan_.label_records:
        rs = C.generate_real_factorized_coefficient_schedule_for_labels([B.compact_label(lab)])
        fr = rs.flat_arrays()
        X = np.zeros((2, 1, rs.block_count, fr["max_block_m_dim"]))
        for bi, s in enumerate(rs.block_specs[0]):
            off = spec.leaf_offset(s["n"], s["l"])
            a = A[:, off:off + 2 * s["l"] + 1]
            if s["kind"] == "leaf":
                vals = a
            else:
                vals = np.zeros((2, 2 * s["Lambda"] + 1))
                for out_c, e, v in SP.real_monomial_entries(s["k_b"], s["l"], s["Lambda"], s["multiplicity_index"]):
                    vals[:, out_c] += v * np.prod(a ** np.asarray(e), axis=1)
            X[:, 0, bi, :vals.shape[1]] = vals[:, ::-1]
        got = _eval(X, fr)[:, ::-1]
        np.testing.assert_allclose(Bf[:, first:first + 2 * L + 1], got, rtol=1e-10, atol=1e-10)


# ------------------------------------------------------------ Sym^2(V_1)
def test_symmetric_square_table_matches_reference_fixture():
    """The fixture's real-tesseral Sym^2(V_1) coefficients (outputs: Lambda=0,
    and Lambda=2 components 0 and 2 in tesseral order) are the builder's table
    with input and output indices reversed."""
    fx = json.load(open(os.path.join(HERE, "golden", "shared_monomial_plan_v1.json")))
    counts = np.asarray(fx["monomial_counts"], dtype=np.int64).reshape(int(fx["monomial_count"]),
                                                                       int(fx["input_dimension"]))
    fixture = {}
    for out, term, value in zip(fx["coefficient_outputs"], fx["coefficient_terms"], fx["coefficient_values"]):
        fixture[(int(out), tuple(int(x) for x in counts[int(term)]))] = float(value)
    outputs = {0: (0, 0), 1: (2, 0), 2: (2, 2)}  # fixture output -> (Lambda, tesseral component)
    ours = {}
    for out, (Lam, comp) in outputs.items():
        for c, e, v in SP.real_monomial_entries(2, 1, Lam, 0):
            if c == 2 * Lam - comp:
                ours[(out, tuple(e[::-1]))] = v
    assert ours.keys() == fixture.keys()
    for key, value in fixture.items():
        assert abs(ours[key] - value) <= 4 * np.spacing(abs(value)), (key, ours[key], value)
