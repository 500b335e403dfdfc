"""The term stream of the device interpreter, checked on the CPU.

``native.stream_encode`` returns the records the HIP interpreter runs (host
code only).  These tests check the encoder's invariants and execute the
records with numpy -- forward as written, forward with each group's reads
hoisted above its stores (what the device kernel does), and the reverse
sweep of the adjoint kernel -- against the pinned oracle.
"""

import numpy as np
import pytest

import oracle
from tests._util import column_rel_error
from ye3t_amd.ace import workloads as W
from ye3t_amd.ace.plan import ACEFeatureSpec, ProductPlan
from ye3t_amd.ace.program import compile_program
from ye3t_amd.runtime import native

FLUSH, CHAIN, CHAINED = 1, 2, 4


def _rank4_spec():
    return ACEFeatureSpec(channel_count=44, l_max=4, nu_max=4, targets=(0,), parity="even",
                          radial_per_species=11, caps={1: (11, 0), 2: (3, 4), 3: (2, 2), 4: (1, 2)})


@pytest.fixture(scope="module", params=[("config4", "f64"), ("config4", "f32"), ("rank4", "f64"), ("config2", "f64")])
def case(request):
    name, dtype = request.param
    spec = {"config4": W.config(4).feature_spec, "rank4": _rank4_spec(), "config2": W.config(2).feature_spec}[name]
    plan = ProductPlan(spec)
    prog = compile_program(plan, dtype)
    return plan, prog, native.stream_encode(prog)


def _decode(prog, st):
    elem = 8 if prog["dtype"] == "f64" else 4
    pitch = 64 * elem
    rec = st["records"]
    if elem == 8:
        coef = (rec[:, 2].astype(np.uint64) | (rec[:, 3].astype(np.uint64) << np.uint64(32))).view(np.float64)
    else:
        coef = rec[:, 2].copy().view(np.float32).astype(np.float64)
    assert np.all(rec[:, 0] % pitch == 0) and np.all(rec[:, 1] % pitch == 0)
    return {"a": rec[:, 0] // pitch, "b": rec[:, 1] // pitch, "c": coef, "f": st["flags"] & 0xFFFF,
            "dst": (st["flags"] >> 16) // pitch, "ld_dst": st["loads"][:, 0] // pitch, "ld_col": st["loads"][:, 1],
            "pitch": pitch}


def test_encoder_invariants(case):
    plan, prog, st = case
    assert st is not None
    d = _decode(prog, st)
    G = st["layout"]["group"]
    slots = prog["workspace_slots"]
    one, sink = slots, slots + 1
    assert st["layout"]["one_off"] == one * d["pitch"]
    for ch in range(prog["chunk_count"]):
        r0, r1 = st["rec_off"][ch], st["rec_off"][ch + 1]
        l0, l1 = st["load_off"][ch], st["load_off"][ch + 1]
        assert (r1 - r0) % G == 0 and (l1 - l0) % 8 == 0
        for g0 in range(r0, r1, G):
            flushed = set()
            for q in range(g0, g0 + G):
                assert d["a"][q] not in flushed and d["b"][q] not in flushed, "a group reads a slot it flushed"
                if d["f"][q] & FLUSH:
                    flushed.add(d["dst"][q])
        for q in range(r0, r1):
            assert d["a"][q] <= sink and d["b"][q] <= sink
            if d["f"][q] & FLUSH:
                assert d["dst"][q] < slots
            if d["f"][q] & CHAINED:
                assert q > r0 and d["f"][q - 1] & CHAIN, "a chained record must follow its chain record"
        assert np.all(d["ld_col"][l0:l1] < prog["a_width"]) and np.all(d["ld_dst"][l0:l1] <= sink)
    assert st["layout"]["lds_bytes"] <= 64 * 1024


def _forward(prog, st, A, grouped):
    """B from the stream; ``grouped``: each group's factors read before its stores."""
    d = _decode(prog, st)
    S = A.shape[0]
    slots = prog["workspace_slots"]
    G = st["layout"]["group"]
    B = np.zeros((S, prog["feature_count"]))
    values = []
    for ch in range(prog["chunk_count"]):
        ws = np.zeros((slots + 2, S))
        ws[slots] = 1.0
        for q in range(st["load_off"][ch], st["load_off"][ch + 1]):
            ws[d["ld_dst"][q]] = A[:, d["ld_col"][q]]
        acc, p = np.zeros(S), np.ones(S)
        r0, r1 = st["rec_off"][ch], st["rec_off"][ch + 1]
        for g0 in range(r0, r1, G):
            if grouped:
                fa = [ws[d["a"][q]].copy() for q in range(g0, g0 + G)]
                fb = [ws[d["b"][q]].copy() for q in range(g0, g0 + G)]
            for k, q in enumerate(range(g0, g0 + G)):
                a = fa[k] if grouped else ws[d["a"][q]]
                b = fb[k] if grouped else ws[d["b"][q]]
                f = d["f"][q]
                if f & CHAIN:
                    p = a * b
                    continue
                t = (p * a) * b if f & CHAINED else a * b
                acc = d["c"][q] * t + acc
                if f & FLUSH:
                    ws[d["dst"][q]] = acc
                    acc = np.zeros(S)
        o0, o1 = prog["chunk_out_offsets"][ch], prog["chunk_out_offsets"][ch + 1]
        c0 = prog["chunk_first_column"][ch]
        B[:, c0:c0 + (o1 - o0)] = ws[prog["out_slots"][o0:o1]].T
        values.append(ws)
    return B, values


def test_stream_forward_matches_the_oracle(case):
    plan, prog, st = case
    A = np.random.default_rng(21).normal(size=(48, plan.a_width))
    if prog["dtype"] == "f32":
        A = A.astype(np.float32).astype(np.float64)
    B_seq, _ = _forward(prog, st, A, grouped=False)
    B_grp, _ = _forward(prog, st, A, grouped=True)
    assert np.array_equal(B_seq, B_grp)  # hazard-free groups: hoisted reads change nothing
    ref = oracle.ace_product_flat(A, plan.flat_arrays())
    # fp64 emulation of the records; fp32 programs only round their coefficients
    assert column_rel_error(B_seq, ref) < (1e-12 if prog["dtype"] == "f64" else 1e-6)


def test_stream_reverse_sweep_matches_the_oracle(case):
    """The adjoint kernel's sweep: g read at the flushing record, plain records
    add c g b / c g a, chained pairs differentiate through p."""
    plan, prog, st = case
    if prog["dtype"] != "f64":
        pytest.skip("fp64 programs cover the sweep")
    rng = np.random.default_rng(22)
    S = 24
    A = rng.normal(size=(S, plan.a_width))
    gB = rng.normal(size=(S, prog["feature_count"]))
    d = _decode(prog, st)
    slots = prog["workspace_slots"]
    _, values = _forward(prog, st, A, grouped=False)
    gA = np.zeros_like(A)
    for ch in range(prog["chunk_count"]):
        ws = values[ch]
        gs = np.zeros_like(ws)
        o0, o1 = prog["chunk_out_offsets"][ch], prog["chunk_out_offsets"][ch + 1]
        c0 = prog["chunk_first_column"][ch]
        for k, slot in enumerate(prog["out_slots"][o0:o1]):
            gs[slot] += gB[:, c0 + k]
        g = np.zeros(S)
        r0, r1 = st["rec_off"][ch], st["rec_off"][ch + 1]
        for q in range(r1 - 1, r0 - 1, -1):
            f = d["f"][q]
            if f & CHAIN:
                continue
            if f & FLUSH:
                g = gs[d["dst"][q]].copy()
            a, b = ws[d["a"][q]], ws[d["b"][q]]
            cg = d["c"][q] * g
            if f & CHAINED:
                a1, b1 = ws[d["a"][q - 1]], ws[d["b"][q - 1]]
                pp, ab = a1 * b1, a * b
                gs[d["a"][q]] += cg * pp * b
                gs[d["b"][q]] += cg * pp * a
                gs[d["a"][q - 1]] += cg * ab * b1
                gs[d["b"][q - 1]] += cg * ab * a1
            else:
                gs[d["a"][q]] += cg * b
                gs[d["b"][q]] += cg * a
        for q in range(st["load_off"][ch], st["load_off"][ch + 1]):
            if d["ld_dst"][q] != slots + 1:
                gA[:, d["ld_col"][q]] += gs[d["ld_dst"][q]]
    ref = oracle.ace_product_flat_adjoint(A, gB, plan.flat_arrays())
    assert column_rel_error(gA, ref) < 1e-12


def test_wide_workspaces_get_no_stream():
    plan = ProductPlan(W.config(4).feature_spec)
    prog = compile_program(plan, "f64", 130)
    # 125 + 2 fp64 slots (63.5 KB) plus the staged density loads and output
    # slots of the widest chunk exceed 64 KB of LDS
    assert prog["workspace_slots"] == 125
    assert native.stream_encode(prog) is None


def test_records_take_no_lds():
    """Records and flags are read through the scalar cache, so only the
    workspace, the density-load list and the output slots must fit 64 KB: a
    120-slot fp64 workspace (61 KB) still gets a term stream."""
    plan = ProductPlan(W.config(4).feature_spec)
    prog = compile_program(plan, "f64", 120)
    st = native.stream_encode(prog)
    assert st is not None
    lay = st["layout"]
    assert lay["rec_at"] == lay["flag_at"] == lay["lds_bytes"] <= 64 * 1024
    assert lay["lds_bytes"] < lay["ws_bytes"] + 16 * len(st["records"])


def test_a_chunk_that_loads_a_column_twice_gets_no_stream():
    """The reverse mode adds a chunk's density gradients eight loads at a time,
    which needs each density column loaded at most once per chunk: the encoder
    refuses a program that breaks this (the plan then runs the word interpreter)."""
    plan = ProductPlan(W.config(2).feature_spec)
    prog = compile_program(plan, "f64")
    assert native.stream_encode(prog) is not None
    words = prog["words"].copy()
    w0 = int(prog["chunk_word_offsets"][0])
    assert words[w0] >> 28 == 1  # the chunk opens with its LOAD block
    n = int(words[w0] & 0xFFFFFF)
    assert n >= 2
    first_col = int(words[w0 + 1]) & 0xFFFF
    # the second load keeps its slot but reads the first load's column
    words[w0 + 2] = (int(words[w0 + 2]) & 0xFFFF0000) | first_col
    bad = dict(prog, words=words)
    assert native.stream_encode(bad) is None
