"""The HIP product program, executed by a CPU emulator of the kernel's semantics.

Checks the DAG lowering (chunking, slot assignment, word encoding) against the
oracle's flat evaluation before any GPU run, and checks every index the kernel
will read against its buffers.
"""

import numpy as np
import pytest

import oracle
from ye3t_amd.ace import workloads as W
from ye3t_amd.ace.plan import ACEFeatureSpec, ProductPlan
from ye3t_amd.ace.program import OP_ACC1, OP_ACC2, OP_ACC3, OP_ACC4, OP_LOAD, compile_program, program_stats


def emulate(prog, A):
    """Execute a compiled program on [S, a_width] rows exactly as product_kernel does."""
    S = A.shape[0]
    F = prog["feature_count"]
    B = np.zeros((S, F))
    words, coeffs = prog["words"], prog["coeffs"].astype(np.float64)
    slots = prog["workspace_slots"]
    for c in range(prog["chunk_count"]):
        ws = np.zeros((slots, S))
        i, end = int(prog["chunk_word_offsets"][c]), int(prog["chunk_word_offsets"][c + 1])
        ci = int(prog["chunk_coeff_offsets"][c])
        while i < end:
            h = int(words[i])
            op, n = h >> 28, h & 0xFFFFFF
            if op == OP_LOAD:
                for t in words[i + 1:i + 1 + n]:
                    t = int(t)
                    assert (t >> 16) < slots and (t & 0xFFFF) < prog["a_width"]
                    ws[t >> 16] = A[:, t & 0xFFFF]
                i += 1 + n
                continue
            dst = int(words[i + 1])
            assert dst < slots
            i += 2
            acc = np.zeros(S)
            for q in range(n):
                if op == OP_ACC1:
                    m = ws[int(words[i + q]) & 0xFFFF]
                elif op == OP_ACC2:
                    t = int(words[i + q])
                    m = ws[t & 0xFFFF] * ws[t >> 16]
                else:
                    t0, t1 = int(words[i + 2 * q]), int(words[i + 2 * q + 1])
                    m = ws[t0 & 0xFFFF] * ws[t0 >> 16] * ws[t1 & 0xFFFF]
                    if op == OP_ACC4:
                        m = m * ws[t1 >> 16]
                acc = acc + coeffs[ci + q] * m
            i += n if op in (OP_ACC1, OP_ACC2) else 2 * n
            ci += n
            ws[dst] = acc
        assert ci == prog["chunk_coeff_offsets"][c + 1]
        o0, o1 = int(prog["chunk_out_offsets"][c]), int(prog["chunk_out_offsets"][c + 1])
        f0 = int(prog["chunk_first_column"][c])
        B[:, f0:f0 + (o1 - o0)] = ws[prog["out_slots"][o0:o1].astype(np.int64)].T
    return B


def _check_cover(prog):
    cols = []
    for c in range(prog["chunk_count"]):
        o0, o1 = prog["chunk_out_offsets"][c], prog["chunk_out_offsets"][c + 1]
        cols.extend(range(prog["chunk_first_column"][c], prog["chunk_first_column"][c] + o1 - o0))
    assert cols == list(range(prog["feature_count"]))


@pytest.mark.parametrize("max_slots", [48, 96, 250])
def test_config4_program_matches_flat_oracle(max_slots):
    cfg = W.config(4)
    plan = ProductPlan(cfg.feature_spec)
    assert plan.feature_count == 161
    prog = compile_program(plan, "f64", max_slots)
    _check_cover(prog)
    A = np.random.default_rng(0).normal(size=(37, plan.a_width))
    np.testing.assert_allclose(emulate(prog, A), oracle.ace_product_flat(A, plan.flat_arrays()),
                               rtol=1e-12, atol=1e-11)


def test_config2_program_matches_flat_oracle():
    cfg = W.config(2)
    plan = ProductPlan(cfg.feature_spec)
    assert plan.feature_count == 3273
    prog = compile_program(plan, "f64")
    _check_cover(prog)
    st = program_stats(prog)
    assert st["workspace_slots"] <= 48
    A = np.random.default_rng(1).normal(size=(5, plan.a_width))
    np.testing.assert_allclose(emulate(prog, A), oracle.ace_product_flat(A, plan.flat_arrays()),
                               rtol=1e-11, atol=1e-10)


def test_rank_four_and_species_program():
    spec = ACEFeatureSpec(channel_count=6, l_max=2, nu_max=4, targets=(0, 1), parity="any",
                          radial_per_species=3, caps={1: (3, 2), 2: (2, 2), 3: (2, 1), 4: (1, 2)})
    plan = ProductPlan(spec)
    prog = compile_program(plan, "f32", 64)
    _check_cover(prog)
    A = np.random.default_rng(2).normal(size=(9, plan.a_width))
    np.testing.assert_allclose(emulate(prog, A), oracle.ace_product_flat(A, plan.flat_arrays()),
                               rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("max_live,per", [(16, 1), (24, 3), (1 << 30, 4)])
def test_generated_parts_cover_the_outputs_in_order(max_live, per):
    """``codegen.generate_parts``: consecutive parts hand over at chunk
    boundaries, cover every output once, and a part's kernel switches over its
    own chunks (mapped from the linear workgroup id) and writes only its
    columns (never the whole-row tile store of a one-chunk plan)."""
    import re

    from ye3t_amd.ace import codegen

    plan = ProductPlan(W.config(4).feature_spec)
    chunks = codegen._chunks(plan, max_live)
    parts = codegen.generate_parts(plan, "f64", max_live=max_live, chunks_per_part=per, out_dtype="f32")
    assert len(parts) == -(-len(chunks) // per)
    assert sum(m["chunks"] for _, m in parts) == len(chunks)
    first = 0
    for k, (src, meta) in enumerate(parts):
        assert meta["first_output"] == first and meta["kernel"] == "ye3t_product_part"
        lo, hi = meta["first_output"], meta["last_output"]
        assert (lo, hi) == (chunks[k * per][0], chunks[min(len(chunks), (k + 1) * per) - 1][1])
        assert src.count("  case ") == meta["chunks"] and "switch (chunk)" in src
        cols = [int(g) for g in re.findall(r"B\[\(s0 \+ r\) \* \d+L \+ (\d+) \+ c\]", src)]
        assert cols and min(cols) == lo and max(cols) < hi
        first = hi
    assert first == plan.feature_count


def test_adjoint_parts_reduction_map():
    """``codegen.generate_adjoint_parts``: every partial row belongs to exactly
    one density column, a column's rows come in chunk order, the parts' row
    ranges tile the partial buffer, and each part writes exactly its rows."""
    import re

    from ye3t_amd.ace import codegen

    plan = ProductPlan(W.config(4).feature_spec)
    parts, red = codegen.generate_adjoint_parts(plan, "f64", max_live=24, chunks_per_part=2, grad_dtype="f32",
                                                in_dtype="f32")
    col_off, rows = red["col_off"], red["rows"]
    assert len(col_off) == plan.a_width + 1 and col_off[0] == 0 and col_off[-1] == len(rows)
    assert sorted(rows.tolist()) == list(range(red["partial_rows"]))
    for k in range(plan.a_width):
        seg = rows[col_off[k]:col_off[k + 1]]
        assert np.all(np.diff(seg) > 0)
    first = 0
    for src, meta in parts:
        assert meta["first_row"] == first
        written = sorted(int(r) for r in re.findall(r"\*\(REAL\*\)\(pt \+ (\d+)L \* pb \+ plane\)", src))
        assert written == list(range(meta["first_row"], meta["last_row"]))
        first = meta["last_row"]
    assert first == red["partial_rows"]


def test_readout_parts_weight_every_feature_once():
    """``codegen.generate_readout_parts``: the parts use the chunks of the
    forward parts, every feature's weight enters exactly one chunk's partial
    sum, each chunk writes its own partial row, and the features are emitted
    with the same text as the forward parts (so they agree bit for bit)."""
    import re

    from ye3t_amd.ace import codegen

    plan = ProductPlan(W.config(4).feature_spec)
    chunks = codegen._chunks(plan, 96)
    parts, count = codegen.generate_readout_parts(plan, "f64", max_live=96, chunks_per_part=3)
    assert count == len(chunks) and len(parts) == -(-count // 3)
    weights, rows = [], []
    for src, meta in parts:
        assert meta["kernel"] == "ye3t_product_readout_part" and src.count("  case ") == meta["chunks"]
        weights += [int(g) for g in re.findall(r"W\[(\d+)\]", src)]
        rows += [int(g) for g in re.findall(r"P\[(\d+)L \* ldp \+ s\]", src)]
    assert sorted(weights) == list(range(plan.feature_count))
    assert rows == list(range(count))
    fwd = "\n".join(s for s, _ in codegen.generate_parts(plan, "f64", max_live=96, chunks_per_part=3))
    node_lines = {ln.strip() for ln in fwd.splitlines() if ln.strip().startswith("const REAL v")}
    for src, _ in parts:
        for ln in src.splitlines():
            if ln.strip().startswith("const REAL v"):
                assert ln.strip() in node_lines
