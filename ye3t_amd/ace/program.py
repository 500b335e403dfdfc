"""Lower a :class:`~ye3t_amd.ace.plan.ProductPlan` DAG to the HIP product program.

The output columns are split into *chunks* (contiguous column ranges).  Each
chunk is an independent straight-line program over a per-sample LDS workspace
of at most ``max_slots`` values:

* ``LOAD n``  -- n words ``slot << 16 | column``: copy density entries into slots;
* ``ACCk n``  -- ``dst`` then n terms of k factors (k = 1..4):
  ``ws[dst] = sum_t coeff_t * prod_q ws[slot_{t,q}]``; words hold two 16-bit
  slots each; coefficients are a separate array consumed in order.

Nodes are emitted in creation order (dependencies first).  A node needed by
several chunks is recomputed in each (chunks are independent so they can run
on different waves); within a chunk every node is computed once.
"""

import numpy as np

OP_LOAD, OP_ACC1, OP_ACC2, OP_ACC3, OP_ACC4 = 1, 2, 3, 4, 5
_ACC = {1: OP_ACC1, 2: OP_ACC2, 3: OP_ACC3, 4: OP_ACC4}
LDS_LIMIT = 64 * 1024
PAD = 65


def default_max_slots(dtype):
    return 96 if dtype == "f32" else 48


def _closure(nodes, root, out):
    stack = [root]
    while stack:
        n = stack.pop()
        if n in out:
            continue
        out.add(n)
        stack.extend(nodes[n]["deps"])
    return out


def compile_program(plan, dtype="f32", max_slots=None):
    """Return the arrays of ``ye3t_product_plan_desc`` for ``plan``."""
    if max_slots is None:
        max_slots = default_max_slots(dtype)
    elem = 8 if dtype == "f64" else 4
    hard_limit = LDS_LIMIT // (PAD * elem)
    max_slots = min(int(max_slots), hard_limit)
    nodes = plan.nodes
    # --- chunking over output columns ---------------------------------------
    chunks = []  # (first_col, last_col_exclusive, node set)
    cur_nodes, cur_first, cur_slots = set(), 0, 0
    for f, (root, _comp) in enumerate(plan.outputs):
        need = _closure(nodes, root, set())
        new = need - cur_nodes
        cost = sum(nodes[n]["dim"] for n in new)
        if cur_nodes and cur_slots + cost > max_slots:
            chunks.append((cur_first, f, cur_nodes))
            cur_nodes, cur_first, cur_slots = set(), f, 0
            new = need
            cost = sum(nodes[n]["dim"] for n in new)
        cur_nodes |= new
        cur_slots += cost
    chunks.append((cur_first, len(plan.outputs), cur_nodes))

    words, coeffs, out_slots = [], [], []
    word_off, coeff_off, out_off, first_col = [0], [0], [0], []
    workspace = 0
    for first, last, members in chunks:
        slot_of = {}
        nxt = 0
        for n in sorted(members):
            slot_of[n] = nxt
            nxt += nodes[n]["dim"]
        if nxt > hard_limit:
            raise ValueError(f"a chunk needs {nxt} workspace slots (> {hard_limit}); lower the plan size")
        workspace = max(workspace, nxt)
        loads = []
        for n in sorted(members):
            nd = nodes[n]
            if nd["kind"] == "leaf":
                for c in range(nd["dim"]):
                    loads.append(((slot_of[n] + c) << 16) | (nd["a_offset"] + c))
        if loads:
            words.append((OP_LOAD << 28) | len(loads))
            words.extend(loads)
        for n in sorted(members):
            nd = nodes[n]
            if nd["kind"] == "leaf":
                continue
            if nd["kind"] == "sym":
                src = slot_of[nd["deps"][0]]
                k = nd["k"]
                per_comp = [[] for _ in range(nd["dim"])]
                for out_c, value, factors in nd["terms"]:
                    per_comp[out_c].append((value, tuple(src + q for q in factors)))
            else:
                a, b = (slot_of[d] for d in nd["deps"])
                k = 2
                per_comp = [[] for _ in range(nd["dim"])]
                for out_c, value, (i, j) in nd["terms"]:
                    per_comp[out_c].append((value, (a + i, b + j)))
            for c, terms in enumerate(per_comp):
                words.append((_ACC[k] << 28) | len(terms))
                words.append(slot_of[n] + c)
                for value, slots in terms:
                    coeffs.append(value)
                    if k == 1:
                        words.append(slots[0])
                    elif k == 2:
                        words.append(slots[0] | (slots[1] << 16))
                    elif k == 3:
                        words.append(slots[0] | (slots[1] << 16))
                        words.append(slots[2])
                    else:
                        words.append(slots[0] | (slots[1] << 16))
                        words.append(slots[2] | (slots[3] << 16))
        for f in range(first, last):
            root, comp = plan.outputs[f]
            out_slots.append(slot_of[root] + comp)
        word_off.append(len(words))
        coeff_off.append(len(coeffs))
        out_off.append(len(out_slots))
        first_col.append(first)
    real = np.float64 if dtype == "f64" else np.float32
    return {
        "dtype": dtype,
        "a_width": int(plan.a_width),
        "feature_count": int(plan.feature_count),
        "chunk_count": len(chunks),
        "workspace_slots": int(workspace),
        "chunk_word_offsets": np.asarray(word_off, dtype=np.int64),
        "chunk_coeff_offsets": np.asarray(coeff_off, dtype=np.int64),
        "chunk_out_offsets": np.asarray(out_off, dtype=np.int64),
        "chunk_first_column": np.asarray(first_col, dtype=np.int64),
        "words": np.asarray(words, dtype=np.uint32),
        "coeffs": np.asarray(coeffs, dtype=real),
        "out_slots": np.asarray(out_slots, dtype=np.uint16),
    }


def program_stats(prog):
    """Per-sample work of a program: terms and factor reads summed over chunks."""
    words = prog["words"]
    terms = factor_reads = loads = 0
    i = 0
    while i < len(words):
        h = int(words[i])
        op, n = h >> 28, h & 0xFFFFFF
        if op == OP_LOAD:
            loads += n
            i += 1 + n
            continue
        k = {OP_ACC1: 1, OP_ACC2: 2, OP_ACC3: 3, OP_ACC4: 4}[op]
        terms += n
        factor_reads += k * n
        i += 2 + (n if k <= 2 else 2 * n)
    return {"chunks": int(prog["chunk_count"]), "workspace_slots": int(prog["workspace_slots"]),
            "terms": terms, "factor_reads": factor_reads, "loads": loads,
            "words": int(len(words))}
