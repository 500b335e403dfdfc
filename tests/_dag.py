"""Factorized-angular DAG fixtures shared by the oracle and GPU tests (not collected)."""

import numpy as np

# Known-answer case of the reference's installed-CUDA smoke test
# (cmake/smoke_installed_cuda.py:106-240): two sources of two l=1 leaves,
# one merge node with three coefficients, one root, two projections.
KAT_PACKED = np.array([[0.25, -0.5, 0.75, 1.0, -0.625, 0.375, -0.25, 0.5, 1.25, 0.75, -1.0, 0.625],
                       [-0.5, 0.125, 1.0, 0.375, 0.75, -0.25, 1.25, -0.75, 0.5, -0.625, 0.25, 1.0]])
KAT_TABLES = {
    "node_offsets": np.array([0, 3, 6]), "node_dimensions": np.array([3, 3, 1]),
    "node_leaf_offsets": np.array([0, 3, -1]), "node_left": np.array([-1, -1, 0]),
    "node_right": np.array([-1, -1, 1]), "node_coefficient_offsets": np.array([0, 0, 0, 3]),
    "coefficient_rows": np.array([0, 4, 8]), "coefficient_columns": np.array([0, 0, 0]),
    "coefficient_values": np.array([0.5 + 0.125j, -0.25 - 0.375j, 0.75 + 0.25j]),
    "root_nodes": np.array([2]),
    "projection_values": np.array([1.0 + 0.25j, 0.5 - 0.125j, -0.25 + 0.5j, 0.75 + 0.375j]),
}
KAT_SOURCES, KAT_WORKSPACE, KAT_OUTPUT = 2, 7, 2
KAT_OUTPUT_ADJOINT = np.array([[0.5 - 0.25j, -1.0 + 0.75j], [1.25 + 0.5j, 0.25 - 0.625j]])
KAT_LINEAR_WEIGHT = np.array([0.75 - 0.25j, -1.125 + 0.5j])
KAT_LINEAR_BIAS = 0.125 + 0.375j


def kat_closed_form(packed, tables=KAT_TABLES):
    """The smoke test's expected value: per source, sum_k conj(c_k) a_k b_k of
    the two leaves, then the projection matrix."""
    src = np.asarray(packed).reshape(2, 2, 6)
    roots = (src[:, :, :3] * src[:, :, 3:] * np.conj(tables["coefficient_values"]).reshape(1, 1, 3)).sum(axis=2)
    return roots @ tables["projection_values"].reshape(2, 2)


def random_dag(seed, *, complex_data, leaves_L=(1, 2, 1, 0), sources=3, projections=2, max_nodes=9):
    """A random valid DAG: leaf nodes over the packed input, then merge nodes of
    two earlier nodes with random sparse coefficient tables, several roots of
    one output dimension.  Returns ``(tables, source_dimension, input_dim)``."""
    rng = np.random.default_rng(seed)
    dims, leaf_off, left, right, offs = [], [], [], [], []
    coef_off, rows, cols, vals = [0], [], [], []
    running_in, running_ws = 0, 0
    for L in leaves_L:
        d = 2 * L + 1
        dims.append(d)
        leaf_off.append(running_in)
        left.append(-1)
        right.append(-1)
        offs.append(running_ws)
        running_in += d
        running_ws += d
        coef_off.append(len(vals))
    root_dim = 3
    while len(dims) < max_nodes:
        a, b = (int(x) for x in rng.integers(0, len(dims), 2))
        d = root_dim if len(dims) >= max_nodes - 3 else int(rng.choice([1, 3, 5]))
        nnz = int(rng.integers(1, dims[a] * dims[b] + 1))
        pairs = rng.choice(dims[a] * dims[b], size=nnz, replace=False)
        for p in pairs:
            rows.append(int(p))
            cols.append(int(rng.integers(0, d)))
            v = rng.normal()
            vals.append(complex(v, rng.normal()) if complex_data else v)
        dims.append(d)
        leaf_off.append(-1)
        left.append(a)
        right.append(b)
        offs.append(running_ws)
        running_ws += d
        coef_off.append(len(vals))
    n = len(dims)
    roots = [i for i in range(n - 3, n)]
    proj = rng.normal(size=sources * projections)
    if complex_data:
        proj = proj + 1j * rng.normal(size=sources * projections)
    tables = {"node_offsets": np.array(offs), "node_dimensions": np.array(dims),
              "node_leaf_offsets": np.array(leaf_off), "node_left": np.array(left), "node_right": np.array(right),
              "node_coefficient_offsets": np.array(coef_off), "coefficient_rows": np.array(rows, dtype=np.int64),
              "coefficient_columns": np.array(cols, dtype=np.int64),
              "coefficient_values": np.array(vals, dtype=np.complex128 if complex_data else np.float64),
              "root_nodes": np.array(roots), "projection_values": proj}
    return tables, sources, running_in


SEGMENT_KEYS = ("segment_source_offsets", "segment_input_offsets", "segment_input_dimensions",
                "segment_workspace_offsets", "segment_workspace_dimensions", "segment_node_offsets",
                "segment_root_offsets", "segment_projection_offsets", "segment_projection_dimensions",
                "segment_output_offsets", "node_offsets", "node_dimensions", "node_leaf_offsets", "node_left",
                "node_right", "node_coefficient_offsets", "coefficient_rows", "coefficient_columns",
                "coefficient_values", "root_nodes", "root_projection_starts", "root_projection_dimensions",
                "root_output_offsets", "projection_values")


def random_segmented(seed, *, complex_data, count=3):
    """Random segmented tables (the reference segmented op's layout): ``count``
    random DAGs with their own source count, leaves and projection width; each
    segment's roots are random nodes of any dimension, each projecting onto a
    random interval of its segment's projection columns, their output blocks
    laid out in a shuffled order.  Returns ``(tables, dims)`` with ``dims`` =
    (packed_input_dimension, total_source_count, workspace_dimension,
    output_dimension)."""
    rng = np.random.default_rng(seed)
    t = {k: [] for k in SEGMENT_KEYS}
    for k in ("segment_source_offsets", "segment_node_offsets", "segment_root_offsets", "segment_output_offsets"):
        t[k].append(0)
    src = in_base = ws_base = proj_base = out_base = node_base = root_base = coef_base = 0
    for k in range(count):
        leaves = tuple(int(x) for x in rng.integers(0, 4, size=int(rng.integers(2, 5))))
        S, P = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        dag, S, D = random_dag(int(seed) * 100 + k, complex_data=complex_data, leaves_L=leaves, sources=S,
                               projections=P, max_nodes=len(leaves) + int(rng.integers(2, 8)))
        dims = np.asarray(dag["node_dimensions"])
        N = int(dims.size)
        W = int(dag["node_offsets"][-1] + dims[-1])
        R = int(rng.integers(1, min(4, N) + 1))
        roots = rng.choice(N, size=R, replace=False)
        ps = rng.integers(0, P, size=R)
        pd = np.array([int(rng.integers(1, P - a + 1)) for a in ps])
        sizes = pd * dims[roots]
        oo = np.zeros(R, dtype=np.int64)
        cursor = 0
        for r in rng.permutation(R):
            oo[r] = cursor
            cursor += int(sizes[r])
        src += S
        t["segment_source_offsets"].append(src)
        t["segment_input_offsets"].append(in_base)
        t["segment_input_dimensions"].append(D)
        t["segment_workspace_offsets"].append(ws_base)
        t["segment_workspace_dimensions"].append(W)
        t["segment_projection_offsets"].append(proj_base)
        t["segment_projection_dimensions"].append(P)
        for n in ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right"):
            t[n].extend(int(v) for v in dag[n])
        offs = [int(v) + coef_base for v in dag["node_coefficient_offsets"]]
        t["node_coefficient_offsets"].extend(offs if k == 0 else offs[1:])
        t["coefficient_rows"].extend(int(v) for v in dag["coefficient_rows"])
        t["coefficient_columns"].extend(int(v) for v in dag["coefficient_columns"])
        t["coefficient_values"].extend(dag["coefficient_values"])
        t["root_nodes"].extend(int(v) for v in roots)
        t["root_projection_starts"].extend(int(v) for v in ps)
        t["root_projection_dimensions"].extend(int(v) for v in pd)
        t["root_output_offsets"].extend(int(v) for v in oo)
        t["projection_values"].extend(dag["projection_values"])
        node_base += N
        root_base += R
        coef_base += len(dag["coefficient_values"])
        proj_base += S * P
        in_base += S * D
        ws_base += S * W
        out_base += cursor
        t["segment_node_offsets"].append(node_base)
        t["segment_root_offsets"].append(root_base)
        t["segment_output_offsets"].append(out_base)
    vdt = np.complex128 if complex_data else np.float64
    tables = {k: np.asarray(v, dtype=vdt if k in ("coefficient_values", "projection_values") else np.int64)
              for k, v in t.items()}
    return tables, (in_base, src, ws_base, out_base)
