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
