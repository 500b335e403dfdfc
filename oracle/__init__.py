"""CPU oracle for the ACE hot path -- TEST INFRASTRUCTURE ONLY.

Thin numpy/ctypes wrappers over ``liboracle.so`` (the C restatement in
``ye3t_oracle.c``) and, where it has been built from the reference sources in
this container, ``_ref/libye3t_ref.so`` (the reference's own CPU core).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this package, and only as the checker / the timed CPU baseline.
The product library (``ye3t_amd``) never imports it.

Pinning status of each function is recorded in ``tests/test_oracle.py``.
"""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

_d = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.POINTER(ctypes.c_int64)
_i32 = ctypes.POINTER(ctypes.c_int32)
_I = ctypes.c_int64


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        _LIB = ctypes.CDLL(path)
        L = _LIB
        L.oracle_radial_table.argtypes = [_d, _d, _d, _I, _I, _d, _d]
        L.oracle_real_sph_table.argtypes = [_d, _I, _I, ctypes.c_double, _d, _d]
        L.oracle_density_accumulate.argtypes = [_d, _i64, _I, _I, _I, _d]
        L.oracle_density_accumulate_adjoint.argtypes = [_d, _i64, _I, _I, _d]
        L.oracle_scheduled_channels.argtypes = [_d, _d, _d, _d, _d, _i64, _i64, _i64, _i64, _d, _I, _I, _I, _I,
                                                _d, _d]
        L.oracle_ace_density_edge_gradient.argtypes = [_I, _I, _i64, _i64, _d, _i32, _d, _d, _I, _I, _I,
                                                       ctypes.c_double, ctypes.c_double, ctypes.c_double, _d, _d]
        L.oracle_ace_density.argtypes = [_I, _I, _i64, _i64, _d, _i32, _d, _d, _I, _I, _I,
                                         ctypes.c_double, ctypes.c_double, ctypes.c_double, _d]
        L.oracle_symmetric_power_monomial.argtypes = [_d, _I, _I, _i64, _i64, _d, _I, _d]
        L.oracle_evaluate_componentwise.argtypes = [_d, _i64, _i64, _i64, _d, _d, _I, _I, _I, _I, _I]
        L.oracle_ace_product_flat.argtypes = [_d, _I, _I, _I, _i64, _d, _i32, _I, _i64, _d, _i32, _d]
        L.oracle_ace_product_flat_adjoint.argtypes = [_d, _d, _I, _I, _I, _i64, _d, _i32, _I, _i64, _d, _i32, _d]
        L.oracle_max_threads.restype = ctypes.c_int
        L.oracle_set_threads.argtypes = [ctypes.c_int]
    return _LIB


def ref_lib():
    """The reference's own CPU core built in ``_ref/`` (None if not built)."""
    global _REF
    if _REF is None:
        path = os.path.join(_HERE, "_ref", "libye3t_ref.so")
        if not os.path.exists(path):
            return None
        _REF = ctypes.CDLL(path)
        _REF.ref_radial_table.argtypes = [_d, _d, _d, _I, _I, _d, _d]
        _REF.ref_real_sph_table.argtypes = [_d, _I, _I, ctypes.c_double, _d, _d]
        _REF.ref_density_accumulate.argtypes = [_d, _i64, _I, _I, _I, _d]
        if hasattr(_REF, "ref_density_accumulate_adjoint"):
            _REF.ref_density_accumulate_adjoint.argtypes = [_d, _i64, _I, _I, _d]
        _REF.ref_symmetric_power_monomial.argtypes = [_d, _I, _I, _i64, _i64, _d, _I, _I, _d]
        if hasattr(_REF, "ref_scheduled_channels"):
            _REF.ref_scheduled_channels.argtypes = [_d, _d, _d, _d, _d, _i64, _i64, _i64, _i64, _d, _I, _I, _I, _I,
                                                    _d, _d]
    return _REF


def _p(a, t=_d):
    return a.ctypes.data_as(t)


def _f64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def _i64a(a):
    return np.ascontiguousarray(a, dtype=np.int64)


def set_threads(n):
    lib().oracle_set_threads(int(n))


def max_threads():
    return int(lib().oracle_max_threads())


def radial_table(radii, cutoffs, lambdas, n_max, *, use_reference=False):
    radii, cutoffs, lambdas = _f64(radii), _f64(cutoffs), _f64(lambdas)
    E = radii.shape[0]
    v = np.zeros((E, n_max + 1))
    d = np.zeros((E, n_max + 1))
    if use_reference:
        ref_lib().ref_radial_table(_p(radii), _p(cutoffs), _p(lambdas), E, n_max, _p(v), _p(d))
    else:
        lib().oracle_radial_table(_p(radii), _p(cutoffs), _p(lambdas), E, n_max, _p(v), _p(d))
    return v, d


def real_sph_table(vectors, l_max, epsilon=1e-12, *, use_reference=False):
    vectors = _f64(vectors).reshape(-1, 3)
    E = vectors.shape[0]
    w = (l_max + 1) ** 2
    v = np.zeros((E, w))
    g = np.zeros((E, w, 3))
    if use_reference:
        ref_lib().ref_real_sph_table(_p(vectors), E, l_max, epsilon, _p(v), _p(g))
    else:
        lib().oracle_real_sph_table(_p(vectors), E, l_max, epsilon, _p(v), _p(g))
    return v, g


def scheduled_channels(radial_values, radial_derivatives, angular_values, angular_derivatives, radial_directions,
                       edge_types, channel_radial_indices, channel_angular_indices, channel_types, channel_scales,
                       *, use_reference=False):
    """Scheduled radial-angular edge channels ``(values [E, K], derivatives [E, K, 3])``
    (``ye3t_runtime_core.cpp:1550-1604``); ``use_reference`` runs the reference core in ``_ref``."""
    rv, rd = _f64(radial_values), _f64(radial_derivatives)
    av, ad, dr = _f64(angular_values), _f64(angular_derivatives), _f64(radial_directions)
    et, cri, cai, ct = (_i64a(a) for a in (edge_types, channel_radial_indices, channel_angular_indices,
                                           channel_types))
    cs = _f64(channel_scales)
    E, NR = rv.shape
    NA, K = av.shape[1], cs.shape[0]
    v = np.zeros((E, K))
    d = np.zeros((E, K, 3))
    f = ref_lib().ref_scheduled_channels if use_reference else lib().oracle_scheduled_channels
    f(_p(rv), _p(rd), _p(av), _p(ad), _p(dr), _p(et, _i64), _p(cri, _i64), _p(cai, _i64), _p(ct, _i64), _p(cs),
      E, NR, NA, K, _p(v), _p(d))
    return v, d


def density_accumulate(edge_values, centers, atom_count, *, use_reference=False):
    ev = _f64(edge_values)
    E, C = ev.shape
    centers = _i64a(centers)
    out = np.zeros((atom_count, C))
    f = ref_lib().ref_density_accumulate if use_reference else lib().oracle_density_accumulate
    f(_p(ev), _p(centers, _i64), E, C, atom_count, _p(out))
    return out


def density_accumulate_adjoint(atomic_adjoint, centers, *, use_reference=False):
    """``edge_adjoint[e] = atomic_adjoint[centers[e]]`` (the adjoint of :func:`density_accumulate`)."""
    adj = _f64(atomic_adjoint)
    N, C = adj.shape
    centers = _i64a(centers)
    if centers.size and (centers.min() < 0 or centers.max() >= N):
        raise ValueError("center index out of range")
    E = centers.shape[0]
    out = np.zeros((E, C))
    f = ref_lib().ref_density_accumulate_adjoint if use_reference else lib().oracle_density_accumulate_adjoint
    f(_p(adj), _p(centers, _i64), E, C, _p(out))
    return out


def ace_density(inp):
    """Stage-1 oracle on a workload dict (see ``ye3t_amd.ace.workloads``)."""
    N, E = int(inp["atom_count"]), int(inp["edge_count"])
    centers = _i64a(inp["centers"])
    neighbors = _i64a(inp["neighbors"])
    vec = _f64(inp["edge_vectors"])
    species = inp.get("species")
    feats = inp.get("node_features")
    mix = inp.get("radial_mix")
    C, n_max, l_max = int(inp["channel_count"]), int(inp["n_max"]), int(inp["l_max"])
    rows = 1 if mix is not None else n_max + 1
    out = np.zeros((N, C, rows, (l_max + 1) ** 2))
    sp = np.ascontiguousarray(species, dtype=np.int32) if species is not None else None
    fe = _f64(feats) if feats is not None else None
    mx = _f64(mix) if mix is not None else None
    lib().oracle_ace_density(N, E, _p(centers, _i64), _p(neighbors, _i64), _p(vec),
                             _p(sp, _i32) if sp is not None else None,
                             _p(fe) if fe is not None else None, _p(mx) if mx is not None else None,
                             C, n_max, l_max, float(inp["cutoff"]), float(inp["lambda"]),
                             float(inp.get("epsilon", 1e-12)), _p(out))
    return out


def ace_density_edge_gradient(inp, density_adjoint):
    """Edge-vector gradient ``[E, 3]`` of ``<density_adjoint, A(edge_vectors)>``
    for a stage-1 workload dict (``oracle_ace_density_edge_gradient``: the
    reference's scheduled channel derivative, ye3t_runtime_core.cpp:1550-1604,
    on the radial and harmonic derivative tables, contracted with the gathered
    density adjoint)."""
    N, E = int(inp["atom_count"]), int(inp["edge_count"])
    centers = _i64a(inp["centers"])
    neighbors = _i64a(inp["neighbors"])
    vec = _f64(inp["edge_vectors"])
    species = inp.get("species")
    feats = inp.get("node_features")
    mix = inp.get("radial_mix")
    C, n_max, l_max = int(inp["channel_count"]), int(inp["n_max"]), int(inp["l_max"])
    rows = 1 if mix is not None else n_max + 1
    gA = _f64(density_adjoint).reshape(N, C * rows * (l_max + 1) ** 2)
    out = np.zeros((E, 3))
    sp = np.ascontiguousarray(species, dtype=np.int32) if species is not None else None
    fe = _f64(feats) if feats is not None else None
    mx = _f64(mix) if mix is not None else None
    lib().oracle_ace_density_edge_gradient(N, E, _p(centers, _i64), _p(neighbors, _i64), _p(vec),
                                           _p(sp, _i32) if sp is not None else None,
                                           _p(fe) if fe is not None else None, _p(mx) if mx is not None else None,
                                           C, n_max, l_max, float(inp["cutoff"]), float(inp["lambda"]),
                                           float(inp.get("epsilon", 1e-12)), _p(gA), _p(out))
    return out


def symmetric_power_monomial(inp, monomial_counts, output_offsets, monomial_values, *, use_reference=False):
    x = _f64(inp)
    B, D = x.shape
    counts = _i64a(monomial_counts)
    offs = _i64a(output_offsets)
    vals = _f64(monomial_values)
    out_dim = offs.shape[0] - 1
    out = np.zeros((B, out_dim))
    if use_reference:
        ref_lib().ref_symmetric_power_monomial(_p(x), B, D, _p(counts, _i64), _p(offs, _i64), _p(vals),
                                               vals.shape[0], out_dim, _p(out))
    else:
        lib().oracle_symmetric_power_monomial(_p(x), B, D, _p(counts, _i64), _p(offs, _i64), _p(vals),
                                              out_dim, _p(out))
    return out


def evaluate_componentwise(block_values, flat):
    """``evaluate_factorized_schedule_cpu`` restatement on a schedule's flat arrays."""
    bv = _f64(block_values)
    B, basis, blocks, mdim = bv.shape
    K = flat["component_offsets"].shape[0] - 1
    out = np.zeros((B, K))
    lib().oracle_evaluate_componentwise(
        _p(bv), _p(_i64a(flat["component_offsets"]), _i64), _p(_i64a(flat["component_label_index"]), _i64),
        _p(_i64a(flat["block_m_indices"]), _i64), _p(_f64(flat["coeffs"])), _p(out), B, basis, mdim, K, blocks)
    return out


def ace_product_flat(A, plan_arrays):
    A = _f64(A)
    S, W = A.shape
    pa = plan_arrays
    K = pa["column_offsets"].shape[0] - 1
    out = np.zeros((S, K))
    lib().oracle_ace_product_flat(
        _p(A), S, W, int(pa["value_count"]), _p(_i64a(pa["value_offsets"]), _i64), _p(_f64(pa["value_coeffs"])),
        _p(np.ascontiguousarray(pa["value_factors"], dtype=np.int32), _i32), K,
        _p(_i64a(pa["column_offsets"]), _i64), _p(_f64(pa["term_coeffs"])),
        _p(np.ascontiguousarray(pa["term_refs"], dtype=np.int32), _i32), _p(out))
    return out


def linear_readout(features, weight, bias):
    """``features @ weight + bias`` -- the reference's materialised readout
    (``execution_plan.py:13838-13845``), in fp64."""
    return _f64(features) @ _f64(weight) + float(bias)


def ace_product_flat_adjoint(A, gB, plan_arrays):
    """``gA[s] = J(A[s])^T gB[s]`` for the flat product (reverse mode of :func:`ace_product_flat`)."""
    A = _f64(A)
    S, W = A.shape
    pa = plan_arrays
    K = pa["column_offsets"].shape[0] - 1
    gB = _f64(gB).reshape(S, K)
    out = np.zeros((S, W))
    lib().oracle_ace_product_flat_adjoint(
        _p(A), _p(gB), S, W, int(pa["value_count"]), _p(_i64a(pa["value_offsets"]), _i64),
        _p(_f64(pa["value_coeffs"])), _p(np.ascontiguousarray(pa["value_factors"], dtype=np.int32), _i32), K,
        _p(_i64a(pa["column_offsets"]), _i64), _p(_f64(pa["term_coeffs"])),
        _p(np.ascontiguousarray(pa["term_refs"], dtype=np.int32), _i32), _p(out))
    return out


def neighbor_list(positions, cutoff):
    """Brute-force neighbour CSR (``oracle_neighbor_list``): dict with
    ``target_offsets``, ``edge_targets``, ``edge_sources``, ``edge_vectors``
    (the last in the positions' dtype)."""
    L = lib()
    pos = np.ascontiguousarray(positions)
    if pos.dtype not in (np.float32, np.float64) or pos.ndim != 2 or pos.shape[1] != 3:
        raise ValueError("positions must be float32/float64 [N, 3]")
    n = int(pos.shape[0])
    is_f32 = int(pos.dtype == np.float32)
    offsets = np.zeros(n + 1, dtype=np.int64)
    vp = ctypes.c_void_p
    L.oracle_neighbor_list.argtypes = [vp, ctypes.c_int, _I, ctypes.c_double, vp, vp, vp, vp]
    L.oracle_neighbor_list(pos.ctypes.data, is_f32, n, float(cutoff), offsets.ctypes.data, None, None, None)
    e = int(offsets[-1])
    centers = np.empty(e, dtype=np.int64)
    nbrs = np.empty(e, dtype=np.int64)
    vecs = np.empty((e, 3), dtype=np.float64)
    if e:
        L.oracle_neighbor_list(pos.ctypes.data, is_f32, n, float(cutoff), offsets.ctypes.data, centers.ctypes.data,
                               nbrs.ctypes.data, vecs.ctypes.data)
    return {"target_offsets": offsets, "edge_targets": centers, "edge_sources": nbrs,
            "edge_vectors": vecs.astype(pos.dtype)}


# ---- factorized angular DAG (ye3t_oracle_dag.c) ------------------------------

FA_TABLE_KEYS = ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
                 "node_coefficient_offsets", "coefficient_rows", "coefficient_columns")


def _fa_args(tables, complex_data):
    """ctypes arguments of the DAG tables (dict of arrays) and the arrays kept alive."""
    keep = {k: _i64a(tables[k]) for k in FA_TABLE_KEYS + ("root_nodes",)}
    ctype = np.complex128 if complex_data else np.float64
    keep["coefficient_values"] = np.ascontiguousarray(tables["coefficient_values"], dtype=ctype)
    keep["projection_values"] = np.ascontiguousarray(tables["projection_values"], dtype=ctype)
    return keep


def _vp(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None and a.size else None


def _fa_dims(packed, tables, source_dimension):
    nodes = int(len(tables["node_offsets"]))
    S = int(source_dimension)
    width = int(packed.shape[1])
    proj = np.asarray(tables["projection_values"]).reshape(-1)
    P = proj.shape[0] // S
    roots = np.asarray(tables["root_nodes"]).reshape(-1)
    rdim = int(np.asarray(tables["node_dimensions"])[roots[0]])
    W = int(tables["node_offsets"][-1] + tables["node_dimensions"][-1])
    return nodes, S, width // S, P, len(roots), rdim, W


def _fa_fn(name, complex_data, use_reference):
    suffix = "c128" if complex_data else "f64"
    if use_reference:
        fn = getattr(ref_lib(), f"ref_{name}_{suffix}")
    else:
        fn = getattr(lib(), f"oracle_{name}_{suffix}")
    fn.restype = None
    return fn


def factorized_angular(packed_slots, tables, source_dimension, *, use_reference=False):
    """``factorized_angular_forward`` (ye3t_runtime_core.cpp:5667-5769) with the
    Torch op's uniform root metadata; returns ``[batch, roots * P * root_dim]``."""
    cplx = np.iscomplexobj(packed_slots) or np.iscomplexobj(tables["coefficient_values"]) or \
        np.iscomplexobj(tables["projection_values"])
    dt = np.complex128 if cplx else np.float64
    x = np.ascontiguousarray(packed_slots, dtype=dt)
    B = int(x.shape[0])
    nodes, S, D, P, R, rdim, W = _fa_dims(x, tables, source_dimension)
    out_dim = R * P * rdim
    k = _fa_args(tables, cplx)
    out = np.zeros((B, out_dim), dtype=dt)
    ws = np.zeros(max(W, 1), dtype=dt)
    I = ctypes.c_int64
    args = [_vp(x), I(B), I(D), I(S)] + [_vp(k[n]) for n in FA_TABLE_KEYS[:6]] + [I(nodes)] + \
        [_vp(k["coefficient_rows"]), _vp(k["coefficient_columns"]), _vp(k["coefficient_values"]),
         _vp(k["root_nodes"]), I(R), _vp(k["projection_values"]), I(P), I(out_dim)]
    if not use_reference:
        args.append(_vp(ws))
    args.append(_vp(out))
    _fa_fn("factorized_angular", cplx, use_reference)(*args)
    return out


def factorized_angular_adjoint(output_adjoint, packed_slots, tables, source_dimension, *, use_reference=False):
    """``factorized_angular_adjoint`` (ye3t_runtime_core.cpp:6481-6643): the
    packed-slot gradient ``[batch, S * input_dim]`` of an output adjoint."""
    cplx = np.iscomplexobj(packed_slots) or np.iscomplexobj(output_adjoint) or \
        np.iscomplexobj(tables["coefficient_values"]) or np.iscomplexobj(tables["projection_values"])
    dt = np.complex128 if cplx else np.float64
    x = np.ascontiguousarray(packed_slots, dtype=dt)
    g = np.ascontiguousarray(output_adjoint, dtype=dt)
    B = int(x.shape[0])
    nodes, S, D, P, R, rdim, W = _fa_dims(x, tables, source_dimension)
    out_dim = R * P * rdim
    k = _fa_args(tables, cplx)
    out = np.zeros((B, S * D), dtype=dt)
    ws = np.zeros(max(W, 1), dtype=dt)
    wa = np.zeros(max(W, 1), dtype=dt)
    I = ctypes.c_int64
    args = [_vp(g), _vp(x), I(B), I(D), I(S)] + [_vp(k[n]) for n in FA_TABLE_KEYS[:6]] + [I(nodes)] + \
        [_vp(k["coefficient_rows"]), _vp(k["coefficient_columns"]), _vp(k["coefficient_values"]),
         _vp(k["root_nodes"]), I(R), _vp(k["projection_values"]), I(P), I(out_dim)]
    if not use_reference:
        args += [_vp(ws), _vp(wa)]
    args.append(_vp(out))
    _fa_fn("factorized_angular_adjoint", cplx, use_reference)(*args)
    return out


def factorized_angular_linear(packed_slots, tables, source_dimension, weight, bias, *, use_reference=False):
    """``factorized_angular_linear_forward`` (ye3t_runtime_core.cpp:7144-7234):
    ``bias + features @ weight`` per sample, accumulated in the reference's order."""
    cplx = any(np.iscomplexobj(a) for a in (packed_slots, weight, tables["coefficient_values"],
                                            tables["projection_values"])) or isinstance(bias, complex)
    dt = np.complex128 if cplx else np.float64
    x = np.ascontiguousarray(packed_slots, dtype=dt)
    B = int(x.shape[0])
    nodes, S, D, P, R, rdim, W = _fa_dims(x, tables, source_dimension)
    k = _fa_args(tables, cplx)
    w = np.ascontiguousarray(weight, dtype=dt)
    b = np.array([bias], dtype=dt)
    out = np.zeros(B, dtype=dt)
    ws = np.zeros(max(W, 1), dtype=dt)
    I = ctypes.c_int64
    args = [_vp(x), I(B), I(D), I(S)] + [_vp(k[n]) for n in FA_TABLE_KEYS[:6]] + [I(nodes)] + \
        [_vp(k["coefficient_rows"]), _vp(k["coefficient_columns"]), _vp(k["coefficient_values"]),
         _vp(k["root_nodes"]), I(R), _vp(k["projection_values"]), I(P), _vp(w)]
    if use_reference:
        args += [_vp(b), _vp(out)]
    else:
        # the C restatement takes the bias by value
        fn = _fa_fn("factorized_angular_linear", cplx, False)
        if cplx:
            class _C(ctypes.Structure):
                _fields_ = [("re", ctypes.c_double), ("im", ctypes.c_double)]
            fn.argtypes = None
            args += [_C(b[0].real, b[0].imag), _vp(ws), _vp(out)]
        else:
            args += [ctypes.c_double(float(b[0])), _vp(ws), _vp(out)]
        fn(*args)
        return out
    _fa_fn("factorized_angular_linear", cplx, True)(*args)
    return out


def factorized_angular_linear_adjoint(output_adjoint, packed_slots, tables, source_dimension, weight, *,
                                      use_reference=False):
    """``factorized_angular_linear_adjoint`` (ye3t_runtime_core.cpp:7237-7399):
    ``(packed_slots_adjoint, weight_adjoint, bias_adjoint)``."""
    cplx = any(np.iscomplexobj(a) for a in (packed_slots, weight, output_adjoint, tables["coefficient_values"],
                                            tables["projection_values"]))
    dt = np.complex128 if cplx else np.float64
    x = np.ascontiguousarray(packed_slots, dtype=dt)
    g = np.ascontiguousarray(output_adjoint, dtype=dt)
    B = int(x.shape[0])
    nodes, S, D, P, R, rdim, W = _fa_dims(x, tables, source_dimension)
    k = _fa_args(tables, cplx)
    w = np.ascontiguousarray(weight, dtype=dt)
    gx = np.zeros((B, S * D), dtype=dt)
    gw = np.zeros(R * P * rdim, dtype=dt)
    gb = np.zeros(1, dtype=dt)
    ws = np.zeros(max(W, 1), dtype=dt)
    wa = np.zeros(max(W, 1), dtype=dt)
    I = ctypes.c_int64
    args = [_vp(g), _vp(x), I(B), I(D), I(S)] + [_vp(k[n]) for n in FA_TABLE_KEYS[:6]] + [I(nodes)] + \
        [_vp(k["coefficient_rows"]), _vp(k["coefficient_columns"]), _vp(k["coefficient_values"]),
         _vp(k["root_nodes"]), I(R), _vp(k["projection_values"]), I(P), _vp(w)]
    if not use_reference:
        args += [_vp(ws), _vp(wa)]
    args += [_vp(gx), _vp(gw), _vp(gb)]
    _fa_fn("factorized_angular_linear_adjoint", cplx, use_reference)(*args)
    return gx, gw, gb[0]


# segmented tables, in the reference op's argument order (execution_plan_torch.cpp:7666-7679)
FA_SEGMENT_KEYS = ("segment_source_offsets", "segment_input_offsets", "segment_input_dimensions",
                   "segment_workspace_offsets", "segment_workspace_dimensions", "segment_node_offsets",
                   "segment_root_offsets", "segment_projection_offsets", "segment_projection_dimensions",
                   "segment_output_offsets", "node_offsets", "node_dimensions", "node_leaf_offsets", "node_left",
                   "node_right", "node_coefficient_offsets", "coefficient_rows", "coefficient_columns",
                   "coefficient_values", "root_nodes", "root_projection_starts", "root_projection_dimensions",
                   "root_output_offsets", "projection_values")


def _fa_seg_args(seg, cplx, packed_dim, out_dim, batch):
    keep = {k: _i64a(seg[k]) for k in FA_SEGMENT_KEYS if k not in ("coefficient_values", "projection_values")}
    dt = np.complex128 if cplx else np.float64
    keep["coefficient_values"] = np.ascontiguousarray(seg["coefficient_values"], dtype=dt)
    keep["projection_values"] = np.ascontiguousarray(seg["projection_values"], dtype=dt)
    I = ctypes.c_int64
    nseg = int(keep["segment_input_offsets"].size)
    args = [I(batch), I(packed_dim), I(nseg)] + [_vp(keep[k]) for k in (
        "segment_source_offsets", "segment_input_offsets", "segment_input_dimensions", "segment_node_offsets",
        "segment_root_offsets", "segment_projection_offsets", "segment_projection_dimensions",
        "segment_output_offsets")] + [I(out_dim)] + [_vp(keep[k]) for k in (
            "node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right",
            "node_coefficient_offsets", "coefficient_rows", "coefficient_columns", "coefficient_values",
            "root_nodes", "root_projection_starts", "root_projection_dimensions", "root_output_offsets",
            "projection_values")]
    W = int(max(np.asarray(seg["segment_workspace_dimensions"]).max(), 1))
    return keep, args, W


def _seg_complex(seg, *arrays):
    return any(np.iscomplexobj(a) for a in arrays) or np.iscomplexobj(seg["coefficient_values"]) or \
        np.iscomplexobj(seg["projection_values"])


def factorized_angular_segmented(packed_slots, seg, output_dimension, *, use_reference=False):
    """``factorized_angular_segmented_forward`` (ye3t_runtime_core.cpp:6977-7021):
    ``seg`` holds the op's segment, node, coefficient, root and projection
    tables (:data:`FA_SEGMENT_KEYS`); returns ``[batch, output_dimension]``."""
    cplx = _seg_complex(seg, packed_slots)
    dt = np.complex128 if cplx else np.float64
    x = np.ascontiguousarray(packed_slots, dtype=dt)
    B, D = x.shape
    out = np.zeros((B, int(output_dimension)), dtype=dt)
    keep, args, W = _fa_seg_args(seg, cplx, D, int(output_dimension), B)
    ws = np.zeros(W, dtype=dt)
    args = [_vp(x)] + args + ([] if use_reference else [_vp(ws)]) + [_vp(out)]
    _fa_fn("factorized_angular_segmented", cplx, use_reference)(*args)
    return out


def factorized_angular_segmented_adjoint(output_adjoint, packed_slots, seg, *, use_reference=False):
    """``factorized_angular_segmented_adjoint`` (ye3t_runtime_core.cpp:7023-7070):
    the packed-slot gradient ``[batch, packed width]``."""
    cplx = _seg_complex(seg, packed_slots, output_adjoint)
    dt = np.complex128 if cplx else np.float64
    x = np.ascontiguousarray(packed_slots, dtype=dt)
    g = np.ascontiguousarray(output_adjoint, dtype=dt)
    B, D = x.shape
    gx = np.zeros((B, D), dtype=dt)
    keep, args, W = _fa_seg_args(seg, cplx, D, int(g.shape[1]), B)
    ws = np.zeros(W, dtype=dt)
    wa = np.zeros(W, dtype=dt)
    args = [_vp(g), _vp(x)] + args + ([] if use_reference else [_vp(ws), _vp(wa)]) + [_vp(gx)]
    _fa_fn("factorized_angular_segmented_adjoint", cplx, use_reference)(*args)
    return gx


# ---- symmetric-power monomial adjoint and shared monomials -------------------

def symmetric_power_monomial_adjoint(output_adjoint, inp, monomial_counts, output_indices, monomial_values,
                                     output_dimension, *, use_reference=False):
    """``symmetric_power_monomial_adjoint`` (ye3t_runtime_core.cpp:5318-5389)."""
    x = _f64(inp)
    B, D = x.shape
    g = _f64(output_adjoint).reshape(B, int(output_dimension))
    counts = _i64a(monomial_counts)
    idx = _i64a(output_indices)
    vals = _f64(monomial_values)
    out = np.zeros((B, D))
    fn = ref_lib().ref_symmetric_power_monomial_adjoint if use_reference else \
        lib().oracle_symmetric_power_monomial_adjoint
    fn.restype = None
    I = ctypes.c_int64
    fn(_vp(g), _vp(x), I(B), I(D), _vp(counts), _vp(idx), _vp(vals), I(vals.shape[0]), I(int(output_dimension)),
       _vp(out))
    return out


def symmetric_power_shared_monomial(inp, monomial_counts, output_offsets, coefficient_terms, coefficient_values,
                                    *, use_reference=False):
    """``symmetric_power_shared_monomial_forward`` (ye3t_runtime_core.cpp:5392-5440)."""
    x = _f64(inp)
    B, D = x.shape
    counts = _i64a(monomial_counts)
    M = counts.shape[0]
    offs = _i64a(output_offsets)
    terms = _i64a(coefficient_terms)
    vals = _f64(coefficient_values)
    O = offs.shape[0] - 1
    out = np.zeros((B, O))
    I = ctypes.c_int64
    if use_reference:
        fn = ref_lib().ref_symmetric_power_shared_monomial
        fn.restype = None
        fn(_vp(x), I(B), I(D), _vp(counts), I(M), _vp(offs), _vp(terms), _vp(vals), I(vals.shape[0]), I(O), _vp(out))
    else:
        fn = lib().oracle_symmetric_power_shared_monomial
        fn.restype = None
        ws = np.zeros(max(M, 1))
        fn(_vp(x), I(B), I(D), _vp(counts), I(M), _vp(offs), _vp(terms), _vp(vals), I(O), _vp(ws), _vp(out))
    return out


def symmetric_power_shared_monomial_adjoint(output_adjoint, inp, monomial_counts, output_offsets,
                                            coefficient_terms, coefficient_values, *, use_reference=False):
    """``symmetric_power_shared_monomial_adjoint`` (ye3t_runtime_core.cpp:5442-5540)."""
    x = _f64(inp)
    B, D = x.shape
    counts = _i64a(monomial_counts)
    M = counts.shape[0]
    offs = _i64a(output_offsets)
    terms = _i64a(coefficient_terms)
    vals = _f64(coefficient_values)
    O = offs.shape[0] - 1
    g = _f64(output_adjoint).reshape(B, O)
    out = np.zeros((B, D))
    I = ctypes.c_int64
    if use_reference:
        fn = ref_lib().ref_symmetric_power_shared_monomial_adjoint
        fn.restype = None
        fn(_vp(g), _vp(x), I(B), I(D), _vp(counts), I(M), _vp(offs), _vp(terms), _vp(vals), I(vals.shape[0]), I(O),
           _vp(out))
    else:
        fn = lib().oracle_symmetric_power_shared_monomial_adjoint
        fn.restype = None
        ws = np.zeros(max(M, 1))
        fn(_vp(g), _vp(x), I(B), I(D), _vp(counts), I(M), _vp(offs), _vp(terms), _vp(vals), I(O), _vp(ws), _vp(out))
    return out


def _sparse_tables(term_offsets, term_components, term_exponents, output_offsets, coefficient_terms,
                   coefficient_values):
    toff, comp, ex = _i64a(term_offsets), _i64a(term_components), _i64a(term_exponents)
    offs, terms = _i64a(output_offsets), _i64a(coefficient_terms)
    outs = np.repeat(np.arange(offs.shape[0] - 1, dtype=np.int64), np.diff(offs))
    return toff, comp, ex, offs, terms, outs, _f64(coefficient_values)


def symmetric_power_shared_sparse_monomial(inp, term_offsets, term_components, term_exponents, output_offsets,
                                           coefficient_terms, coefficient_values):
    """``symmetric_power_shared_sparse_monomial`` (execution_plan_cuda.cu:5720-5755, 5962-6000)."""
    x = _f64(inp)
    B, D = x.shape
    toff, comp, ex, offs, terms, _, vals = _sparse_tables(term_offsets, term_components, term_exponents,
                                                           output_offsets, coefficient_terms, coefficient_values)
    M, O = toff.shape[0] - 1, offs.shape[0] - 1
    out = np.zeros((B, O))
    fn = lib().oracle_symmetric_power_shared_sparse_monomial
    fn.restype = None
    ws = np.zeros(max(M, 1))
    fn(_vp(x), _I(B), _I(D), _vp(toff), _vp(comp), _vp(ex), _I(M), _vp(offs), _vp(terms), _vp(vals), _I(O),
       _vp(ws), _vp(out))
    return out


def symmetric_power_shared_sparse_monomial_adjoint(output_adjoint, inp, term_offsets, term_components,
                                                   term_exponents, output_offsets, coefficient_terms,
                                                   coefficient_values):
    """``..._sparse_monomial_adjoint`` (execution_plan_cuda.cu:5757-5813, 6002-6030)."""
    x = _f64(inp)
    B, D = x.shape
    toff, comp, ex, offs, terms, outs, vals = _sparse_tables(term_offsets, term_components, term_exponents,
                                                              output_offsets, coefficient_terms, coefficient_values)
    M, O, C = toff.shape[0] - 1, offs.shape[0] - 1, terms.shape[0]
    g = _f64(output_adjoint).reshape(B, O)
    out = np.zeros((B, D))
    fn = lib().oracle_symmetric_power_shared_sparse_monomial_adjoint
    fn.restype = None
    ws = np.zeros(max(M, 1))
    fn(_vp(g), _vp(x), _I(B), _I(D), _vp(toff), _vp(comp), _vp(ex), _I(M), _vp(terms), _vp(outs), _vp(vals), _I(C),
       _I(O), _vp(ws), _vp(out))
    return out


def symmetric_power_shared_sparse_monomial_double_backward(input_adjoint_tangent, output_adjoint, inp,
                                                           term_offsets, term_components, term_exponents,
                                                           output_offsets, coefficient_terms, coefficient_values):
    """``..._sparse_monomial_double_backward`` (execution_plan_cuda.cu:5815-5955, host :11206-11330):
    returns ``(output_tangent, input_tangent)``."""
    x = _f64(inp)
    B, D = x.shape
    toff, comp, ex, offs, terms, outs, vals = _sparse_tables(term_offsets, term_components, term_exponents,
                                                              output_offsets, coefficient_terms, coefficient_values)
    M, O, C = toff.shape[0] - 1, offs.shape[0] - 1, terms.shape[0]
    v = _f64(input_adjoint_tangent).reshape(B, D)
    g = _f64(output_adjoint).reshape(B, O)
    ot, it = np.zeros((B, O)), np.zeros((B, D))
    fn = lib().oracle_symmetric_power_shared_sparse_monomial_double_backward
    fn.restype = None
    ws = np.zeros(max(M, 1))
    fn(_vp(v), _vp(g), _vp(x), _I(B), _I(D), _vp(toff), _vp(comp), _vp(ex), _I(M), _vp(offs), _vp(terms),
       _vp(outs), _vp(vals), _I(C), _I(O), _vp(ws), _vp(ot), _vp(it))
    return ot, it
