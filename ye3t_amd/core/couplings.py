"""Factorized (collapsed-block) CG coefficient schedules for ACE labels.

Host-side compiler that produces the same arrays as the reference's
``generate_factorized_coefficient_schedules_by_L``
(``ye3t/core/couplings.py:2066-2122``):

* low-rank fast paths (rank 1 identity, rank 2 symmetric square / direct CG),
  ``ye3t/core/couplings.py:1465-1636``;
* general rank: labels from :mod:`ye3t_amd.core.basis`, path expansion per
  angular key (``ye3t/core/factorized_dag.py:73-131``) and assembly label-major,
  ``M`` ascending, terms in expansion order (``core/couplings.py:1638-1753``).

``evaluate_factorized_schedule_torch`` mirrors the reference evaluator's
contract (``ye3t/core/couplings.py:481-567``); on a GPU tensor it runs the HIP
kernel through the C-ABI library, on a CPU tensor it runs the plain Torch
gather/product/index-add path the reference also ships.
"""

import os
from collections import OrderedDict
from dataclasses import dataclass

import numpy as np

from ye3t_amd.core import basis as _basis
from ye3t_amd.core.cg import cg_matrix


class _BoundedCache:
    def __init__(self, max_entries):
        self.max_entries = int(max_entries)
        self._items = OrderedDict()

    def get(self, key):
        item = self._items.get(key)
        if item is not None:
            self._items.move_to_end(key)
        return item

    def put(self, key, value):
        if self.max_entries <= 0:
            return
        self._items.pop(key, None)
        self._items[key] = value
        while len(self._items) > self.max_entries:
            self._items.popitem(last=False)

    def clear(self):
        self._items.clear()


_FACTORIZED_SCHEDULES_CACHE = _BoundedCache(64)


def angular_key(l_tuple, internal_Ls, tree_type="balanced", basis_key=()):
    """``CompactLabel.angular_key`` (reference ``ye3t/core/labels.py:116-123``)."""
    l_str = ",".join(str(x) for x in l_tuple)
    L_str = ",".join(str(x) for x in internal_Ls)
    basis_str = "" if not basis_key else f"|{tuple(basis_key)!r}"
    if tree_type == "balanced":
        return f"{l_str}_{L_str}{basis_str}"
    return f"{tree_type}:{l_str}_{L_str}{basis_str}"


@dataclass(eq=False)
class FactorizedCoefficientSchedule:
    """Inter-block CG schedule with symmetric blocks collapsed.

    Field meaning follows the reference record (``ye3t/core/couplings.py:164-256``).
    """

    rank: int
    block_count: int
    L_R: int
    n_tuple: tuple
    l_tuple: tuple
    tree_type: str
    block_specs: tuple
    angular_keys: tuple
    basis_keys: tuple
    M_R_values: np.ndarray
    component_label_index: np.ndarray
    component_M_R: np.ndarray
    component_offsets: np.ndarray
    block_m_tuples: np.ndarray
    coeffs: np.ndarray
    structured_labels: tuple = ()

    @property
    def basis_count(self):
        return int(len(self.angular_keys))

    @property
    def component_count(self):
        return int(len(self.component_label_index))

    @property
    def term_count(self):
        return int(len(self.coeffs))

    def component_terms(self, component_index):
        start = int(self.component_offsets[int(component_index)])
        stop = int(self.component_offsets[int(component_index) + 1])
        return self.block_m_tuples[start:stop], self.coeffs[start:stop]

    def block_L_by_label(self, *, dtype=np.int16):
        values = [[int(s["Lambda"] if s["kind"] == "sym" else s["l"]) for s in specs]
                  for specs in self.block_specs]
        if not values:
            return np.zeros((0, int(self.block_count)), dtype=dtype)
        return np.asarray(values, dtype=dtype)

    def flat_arrays(self):
        """Runtime arrays of ``to_torch`` (``core/couplings.py:211-256``) as numpy."""
        offsets = np.asarray(self.component_offsets, dtype=np.int64)
        term_component = np.repeat(np.arange(self.component_count, dtype=np.int64), np.diff(offsets))
        label_index = np.asarray(self.component_label_index, dtype=np.int64)
        term_label = label_index[term_component] if term_component.size else np.zeros(0, np.int64)
        block_L = self.block_L_by_label(dtype=np.int64)
        if self.term_count and self.block_count:
            block_m_indices = np.asarray(self.block_m_tuples, dtype=np.int64) + block_L[term_label]
        else:
            block_m_indices = np.zeros((0, int(self.block_count)), dtype=np.int64)
        coeffs = np.asarray(self.coeffs)
        if np.iscomplexobj(coeffs):
            if coeffs.size and np.max(np.abs(coeffs.imag)) > 1e-12:
                raise ValueError("genuinely complex factorized coefficients")
            coeffs = coeffs.real
        max_m = int(2 * int(block_L.max()) + 1) if block_L.size else 0
        return {
            "component_offsets": offsets,
            "component_label_index": label_index,
            "term_component_index": term_component,
            "term_label_index": term_label,
            "block_m_indices": np.ascontiguousarray(block_m_indices),
            "coeffs": np.ascontiguousarray(coeffs, dtype=np.float64),
            "max_block_m_dim": max_m,
        }


def _leaf_spec(n, l):
    return {"kind": "leaf", "n": int(n), "l": int(l), "k_b": 1, "Lambda": int(l),
            "multiplicity_index": 0, "basis_key": ()}


def _sym_spec(n, l, k, Lam, copy=0):
    return {"kind": "sym", "n": int(n), "l": int(l), "k_b": int(k), "Lambda": int(Lam),
            "multiplicity_index": int(copy), "basis_key": ("sym", int(Lam), int(copy))}


def _identity_schedule(rank, L_R, n_tuple, l_tuple, tree_type, spec, basis_key, coeff_tol, structured):
    """Reference ``_identity_factorized_schedule_for_one_block`` (``couplings.py:1478-1522``)."""
    internal = () if rank == 1 else (int(L_R),)
    M = np.arange(-L_R, L_R + 1, dtype=np.int64)
    count = int(M.shape[0])
    keep = not (coeff_tol > 0.0 and 1.0 <= float(coeff_tol))
    if keep:
        offsets = np.arange(count + 1, dtype=np.int64)
        tuples = M.astype(np.int16).reshape(-1, 1)
        coeffs = np.ones(count, dtype=np.complex128)
    else:
        offsets = np.zeros(count + 1, dtype=np.int64)
        tuples = np.zeros((0, 1), dtype=np.int16)
        coeffs = np.zeros(0, dtype=np.complex128)
    return FactorizedCoefficientSchedule(
        rank=rank, block_count=1, L_R=int(L_R), n_tuple=tuple(n_tuple), l_tuple=tuple(l_tuple),
        tree_type=tree_type, block_specs=((spec,),),
        angular_keys=(angular_key(l_tuple, internal, tree_type, basis_key),),
        basis_keys=(tuple(basis_key),), M_R_values=M,
        component_label_index=np.zeros(count, dtype=np.int64), component_M_R=M.copy(),
        component_offsets=offsets, block_m_tuples=tuples, coeffs=coeffs,
        structured_labels=(structured,))


def _rank_two_direct(n_tuple, l_tuple, L_R, tree_type, coeff_tol):
    """Reference ``_rank_two_direct_cg_schedule`` (``couplings.py:1525-1570``)."""
    l_left, l_right = int(l_tuple[0]), int(l_tuple[1])
    M = np.arange(-L_R, L_R + 1, dtype=np.int64)
    offsets, rows, coeffs = [0], [], []
    cg = cg_matrix(l_left, l_right, L_R)
    for M_R in M.tolist():
        for m_left in range(-l_left, l_left + 1):
            m_right = M_R - m_left
            if m_right < -l_right or m_right > l_right:
                continue
            c = cg[m_left + l_left, m_right + l_right]
            if coeff_tol > 0.0 and abs(c) <= coeff_tol:
                continue
            rows.append((m_left, m_right))
            coeffs.append(c)
        offsets.append(len(coeffs))
    structured = ("node", ("leaf", n_tuple[0], l_left), ("leaf", n_tuple[1], l_right), int(L_R))
    return FactorizedCoefficientSchedule(
        rank=2, block_count=2, L_R=int(L_R), n_tuple=tuple(n_tuple), l_tuple=tuple(l_tuple),
        tree_type=tree_type,
        block_specs=((_leaf_spec(n_tuple[0], l_left), _leaf_spec(n_tuple[1], l_right)),),
        angular_keys=(angular_key(l_tuple, (int(L_R),), tree_type, ()),), basis_keys=((),),
        M_R_values=M, component_label_index=np.zeros(int(M.shape[0]), dtype=np.int64),
        component_M_R=M.copy(), component_offsets=np.asarray(offsets, dtype=np.int64),
        block_m_tuples=np.asarray(rows, dtype=np.int16).reshape(-1, 2),
        coeffs=np.asarray(coeffs, dtype=np.complex128), structured_labels=(structured,))


def _low_rank_schedules(n_tuple, l_tuple, tree_type, coeff_tol):
    if os.getenv("YE3T_DISABLE_LOW_RANK_FACTORIZED_FAST_PATHS", "").strip().lower() in {"1", "true", "yes", "on"}:
        return None
    rank = len(l_tuple)
    if rank == 1:
        L = int(l_tuple[0])
        return {L: _identity_schedule(1, L, n_tuple, l_tuple, tree_type, _leaf_spec(n_tuple[0], L), (),
                                      coeff_tol, ("leaf", n_tuple[0], L))}
    if rank != 2:
        return None
    (n0, n1), (l0, l1) = n_tuple, l_tuple
    if n0 == n1 and l0 == l1:
        out = {}
        for L in range(0, 2 * l0 + 1, 2):
            out[L] = _identity_schedule(2, L, n_tuple, l_tuple, tree_type, _sym_spec(n0, l0, 2, L),
                                        ("sym", L, 0), coeff_tol, ("sym", n0, l0, 2, L, 0))
        return out
    return {L: _rank_two_direct(n_tuple, l_tuple, L, tree_type, coeff_tol)
            for L in range(abs(l0 - l1), l0 + l1 + 1)}


_PATH_CACHE = {}


def expand_path_key(key):
    """Root ``M``, block ``m`` tuples and coefficients of one angular path key.

    Reference ``_expand_block_m_path_arrays_from_key`` (``factorized_dag.py:73-131``):
    rows ordered (left term, right term) lexicographically, CG nonzeros kept
    where ``|cg| > 1e-14``, coefficient ``left * right * cg``.
    """
    cached = _PATH_CACHE.get(key)
    if cached is not None:
        return cached
    kind = key[0]
    if kind in ("leaf", "sym"):
        L = int(key[1])
        m = np.arange(-L, L + 1, dtype=np.int16)
        out = (m.copy(), m.reshape(-1, 1), np.ones(m.shape[0], dtype=np.float64))
    else:
        left_key, right_key, L_out = key[1], key[2], int(key[3])
        lM, lT, lC = expand_path_key(left_key)
        rM, rT, rC = expand_path_key(right_key)
        width = lT.shape[1] + rT.shape[1]
        empty = (np.zeros(0, np.int16), np.zeros((0, width), np.int16), np.zeros(0, np.float64))
        if lM.shape[0] == 0 or rM.shape[0] == 0:
            out = empty
        else:
            lt, rt = _path_total(left_key), _path_total(right_key)
            li = np.repeat(np.arange(lM.shape[0]), rM.shape[0])
            ri = np.tile(np.arange(rM.shape[0]), lM.shape[0])
            M = lM[li].astype(np.int16) + rM[ri].astype(np.int16)
            valid = np.abs(M) <= L_out
            li, ri, M = li[valid], ri[valid], M[valid]
            cg = cg_matrix(lt, rt, L_out)[lM[li].astype(np.int64) + lt, rM[ri].astype(np.int64) + rt]
            nz = np.abs(cg) > 1e-14
            if not np.any(nz):
                out = empty
            else:
                li, ri, M = li[nz], ri[nz], M[nz]
                tuples = np.concatenate((lT[li], rT[ri]), axis=1)
                coeffs = lC[li] * rC[ri] * cg[nz]
                out = (M.astype(np.int16), tuples.astype(np.int16), coeffs)
    _PATH_CACHE[key] = out
    return out


def _path_total(key):
    return int(key[1]) if key[0] in ("leaf", "sym") else int(key[3])


def _schedule_from_structured(structured_labels, L_R, tree_type, coeff_tol):
    compact = [_basis.compact_label(lab, tree_type) for lab in structured_labels]
    first = structured_labels[0]
    n_tuple, l_tuple = _basis.n_sequence(first), _basis.l_sequence(first)
    specs = tuple(_basis.block_specs(lab) for lab in structured_labels)
    block_count = len(specs[0])
    M_values = tuple(range(-L_R, L_R + 1))
    comp_label, comp_M, offsets = [], [], [0]
    tuple_chunks, coeff_chunks = [], []
    for label_index, lab in enumerate(structured_labels):
        root_M, tuples, coeffs = expand_path_key(_basis.path_key(lab))
        for M_R in M_values:
            comp_label.append(label_index)
            comp_M.append(M_R)
            keep = root_M == M_R
            if coeff_tol > 0.0:
                keep = keep & (np.abs(coeffs) > coeff_tol)
            count = int(np.count_nonzero(keep))
            if count:
                tuple_chunks.append(tuples[keep])
                coeff_chunks.append(coeffs[keep])
            offsets.append(offsets[-1] + count)
    block_m = (np.concatenate(tuple_chunks, axis=0).astype(np.int16) if tuple_chunks
               else np.zeros((0, block_count), np.int16))
    coeffs = (np.concatenate(coeff_chunks).astype(np.complex128) if coeff_chunks
              else np.zeros(0, np.complex128))
    keys = []
    for lab, comp in zip(structured_labels, compact):
        basis_key = comp[4] if len(comp) == 5 else ()
        keys.append((angular_key(comp[1], comp[2], tree_type, basis_key), tuple(basis_key)))
    return FactorizedCoefficientSchedule(
        rank=len(l_tuple), block_count=block_count, L_R=int(L_R), n_tuple=n_tuple, l_tuple=l_tuple,
        tree_type=tree_type, block_specs=specs, angular_keys=tuple(k for k, _ in keys),
        basis_keys=tuple(b for _, b in keys), M_R_values=np.asarray(M_values, dtype=np.int64),
        component_label_index=np.asarray(comp_label, dtype=np.int64),
        component_M_R=np.asarray(comp_M, dtype=np.int64),
        component_offsets=np.asarray(offsets, dtype=np.int64), block_m_tuples=block_m, coeffs=coeffs,
        structured_labels=tuple(structured_labels))


def generate_factorized_coefficient_schedules_by_L(n_in, l_in, *, tree_type="balanced", coeff_tol=1e-14,
                                                   constructor_backend="auto"):
    """All target-``L`` schedules of one ACE signature (``core/couplings.py:2066-2122``)."""
    n_sig = tuple(int(x) for x in n_in)
    l_sig = tuple(int(x) for x in l_in)
    tree_type = _basis.validate_tree_type(tree_type)
    key = (n_sig, l_sig, tree_type, float(coeff_tol))
    cached = _FACTORIZED_SCHEDULES_CACHE.get(key)
    if cached is not None:
        return cached
    low = _low_rank_schedules(n_sig, l_sig, tree_type, coeff_tol)
    if low is not None:
        _FACTORIZED_SCHEDULES_CACHE.put(key, low)
        return low
    labels = _basis.structured_labels_by_L(n_sig, l_sig, tree_type)
    out = {int(L): _schedule_from_structured(list(labs), int(L), tree_type, coeff_tol)
           for L, labs in labels.items()}
    _FACTORIZED_SCHEDULES_CACHE.put(key, out)
    return out


def _torch_flat(schedule, device, dtype):
    import torch

    flat = schedule.flat_arrays()
    return {k: (torch.as_tensor(v, device=device) if isinstance(v, np.ndarray) else v) for k, v in flat.items()}


def evaluate_factorized_schedule_torch(block_values, schedule, *, backend="auto"):
    """``out[b, k] = sum_{t in k} c_t prod_blk block_values[b, label_k, blk, m_t,blk]``.

    Contract of the reference evaluator (``ye3t/core/couplings.py:481-567``):
    ``block_values`` is ``[batch, basis, block, max_m]`` and the result is
    ``[batch, component_count]``.  ``backend``: ``"auto"`` (HIP on a GPU tensor,
    Torch on CPU), ``"hip"`` (raise unless the HIP library runs it) or ``"torch"``.
    """
    import torch

    if block_values.ndim != 4:
        raise ValueError("block_values must have shape [batch, basis_count, block_count, max_block_m_dim].")
    flat = schedule.flat_arrays()
    if int(block_values.shape[1]) < schedule.basis_count:
        raise ValueError("block_values basis dimension is smaller than schedule.basis_count.")
    if int(block_values.shape[2]) != int(schedule.block_count):
        raise ValueError("block_values block dimension must equal schedule.block_count.")
    if int(block_values.shape[3]) < int(flat["max_block_m_dim"]):
        raise ValueError("block_values magnetic dimension is smaller than schedule.max_block_m_dim.")
    selected = str(backend or "auto").strip().lower()
    if selected == "auto":
        env = os.getenv("YE3T_FACTORIZED_RUNTIME_BACKEND", "auto").strip().lower()
        selected = env if env not in {"", "auto"} else ("hip" if block_values.device.type == "cuda" else "torch")
    if selected in {"hip", "native"}:
        from ye3t_amd.runtime import native

        return native.evaluate_factorized_schedule(block_values, schedule)
    if selected not in {"torch", "pytorch"}:
        raise ValueError(f"Unknown factorized runtime backend: {backend!r}")
    device, dtype = block_values.device, block_values.dtype
    out = torch.zeros((int(block_values.shape[0]), schedule.component_count), dtype=dtype, device=device)
    if schedule.term_count == 0:
        return out
    coeffs = torch.as_tensor(flat["coeffs"], dtype=dtype, device=device)
    term_label = torch.as_tensor(flat["term_label_index"], device=device)
    m_idx = torch.as_tensor(flat["block_m_indices"], device=device)
    term_comp = torch.as_tensor(flat["term_component_index"], device=device)
    values = coeffs.unsqueeze(0).expand(int(block_values.shape[0]), -1)
    batch_index = torch.arange(int(block_values.shape[0]), device=device).unsqueeze(1)
    for blk in range(schedule.block_count):
        values = values * block_values[batch_index, term_label.unsqueeze(0), blk, m_idx[:, blk].unsqueeze(0)]
    out.index_add_(1, term_comp, values)
    return out


# ------------------------------------------------------------ real tesseral
@dataclass(eq=False)
class RealFactorizedCoefficientSchedule:
    """Real-tesseral inter-block CG schedule for collapsed ACE blocks.

    Fields of the reference record (``ye3t/core/couplings.py:313-420``).  Block
    and output components are real indices in the reference's tesseral ordering
    (:func:`ye3t_amd.core.cg.tesseral_unitary`), so ``block_real_tuples`` index
    the block values directly.
    """

    rank: int
    block_count: int
    L_R: int
    n_tuple: tuple
    l_tuple: tuple
    tree_type: str
    block_specs: tuple
    angular_keys: tuple
    basis_keys: tuple
    component_indices: np.ndarray
    component_label_index: np.ndarray
    component_offsets: np.ndarray
    block_real_tuples: np.ndarray
    coeffs: np.ndarray
    basis_convention: str = "real_tesseral"
    permutation_sector: str = "trivial"
    backend_provenance: str = "real_cg_direct"
    complex_term_count: int = -1
    fallback_reason: object = None
    structured_labels: tuple = ()

    @property
    def basis_count(self):
        return int(len(self.angular_keys))

    @property
    def component_count(self):
        return int(len(self.component_label_index))

    @property
    def term_count(self):
        return int(len(self.coeffs))

    def component_terms(self, component_index):
        start = int(self.component_offsets[int(component_index)])
        stop = int(self.component_offsets[int(component_index) + 1])
        return self.block_real_tuples[start:stop], self.coeffs[start:stop]

    def block_L_by_label(self, *, dtype=np.int16):
        values = [[int(s["Lambda"] if s["kind"] == "sym" else s["l"]) for s in specs]
                  for specs in self.block_specs]
        if not values:
            return np.zeros((0, int(self.block_count)), dtype=dtype)
        return np.asarray(values, dtype=dtype)

    def metadata(self):
        return {"basis_convention": str(self.basis_convention),
                "permutation_sector": str(self.permutation_sector),
                "backend_provenance": str(self.backend_provenance),
                "term_count": int(self.term_count),
                "complex_term_count": int(self.complex_term_count),
                "fallback_reason": None if self.fallback_reason is None else str(self.fallback_reason)}

    def flat_arrays(self):
        """Runtime arrays of ``to_torch`` (``core/couplings.py:378-420``) as numpy;
        ``block_m_indices`` are the real component indices themselves."""
        offsets = np.asarray(self.component_offsets, dtype=np.int64)
        term_component = np.repeat(np.arange(self.component_count, dtype=np.int64), np.diff(offsets))
        label_index = np.asarray(self.component_label_index, dtype=np.int64)
        term_label = label_index[term_component] if term_component.size else np.zeros(0, np.int64)
        block_L = self.block_L_by_label(dtype=np.int64)
        if self.term_count and self.block_count:
            idx = np.asarray(self.block_real_tuples, dtype=np.int64)
        else:
            idx = np.zeros((0, int(self.block_count)), dtype=np.int64)
        return {
            "component_offsets": offsets,
            "component_label_index": label_index,
            "term_component_index": term_component,
            "term_label_index": term_label,
            "block_m_indices": np.ascontiguousarray(idx),
            "coeffs": np.ascontiguousarray(self.coeffs, dtype=np.float64),
            "max_block_m_dim": int(2 * int(block_L.max()) + 1) if block_L.size else 0,
        }


def _as_tuple(value):
    if isinstance(value, (list, tuple)):
        return tuple(_as_tuple(v) for v in value)
    return value


def structured_label_from_compact(compact):
    """The structured label whose ``compact_label`` is ``compact`` (its ``count`` order).

    ``compact`` is a :class:`~ye3t_amd.core.basis.CompactLabel`, its dict form
    or a 3-, 4- or 5-part tuple.
    """
    record = _basis.normalize_compact_label(_as_tuple(compact) if isinstance(compact, list) else compact)
    compact = record.compact_label()
    n_seq, l_seq, internal = compact[0], compact[1], compact[2]
    tree_type = record.tree_type
    target = int(internal[-1]) if internal else int(l_seq[0])
    for lab in _basis.structured_labels_by_L(tuple(n_seq), tuple(l_seq), tree_type).get(target, ()):
        if _basis.compact_label(lab, tree_type) == compact:
            return lab
    raise ValueError(f"Could not recover structured label for {compact!r}.")


def _label_total_L(label):
    return int(label[2] if label[0] == "leaf" else label[4] if label[0] == "sym" else label[3])


_REAL_PATH_CACHE = {}


def expand_real_path(label):
    """Root component, block real tuples and coefficients of one structured label.

    Reference ``_expand_block_real_path_arrays`` (``core/couplings.py:1339-1403``):
    leaves and collapsed sym blocks are identities on their ``2L+1``
    components; a node walks the tesseral CG nonzeros in ``(a, b, c)`` order
    and, for each, pairs every left term ending in ``a`` with every right term
    ending in ``b`` (left outer), keeping ``|product| > 1e-14``.
    """
    key = _basis.path_key(label)
    cached = _REAL_PATH_CACHE.get(key)
    if cached is not None:
        return cached
    if label[0] in ("leaf", "sym"):
        dim = 2 * _label_total_L(label) + 1
        idx = np.arange(dim, dtype=np.int16)
        out = (idx, idx.reshape(dim, 1), np.ones(dim, dtype=np.float64))
    else:
        from ye3t_amd.core.cg import tesseral_cg_entries

        l_out, l_tup, l_co = expand_real_path(label[1])
        r_out, r_tup, r_co = expand_real_path(label[2])
        width = l_tup.shape[1] + r_tup.shape[1]
        entries = tesseral_cg_entries(_label_total_L(label[1]), _label_total_L(label[2]), int(label[3]))
        outs, tups, cos = [], [], []
        if entries and l_out.size and r_out.size:
            l_by = {}
            r_by = {}
            for i, c in enumerate(l_out.tolist()):
                l_by.setdefault(int(c), []).append(i)
            for i, c in enumerate(r_out.tolist()):
                r_by.setdefault(int(c), []).append(i)
            for a, b, c, v in entries:
                li, ri = l_by.get(a), r_by.get(b)
                if not li or not ri:
                    continue
                fl = np.repeat(np.asarray(li, np.int64), len(ri))
                fr = np.tile(np.asarray(ri, np.int64), len(li))
                co = l_co[fl] * r_co[fr] * float(v)
                keep = np.abs(co) > 1.0e-14
                if not np.any(keep):
                    continue
                outs.append(np.full(int(np.count_nonzero(keep)), c, dtype=np.int16))
                tups.append(np.concatenate((l_tup[fl], r_tup[fr]), axis=1)[keep])
                cos.append(co[keep])
        if outs:
            out = (np.concatenate(outs).astype(np.int16), np.concatenate(tups).astype(np.int16),
                   np.concatenate(cos))
        else:
            out = (np.zeros(0, np.int16), np.zeros((0, width), np.int16), np.zeros(0, np.float64))
    _REAL_PATH_CACHE[key] = out
    return out


def generate_real_factorized_coefficient_schedule_for_labels(labels, component_indices=None, coeff_tol=1e-14, *,
                                                             coeff_dtype=np.float64, real_index_dtype=np.int16):
    """Real-tesseral factorized ACE schedule of compact labels.

    Reference ``generate_real_factorized_coefficient_schedule_for_labels`` /
    ``_real_factorized_schedule_from_structured_labels``
    (``core/couplings.py:1818-1966``): assembled label-major, components in
    ``component_indices`` order, terms in :func:`expand_real_path` order.
    """
    labels = [_basis.normalize_compact_label(_as_tuple(lab) if isinstance(lab, list) else lab).payload()
              for lab in labels]
    if not labels:
        return RealFactorizedCoefficientSchedule(
            rank=0, block_count=0, L_R=0, n_tuple=(), l_tuple=(), tree_type="balanced", block_specs=(),
            angular_keys=(), basis_keys=(), component_indices=np.asarray([0], dtype=np.int64),
            component_label_index=np.zeros(0, np.int64), component_offsets=np.zeros(1, np.int64),
            block_real_tuples=np.zeros((0, 0), dtype=real_index_dtype), coeffs=np.zeros(0, dtype=coeff_dtype))
    structured = [structured_label_from_compact(lab) for lab in labels]
    first = labels[0]
    tree_type = first[3] if len(first) > 3 else "balanced"
    L_R = _label_total_L(structured[0])
    rank = len(first[0])
    if component_indices is None:
        component_indices = range(0, 2 * L_R + 1)
    component_indices = tuple(int(c) for c in component_indices)
    for c in component_indices:
        if c < 0 or c >= 2 * L_R + 1:
            raise ValueError(f"Real component index {c} is outside V_{L_R}.")
    for lab, s in zip(labels, structured):
        if _label_total_L(s) != L_R:
            raise ValueError("All labels must share one final L_R.")
        if len(lab[0]) != rank:
            raise ValueError("All labels must have the same rank.")
    specs = tuple(_basis.block_specs(s) for s in structured)
    block_count = len(specs[0])
    comp_label, offsets, tup_chunks, co_chunks = [], [0], [], []
    for label_index, s in enumerate(structured):
        root, tuples, coeffs = expand_real_path(s)
        for c in component_indices:
            comp_label.append(label_index)
            keep = root == c
            if coeff_tol > 0.0:
                keep = keep & (np.abs(coeffs) > float(coeff_tol))
            count = int(np.count_nonzero(keep))
            if count:
                tup_chunks.append(tuples[keep])
                co_chunks.append(coeffs[keep])
            offsets.append(offsets[-1] + count)
    block_real = (np.concatenate(tup_chunks).astype(real_index_dtype) if tup_chunks
                  else np.zeros((0, block_count), dtype=real_index_dtype))
    coeffs = (np.concatenate(co_chunks).astype(coeff_dtype) if co_chunks else np.zeros(0, dtype=coeff_dtype))
    keys = []
    for lab in labels:
        basis_key = lab[4] if len(lab) == 5 else ()
        keys.append((angular_key(lab[1], lab[2], tree_type, basis_key), tuple(basis_key)))
    complex_terms = _schedule_from_structured(structured, L_R, tree_type, coeff_tol).term_count
    return RealFactorizedCoefficientSchedule(
        rank=rank, block_count=block_count, L_R=L_R, n_tuple=tuple(first[0]), l_tuple=tuple(first[1]),
        tree_type=tree_type, block_specs=specs, angular_keys=tuple(k for k, _ in keys),
        basis_keys=tuple(b for _, b in keys), component_indices=np.asarray(component_indices, dtype=np.int64),
        component_label_index=np.asarray(comp_label, dtype=np.int64),
        component_offsets=np.asarray(offsets, dtype=np.int64), block_real_tuples=block_real, coeffs=coeffs,
        complex_term_count=int(complex_terms), structured_labels=tuple(structured))


def evaluate_real_factorized_schedule_torch(block_values, schedule, *, backend="auto"):
    """Evaluate a real-tesseral schedule (reference ``core/couplings.py:570-610``).

    Same contract as :func:`evaluate_factorized_schedule_torch`; real block
    values only.  ``"auto"`` runs the HIP kernel on a GPU tensor.
    """
    import torch

    if torch.is_complex(block_values):
        raise ValueError("Real factorized schedule evaluation requires real block values.")
    return evaluate_factorized_schedule_torch(block_values, schedule, backend=backend)
