"""ACE product plans: which B-features to compute from a density row, and how.

A *sample* is one row of the density ``A`` (an atom, or an (atom, channel)
pair for channel-wise products).  The row holds ``channel_count`` radial
channels, each with all real SH components ``l <= l_max`` (``(l_max+1)^2``
values, degree ``l`` at ``[l^2, (l+1)^2)``, ``m`` ascending), i.e. one
``A[i, c, n, l, m]`` slice flattened over ``(c, n)``.

Features are the reference's ACE labels (``ye3t/couplings/__init__.py:2617``
compiler, see :mod:`ye3t_amd.core.couplings`) of every content (multiset of
``(n, l)`` leaves), evaluated in the real spherical-harmonic basis of the SH
table.  Ordering: target ``L`` ascending, then content (canonical leaf tuple,
lexicographic, rank ascending), then label order, then component.

Two equivalent evaluation forms are produced:

* ``flat``: per output column a list of terms ``c * prod_blocks value`` over
  *block values* (leaves and symmetric blocks) -- the structure of the
  reference's ``evaluate_factorized_schedule_cpu`` plus
  ``symmetric_power_monomial_forward`` (``factorized_runtime.cpp:251-285``,
  ``ye3t_runtime_core.cpp:5279-5315``); used by the CPU oracle.
* ``dag``: hash-consed nodes (leaf, symmetric block, pair coupling) shared
  across labels and contents -- the factorized-angular DAG form with shared
  intermediate couplings (``ye3t/runtime/execution_plan.py:6303, 13550-13903``);
  executed by the HIP product kernel.
"""

import itertools
import json
import hashlib
from dataclasses import dataclass, field

import numpy as np

from ye3t_amd.core import basis as _basis
from ye3t_amd.core.cg import real_cg_entries
from ye3t_amd.core.couplings import generate_factorized_coefficient_schedules_by_L
from ye3t_amd.core.symmetric_power import real_monomial_entries


@dataclass
class ACEFeatureSpec:
    """What to compute per sample.

    ``caps`` maps rank -> ``(max_radial, max_l)``; a content of that rank uses
    only channels whose radial index (0-based within its species block) is
    ``< max_radial`` and degrees ``<= max_l`` -- the per-rank ``eta``/``l``
    truncation knobs of the reference's representation config
    (``ye3t/representation_config.py:94-147``).
    """

    channel_count: int            # channels (n) per sample row
    l_max: int
    nu_max: int
    targets: tuple = (0,)
    parity: str = "any"           # "any" or "even" (O(3) even for scalar ACE)
    nu_min: int = 1
    radial_per_species: int = 0   # 0: no species blocks; else channels = species*radial
    caps: dict = field(default_factory=dict)
    channel_ids: tuple = ()       # optional explicit one-based channel ids (default 1..C)

    def row_width(self):
        return self.channel_count * (self.l_max + 1) ** 2

    def leaf_offset(self, n, l):
        return (int(n) - 1) * (self.l_max + 1) ** 2 + int(l) * int(l)

    def _allowed_pairs(self, rank):
        cap_r, cap_l = self.caps.get(rank, (None, None))
        out = []
        ids = self.channel_ids or tuple(range(1, self.channel_count + 1))
        for n in ids:
            radial = (n - 1) % self.radial_per_species if self.radial_per_species else n - 1
            if cap_r is not None and radial >= cap_r:
                continue
            for l in range(self.l_max + 1):
                if cap_l is not None and l > cap_l:
                    continue
                out.append((n, l))
        return out

    def contents(self):
        for rank in range(self.nu_min, self.nu_max + 1):
            for combo in itertools.combinations_with_replacement(self._allowed_pairs(rank), rank):
                ls = tuple(p[1] for p in combo)
                if self.parity == "even" and sum(ls) % 2:
                    continue
                if rank == 1 and ls[0] not in self.targets:
                    continue
                n_c, l_c = _basis.canonicalize_leaf_quantum_numbers(tuple(p[0] for p in combo), ls)
                yield n_c, l_c

    def to_dict(self):
        return {"channel_count": self.channel_count, "l_max": self.l_max, "nu_max": self.nu_max,
                "nu_min": self.nu_min, "targets": list(self.targets), "parity": self.parity,
                "radial_per_species": self.radial_per_species,
                "caps": {str(k): list(v) for k, v in sorted(self.caps.items())},
                "channel_ids": list(self.channel_ids)}


def _label_phase_odd(label):
    """Count of odd-parity couplings along a label (nodes and symmetric blocks)."""
    kind = label[0]
    if kind == "leaf":
        return 0
    if kind == "sym":
        return (label[3] * label[2] + label[4]) % 2
    return (_label_phase_odd(label[1]) + _label_phase_odd(label[2])
            + (_basis.total_L(label[1]) + _basis.total_L(label[2]) - label[3]) % 2)


class ProductPlan:
    """Compiled features of one :class:`ACEFeatureSpec` (both evaluation forms)."""

    def __init__(self, spec):
        self.spec = spec
        self.a_width = spec.row_width()
        self.features = []          # (L, content_index, label_index, component)
        self.label_records = []     # (L, content, structured label, first column)
        self.contents = []
        by_content = {}
        for n_c, l_c in spec.contents():
            by_content[(n_c, l_c)] = generate_factorized_coefficient_schedules_by_L(n_c, l_c)
            self.contents.append((n_c, l_c))
        order = sorted(range(len(self.contents)),
                       key=lambda i: (len(self.contents[i][0]), tuple(zip(*self.contents[i]))))
        self.contents = [self.contents[i] for i in order]
        for L in sorted(spec.targets):
            for ci, content in enumerate(self.contents):
                sched = by_content[content].get(L)
                if sched is None:
                    continue
                for li, lab in enumerate(sched.structured_labels):
                    self.label_records.append((L, ci, lab, len(self.features)))
                    for comp in range(2 * L + 1):
                        self.features.append((L, ci, li, comp))
        self.feature_count = len(self.features)
        self._build_dag()
        self._flat = None

    # ------------------------------------------------------------------ DAG
    def _build_dag(self):
        spec = self.spec
        self.nodes = []            # dicts: kind, dim, terms [(component, coeff, (slots...))], operands
        self.node_index = {}
        self.outputs = []          # (node id, component) per feature column

        def leaf(n, l):
            key = ("leaf", n, l)
            if key not in self.node_index:
                self.node_index[key] = len(self.nodes)
                self.nodes.append({"kind": "leaf", "key": key, "dim": 2 * l + 1,
                                   "a_offset": spec.leaf_offset(n, l), "deps": ()})
            return self.node_index[key]

        def sym(n, l, k, Lam, copy):
            key = ("sym", n, l, k, Lam, copy)
            if key not in self.node_index:
                src = leaf(n, l)
                terms = []
                for out_c, exps, value in real_monomial_entries(k, l, Lam, copy):
                    factors = tuple(m for m, e in enumerate(exps) for _ in range(e))
                    terms.append((out_c, value, factors))
                self.node_index[key] = len(self.nodes)
                self.nodes.append({"kind": "sym", "key": key, "dim": 2 * Lam + 1, "terms": terms,
                                   "deps": (src,), "k": k})
            return self.node_index[key]

        def build(label):
            kind = label[0]
            if kind == "leaf":
                return leaf(label[1], label[2])
            if kind == "sym":
                return sym(*label[1:])
            a, b = build(label[1]), build(label[2])
            La, Lb, L = _basis.total_L(label[1]), _basis.total_L(label[2]), label[3]
            key = ("pair", a, b, L)
            if key not in self.node_index:
                terms = [(c, v, (i, j)) for i, j, c, v in real_cg_entries(La, Lb, L)]
                self.node_index[key] = len(self.nodes)
                self.nodes.append({"kind": "pair", "key": key, "dim": 2 * L + 1, "terms": terms,
                                   "deps": (a, b)})
            return self.node_index[key]

        for L, ci, lab, first in self.label_records:
            root = build(lab)
            for comp in range(2 * L + 1):
                self.outputs.append((root, comp))

    def dag_stats(self):
        counts = {"leaf": 0, "sym": 0, "pair": 0}
        terms = {"sym": 0, "pair": 0}
        factors = 0
        for nd in self.nodes:
            counts[nd["kind"]] += 1
            if nd["kind"] != "leaf":
                terms[nd["kind"]] += len(nd["terms"])
                factors += sum(len(t[2]) for t in nd["terms"])
        return {"nodes": counts, "terms": terms, "factor_reads": factors,
                "features": self.feature_count, "a_width": self.a_width}

    # ----------------------------------------------------------------- flat
    def flat(self):
        """Flat real schedule: block values + per-column term lists.

        ``block_values``: list of ``(kind, key)``; a leaf block value vector is
        read from the row, a sym block value vector is the monomial contraction.
        ``terms``: per column, ``(coeff, (block_value_ref, component), ...)``.
        The expansion restates ``_expand_block_real_path_arrays``
        (``ye3t/core/couplings.py:1339-1402``) in this package's real basis.
        """
        if self._flat is not None:
            return self._flat
        blocks, block_index = [], {}

        def block_ref(spec_key):
            if spec_key not in block_index:
                block_index[spec_key] = len(blocks)
                blocks.append(spec_key)
            return block_index[spec_key]

        cache = {}

        def expand(label):
            kind = label[0]
            if kind in ("leaf", "sym"):
                ref = block_ref(label)
                dim = 2 * _basis.total_L(label) + 1
                return [(c, 1.0, ((ref, c),)) for c in range(dim)]
            key = label
            if key in cache:
                return cache[key]
            left, right = expand(label[1]), expand(label[2])
            La, Lb, L = _basis.total_L(label[1]), _basis.total_L(label[2]), label[3]
            by_l, by_r = {}, {}
            for t in left:
                by_l.setdefault(t[0], []).append(t)
            for t in right:
                by_r.setdefault(t[0], []).append(t)
            out = []
            for a, b, c, v in sorted(real_cg_entries(La, Lb, L), key=lambda e: (e[0], e[1], e[2])):
                for tl in by_l.get(a, ()):
                    for tr in by_r.get(b, ()):
                        coeff = tl[1] * tr[1] * v
                        if abs(coeff) > 1e-14:
                            out.append((c, coeff, tl[2] + tr[2]))
            cache[key] = out
            return out

        columns = []
        for L, ci, lab, first in self.label_records:
            expanded = expand(lab)
            for comp in range(2 * L + 1):
                columns.append([(coeff, refs) for c, coeff, refs in expanded if c == comp])
        block_tables = []
        for key in blocks:
            if key[0] == "leaf":
                block_tables.append({"kind": "leaf", "a_offset": self.spec.leaf_offset(key[1], key[2]),
                                     "dim": 2 * key[2] + 1})
            else:
                _, n, l, k, Lam, copy = key
                block_tables.append({"kind": "sym", "a_offset": self.spec.leaf_offset(n, l), "in_dim": 2 * l + 1,
                                     "dim": 2 * Lam + 1, "k": k,
                                     "entries": real_monomial_entries(k, l, Lam, copy)})
        self._flat = {"blocks": block_tables, "columns": columns}
        return self._flat

    def flat_arrays(self):
        """Flat form packed as arrays for the C oracle."""
        flat = self.flat()
        blk_off = [0]
        for b in flat["blocks"]:
            blk_off.append(blk_off[-1] + b["dim"])
        # symmetric-block monomial tables (exponent counts over the input multiplet)
        sym_rows = []
        for bi, b in enumerate(flat["blocks"]):
            if b["kind"] == "leaf":
                for c in range(b["dim"]):
                    sym_rows.append((bi, c, 1.0, (c,)))
            else:
                for out_c, exps, value in b["entries"]:
                    factors = tuple(m for m, e in enumerate(exps) for _ in range(e))
                    sym_rows.append((bi, out_c, value, factors))
        # value slot v = blk_off[bi] + c, computed from factors over A row
        n_vals = blk_off[-1]
        vt_offsets = np.zeros(n_vals + 1, dtype=np.int64)
        counts = np.zeros(n_vals, dtype=np.int64)
        for bi, c, value, factors in sym_rows:
            counts[blk_off[bi] + c] += 1
        vt_offsets[1:] = np.cumsum(counts)
        vt_coeff = np.zeros(int(vt_offsets[-1]), dtype=np.float64)
        vt_fac = np.full((int(vt_offsets[-1]), 4), -1, dtype=np.int32)
        fill = vt_offsets[:-1].copy()
        for bi, c, value, factors in sym_rows:
            v = blk_off[bi] + c
            pos = fill[v]
            fill[v] += 1
            vt_coeff[pos] = value
            base = flat["blocks"][bi]["a_offset"]
            for q, f in enumerate(factors):
                vt_fac[pos, q] = base + f
        col_off = np.zeros(len(flat["columns"]) + 1, dtype=np.int64)
        col_off[1:] = np.cumsum([len(c) for c in flat["columns"]])
        t_coeff = np.zeros(int(col_off[-1]), dtype=np.float64)
        t_ref = np.full((int(col_off[-1]), 4), -1, dtype=np.int32)
        pos = 0
        for col in flat["columns"]:
            for coeff, refs in col:
                t_coeff[pos] = coeff
                for q, (bi, c) in enumerate(refs):
                    t_ref[pos, q] = blk_off[bi] + c
                pos += 1
        return {"value_offsets": vt_offsets, "value_coeffs": vt_coeff, "value_factors": vt_fac,
                "value_count": n_vals, "column_offsets": col_off, "term_coeffs": t_coeff,
                "term_refs": t_ref}

    def convention_hash(self):
        payload = {"spec": self.spec.to_dict(), "features": self.feature_count,
                   "labels": [[L, list(map(list, self.contents[ci])), repr(lab)]
                              for L, ci, lab, _ in self.label_records]}
        return hashlib.sha256(json.dumps(payload, sort_keys=True).encode()).hexdigest()[:16]
