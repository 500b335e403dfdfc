"""Exact ACE label enumeration for the globally trivial (fully symmetric) sector.

Restates the reference's label construction without SymPy:

* canonical leaf order, ``l``-first (reference ``ye3t/core/basis/validation.py:37-61``);
* Young-subgroup blocks = runs of identical ``(n, l)`` (``theory.py:203-225``);
* ``Sym^k(V_l)`` irrep multiplicities from weight counts
  (``ye3t/core/basis/multiplicity.py:15-87``);
* block-coupling tree shapes (``ye3t/core/basis/tree.py:124-180``);
* block subspaces coupled by CG ranges and ordered by the Python tuple order of
  ``compact_label()`` (``young_exact.py:337-342, 413-457``, ``basis/labels.py``).

Label records are plain tuples-of-ints so ordering is Python's tuple order, the
same order the reference's ``sorted(compact_label)`` produces.
"""

from collections import Counter
from collections.abc import Mapping
from dataclasses import dataclass
from functools import lru_cache


def validate_tree_type(tree_type):
    normalized = "balanced" if tree_type is None else str(tree_type).strip().lower()
    if normalized in {"balanced", "balanced_pairwise", "pairwise"}:
        return "balanced"
    if normalized in {"left", "left_justified", "left-justified"}:
        return "left"
    raise ValueError(f"Unknown tree_type '{tree_type}'. Use 'balanced' or 'left'.")


def validate_leaf_quantum_numbers(nin, lin):
    if len(nin) != len(lin):
        raise ValueError("nin and lin must have the same length.")
    if len(nin) == 0:
        raise ValueError("nin and lin must be non-empty.")
    if any(int(n) < 1 for n in nin):
        raise ValueError(f"All radial quantum numbers n must be positive integers; got nin={tuple(nin)}")
    if any(int(l) < 0 for l in lin):
        raise ValueError(f"All angular quantum numbers l must be non-negative integers; got lin={tuple(lin)}")


def canonicalize_leaf_quantum_numbers(nin, lin):
    """Order leaves by (-multiplicity of l, l, n) -- reference ``validation.py:37-61``."""
    validate_leaf_quantum_numbers(nin, lin)
    counts = Counter(int(l) for l in lin)
    pairs = sorted(((int(n), int(l)) for n, l in zip(nin, lin)),
                   key=lambda p: (-counts[p[1]], p[1], p[0]))
    return tuple(n for n, _ in pairs), tuple(l for _, l in pairs)


def young_blocks(nin, lin):
    """Runs of identical ``(n, l)`` in first-appearance order -> ``[(n, l, k)]``."""
    counts = {}
    for n, l in zip(nin, lin):
        counts[(int(n), int(l))] = counts.get((int(n), int(l)), 0) + 1
    return tuple((n, l, k) for (n, l), k in counts.items())


@lru_cache(maxsize=512)
def symmetric_power_weight_counts(l, k):
    """Weight multiplicities of ``Sym^k(V_l)`` (reference ``multiplicity.py:19-60``)."""
    l, k = int(l), int(k)
    if k == 0 or l == 0:
        return {0: 1}
    polys = [{0: 1}] + [dict() for _ in range(k)]
    for weight in range(-l, l + 1):
        for degree in range(1, k + 1):
            source, target = polys[degree - 1], polys[degree]
            for exponent, coeff in source.items():
                target[exponent + weight] = target.get(exponent + weight, 0) + coeff
    return {w: c for w, c in polys[k].items() if c}


@lru_cache(maxsize=512)
def symmetric_power_irrep_multiplicities(l, k):
    """``d_Lambda`` of ``Sym^k(V_l) = sum d_Lambda V_Lambda`` (``multiplicity.py:63-80``)."""
    weights = symmetric_power_weight_counts(int(l), int(k))
    out = {}
    for L in range(int(l) * int(k), -1, -1):
        d = weights.get(L, 0) - weights.get(L + 1, 0)
        if d > 0:
            out[L] = d
    return dict(sorted(out.items()))


def couple_multiplicities(left, right):
    """CG-range convolution of two SO(3) multiplicity maps (``multiplicity.py:83-108``)."""
    out = {}
    for a, ma in left.items():
        for b, mb in right.items():
            for L in range(abs(a - b), a + b + 1):
                out[L] = out.get(L, 0) + ma * mb
    return dict(sorted((L, v) for L, v in out.items() if v))


# ----------------------------------------------------------------------------
# Tree shapes over blocks
# ----------------------------------------------------------------------------

def block_tree_shape(block_count, tree_type="balanced"):
    """Nested tuple shape; ``None`` marks a leaf (reference ``tree.py:124-180``)."""
    tree_type = validate_tree_type(tree_type)
    level = [None] * int(block_count)
    while len(level) > 1:
        if tree_type == "balanced":
            nxt, i = [], 0
            while i < len(level):
                if i + 1 < len(level):
                    nxt.append((level[i], level[i + 1]))
                    i += 2
                else:
                    nxt.append(level[i])
                    i += 1
            level = nxt
        else:
            level = [(level[0], level[1])] + level[2:]
    return level[0]


# ----------------------------------------------------------------------------
# Structured labels
# ----------------------------------------------------------------------------
# Leaf:  ("leaf", n, l)
# Sym:   ("sym", n, l, k, Lambda, copy)
# Node:  ("node", left, right, L)

def total_L(label):
    kind = label[0]
    if kind == "leaf":
        return label[2]
    if kind == "sym":
        return label[4]
    return label[3]


def n_sequence(label):
    kind = label[0]
    if kind == "leaf":
        return (label[1],)
    if kind == "sym":
        return (label[1],) * label[3]
    return n_sequence(label[1]) + n_sequence(label[2])


def l_sequence(label):
    kind = label[0]
    if kind == "leaf":
        return (label[2],)
    if kind == "sym":
        return (label[2],) * label[3]
    return l_sequence(label[1]) + l_sequence(label[2])


def internal_Ls_postorder(label):
    kind = label[0]
    if kind == "leaf":
        return ()
    if kind == "sym":
        return (label[4],)
    return internal_Ls_postorder(label[1]) + internal_Ls_postorder(label[2]) + (label[3],)


def compact_basis_key(label):
    kind = label[0]
    if kind == "leaf":
        return ()
    if kind == "sym":
        return ("sym", label[4], label[5])
    left, right = compact_basis_key(label[1]), compact_basis_key(label[2])
    if not left and not right:
        return ()
    return ("node", left, right)


def compact_label(label, tree_type="balanced"):
    """Reference ``basis/labels.py:18-24, 49-56, 114-120``."""
    key = compact_basis_key(label)
    head = (n_sequence(label), l_sequence(label), internal_Ls_postorder(label))
    if not key and tree_type == "balanced":
        return head
    if not key:
        return head + (tree_type,)
    return head + (tree_type, key)


def block_specs(label):
    """Per-block spec dicts in tree order (reference ``factorized_dag.py:18-45``)."""
    kind = label[0]
    if kind == "leaf":
        return ({"kind": "leaf", "n": label[1], "l": label[2], "k_b": 1, "Lambda": label[2],
                 "multiplicity_index": 0, "basis_key": ()},)
    if kind == "sym":
        return ({"kind": "sym", "n": label[1], "l": label[2], "k_b": label[3], "Lambda": label[4],
                 "multiplicity_index": label[5], "basis_key": ("sym", label[4], label[5])},)
    return block_specs(label[1]) + block_specs(label[2])


def path_key(label):
    """Angular-only key (reference ``factorized_dag.py:48-60``)."""
    kind = label[0]
    if kind == "leaf":
        return ("leaf", label[2])
    if kind == "sym":
        return ("sym", label[4])
    return ("node", path_key(label[1]), path_key(label[2]), label[3])


def _block_label_map(n, l, k):
    if k == 1:
        return {l: [("leaf", n, l)]}
    out = {}
    for Lam, mult in symmetric_power_irrep_multiplicities(l, k).items():
        out[Lam] = [("sym", n, l, k, Lam, c) for c in range(mult)]
    return out


def _dedupe_sorted(labels, tree_type):
    uniq = {}
    for lab in labels:
        uniq.setdefault(compact_label(lab, tree_type), lab)
    return [uniq[key] for key in sorted(uniq)]


def _combine(left_map, right_map, tree_type):
    out = {}
    for Jl, left_labels in left_map.items():
        for Jr, right_labels in right_map.items():
            for a in left_labels:
                for b in right_labels:
                    for L in range(abs(Jl - Jr), Jl + Jr + 1):
                        out.setdefault(L, []).append(("node", a, b, L))
    return {L: _dedupe_sorted(labs, tree_type) for L, labs in out.items()}


@lru_cache(maxsize=256)
def structured_labels_by_L(nin, lin, tree_type="balanced"):
    """``{L: [structured label, ...]}`` in the reference's canonical order.

    Reference: ``YoungSymmetrizerBackend._labels_on_block_shape`` /
    ``_ensure_lightweight_structured_labels`` (``young_exact.py:441-457, 597-612``).
    """
    tree_type = validate_tree_type(tree_type)
    n_c, l_c = canonicalize_leaf_quantum_numbers(nin, lin)
    blocks = young_blocks(n_c, l_c)
    maps = [_block_label_map(n, l, k) for n, l, k in blocks]
    shape = block_tree_shape(len(blocks), tree_type)

    def walk(shape_node, idx):
        if shape_node is None:
            return maps[idx], idx + 1
        left, idx = walk(shape_node[0], idx)
        right, idx = walk(shape_node[1], idx)
        return _combine(left, right, tree_type), idx

    full, used = walk(shape, 0)
    if used != len(blocks):
        raise RuntimeError("block tree did not consume every block")
    return {int(L): tuple(_dedupe_sorted(labs, tree_type)) for L, labs in sorted(full.items()) if labs}


def compact_labels_by_L(nin, lin, tree_type="balanced"):
    tree_type = validate_tree_type(tree_type)
    return {L: [compact_label(lab, tree_type) for lab in labs]
            for L, labs in structured_labels_by_L(tuple(nin), tuple(lin), tree_type).items()}


def _freeze_key(value):
    if isinstance(value, Mapping):
        raise TypeError("Compact-label basis keys cannot contain mappings.")
    if isinstance(value, (tuple, list)):
        return tuple(_freeze_key(v) for v in value)
    return value


def _label_int(value, name):
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError(f"{name} values must be integers, not {value!r}.")
    return int(value)


def _key_from_json(value):
    """A basis key read back from its JSON list form (``sym`` / ``sym_numeric`` / ``node`` tags)."""
    if not isinstance(value, (tuple, list)):
        raise TypeError("Compact-label basis_key must be a recursive sequence.")
    key = tuple(value)
    if not key:
        return ()
    if not isinstance(key[0], str):
        raise TypeError("Compact-label basis-key tags must be strings.")
    if key[0] in {"sym", "sym_numeric"}:
        if len(key) != 3:
            raise ValueError(f"Compact-label {key[0]} basis keys require tag, L, and copy index.")
        L, copy = _label_int(key[1], "basis_key.L"), _label_int(key[2], "basis_key.copy_index")
        if L < 0 or copy < 0:
            raise ValueError("Compact-label symmetric basis-key indices must be non-negative.")
        return (key[0], L, copy)
    if key[0] == "node":
        if len(key) != 3:
            raise ValueError("Compact-label node basis keys require tag, left key, and right key.")
        return ("node", _key_from_json(key[1]), _key_from_json(key[2]))
    raise ValueError(f"Unknown compact-label basis-key tag {key[0]!r}.")


def _key_to_json(value):
    if isinstance(value, tuple):
        return [_key_to_json(v) for v in value]
    return value


@dataclass(frozen=True)
class CompactLabel:
    """One exact ACE label as ``count`` reports it (reference ``ye3t/core/labels.py:65-211``).

    ``n_tuple`` / ``l_tuple`` are the canonical leaf order, ``internal_Ls`` the
    post-order internal couplings ending in ``L_R``, ``basis_key`` the nested
    symmetric-block copy selectors (empty when every block takes copy 0).
    """

    n_tuple: tuple
    l_tuple: tuple
    internal_Ls: tuple
    tree_type: str = "balanced"
    basis_key: tuple = ()

    def __post_init__(self):
        object.__setattr__(self, "n_tuple", tuple(_label_int(v, "n_tuple") for v in self.n_tuple))
        object.__setattr__(self, "l_tuple", tuple(_label_int(v, "l_tuple") for v in self.l_tuple))
        object.__setattr__(self, "internal_Ls", tuple(_label_int(v, "internal_Ls") for v in self.internal_Ls))
        if not isinstance(self.tree_type, str):
            raise TypeError("Compact-label tree_type must be a string.")
        object.__setattr__(self, "tree_type", validate_tree_type(self.tree_type))
        object.__setattr__(self, "basis_key", _freeze_key(self.basis_key))
        if not self.n_tuple or len(self.n_tuple) != len(self.l_tuple):
            raise ValueError("Compact labels require equally sized non-empty n_tuple and l_tuple.")
        if any(v < 0 for v in self.n_tuple):
            raise ValueError("Compact-label radial indices must be non-negative.")
        if any(v < 0 for v in self.l_tuple + self.internal_Ls):
            raise ValueError("Compact-label angular momenta must be non-negative.")

    @property
    def rank(self):
        return len(self.l_tuple)

    @property
    def L_R(self):
        return self.internal_Ls[-1] if self.internal_Ls else self.l_tuple[0]

    def angular_key(self):
        ls = ",".join(str(x) for x in self.l_tuple)
        Ls = ",".join(str(x) for x in self.internal_Ls)
        key = "" if not self.basis_key else f"|{self.basis_key!r}"
        return f"{ls}_{Ls}{key}" if self.tree_type == "balanced" else f"{self.tree_type}:{ls}_{Ls}{key}"

    def full_key(self):
        return ",".join(str(x) for x in self.n_tuple) + "|" + self.angular_key()

    def compact_label(self):
        """The 3-, 4- or 5-part tuple form (``basis/labels.py:49-56``)."""
        head = (self.n_tuple, self.l_tuple, self.internal_Ls)
        if not self.basis_key:
            return head if self.tree_type == "balanced" else head + (self.tree_type,)
        return head + (self.tree_type, self.basis_key)

    def payload(self):
        """The five-field tuple a report hashes (``couplings/__init__.py:428-440``)."""
        return (self.n_tuple, self.l_tuple, self.internal_Ls, self.tree_type, self.basis_key)

    def to_dict(self):
        return {"n_tuple": list(self.n_tuple), "l_tuple": list(self.l_tuple), "internal_Ls": list(self.internal_Ls),
                "L_R": int(self.L_R), "tree_type": str(self.tree_type), "basis_key": _key_to_json(self.basis_key)}

    @classmethod
    def from_dict(cls, payload):
        if not isinstance(payload, Mapping):
            raise TypeError("Compact-label payload must be a mapping.")
        unknown = set(payload) - {"n_tuple", "l_tuple", "internal_Ls", "L_R", "tree_type", "basis_key"}
        if unknown:
            raise ValueError("Compact-label payload has unknown fields: " + ", ".join(sorted(map(str, unknown))))
        missing = {"n_tuple", "l_tuple", "internal_Ls"} - set(payload)
        if missing:
            raise ValueError("Compact-label payload is missing fields: " + ", ".join(sorted(missing)))
        label = cls(tuple(payload["n_tuple"]), tuple(payload["l_tuple"]), tuple(payload["internal_Ls"]),
                    payload.get("tree_type", "balanced"), _key_from_json(payload.get("basis_key", ())))
        if "L_R" in payload and _label_int(payload["L_R"], "L_R") != int(label.L_R):
            raise ValueError("Compact-label L_R does not match its coupling label.")
        return label

    @classmethod
    def from_tuple(cls, value):
        value = tuple(value)
        if len(value) == 3:
            return cls(tuple(value[0]), tuple(value[1]), tuple(value[2]))
        if len(value) == 4:
            if isinstance(value[3], str):
                return cls(tuple(value[0]), tuple(value[1]), tuple(value[2]), value[3])
            return cls(tuple(value[0]), tuple(value[1]), tuple(value[2]), basis_key=_freeze_key(value[3]))
        if len(value) == 5:
            return cls(tuple(value[0]), tuple(value[1]), tuple(value[2]), str(value[3]), _freeze_key(value[4]))
        raise ValueError("Compact label must have 3, 4, or 5 parts: "
                         "(n_tuple, l_tuple, internal_Ls[, tree_type][, basis_key])")


def normalize_compact_label(value):
    """A :class:`CompactLabel` from a label, its dict form or its tuple form."""
    if isinstance(value, CompactLabel):
        return value
    if isinstance(value, Mapping):
        return CompactLabel.from_dict(value)
    return CompactLabel.from_tuple(value)


def counts_by_L(nin, lin):
    """Closed-form ``alpha_L`` (reference ``multiplicity.py:111-116``)."""
    n_c, l_c = canonicalize_leaf_quantum_numbers(nin, lin)
    current = {0: 1}
    for _, l, k in young_blocks(n_c, l_c):
        current = couple_multiplicities(current, symmetric_power_irrep_multiplicities(l, k))
    return current
