"""Exact symmetric-power block bases ``Sym^k(V_l) -> V_Lambda`` and monomial tables.

Restates the reference's independent (non-orthogonalised) homogeneous basis
(``ye3t/core/basis/homogeneous.py:182-256, 468-505, 555-594``):

1. occupancy basis of each weight space, in the reference's recursion order;
2. highest-weight vectors = nullspace of ``J_+`` at weight ``Lambda`` in the
   reduced-row-echelon basis (one vector per free column), pivot-normalised
   (first nonzero entry = 1) and ordered by ``(pivot, srepr(entries))``;
3. lowering ``v_{M} = J_- v_{M+1} / sqrt((Lambda+M+1)(Lambda-M))``.

The reference does this in SymPy.  Here it is exact without SymPy: with the
diagonal scaling ``D(alpha)^2 = prod_j alpha_j! * prod_j h_j^(2 alpha_j)``,
``h_{j+1}^2 = h_j^2 (l-m_j)(l+m_j+1)``, the ladder operator factors as
``J_+ = D_{M+1} Q D_M^{-1}`` with an *integer* matrix ``Q``, so every entry of
every basis vector is a single radical ``q * sqrt(r)`` with rational ``q, r``.
The ``srepr`` tie-break is reproduced for that radical form.

Monomial tables follow ``_complex_symmetric_power_monomial_entries``
(``ye3t/couplings/__init__.py:3279-3328``): coefficient of ``prod_m A_m^alpha_m``
is ``float(c) * sqrt(k! / prod alpha!)``.
"""

from fractions import Fraction
from functools import lru_cache
from math import factorial, isqrt, sqrt

import numpy as np

from ye3t_amd.core.basis import symmetric_power_irrep_multiplicities
from ye3t_amd.core.cg import _squarefree_split, parity_phase, real_to_complex_unitary


@lru_cache(maxsize=None)
def occupancy_basis_by_weight(l, k):
    """``{M: (alpha, ...)}`` with ``alpha`` counts over ``m=-l..l`` (``homogeneous.py:182-203``)."""
    l, k = int(l), int(k)
    m_values = tuple(range(-l, l + 1))
    out = {}

    def recurse(slot, remaining, occ, weight):
        if slot == len(m_values) - 1:
            occ.append(remaining)
            out.setdefault(weight + remaining * m_values[slot], []).append(tuple(occ))
            occ.pop()
            return
        for count in range(remaining + 1):
            occ.append(count)
            recurse(slot + 1, remaining - count, occ, weight + count * m_values[slot])
            occ.pop()

    recurse(0, k, [], 0)
    return {M: tuple(items) for M, items in sorted(out.items())}


@lru_cache(maxsize=None)
def _h_squared(l):
    """``h_j^2`` for ``j = 0..2l`` with ``h_0 = 1``, ``h_{j+1}^2 = h_j^2 (l-m_j)(l+m_j+1)``."""
    out = [Fraction(1)]
    for j in range(2 * l):
        m = j - l
        out.append(out[-1] * (l - m) * (l + m + 1))
    return tuple(out)


def _d_squared(l, alpha):
    h2 = _h_squared(l)
    value = Fraction(1)
    for j, a in enumerate(alpha):
        value *= factorial(a) * h2[j] ** a
    return value


@lru_cache(maxsize=None)
def _q_matrix(l, k, M):
    """Integer ``Q`` with ``J_+(M) = D_{M+1} Q D_M^{-1}``; rows weight ``M+1``, cols ``M``."""
    basis = occupancy_basis_by_weight(l, k)
    src = basis.get(M, ())
    dst = basis.get(M + 1, ())
    index = {alpha: i for i, alpha in enumerate(dst)}
    Q = [[0] * len(src) for _ in range(len(dst))]
    for col, alpha in enumerate(src):
        for i in range(2 * l):
            if alpha[i] == 0:
                continue
            new = list(alpha)
            new[i] -= 1
            new[i + 1] += 1
            Q[index[tuple(new)]][col] += alpha[i]
    return Q


def _rref_nullspace(Q, cols):
    """Reduced-row-echelon nullspace basis (SymPy ``Matrix.nullspace`` convention)."""
    rows = [[Fraction(x) for x in row] for row in Q]
    pivots = []
    r = 0
    for c in range(cols):
        pivot_row = next((i for i in range(r, len(rows)) if rows[i][c] != 0), None)
        if pivot_row is None:
            continue
        rows[r], rows[pivot_row] = rows[pivot_row], rows[r]
        inv = 1 / rows[r][c]
        rows[r] = [x * inv for x in rows[r]]
        for i in range(len(rows)):
            if i != r and rows[i][c] != 0:
                f = rows[i][c]
                rows[i] = [a - f * b for a, b in zip(rows[i], rows[r])]
        pivots.append(c)
        r += 1
        if r == len(rows):
            break
    free = [c for c in range(cols) if c not in set(pivots)]
    vectors = []
    for f in free:
        u = [Fraction(0)] * cols
        u[f] = Fraction(1)
        for i, p in enumerate(pivots):
            u[p] = -rows[i][f]
        vectors.append((f, u))
    return vectors


def _radical(q, r):
    """Normalise ``q*sqrt(r)`` to ``(coefficient, squarefree_int)``."""
    if q == 0 or r == 0:
        return Fraction(0), 1
    a, r1 = _squarefree_split(r.numerator)
    b, r2 = _squarefree_split(r.denominator)
    return q * Fraction(a, b * r2), r1 * r2


def _srepr_rational(q):
    if q.denominator == 1:
        return f"Integer({q.numerator})"
    return f"Rational({q.numerator}, {q.denominator})"


def srepr_radical(coefficient, radicand):
    """SymPy ``srepr`` of ``coefficient*sqrt(radicand)`` (radicand squarefree)."""
    if coefficient == 0:
        return "Integer(0)"
    if radicand == 1:
        return _srepr_rational(coefficient)
    root = f"Pow(Integer({radicand}), Rational(1, 2))"
    if coefficient == 1:
        return root
    return f"Mul({_srepr_rational(coefficient)}, {root})"


def _radical_to_float(coefficient, radicand):
    """Correctly rounded ``coefficient*sqrt(radicand)`` (SymPy ``evalf(30)`` then float)."""
    if coefficient == 0:
        return 0.0
    value2 = coefficient * coefficient * radicand
    scale = 1 << 128
    root = isqrt((value2.numerator * scale * scale) // value2.denominator)
    out = float(Fraction(root, scale))
    return out if coefficient > 0 else -out


@lru_cache(maxsize=None)
def highest_weight_vectors(l, k, Lam):
    """Independent highest-weight basis at weight ``Lambda`` in the reference's order.

    Returns ``(basis, [(u, f), ...])``: each vector is ``v = D u / D[f]`` with
    rational ``u`` (``u[f] = 1``); entries of ``v`` are single radicals.
    """
    l, k, Lam = int(l), int(k), int(Lam)
    basis = occupancy_basis_by_weight(l, k)
    weight_basis = basis.get(Lam, ())
    if not weight_basis:
        return weight_basis, []
    d2 = [_d_squared(l, a) for a in weight_basis]
    if not basis.get(Lam + 1):
        kernel = []
        for f in range(len(weight_basis)):
            u = [Fraction(0)] * len(weight_basis)
            u[f] = Fraction(1)
            kernel.append((f, u))
    else:
        kernel = _rref_nullspace(_q_matrix(l, k, Lam), len(weight_basis))
    keyed = []
    for f, u in kernel:
        entries = [_radical(u[j], d2[j] / d2[f]) for j in range(len(u))]
        pivot = next(j for j, (c, _) in enumerate(entries) if c != 0)
        pc, pr = entries[pivot]
        normalized = [_radical(c / pc, Fraction(r, pr)) if c != 0 else (Fraction(0), 1) for c, r in entries]
        key = (pivot, tuple(srepr_radical(c, r) for c, r in normalized))
        # pivot-normalised vector expressed again as D * u' / D[f'] with u' rational
        scale_u = u[pivot]
        u_norm = [x / scale_u for x in u]
        keyed.append((key, (u_norm, pivot)))
    keyed.sort(key=lambda item: item[0])
    out, seen = [], set()
    for key, vec in keyed:
        if key in seen:
            continue
        seen.add(key)
        out.append(vec)
    return weight_basis, out


@lru_cache(maxsize=None)
def occupancy_expansion(l, k, Lam, copy):
    """``{M: {alpha: (coefficient, radicand)}}`` of one basis state (exact).

    Each state is pivot-normalised at weight ``Lambda`` and lowered with
    ``J_- / sqrt((Lambda+M+1)(Lambda-M))`` (reference ``homogeneous.py:495-505``).
    """
    l, k, Lam, copy = int(l), int(k), int(Lam), int(copy)
    weight_basis, vectors = highest_weight_vectors(l, k, Lam)
    if copy < 0 or copy >= len(vectors):
        raise ValueError(f"Sym^{k}(V_{l}) -> V_{Lam} has no multiplicity index {copy}.")
    u, pivot = vectors[copy]
    basis = occupancy_basis_by_weight(l, k)
    # v_M[j] = sqrt(D2_M[j]) * u_M[j] * kappa_M ; kappa_Lam = 1/sqrt(D2_Lam[pivot])
    d2_top = [_d_squared(l, a) for a in weight_basis]
    kappa2 = 1 / d2_top[pivot]
    expansion = {}

    def record(M, u_vec, d2_vec, kappa_sq):
        block = {}
        for alpha, uj, dj in zip(basis[M], u_vec, d2_vec):
            if uj != 0:
                block[alpha] = _radical(uj, dj * kappa_sq)
        expansion[M] = block

    record(Lam, u, d2_top, kappa2)
    u_cur, d2_cur = u, d2_top
    for M in range(Lam - 1, -Lam - 1, -1):
        # J_-(M+1) = J_+(M)^T = D_M^{-1} Q^T D_{M+1}:  u_M = D_M^{-2} Q^T D_{M+1}^2 u_{M+1}
        Q = _q_matrix(l, k, M)
        src = basis[M]
        d2_new = [_d_squared(l, a) for a in src]
        weighted = [d * x for d, x in zip(d2_cur, u_cur)]
        u_new = []
        for col in range(len(src)):
            acc = Fraction(0)
            for row in range(len(weighted)):
                q = Q[row][col]
                if q:
                    acc += q * weighted[row]
            u_new.append(acc / d2_new[col])
        kappa2 = kappa2 / ((Lam + M + 1) * (Lam - M))
        record(M, u_new, d2_new, kappa2)
        u_cur, d2_cur = u_new, d2_new
    return {M: expansion[M] for M in sorted(expansion)}


@lru_cache(maxsize=None)
def complex_monomial_entries(power, input_L, output_L, copy):
    """``(output_index, exponents, value)`` rows, reference ordering and rounding.

    Mirrors ``_complex_symmetric_power_monomial_entries``
    (``ye3t/couplings/__init__.py:3279-3328``): ``M`` ascending, occupancies in
    tuple order, ``value = float(c) * sqrt(k!/prod alpha!)``, kept if ``|value| > 1e-12``.
    """
    expansion = occupancy_expansion(int(input_L), int(power), int(output_L), int(copy))
    fk = factorial(int(power))
    rows = []
    for M, block in expansion.items():
        for alpha in sorted(block):
            c, r = block[alpha]
            den = 1
            for a in alpha:
                den *= factorial(a)
            value = _radical_to_float(c, r) * sqrt(float(fk) / float(den))
            if abs(value) > 1.0e-12:
                rows.append((int(M) + int(output_L), tuple(int(a) for a in alpha), float(value)))
    return tuple(rows)


def _poly_mul(p, q):
    out = {}
    for ea, ca in p.items():
        for eb, cb in q.items():
            e = tuple(x + y for x, y in zip(ea, eb))
            out[e] = out.get(e, 0j) + ca * cb
    return out


@lru_cache(maxsize=None)
def real_monomial_entries(power, input_L, output_L, copy, tol=1e-13):
    """Sym block in this package's real SH basis: ``(out_real, exponents, value)``.

    ``S^r = (-i)^{(k l + Lambda) mod 2} * W_Lambda^dagger S^c(W_l A^r)`` with the
    complex-basis monomials of :func:`complex_monomial_entries`.  The real-form
    lowering follows the reference's ``symmetric_power_coefficient_entries``
    (``ye3t/couplings/__init__.py:3481-3540``) with the parity phase applied so
    the coefficients are real.
    """
    k, l, Lam = int(power), int(input_L), int(output_L)
    W_in = real_to_complex_unitary(l)
    W_out = real_to_complex_unitary(Lam)
    width = 2 * l + 1
    # powers of A^c_m as polynomials in the real components
    linear = []
    for m in range(width):
        poly = {}
        for a in range(width):
            if abs(W_in[m, a]) > 0:
                e = [0] * width
                e[a] = 1
                poly[tuple(e)] = complex(W_in[m, a])
        linear.append(poly)
    power_cache = {}

    def monomial(alpha):
        poly = {tuple([0] * width): 1 + 0j}
        for m, a in enumerate(alpha):
            for _ in range(a):
                poly = _poly_mul(poly, linear[m])
        return poly

    complex_rows = complex_monomial_entries(k, l, Lam, copy)
    per_output = [dict() for _ in range(2 * Lam + 1)]
    for out_c, alpha, value in complex_rows:
        key = alpha
        if key not in power_cache:
            power_cache[key] = monomial(alpha)
        for nu in range(2 * Lam + 1):
            factor = np.conj(W_out[out_c, nu])
            if abs(factor) == 0:
                continue
            target = per_output[nu]
            for e, c in power_cache[key].items():
                target[e] = target.get(e, 0j) + value * factor * c
    phase = parity_phase((k * l + Lam) % 2)
    rows = []
    for nu in range(2 * Lam + 1):
        for e in sorted(per_output[nu]):
            v = per_output[nu][e] * phase
            if abs(v.imag) > 1e-10 * max(1.0, abs(v.real)):
                raise ArithmeticError("real-basis symmetric block has a complex coefficient")
            if abs(v.real) > tol:
                rows.append((nu, e, float(v.real)))
    return tuple(rows)


def block_copies(l, k, Lam):
    return int(symmetric_power_irrep_multiplicities(int(l), int(k)).get(int(Lam), 0))
