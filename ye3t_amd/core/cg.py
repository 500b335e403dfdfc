"""Clebsch--Gordan coefficients (Condon--Shortley) and real-basis lowering.

The complex CG values are computed exactly (rational arithmetic, Racah's
formula) and converted to float the same way the reference converts its exact
radicals: ``float(rational_coefficient) * float(squarefree_radicand) ** 0.5``
(reference: ``ye3t/core/cg.py:120-160`` builds ``rational(total) *
sqrt(prefactor)``; ``ye3t/exact_scalars.py:60-84,162-166`` normalises the
radicand and evaluates the float).  Reproducing that conversion keeps the
factorized schedule coefficients bit-identical to the reference's Python
constructor path (``ye3t/core/factorized_dag.py:63-70``).

The real-basis coupling tensors (``real_cg_entries``) use this package's
real spherical-harmonic convention, i.e. the one produced by the reference's
real SH table (``ye3t_runtime_core.cpp:224-286``): cos-type components at
``+m``, sin-type at ``-m`` with ``Y_{l,-m} = -sqrt(2) N P^{(m)} Im(x+iy)^m``.
"""

from fractions import Fraction
from functools import lru_cache
from math import factorial

import numpy as np


@lru_cache(maxsize=4096)
def _squarefree_split(value):
    """Return ``(s, r)`` with ``value = s*s*r`` and ``r`` squarefree."""
    value = int(value)
    if value in (0, 1):
        return 1, value
    square, rest, factor = 1, value, 2
    while factor * factor <= rest:
        fsq = factor * factor
        while rest % fsq == 0:
            square *= factor
            rest //= fsq
        factor += 1 if factor == 2 else 2
    return square, rest


def _radical_float(coefficient, radicand):
    """float(coefficient * sqrt(radicand)) the way the reference evaluates it.

    ``sqrt(p/q)`` is normalised to ``a/(b*r2) * sqrt(r1*r2)`` with ``p=a^2 r1``
    and ``q=b^2 r2`` (reference ``exact_scalars.py:64-84``).
    """
    coefficient = Fraction(coefficient)
    radicand = Fraction(radicand)
    if coefficient == 0 or radicand == 0:
        return 0.0
    a, r1 = _squarefree_split(radicand.numerator)
    b, r2 = _squarefree_split(radicand.denominator)
    scale = Fraction(a, b * r2)
    return float(coefficient * scale) * float(r1 * r2) ** 0.5


@lru_cache(maxsize=None)
def cg_exact(j1, m1, j2, m2, j3, m3):
    """Exact integer-spin CG as ``(rational, radicand)`` with value ``q*sqrt(r)``.

    Racah's closed form; reference ``ye3t/core/cg.py:100-160`` (integer branch)
    and ``factorized_runtime.cpp:86-114`` (same formula in log-factorials).
    """
    if m1 + m2 != m3 or abs(m1) > j1 or abs(m2) > j2 or abs(m3) > j3:
        return Fraction(0), Fraction(0)
    if j3 < abs(j1 - j2) or j3 > j1 + j2:
        return Fraction(0), Fraction(0)
    f = factorial
    prefactor = Fraction(
        (2 * j3 + 1) * f(j1 + j2 - j3) * f(j1 - j2 + j3) * f(-j1 + j2 + j3)
        * f(j1 + m1) * f(j1 - m1) * f(j2 + m2) * f(j2 - m2) * f(j3 + m3) * f(j3 - m3),
        f(j1 + j2 + j3 + 1),
    )
    z_min = max(0, j2 - j3 - m1, j1 - j3 + m2)
    z_max = min(j1 + j2 - j3, j1 - m1, j2 + m2)
    total = Fraction(0)
    for z in range(z_min, z_max + 1):
        den = (f(z) * f(j1 + j2 - j3 - z) * f(j1 - m1 - z) * f(j2 + m2 - z)
               * f(j3 - j2 + m1 + z) * f(j3 - j1 - m2 + z))
        total += Fraction(-1 if z % 2 else 1, den)
    if total == 0:
        return Fraction(0), Fraction(0)
    return total, prefactor


@lru_cache(maxsize=None)
def cg_float(j1, m1, j2, m2, j3, m3):
    q, r = cg_exact(int(j1), int(m1), int(j2), int(m2), int(j3), int(m3))
    return _radical_float(q, r)


@lru_cache(maxsize=None)
def cg_matrix(left_L, right_L, output_L):
    """``[2l1+1, 2l2+1]`` matrix of ``<l1 m1 l2 m2 | L m1+m2>`` (zeros elsewhere).

    Mirrors ``cg_matrix_for_node`` (reference ``ye3t/core/factorized_dag.py:63-70``).
    """
    l1, l2, L = int(left_L), int(right_L), int(output_L)
    out = np.zeros((2 * l1 + 1, 2 * l2 + 1), dtype=np.float64)
    if not (abs(l1 - l2) <= L <= l1 + l2):
        return out
    for m1 in range(-l1, l1 + 1):
        for m2 in range(-l2, l2 + 1):
            if abs(m1 + m2) > L:
                continue
            out[m1 + l1, m2 + l2] = cg_float(l1, m1, l2, m2, L, m1 + m2)
    out.setflags(write=False)
    return out


@lru_cache(maxsize=None)
def real_to_complex_unitary(L):
    """``W`` with ``Y^c_{l,m} = sum_a W[m+l, a] Y^r_{l,a}`` (complex CS from real).

    For ``m>0``: ``Y^c_{+m} = (-1)^m (Y^r_{+m} - i Y^r_{-m}) / sqrt 2`` and
    ``Y^c_{-m} = (Y^r_{+m} + i Y^r_{-m}) / sqrt 2``; ``Y^c_0 = Y^r_0``.

    This is the ordering of the real spherical-harmonic tables (cosine-type
    ``Re[(x+iy)^m]`` at index ``l+m``, ``ye3t_runtime_core.cpp:226-290`` and
    ``runtime/execution_plan.py:6919-6962``), so a density built from those
    tables is a real multiplet in this basis.  The reference's tesseral map
    (``core/tesseral.py:13-24, 124-140``) stores the cosine type at ``l-m``
    instead: its ``W_tess[m, a] = W[m, 2l-a]`` (see :func:`tesseral_unitary`).
    """
    L = int(L)
    W = np.zeros((2 * L + 1, 2 * L + 1), dtype=np.complex128)
    W[L, L] = 1.0
    r = 2.0 ** -0.5
    for m in range(1, L + 1):
        sign = -1.0 if m % 2 else 1.0
        W[L + m, L + m] = sign * r
        W[L + m, L - m] = -sign * 1j * r
        W[L - m, L + m] = r
        W[L - m, L - m] = 1j * r
    W.setflags(write=False)
    return W


@lru_cache(maxsize=None)
def tesseral_unitary(L):
    """The reference's tesseral-to-Condon--Shortley map (``core/tesseral.py:124-140``).

    ``c_{-m} = (t_{l-m} + i t_{l+m}) / sqrt 2``, ``c_{+m} = (-1)^m (t_{l-m} - i t_{l+m}) / sqrt 2``,
    ``c_0 = t_l`` -- the formula the reference's own test spells out
    (``tests/test_numeric_structured_expansion.py:503-520``).  It is
    :func:`real_to_complex_unitary` with the real index reversed.
    """
    L = int(L)
    W = np.ascontiguousarray(real_to_complex_unitary(L)[:, ::-1])
    W.setflags(write=False)
    return W


def parity_phase(odd):
    """Phase that makes an odd-parity real-basis coupling real: ``(-i)^odd``."""
    return (-1j) if (int(odd) % 2) else 1.0


@lru_cache(maxsize=None)
def real_cg_tensor(left_L, right_L, output_L):
    """Dense real coupling tensor ``T[a, b, c]`` in this package's real basis.

    ``T = (-i)^{(l1+l2-L) mod 2} * sum_{m1,m2} C^{L,M}_{l1 m1 l2 m2}
    W1[m1,a] W2[m2,b] conj(W3[M,c])`` -- the reference's real-form lowering of
    the canonical complex CG (``ye3t/core/tesseral.py:48-82``) expressed with
    the unitary that maps this package's real SH table to Condon--Shortley.
    """
    l1, l2, L = int(left_L), int(right_L), int(output_L)
    C = cg_matrix(l1, l2, L)
    W1, W2, W3 = (real_to_complex_unitary(x) for x in (l1, l2, L))
    T = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * L + 1), dtype=np.complex128)
    for i1 in range(2 * l1 + 1):
        for i2 in range(2 * l2 + 1):
            c = C[i1, i2]
            if c == 0.0:
                continue
            M = (i1 - l1) + (i2 - l2)
            T += c * np.einsum("a,b,c->abc", W1[i1], W2[i2], np.conj(W3[M + L]))
    T *= parity_phase((l1 + l2 - L) % 2)
    if np.max(np.abs(T.imag), initial=0.0) > 1e-12:
        raise ArithmeticError("real-basis CG lowering produced a complex coefficient")
    real = np.ascontiguousarray(T.real)
    real[np.abs(real) < 1e-15] = 0.0
    real.setflags(write=False)
    return real


@lru_cache(maxsize=None)
def tesseral_cg_entries(left_L, right_L, output_L, tol=1e-14):
    """Real CG nonzeros ``(a, b, c, value)`` in the reference's tesseral ordering.

    The table of ``_real_cg_entries_exact`` (``core/tesseral.py:48-82``, via
    ``paired_cg.py:62-72``): the same lowering as :func:`real_cg_tensor` with
    every index reversed (``a -> 2l-a``), sorted by ``(a, b, c)`` and filtered
    at ``|value| > tol``.
    """
    T = real_cg_tensor(left_L, right_L, output_L)[::-1, ::-1, ::-1]
    entries = []
    for a in range(T.shape[0]):
        for b in range(T.shape[1]):
            for c in range(T.shape[2]):
                v = float(T[a, b, c])
                if abs(v) > tol:
                    entries.append((a, b, c, v))
    return tuple(entries)


@lru_cache(maxsize=None)
def real_cg_entries(left_L, right_L, output_L, tol=1e-14):
    """Nonzeros ``(a, b, c, value)`` of :func:`real_cg_tensor`, sorted by (c, a, b)."""
    T = real_cg_tensor(left_L, right_L, output_L)
    entries = []
    for c in range(T.shape[2]):
        for a in range(T.shape[0]):
            for b in range(T.shape[1]):
                v = float(T[a, b, c])
                if abs(v) > tol:
                    entries.append((a, b, c, v))
    return tuple(entries)
