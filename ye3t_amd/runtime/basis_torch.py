"""Differentiable Torch expressions of the radial and harmonic bases.

The HIP kernels give the radial table, the harmonic table and their first
derivatives; these expressions exist only for second derivatives through the
``ye3t_runtime`` operators (a backward differentiated again), the role the
reference's Torch expressions play for it (``execution_plan.py:2534-2935``).
They run on the tensors' own device and follow the same conventions:

* ChebExpCos: ``R_0 = 1``, ``R_1 = (1 + cos(pi s)) / 2``,
  ``R_n = (1 - T_n(x)) (1 + cos(pi s)) / 4`` with ``s = r / rc`` and
  ``x = 1 - 2 expm1(-lambda (s - 1)) / expm1(lambda)``, zero for ``s > 1``
  (``ye3t_runtime_core.cpp:321-423``);
* real harmonics of the unit vector ``u = v / max(|v|, eps)``:
  ``R_l0 = N_l0 P_l(z)``, ``R_lm = sqrt2 N_lm P_l^(m)(z) Re (x + iy)^m`` and
  ``R_l,-m = -sqrt2 N_lm P_l^(m)(z) Im (x + iy)^m`` for ``m > 0``, with
  ``P_l^(m)`` the m-th derivative of the Legendre polynomial and
  ``N_lm = sqrt((2l + 1) / (4 pi) (l - m)! / (l + m)!)`` (Condon-Shortley
  convention, DLMF 14.30), packed ``l^2 + l + m``.
"""

import math
from functools import lru_cache


@lru_cache(maxsize=None)
def _legendre_derivative(l, m):
    """Ascending coefficients of d^m/dz^m P_l(z) (Bonnet's recurrence)."""
    p0, p1 = [1.0], [0.0, 1.0]
    if l == 0:
        poly = p0
    else:
        for n in range(1, l):
            nxt = [0.0] * (n + 2)
            for k, c in enumerate(p1):
                nxt[k + 1] += (2 * n + 1) / (n + 1) * c
            for k, c in enumerate(p0):
                nxt[k] -= n / (n + 1) * c
            p0, p1 = p1, nxt
        poly = p1
    for _ in range(m):
        poly = [k * poly[k] for k in range(1, len(poly))] or [0.0]
    return tuple(poly)


def _horner(coeffs, z):
    out = z.new_zeros(z.shape) + coeffs[-1]
    for c in reversed(coeffs[:-1]):
        out = out * z + c
    return out


def real_harmonics(edge_vectors, l_max, epsilon=1.0e-12):
    """``[E, (l_max + 1)^2]`` real harmonics, differentiable in ``edge_vectors``."""
    import torch

    r = torch.linalg.norm(edge_vectors, dim=-1, keepdim=True)
    u = edge_vectors / torch.clamp(r, min=float(epsilon))
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    cols = []
    for l in range(int(l_max) + 1):
        row = [None] * (2 * l + 1)
        row[l] = math.sqrt((2 * l + 1) / (4 * math.pi)) * _horner(_legendre_derivative(l, 0), z)
        re, im = torch.ones_like(x), torch.zeros_like(x)
        for m in range(1, l + 1):
            re, im = re * x - im * y, re * y + im * x  # (x + iy)^m
            norm = math.sqrt(2.0 * (2 * l + 1) / (4 * math.pi) * math.factorial(l - m) / math.factorial(l + m))
            d = _horner(_legendre_derivative(l, m), z)
            row[l + m] = norm * d * re
            row[l - m] = -norm * d * im
        cols.extend(row)
    return torch.stack(cols, dim=1)


def cheb_exp_cos_radial(radii, cutoffs, lambdas, max_index):
    """``[..., max_index + 1]`` radial functions, differentiable in ``radii``."""
    import torch

    eps = torch.finfo(radii.dtype).eps
    s = radii / torch.clamp(cutoffs, min=eps)
    env = 1.0 + torch.cos(math.pi * s)
    cols = [torch.ones_like(radii)]
    if max_index >= 1:
        cols.append(0.5 * env)
    if max_index >= 2:
        x = 1.0 - 2.0 * torch.expm1(-lambdas * (s - 1.0)) / torch.expm1(lambdas)
        t0, t1 = torch.ones_like(x), x
        for _ in range(2, int(max_index) + 1):
            t0, t1 = t1, 2.0 * x * t1 - t0
            cols.append(0.25 * (1.0 - t1) * env)
    out = torch.stack(cols, dim=-1)
    return torch.where((s <= 1.0).unsqueeze(-1), out, torch.zeros_like(out))
