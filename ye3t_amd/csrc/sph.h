// Real spherical harmonics for gfx950, in registers.
//
// Convention (the reference's real SH table, ye3t_runtime_core.cpp:224-286):
//   Y_{l,0}  = N_l0 Q_l^0(z)
//   Y_{l,+m} = sqrt2 N_lm Q_l^m(z) Re (x+iy)^m
//   Y_{l,-m} = -sqrt2 N_lm Q_l^m(z) Im (x+iy)^m
// with Q_l^m = d^m P_l / dz^m on the unit sphere.  The reference evaluates
// Q_l^m from Legendre coefficient polynomials; here Q_l^m comes from the
// three-term recurrence (l-m) Q_l^m = (2l-1) z Q_{l-1}^m - (l+m-1) Q_{l-2}^m,
// Q_m^m = (2m-1)!!, which is cheaper and better conditioned.
#pragma once

#include "common.h"

namespace ye3t {

// Writes the (lmax+1)^2 values of one unit vector to out[stride * k],
// computing in `Real` and storing as `Out`.
template <typename Real, typename Out = Real>
__device__ inline void real_sph_row(Real x, Real y, Real z, int lmax, const NormTable& nt, Out* out,
                                    int stride) {
  const Real sqrt2 = Real(1.4142135623730950488016887242096981);
  Real cr = Real(1), ci = Real(0);  // (x + i y)^m
  Real qmm = Real(1);               // Q_m^m
  for (int m = 0; m <= lmax; ++m) {
    if (m > 0) {
      qmm *= Real(2 * m - 1);
      const Real nr = cr * x - ci * y;
      const Real ni = cr * y + ci * x;
      cr = nr;
      ci = ni;
    }
    Real q2 = Real(0), q1 = Real(0);
    for (int l = m; l <= lmax; ++l) {
      Real q;
      if (l == m) {
        q = qmm;
      } else if (l == m + 1) {
        q = Real(2 * m + 1) * z * qmm;
      } else {
        q = (Real(2 * l - 1) * z * q1 - Real(l + m - 1) * q2) * Real(nt.inv[l - m]);
      }
      q2 = q1;
      q1 = q;
      const Real n = Real(nt.v[l * (kMaxL + 1) + m]);
      const int base = l * l + l;
      if (m == 0) {
        out[stride * base] = Out(n * q);
      } else {
        const Real s = sqrt2 * n * q;
        out[stride * (base + m)] = Out(s * cr);
        out[stride * (base - m)] = Out(-s * ci);
      }
    }
  }
}

// The same row for a compile-time LMAX, both loops unrolled so that `out`
// may be a register array (every index a constant).
template <int LMAX, typename Real, typename Out = Real>
__device__ inline void real_sph_row_fixed(Real x, Real y, Real z, const NormTable& nt, Out* out) {
  const Real sqrt2 = Real(1.4142135623730950488016887242096981);
  Real cr = Real(1), ci = Real(0);  // (x + i y)^m
  Real qmm = Real(1);               // Q_m^m
#pragma unroll
  for (int m = 0; m <= LMAX; ++m) {
    if (m > 0) {
      qmm *= Real(2 * m - 1);
      const Real nr = cr * x - ci * y;
      const Real ni = cr * y + ci * x;
      cr = nr;
      ci = ni;
    }
    Real q2 = Real(0), q1 = Real(0);
#pragma unroll
    for (int l = m; l <= LMAX; ++l) {
      Real q;
      if (l == m) {
        q = qmm;
      } else if (l == m + 1) {
        q = Real(2 * m + 1) * z * qmm;
      } else {
        q = (Real(2 * l - 1) * z * q1 - Real(l + m - 1) * q2) * Real(nt.inv[l - m]);
      }
      q2 = q1;
      q1 = q;
      const Real n = Real(nt.v[l * (kMaxL + 1) + m]);
      const int base = l * l + l;
      if (m == 0) {
        out[base] = Out(n * q);
      } else {
        const Real s = sqrt2 * n * q;
        out[base + m] = Out(s * cr);
        out[base - m] = Out(-s * ci);
      }
    }
  }
}

}  // namespace ye3t
