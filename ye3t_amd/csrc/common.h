// Shared helpers of the ye3t_hip library (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "ye3t_hip.h"

namespace ye3t {

int set_error(int code, const char* fmt, ...);
void clear_error();
// records the kernel an ace_density_forward call launched (static string)
void set_density_kernel(const char* name);

#define YE3T_CHECK_HIP(expr)                                                              \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess) {                                                               \
      return ::ye3t::set_error(YE3T_ELAUNCH, "%s failed: %s", #expr, hipGetErrorString(_e)); \
    }                                                                                     \
  } while (0)

#define YE3T_REQUIRE(cond, ...)                                  \
  do {                                                           \
    if (!(cond)) return ::ye3t::set_error(YE3T_EINVAL, __VA_ARGS__); \
  } while (0)

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(YE3T_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return YE3T_OK;
}

inline hipStream_t as_stream(ye3t_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---- device math, overloaded for float / double ----------------------------
__device__ inline float d_exp(float x) { return expf(x); }
__device__ inline double d_exp(double x) { return exp(x); }
__device__ inline float d_expm1(float x) { return expm1f(x); }
__device__ inline double d_expm1(double x) { return expm1(x); }
__device__ inline float d_cos(float x) { return cosf(x); }
__device__ inline double d_cos(double x) { return cos(x); }
__device__ inline float d_sin(float x) { return sinf(x); }
__device__ inline double d_sin(double x) { return sin(x); }
__device__ inline float d_sqrt(float x) { return sqrtf(x); }
__device__ inline double d_sqrt(double x) { return sqrt(x); }
__device__ inline float d_fma(float a, float b, float c) { return fmaf(a, b, c); }
__device__ inline double d_fma(double a, double b, double c) { return fma(a, b, c); }

template <typename Real>
struct Eps;
template <>
struct Eps<float> {
  static constexpr float value = 1.1920928955078125e-07f;
};
template <>
struct Eps<double> {
  static constexpr double value = 2.220446049250313e-16;
};

// Real-SH normalisation N_lm = sqrt((2l+1)/(4 pi) (l-m)!/(l+m)!) for l <= kMaxL,
// passed by value as a kernel argument (lives in the scalar/constant cache).
constexpr int kMaxL = 12;
struct NormTable {
  double v[(kMaxL + 1) * (kMaxL + 1)];  // N_lm at l*(kMaxL+1)+m
  double inv[2 * kMaxL + 2];            // 1/k, k = 0..2 kMaxL+1 (inv[0] unused)
};
const NormTable& norm_table();

// Radial ChebExpCos values (and d/dr) for n = 0..n_max, same algebra as the
// reference CPU core (ye3t_runtime_core.cpp:321-423) but one Chebyshev pass.
// Value n goes to v[n * vs], its derivative to d[n * ds].
template <typename Real, bool WithDeriv, typename Out = Real>
__device__ inline void cheb_exp_cos_row(Real r, Real rc_in, Real lam, int n_max, Out* v, Out* d, int vs = 1,
                                      int ds = 1) {
  const Real pi = Real(3.141592653589793238462643383279502884);
  const Real rc = rc_in > Eps<Real>::value ? rc_in : Eps<Real>::value;
  const Real s = r / rc;
  if (s > Real(1)) {
    for (int n = 0; n <= n_max; ++n) {
      v[n * vs] = Out(0);
      if (WithDeriv) d[n * ds] = Out(0);
    }
    return;
  }
  // the envelope is evaluated in the output precision (it enters linearly);
  // the warped variable stays in `Real` because T_n amplifies its error by n^2
  const Real c = (sizeof(Out) < sizeof(Real) && !WithDeriv) ? Real(d_cos(float(pi * s))) : d_cos(pi * s);
  const Real sn = WithDeriv ? d_sin(pi * s) : Real(0);
  v[0] = Out(1);
  if (WithDeriv) d[0] = Out(0);
  if (n_max >= 1) {
    v[vs] = Out(Real(0.5) * (Real(1) + c));
    if (WithDeriv) d[ds] = Out(-Real(0.5) * pi * sn / rc);
  }
  if (n_max >= 2) {
    const Real den = d_expm1(lam);
    const Real em1 = d_expm1(-lam * (s - Real(1)));
    const Real x = Real(1) - Real(2) * em1 / den;
    const Real dx = WithDeriv ? Real(2) * lam * d_exp(-lam * (s - Real(1))) / (den * rc) : Real(0);
    const Real env = Real(1) + c;
    const Real denv = -pi * sn / rc;
    Real t0 = Real(1), t1 = x;     // T_{n-2}, T_{n-1}
    Real u0 = Real(1), u1 = Real(2) * x;  // U_{n-2}, U_{n-1} (at the top of iteration n)
    for (int n = 2; n <= n_max; ++n) {
      const Real t2 = Real(2) * x * t1 - t0;
      // derivative of T_n is n U_{n-1}; U_{n-1} is u1 here
      v[n * vs] = Out(Real(0.25) * (Real(1) - t2) * env);
      if (WithDeriv) d[n * ds] = Out(Real(0.25) * (-(Real(n) * u1) * dx * env + (Real(1) - t2) * denv));
      t0 = t1;
      t1 = t2;
      const Real u2 = Real(2) * x * u1 - u0;
      u0 = u1;
      u1 = u2;
    }
  }
}

}  // namespace ye3t
