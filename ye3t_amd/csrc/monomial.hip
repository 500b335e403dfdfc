// Symmetric-power monomial contractions (the reference's symmetric_power_*
// ops; CPU core ye3t_runtime_core.cpp:5279-5540, CUDA execution_plan_cuda.cu:
// 5229, 5931-6000): the grouped table S[b, o] = sum_{t in o} v_t prod_c
// x[b, c]^e[t, c], its adjoint, the shared form in which outputs are sparse
// combinations of unique monomials, and that form with sparse monomial supports
// (with its second order).  These are the reference's stand-alone ops;
// the ACE product plan evaluates its symmetric blocks inside its own kernels.
//
// Forward: one thread per (row, output).  Adjoints: one thread per row, which
// owns its row of the input gradient (no atomics, fixed order).  The tables are
// validated by the caller (ye3t_amd.runtime checks them on the host).
#include "common.h"

namespace ye3t {
namespace {

// Complex scalar of the sparse kernels (YE3T_C64 / YE3T_C128: interleaved
// (re, im) pairs, as torch stores complex tensors), with the arithmetic the
// kernels use.  Division is Smith's algorithm (R. L. Smith, "Algorithm 116:
// Complex division", CACM 5(8), 1962): the larger of |c| and |d| scales the
// denominator, so no intermediate overflows for finite operands.
template <typename R>
struct cplx {
  R re, im;
  cplx() = default;
  __device__ constexpr cplx(R r, R i) : re(r), im(i) {}
  __device__ constexpr cplx(int v) : re(R(v)), im(R(0)) {}
  __device__ constexpr cplx(int64_t v) : re(R(v)), im(R(0)) {}
};
template <typename R>
__device__ inline cplx<R> operator+(cplx<R> a, cplx<R> b) { return {a.re + b.re, a.im + b.im}; }
template <typename R>
__device__ inline cplx<R> operator-(cplx<R> a, cplx<R> b) { return {a.re - b.re, a.im - b.im}; }
template <typename R>
__device__ inline cplx<R> operator*(cplx<R> a, cplx<R> b) {
  return {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
}
template <typename R>
__device__ inline cplx<R> operator/(cplx<R> a, cplx<R> b) {
  if (fabs(b.re) >= fabs(b.im)) {
    const R t = b.im / b.re, s = R(1) / (b.re + b.im * t);
    return {(a.re + a.im * t) * s, (a.im - a.re * t) * s};
  }
  const R t = b.re / b.im, s = R(1) / (b.im + b.re * t);
  return {(a.re * t + a.im) * s, (a.im * t - a.re) * s};
}
template <typename R>
__device__ inline cplx<R>& operator+=(cplx<R>& a, cplx<R> b) { return a = a + b; }
template <typename R>
__device__ inline cplx<R>& operator*=(cplx<R>& a, cplx<R> b) { return a = a * b; }
template <typename R>
__device__ inline bool operator==(cplx<R> a, cplx<R> b) { return a.re == b.re && a.im == b.im; }

// conjugate (the identity for real scalars): the adjoints multiply by the
// conjugates of coefficients and derivatives, as the reference's complex
// kernels do (execution_plan_cuda.cu:5757-5955, 6002-6033)
template <typename Real>
__device__ inline Real conjv(Real a) { return a; }
template <typename R>
__device__ inline cplx<R> conjv(cplx<R> a) { return {a.re, -a.im}; }

// integer_power of the reference core (ye3t_runtime_core.cpp:98-110): square and multiply
template <typename Real>
__device__ inline Real ipow(Real b, int64_t e) {
  Real v = Real(1);
  while (e > 0) {
    if (e & 1) v *= b;
    e >>= 1;
    if (e > 0) b *= b;
  }
  return v;
}

inline unsigned grid_for(int64_t work, int threads) {
  int64_t g = (work + threads - 1) / threads;
  if (g < 1) g = 1;
  if (g > (1 << 20)) g = 1 << 20;
  return unsigned(g);
}

template <typename Real>
__global__ __launch_bounds__(256) void sym_monomial_kernel(const Real* __restrict__ x, int64_t batch, int64_t D,
                                                           const int64_t* __restrict__ counts,
                                                           const int64_t* __restrict__ offsets,
                                                           const Real* __restrict__ values, int64_t O,
                                                           Real* __restrict__ out) {
  const int64_t total = batch * O;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int64_t b = idx / O, o = idx - (idx / O) * O;
    const Real* row = x + b * D;
    Real acc = Real(0);
    for (int64_t t = offsets[o]; t < offsets[o + 1]; ++t) {
      Real m = values[t];
      for (int64_t c = 0; c < D; ++c) m *= ipow(row[c], counts[t * D + c]);
      acc += m;
    }
    out[idx] = acc;
  }
}

// The adjoint rule of one monomial m = scale * prod x_c^e_c (ye3t_runtime_core.cpp:
// 5331-5388): zero factors are left out of the product; two or more of them
// give no gradient, one of exponent 1 gives the cofactor, otherwise factor c
// gets e_c m / x_c.  `g` multiplies every contribution.
template <typename Real>
__device__ inline void monomial_gradient(const Real* __restrict__ row, const int64_t* __restrict__ e, int64_t D,
                                         Real scale, Real g, Real* __restrict__ grad) {
  Real mono = scale;
  int zeros = 0;
  int64_t zc = -1;
  for (int64_t c = 0; c < D; ++c) {
    if (e[c] == 0) continue;
    if (row[c] == Real(0)) {
      ++zeros;
      zc = c;
      continue;
    }
    mono *= ipow(row[c], e[c]);
  }
  if (zeros >= 2) return;
  if (zeros == 1) {
    if (e[zc] == 1) grad[zc] += g * mono;
    return;
  }
  for (int64_t c = 0; c < D; ++c) {
    if (e[c] == 0) continue;
    grad[c] += g * (Real(e[c]) * mono / row[c]);
  }
}

template <typename Real>
__global__ __launch_bounds__(256) void sym_monomial_adjoint_kernel(
    const Real* __restrict__ gout, const Real* __restrict__ x, int64_t batch, int64_t D,
    const int64_t* __restrict__ counts, const int64_t* __restrict__ out_index, const Real* __restrict__ values,
    int64_t T, int64_t O, Real* __restrict__ gin) {
  for (int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; b < batch; b += int64_t(gridDim.x) * blockDim.x) {
    const Real* row = x + b * D;
    Real* grad = gin + b * D;
    for (int64_t c = 0; c < D; ++c) grad[c] = Real(0);
    for (int64_t t = 0; t < T; ++t)
      monomial_gradient(row, counts + t * D, D, values[t], gout[b * O + out_index[t]], grad);
  }
}

template <typename Real>
__global__ __launch_bounds__(256) void shared_monomial_kernel(const Real* __restrict__ x, int64_t batch, int64_t D,
                                                              const int64_t* __restrict__ counts,
                                                              const int64_t* __restrict__ offsets,
                                                              const int64_t* __restrict__ terms,
                                                              const Real* __restrict__ values, int64_t O,
                                                              Real* __restrict__ out) {
  const int64_t total = batch * O;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int64_t b = idx / O, o = idx - (idx / O) * O;
    const Real* row = x + b * D;
    Real acc = Real(0);
    for (int64_t k = offsets[o]; k < offsets[o + 1]; ++k) {
      const int64_t* e = counts + terms[k] * D;
      Real m = Real(1);
      for (int64_t c = 0; c < D; ++c) m *= ipow(row[c], e[c]);
      acc += values[k] * m;
    }
    out[idx] = acc;
  }
}

// Shared monomials' adjoint: coefficient k of output o contributes
// g[b, o] v_k d(monomial terms[k]) -- the reference's per-monomial adjoint
// (ye3t_runtime_core.cpp:5442-5540) with its sum over coefficients taken
// term by term.
template <typename Real>
__global__ __launch_bounds__(256) void shared_monomial_adjoint_kernel(
    const Real* __restrict__ gout, const Real* __restrict__ x, int64_t batch, int64_t D,
    const int64_t* __restrict__ counts, const int64_t* __restrict__ offsets, const int64_t* __restrict__ terms,
    const Real* __restrict__ values, int64_t O, Real* __restrict__ gin) {
  for (int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; b < batch; b += int64_t(gridDim.x) * blockDim.x) {
    const Real* row = x + b * D;
    Real* grad = gin + b * D;
    for (int64_t c = 0; c < D; ++c) grad[c] = Real(0);
    for (int64_t o = 0; o < O; ++o) {
      const Real g = gout[b * O + o];
      for (int64_t k = offsets[o]; k < offsets[o + 1]; ++k)
        monomial_gradient(row, counts + terms[k] * D, D, Real(1), g * values[k], grad);
    }
  }
}

// Sparse shared monomials (the reference's symmetric_power_shared_sparse_*
// ops, execution_plan_cuda.cu:5720-5955 and host :11012-11330): monomial t is
// prod_{q in [toff[t], toff[t+1])} x[comp[q]]^ex[q], stored as a support list
// instead of a dense exponent row.  Zero factors add their exponents to a
// "zero degree" that selects the derivative rule.
template <typename Real>
__device__ inline Real sparse_monomial(const Real* __restrict__ row, const int64_t* __restrict__ toff,
                                       const int64_t* __restrict__ comp, const int64_t* __restrict__ ex, int64_t t) {
  Real v = Real(1);
  for (int64_t q = toff[t]; q < toff[t + 1]; ++q) v *= ipow(row[comp[q]], ex[q]);
  return v;
}

// Product of the nonzero factors, the zero degree and the first two zero
// components of monomial t.
template <typename Real>
struct SparseFactors {
  Real mono;
  int64_t zdeg, z1, z2;
};

template <typename Real>
__device__ inline SparseFactors<Real> sparse_factors(const Real* __restrict__ row, const int64_t* __restrict__ toff,
                                                     const int64_t* __restrict__ comp,
                                                     const int64_t* __restrict__ ex, int64_t t) {
  SparseFactors<Real> f{Real(1), 0, -1, -1};
  for (int64_t q = toff[t]; q < toff[t + 1]; ++q) {
    const Real xv = row[comp[q]];
    if (xv == Real(0)) {
      f.zdeg += ex[q];
      if (f.z1 < 0) f.z1 = comp[q];
      else if (f.z2 < 0) f.z2 = comp[q];
    } else {
      f.mono *= ipow(xv, ex[q]);
    }
  }
  return f;
}

template <typename Real>
__global__ __launch_bounds__(256) void sparse_monomial_kernel(const Real* __restrict__ x, int64_t batch, int64_t D,
                                                              const int64_t* __restrict__ toff,
                                                              const int64_t* __restrict__ comp,
                                                              const int64_t* __restrict__ ex,
                                                              const int64_t* __restrict__ offsets,
                                                              const int64_t* __restrict__ terms,
                                                              const Real* __restrict__ values, int64_t O,
                                                              Real* __restrict__ out) {
  const int64_t total = batch * O;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int64_t b = idx / O, o = idx - (idx / O) * O;
    const Real* row = x + b * D;
    Real acc = Real(0);
    for (int64_t k = offsets[o]; k < offsets[o + 1]; ++k) acc += values[k] * sparse_monomial(row, toff, comp, ex, terms[k]);
    out[idx] = acc;
  }
}

// One thread per row owns its input-gradient row: coefficient k of output o
// adds g[b, o] v_k times the gradient of monomial terms[k] (zero degree one:
// the cofactor to the zero component; zero degree zero: e m / x per entry).
template <typename Real>
__global__ __launch_bounds__(256) void sparse_monomial_adjoint_kernel(
    const Real* __restrict__ gout, const Real* __restrict__ x, int64_t batch, int64_t D,
    const int64_t* __restrict__ toff, const int64_t* __restrict__ comp, const int64_t* __restrict__ ex,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ terms, const Real* __restrict__ values,
    int64_t O, Real* __restrict__ gin) {
  for (int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; b < batch; b += int64_t(gridDim.x) * blockDim.x) {
    const Real* row = x + b * D;
    Real* grad = gin + b * D;
    for (int64_t c = 0; c < D; ++c) grad[c] = Real(0);
    for (int64_t o = 0; o < O; ++o) {
      const Real g = gout[b * O + o];
      for (int64_t k = offsets[o]; k < offsets[o + 1]; ++k) {
        const int64_t t = terms[k];
        const Real w = g * conjv(values[k]);
        const SparseFactors<Real> f = sparse_factors(row, toff, comp, ex, t);
        if (f.zdeg == 1) {
          grad[f.z1] += w * conjv(f.mono);
        } else if (f.zdeg == 0) {
          for (int64_t q = toff[t]; q < toff[t + 1]; ++q)
            grad[comp[q]] += w * conjv(Real(ex[q]) * f.mono / row[comp[q]]);
        }
      }
    }
  }
}

// Directional derivative of monomial t along v.
template <typename Real>
__device__ inline Real sparse_directional(const Real* __restrict__ row, const Real* __restrict__ v,
                                          const int64_t* __restrict__ toff, const int64_t* __restrict__ comp,
                                          const int64_t* __restrict__ ex, int64_t t) {
  const SparseFactors<Real> f = sparse_factors(row, toff, comp, ex, t);
  if (f.zdeg == 1) return v[f.z1] * f.mono;
  if (f.zdeg != 0) return Real(0);
  Real logdir = Real(0);
  for (int64_t q = toff[t]; q < toff[t + 1]; ++q) logdir += Real(ex[q]) * v[comp[q]] / row[comp[q]];
  return f.mono * logdir;
}

// Output tangent of the double backward: the forward's linearisation along v.
template <typename Real>
__global__ __launch_bounds__(256) void sparse_monomial_tangent_kernel(
    const Real* __restrict__ tangent, const Real* __restrict__ x, int64_t batch, int64_t D,
    const int64_t* __restrict__ toff, const int64_t* __restrict__ comp, const int64_t* __restrict__ ex,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ terms, const Real* __restrict__ values,
    int64_t O, Real* __restrict__ out_tangent) {
  const int64_t total = batch * O;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int64_t b = idx / O, o = idx - (idx / O) * O;
    const Real* row = x + b * D;
    const Real* v = tangent + b * D;
    Real acc = Real(0);
    for (int64_t k = offsets[o]; k < offsets[o + 1]; ++k)
      acc += values[k] * sparse_directional(row, v, toff, comp, ex, terms[k]);
    out_tangent[idx] = acc;
  }
}

// Input tangent of the double backward: sum over coefficients of
// g[b, o] v_k (Hessian of monomial terms[k]) v, one thread per row.
template <typename Real>
__global__ __launch_bounds__(256) void sparse_monomial_hessian_kernel(
    const Real* __restrict__ tangent, const Real* __restrict__ gout, const Real* __restrict__ x, int64_t batch,
    int64_t D, const int64_t* __restrict__ toff, const int64_t* __restrict__ comp, const int64_t* __restrict__ ex,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ terms, const Real* __restrict__ values,
    int64_t O, Real* __restrict__ in_tangent) {
  for (int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; b < batch; b += int64_t(gridDim.x) * blockDim.x) {
    const Real* row = x + b * D;
    const Real* v = tangent + b * D;
    Real* it = in_tangent + b * D;
    for (int64_t c = 0; c < D; ++c) it[c] = Real(0);
    for (int64_t o = 0; o < O; ++o) {
      const Real g = gout[b * O + o];
      for (int64_t k = offsets[o]; k < offsets[o + 1]; ++k) {
        const int64_t t = terms[k];
        const Real w = g * conjv(values[k]);
        const SparseFactors<Real> f = sparse_factors(row, toff, comp, ex, t);
        if (f.zdeg == 0) {
          Real logdir = Real(0);
          for (int64_t q = toff[t]; q < toff[t + 1]; ++q) logdir += Real(ex[q]) * v[comp[q]] / row[comp[q]];
          for (int64_t q = toff[t]; q < toff[t + 1]; ++q) {
            const int64_t c = comp[q];
            it[c] += w * conjv(Real(ex[q]) * f.mono / row[c] * (logdir - v[c] / row[c]));
          }
        } else if (f.zdeg == 1) {
          Real zdir = Real(0);
          for (int64_t q = toff[t]; q < toff[t + 1]; ++q) {
            const int64_t c = comp[q];
            if (c == f.z1) continue;
            const Real d = Real(ex[q]) * f.mono / row[c];
            zdir += v[c] * d;
            it[c] += w * conjv(v[f.z1] * d);
          }
          it[f.z1] += w * conjv(zdir);
        } else if (f.zdeg == 2) {
          if (f.z2 < 0) {
            it[f.z1] += w * conjv(Real(2) * f.mono * v[f.z1]);
          } else {
            it[f.z1] += w * conjv(f.mono * v[f.z2]);
            it[f.z2] += w * conjv(f.mono * v[f.z1]);
          }
        }
      }
    }
  }
}

}  // namespace
}  // namespace ye3t

using namespace ye3t;

extern "C" {

int ye3t_hip_symmetric_power_monomial(int dtype, const void* x, int64_t batch, int64_t D, const int64_t* counts,
                                      const int64_t* offsets, const int64_t* output_indices, const void* values,
                                      int64_t T, int64_t O, void* out, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(batch >= 0 && D >= 0 && O >= 0 && T >= 0, "negative size");
  if (batch * O == 0) return YE3T_OK;
  YE3T_REQUIRE(x && offsets && out && (T == 0 || (counts && values && output_indices)), "NULL argument");
  const unsigned grid = grid_for(batch * O, 256);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(sym_monomial_kernel<double>, dim3(grid), dim3(256), 0, as_stream(stream), (const double*)x,
                       batch, D, counts, offsets, (const double*)values, O, (double*)out);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(sym_monomial_kernel<float>, dim3(grid), dim3(256), 0, as_stream(stream), (const float*)x,
                       batch, D, counts, offsets, (const float*)values, O, (float*)out);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("sym_monomial_kernel");
}

int ye3t_hip_symmetric_power_monomial_adjoint(int dtype, const void* output_adjoint, const void* x, int64_t batch,
                                              int64_t D, const int64_t* counts, const int64_t* output_indices,
                                              const void* values, int64_t T, int64_t O, void* input_adjoint,
                                              ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(batch >= 0 && D >= 0 && O >= 0 && T >= 0, "negative size");
  if (batch * D == 0) return YE3T_OK;
  YE3T_REQUIRE(x && input_adjoint && (T == 0 || (output_adjoint && counts && values && output_indices)),
               "NULL argument");
  const unsigned grid = grid_for(batch, 256);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(sym_monomial_adjoint_kernel<double>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const double*)output_adjoint, (const double*)x, batch, D, counts, output_indices,
                       (const double*)values, T, O, (double*)input_adjoint);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(sym_monomial_adjoint_kernel<float>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const float*)output_adjoint, (const float*)x, batch, D, counts, output_indices,
                       (const float*)values, T, O, (float*)input_adjoint);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("sym_monomial_adjoint_kernel");
}

int ye3t_hip_symmetric_power_shared_monomial(int dtype, const void* x, int64_t batch, int64_t D,
                                             const int64_t* counts, int64_t M, const int64_t* output_offsets,
                                             const int64_t* coefficient_terms, const void* coefficient_values,
                                             int64_t C, int64_t O, void* out, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(batch >= 0 && D >= 0 && O >= 0 && M >= 0 && C >= 0, "negative size");
  if (batch * O == 0) return YE3T_OK;
  YE3T_REQUIRE(x && output_offsets && out && (C == 0 || (counts && coefficient_terms && coefficient_values)),
               "NULL argument");
  const unsigned grid = grid_for(batch * O, 256);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(shared_monomial_kernel<double>, dim3(grid), dim3(256), 0, as_stream(stream), (const double*)x,
                       batch, D, counts, output_offsets, coefficient_terms, (const double*)coefficient_values, O,
                       (double*)out);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(shared_monomial_kernel<float>, dim3(grid), dim3(256), 0, as_stream(stream), (const float*)x,
                       batch, D, counts, output_offsets, coefficient_terms, (const float*)coefficient_values, O,
                       (float*)out);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  (void)M;
  return check_launch("shared_monomial_kernel");
}

int ye3t_hip_symmetric_power_shared_monomial_adjoint(int dtype, const void* output_adjoint, const void* x,
                                                     int64_t batch, int64_t D, const int64_t* counts, int64_t M,
                                                     const int64_t* output_offsets, const int64_t* coefficient_terms,
                                                     const void* coefficient_values, int64_t C, int64_t O,
                                                     void* input_adjoint, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(batch >= 0 && D >= 0 && O >= 0 && M >= 0 && C >= 0, "negative size");
  if (batch * D == 0) return YE3T_OK;
  YE3T_REQUIRE(x && input_adjoint && output_offsets &&
                   (C == 0 || (output_adjoint && counts && coefficient_terms && coefficient_values)),
               "NULL argument");
  const unsigned grid = grid_for(batch, 256);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(shared_monomial_adjoint_kernel<double>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const double*)output_adjoint, (const double*)x, batch, D, counts, output_offsets,
                       coefficient_terms, (const double*)coefficient_values, O, (double*)input_adjoint);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(shared_monomial_adjoint_kernel<float>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const float*)output_adjoint, (const float*)x, batch, D, counts, output_offsets,
                       coefficient_terms, (const float*)coefficient_values, O, (float*)input_adjoint);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  (void)M;
  return check_launch("shared_monomial_adjoint_kernel");
}

#define SPARSE_DISPATCH(KERNEL, GRID, ...)                                                                 \
  do {                                                                                                     \
    if (dtype == YE3T_F64) {                                                                               \
      using Real = double;                                                                                 \
      hipLaunchKernelGGL(KERNEL<double>, dim3(GRID), dim3(256), 0, as_stream(stream), __VA_ARGS__);        \
    } else if (dtype == YE3T_F32) {                                                                        \
      using Real = float;                                                                                  \
      hipLaunchKernelGGL(KERNEL<float>, dim3(GRID), dim3(256), 0, as_stream(stream), __VA_ARGS__);         \
    } else if (dtype == YE3T_C128) {                                                                       \
      using Real = cplx<double>;                                                                           \
      hipLaunchKernelGGL(KERNEL<Real>, dim3(GRID), dim3(256), 0, as_stream(stream), __VA_ARGS__);          \
    } else if (dtype == YE3T_C64) {                                                                        \
      using Real = cplx<float>;                                                                            \
      hipLaunchKernelGGL(KERNEL<Real>, dim3(GRID), dim3(256), 0, as_stream(stream), __VA_ARGS__);          \
    } else {                                                                                               \
      return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);                                        \
    }                                                                                                      \
  } while (0)

int ye3t_hip_symmetric_power_shared_sparse_monomial(int dtype, const void* x, int64_t batch, int64_t D,
                                                    const int64_t* term_offsets, const int64_t* term_components,
                                                    const int64_t* term_exponents, int64_t M, int64_t S,
                                                    const int64_t* output_offsets, const int64_t* coefficient_terms,
                                                    const void* coefficient_values, int64_t C, int64_t O, void* out,
                                                    ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(batch >= 0 && D >= 0 && M >= 0 && S >= 0 && C >= 0 && O >= 0, "negative size");
  if (batch * O == 0) return YE3T_OK;
  YE3T_REQUIRE(x && output_offsets && out && term_offsets &&
                   (C == 0 || (coefficient_terms && coefficient_values)) && (S == 0 || (term_components && term_exponents)),
               "NULL argument");
  SPARSE_DISPATCH(sparse_monomial_kernel, grid_for(batch * O, 256), (const Real*)x, batch, D, term_offsets,
                  term_components, term_exponents, output_offsets, coefficient_terms, (const Real*)coefficient_values,
                  O, (Real*)out);
  (void)M;
  return check_launch("sparse_monomial_kernel");
}

int ye3t_hip_symmetric_power_shared_sparse_monomial_adjoint(
    int dtype, const void* output_adjoint, const void* x, int64_t batch, int64_t D, const int64_t* term_offsets,
    const int64_t* term_components, const int64_t* term_exponents, int64_t M, int64_t S,
    const int64_t* output_offsets, const int64_t* coefficient_terms, const void* coefficient_values, int64_t C,
    int64_t O, void* input_adjoint, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(batch >= 0 && D >= 0 && M >= 0 && S >= 0 && C >= 0 && O >= 0, "negative size");
  if (batch * D == 0) return YE3T_OK;
  YE3T_REQUIRE(x && input_adjoint && output_offsets && term_offsets &&
                   (C == 0 || (output_adjoint && coefficient_terms && coefficient_values)) &&
                   (S == 0 || (term_components && term_exponents)),
               "NULL argument");
  SPARSE_DISPATCH(sparse_monomial_adjoint_kernel, grid_for(batch, 256), (const Real*)output_adjoint, (const Real*)x,
                  batch, D, term_offsets, term_components, term_exponents, output_offsets, coefficient_terms,
                  (const Real*)coefficient_values, O, (Real*)input_adjoint);
  (void)M;
  return check_launch("sparse_monomial_adjoint_kernel");
}

int ye3t_hip_symmetric_power_shared_sparse_monomial_double_backward(
    int dtype, const void* input_adjoint_tangent, const void* output_adjoint, const void* x, int64_t batch,
    int64_t D, const int64_t* term_offsets, const int64_t* term_components, const int64_t* term_exponents, int64_t M,
    int64_t S, const int64_t* output_offsets, const int64_t* coefficient_terms, const void* coefficient_values,
    int64_t C, int64_t O, void* output_tangent, void* input_tangent, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(batch >= 0 && D >= 0 && M >= 0 && S >= 0 && C >= 0 && O >= 0, "negative size");
  YE3T_REQUIRE((batch * O == 0 || output_tangent) && (batch * D == 0 || input_tangent), "NULL argument");
  if (batch == 0) return YE3T_OK;
  YE3T_REQUIRE(x && output_offsets && term_offsets && (D == 0 || input_adjoint_tangent) &&
                   (C == 0 || (output_adjoint && coefficient_terms && coefficient_values)) &&
                   (S == 0 || (term_components && term_exponents)),
               "NULL argument");
  if (O > 0) {
    SPARSE_DISPATCH(sparse_monomial_tangent_kernel, grid_for(batch * O, 256), (const Real*)input_adjoint_tangent,
                    (const Real*)x, batch, D, term_offsets, term_components, term_exponents, output_offsets,
                    coefficient_terms, (const Real*)coefficient_values, O, (Real*)output_tangent);
    const int rc = check_launch("sparse_monomial_tangent_kernel");
    if (rc != YE3T_OK) return rc;
  }
  if (D > 0) {
    SPARSE_DISPATCH(sparse_monomial_hessian_kernel, grid_for(batch, 256), (const Real*)input_adjoint_tangent,
                    (const Real*)output_adjoint, (const Real*)x, batch, D, term_offsets, term_components,
                    term_exponents, output_offsets, coefficient_terms, (const Real*)coefficient_values, O,
                    (Real*)input_tangent);
    return check_launch("sparse_monomial_hessian_kernel");
  }
  (void)M;
  return YE3T_OK;
}

}  // extern "C"
