// Symmetric-power monomial contractions (the reference's symmetric_power_*
// ops; CPU core ye3t_runtime_core.cpp:5279-5540, CUDA execution_plan_cuda.cu:
// 5229, 5931-6000): the grouped table S[b, o] = sum_{t in o} v_t prod_c
// x[b, c]^e[t, c], its adjoint, and the shared form in which outputs are sparse
// combinations of unique monomials.  These are the reference's stand-alone ops;
// the ACE product plan evaluates its symmetric blocks inside its own kernels.
//
// Forward: one thread per (row, output).  Adjoints: one thread per row, which
// owns its row of the input gradient (no atomics, fixed order).  The tables are
// validated by the caller (ye3t_amd.runtime checks them on the host).
#include "common.h"

namespace ye3t {
namespace {

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

}  // extern "C"
