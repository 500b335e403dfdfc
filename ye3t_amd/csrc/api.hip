// ye3t_hip: library bookkeeping (errors, ABI, device caps, SH normalisation)
// and the standalone per-edge tables (radial, real SH) and CSR density scatter.
#include <cmath>
#include <mutex>

#include "common.h"
#include "sph.h"

namespace ye3t {

namespace {
thread_local std::string g_last_error;
thread_local const char* g_last_density_kernel = "";
}

void set_density_kernel(const char* name) { g_last_density_kernel = name; }

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

const NormTable& norm_table() {
  static NormTable table;
  static std::once_flag once;
  std::call_once(once, [] {
    for (int l = 0; l <= kMaxL; ++l) {
      for (int m = 0; m <= kMaxL; ++m) {
        double v = 0.0;
        if (m <= l) {
          // (2l+1)/(4 pi) * (l-m)!/(l+m)!  computed as a product of reciprocals
          double ratio = 1.0;
          for (int k = l - m + 1; k <= l + m; ++k) ratio /= double(k);
          v = std::sqrt((2.0 * l + 1.0) / (4.0 * M_PI) * ratio);
        }
        table.v[l * (kMaxL + 1) + m] = v;
      }
    }
    table.inv[0] = 0.0;
    for (int k = 1; k < 2 * kMaxL + 2; ++k) table.inv[k] = 1.0 / double(k);
  });
  return table;
}

// ---------------------------------------------------------------------------
// Radial table: one thread per edge, one Chebyshev pass over n.
template <typename Real>
__global__ __launch_bounds__(256) void radial_table_kernel(const Real* __restrict__ radii,
                                                           const Real* __restrict__ cutoffs,
                                                           const Real* __restrict__ lambdas, int64_t E,
                                                           int n_max, Real* __restrict__ values,
                                                           Real* __restrict__ derivs) {
  // The basis is evaluated in fp64 for both storage types: the Chebyshev
  // recurrence amplifies rounding of the warped variable by ~n^2.
  double v[16], d[16];
  for (int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < E; e += int64_t(gridDim.x) * blockDim.x) {
    if (derivs) {
      cheb_exp_cos_row<double, true>(double(radii[e]), double(cutoffs[e]), double(lambdas[e]), n_max, v, d);
      for (int n = 0; n <= n_max; ++n) {
        values[e * (n_max + 1) + n] = Real(v[n]);
        derivs[e * (n_max + 1) + n] = Real(d[n]);
      }
    } else {
      cheb_exp_cos_row<double, false>(double(radii[e]), double(cutoffs[e]), double(lambdas[e]), n_max, v, d);
      for (int n = 0; n <= n_max; ++n) values[e * (n_max + 1) + n] = Real(v[n]);
    }
  }
}

// Scheduled radial-angular edge channels: output (e, k) is
// scale_k R[e, ri_k] Y[e, ai_k] when channel k takes every edge type
// (type -1) or edge e's type, zero otherwise, with its Cartesian derivative
// scale_k (dR[e, ri_k] dir[e] Y[e, ai_k] + R[e, ri_k] dY[e, ai_k]).  One thread
// per output.  The products are rounded in the reference core's order
// (ye3t_runtime_core.cpp:1550-1604) with no fused multiply-adds, so the
// results are the core's bit for bit.  Indices are validated by the caller;
// the kernel clamps them into the tables rather than faulting.
template <typename Real>
__global__ __launch_bounds__(256) void scheduled_channels_kernel(
    const Real* __restrict__ rv, const Real* __restrict__ rd, const Real* __restrict__ av,
    const Real* __restrict__ ad, const Real* __restrict__ dir, const int64_t* __restrict__ edge_types,
    const int64_t* __restrict__ cri, const int64_t* __restrict__ cai, const int64_t* __restrict__ ctype,
    const Real* __restrict__ cscale, int64_t E, int64_t NR, int64_t NA, int64_t K, Real* __restrict__ values,
    Real* __restrict__ derivs) {
#pragma clang fp contract(off)
  const int64_t total = E * K;
  for (int64_t o = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; o < total; o += int64_t(gridDim.x) * blockDim.x) {
    const int64_t e = o / K, k = o - e * K;
    const int64_t t = ctype[k];
    Real* const d = derivs + 3 * o;
    if (t >= 0 && edge_types[e] != t) {
      values[o] = Real(0);
      d[0] = d[1] = d[2] = Real(0);
      continue;
    }
    int64_t ri = cri[k], ai = cai[k];
    ri = ri < 0 ? 0 : (ri >= NR ? NR - 1 : ri);
    ai = ai < 0 ? 0 : (ai >= NA ? NA - 1 : ai);
    const Real r = rv[e * NR + ri], a = av[e * NA + ai], sc = cscale[k];
    const Real dr = rd[e * NR + ri];
    values[o] = sc * r * a;
    const Real* const ya = ad + 3 * (e * NA + ai);
    const Real* const u = dir + 3 * e;
    for (int x = 0; x < 3; ++x) d[x] = sc * (dr * u[x] * a + r * ya[x]);
  }
}

// Real SH table with optional Cartesian gradient.  Gradients w.r.t. the unit
// vector use d/dz Q_l^m = Q_l^{m+1}, projected with (I - u u^T)/|r|
// (reference ye3t_runtime_core.cpp:226-286, 808-843).
template <typename Real>
__global__ __launch_bounds__(128) void real_sph_table_kernel(const Real* __restrict__ vec, int64_t E, int lmax,
                                                             double eps, NormTable nt, Real* __restrict__ values,
                                                             Real* __restrict__ grads) {
  const int width = (lmax + 1) * (lmax + 1);
  const double sqrt2 = double(1.4142135623730950488016887242096981);
  for (int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < E; e += int64_t(gridDim.x) * blockDim.x) {
    const double x0 = double(vec[3 * e]), y0 = double(vec[3 * e + 1]), z0 = double(vec[3 * e + 2]);
    const double r = d_sqrt(x0 * x0 + y0 * y0 + z0 * z0);
    const double sr = r > eps ? r : eps;
    const double u[3] = {x0 / sr, y0 / sr, z0 / sr};
    Real* row = values + e * width;
    if (!grads) {
      double yrow[(kMaxL + 1) * (kMaxL + 1)];
      real_sph_row<double>(u[0], u[1], u[2], lmax, nt, yrow, 1);
      for (int k = 0; k < width; ++k) row[k] = Real(yrow[k]);
      continue;
    }
    // Q[l][m] for m <= l+1 (Q_l^{l+1} = 0)
    double Q[kMaxL + 2][kMaxL + 2];
    double qmm = double(1);
    for (int m = 0; m <= lmax + 1; ++m) {
      if (m > 0) qmm *= double(2 * m - 1);
      double q2 = double(0), q1 = double(0);
      for (int l = 0; l <= lmax; ++l) {
        double q;
        if (l < m) {
          q = double(0);
        } else if (l == m) {
          q = qmm;
        } else if (l == m + 1) {
          q = double(2 * m + 1) * u[2] * qmm;
        } else {
          q = (double(2 * l - 1) * u[2] * q1 - double(l + m - 1) * q2) / double(l - m);
        }
        if (l >= m) {
          q2 = q1;
          q1 = q;
        }
        Q[l][m] = q;
      }
    }
    double cr = double(1), ci = double(0), pr = double(1), pi = double(0);
    for (int m = 0; m <= lmax; ++m) {
      if (m > 0) {
        pr = cr;
        pi = ci;
        const double nr = cr * u[0] - ci * u[1];
        const double ni = cr * u[1] + ci * u[0];
        cr = nr;
        ci = ni;
      }
      for (int l = m; l <= lmax; ++l) {
        const double n = double(nt.v[l * (kMaxL + 1) + m]);
        const int base = l * l + l;
        double ug[2][3];
        int idx[2];
        int count;
        if (m == 0) {
          row[base] = Real(n * Q[l][0]);
          ug[0][0] = double(0);
          ug[0][1] = double(0);
          ug[0][2] = n * Q[l][1];
          idx[0] = base;
          count = 1;
        } else {
          const double s = sqrt2 * n;
          const double q = Q[l][m], qz = Q[l][m + 1];
          row[base + m] = Real(s * q * cr);
          row[base - m] = Real(-s * q * ci);
          ug[0][0] = s * q * (double(m) * pr);
          ug[0][1] = s * q * (-double(m) * pi);
          ug[0][2] = s * qz * cr;
          ug[1][0] = -s * q * (double(m) * pi);
          ug[1][1] = -s * q * (double(m) * pr);
          ug[1][2] = -s * qz * ci;
          idx[0] = base + m;
          idx[1] = base - m;
          count = 2;
        }
        for (int c = 0; c < count; ++c) {
          for (int a = 0; a < 3; ++a) {
            double g = double(0);
            for (int b = 0; b < 3; ++b) {
              double jac;
              if (r > eps) {
                jac = ((a == b ? double(1) : double(0)) - u[a] * u[b]) / sr;
              } else {
                jac = (a == b) ? double(1) / sr : double(0);
              }
              g += ug[c][b] * jac;
            }
            grads[(e * width + idx[c]) * 3 + a] = Real(g);
          }
        }
      }
    }
  }
}

// CSR segment reduction: thread per (atom, channel), edges summed in order.
template <typename Real>
__global__ __launch_bounds__(256) void density_csr_kernel(const Real* __restrict__ ev,
                                                          const int64_t* __restrict__ offsets, int64_t N,
                                                          int64_t C, Real* __restrict__ out) {
  const int64_t total = N * C;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int64_t i = idx / C, c = idx - (idx / C) * C;
    Real acc = Real(0);
    for (int64_t e = offsets[i]; e < offsets[i + 1]; ++e) acc += ev[e * C + c];
    out[idx] = acc;
  }
}

// Gather of centre-row adjoints to edge rows.  A workgroup of 256 threads
// copies whole edge rows: 256 / CV rows at a time when a row is at most 256
// vectors (V = 16 bytes when the rows allow it), else one row in a loop;
// indices within the group are 32-bit.  The output is streamed with
// non-temporal stores (written once, not re-read here).  Centres are validated
// by the caller; an index outside [0, N) is clamped so that no access leaves
// the array.
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename V>
__global__ __launch_bounds__(256) void density_adjoint_kernel(const V* __restrict__ adj,
                                                              const int64_t* __restrict__ centers, int64_t E,
                                                              int CV, int64_t N, V* __restrict__ out) {
  const int epb = CV >= 256 ? 1 : 256 / CV;  // edge rows per pass of the workgroup
  const int span = epb * CV;
  for (int64_t e0 = int64_t(blockIdx.x) * epb; e0 < E; e0 += int64_t(gridDim.x) * epb) {
    for (int t = threadIdx.x; t < span; t += 256) {
      const int de = t / CV;
      const int c = t - de * CV;
      const int64_t e = e0 + de;
      if (e < E) {
        int64_t i = centers[e];
        i = i < 0 ? 0 : (i >= N ? N - 1 : i);
        __builtin_nontemporal_store(adj[i * CV + c], out + e * CV + c);
      }
    }
  }
}

inline unsigned grid_for(int64_t work, int threads) {
  int64_t g = (work + threads - 1) / threads;
  if (g < 1) g = 1;
  if (g > (1 << 20)) g = 1 << 20;
  return unsigned(g);
}

}  // namespace ye3t

using namespace ye3t;

extern "C" {

int ye3t_hip_abi_version(void) { return YE3T_HIP_ABI_VERSION; }

int ye3t_hip_has_hip(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return count > 0 ? 1 : 0;
}

int ye3t_hip_has_cpu(void) { return 0; }

const char* ye3t_hip_last_error(void) { return g_last_error.c_str(); }

const char* ye3t_hip_last_density_kernel(void) { return g_last_density_kernel; }

int ye3t_hip_device_caps(int device, ye3t_hip_caps* out) {
  YE3T_REQUIRE(out != nullptr, "caps output is NULL");
  hipDeviceProp_t prop;
  YE3T_CHECK_HIP(hipGetDeviceProperties(&prop, device));
  std::snprintf(out->arch, sizeof out->arch, "%s", prop.gcnArchName);
  out->device = device;
  out->cu_count = prop.multiProcessorCount;
  out->wavefront_size = prop.warpSize;
  out->lds_bytes_per_block = int(prop.sharedMemPerBlock);
  out->clock_khz = prop.clockRate;
  out->hbm_bytes = int64_t(prop.totalGlobalMem);
  out->hbm_peak_gbs = 8000.0;  // MI355X nominal HBM3E peak
  return YE3T_OK;
}

int ye3t_hip_radial_table(int dtype, const void* radii, const void* cutoffs, const void* lambdas, int64_t E,
                          int64_t n_max, void* values, void* derivs, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(E >= 0, "edge_count must be non-negative");
  YE3T_REQUIRE(n_max >= 0 && n_max < 16, "max_radial_index must be in [0, 15], got %lld", (long long)n_max);
  if (E == 0) return YE3T_OK;
  YE3T_REQUIRE(radii && cutoffs && lambdas && values, "NULL input or output");
  const unsigned grid = grid_for(E, 256);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(radial_table_kernel<double>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const double*)radii, (const double*)cutoffs, (const double*)lambdas, E, int(n_max),
                       (double*)values, (double*)derivs);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(radial_table_kernel<float>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const float*)radii, (const float*)cutoffs, (const float*)lambdas, E, int(n_max),
                       (float*)values, (float*)derivs);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("radial_table_kernel");
}

int ye3t_hip_scheduled_radial_angular_channels(int dtype, int64_t edge_count, int64_t radial_width,
                                               int64_t angular_width, int64_t channel_count,
                                               const void* radial_values, const void* radial_derivatives,
                                               const void* angular_values, const void* angular_derivatives,
                                               const void* radial_directions, const int64_t* edge_types,
                                               const int64_t* channel_radial_indices,
                                               const int64_t* channel_angular_indices,
                                               const int64_t* channel_types, const void* channel_scales,
                                               void* edge_values, void* edge_derivatives, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(edge_count >= 0 && channel_count >= 0, "edge and channel counts must be non-negative");
  if (edge_count == 0 || channel_count == 0) return YE3T_OK;
  YE3T_REQUIRE(radial_width > 0 && angular_width > 0, "radial and angular tables must not be empty");
  YE3T_REQUIRE(edge_count <= INT64_MAX / channel_count / 3, "edge_count * channel_count overflows");
  YE3T_REQUIRE(radial_values && radial_derivatives && angular_values && angular_derivatives && radial_directions &&
                   edge_types && channel_radial_indices && channel_angular_indices && channel_types &&
                   channel_scales && edge_values && edge_derivatives,
               "NULL input or output");
  const unsigned grid = grid_for(edge_count * channel_count, 256);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(scheduled_channels_kernel<double>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const double*)radial_values, (const double*)radial_derivatives,
                       (const double*)angular_values, (const double*)angular_derivatives,
                       (const double*)radial_directions, edge_types, channel_radial_indices,
                       channel_angular_indices, channel_types, (const double*)channel_scales, edge_count,
                       radial_width, angular_width, channel_count, (double*)edge_values, (double*)edge_derivatives);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(scheduled_channels_kernel<float>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const float*)radial_values, (const float*)radial_derivatives,
                       (const float*)angular_values, (const float*)angular_derivatives,
                       (const float*)radial_directions, edge_types, channel_radial_indices,
                       channel_angular_indices, channel_types, (const float*)channel_scales, edge_count,
                       radial_width, angular_width, channel_count, (float*)edge_values, (float*)edge_derivatives);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("scheduled_channels_kernel");
}

int ye3t_hip_real_sph_table(int dtype, const void* vec, int64_t E, int64_t lmax, double eps, void* values,
                            void* grads, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(E >= 0, "edge_count must be non-negative");
  YE3T_REQUIRE(lmax >= 0 && lmax <= kMaxL, "maximum_angular_momentum must be in [0, %d]", kMaxL);
  if (E == 0) return YE3T_OK;
  YE3T_REQUIRE(vec && values, "NULL input or output");
  const unsigned grid = grid_for(E, 128);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(real_sph_table_kernel<double>, dim3(grid), dim3(128), 0, as_stream(stream),
                       (const double*)vec, E, int(lmax), eps, norm_table(), (double*)values, (double*)grads);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(real_sph_table_kernel<float>, dim3(grid), dim3(128), 0, as_stream(stream),
                       (const float*)vec, E, int(lmax), eps, norm_table(), (float*)values, (float*)grads);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("real_sph_table_kernel");
}

int ye3t_hip_density_accumulate_csr(int dtype, const void* ev, const int64_t* offsets, int64_t N, int64_t C,
                                    void* out, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(N >= 0 && C >= 0, "negative size");
  if (N * C == 0) return YE3T_OK;
  YE3T_REQUIRE(offsets && out, "NULL offsets or output");
  const unsigned grid = grid_for(N * C, 256);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(density_csr_kernel<double>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const double*)ev, offsets, N, C, (double*)out);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(density_csr_kernel<float>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const float*)ev, offsets, N, C, (float*)out);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("density_csr_kernel");
}

int ye3t_hip_density_accumulate_adjoint(int dtype, const void* adj, const int64_t* centers, int64_t E, int64_t C,
                                        int64_t N, void* out, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(E >= 0 && C >= 0 && N >= 0, "negative size");
  if (E * C == 0) return YE3T_OK;
  YE3T_REQUIRE(N >= 1, "edges need at least one atom");
  YE3T_REQUIRE(adj && centers && out, "NULL input or output");
  const size_t elem = dtype == YE3T_F64 ? 8 : 4;
  YE3T_REQUIRE(dtype == YE3T_F64 || dtype == YE3T_F32, "unsupported dtype %d", dtype);
  const bool vec = (size_t(C) * elem) % 16 == 0 && reinterpret_cast<uintptr_t>(adj) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0;
  const hipStream_t s = as_stream(stream);
  const int64_t CV = vec ? int64_t(size_t(C) * elem / 16) : C;
  YE3T_REQUIRE(CV < (int64_t(1) << 30), "channel_count too large");
  const int64_t epb = CV >= 256 ? 1 : 256 / CV;
  const unsigned grid = grid_for((E + epb - 1) / epb, 1);
  if (vec) {
    hipLaunchKernelGGL(density_adjoint_kernel<f32x4>, dim3(grid), dim3(256), 0, s, (const f32x4*)adj, centers, E,
                       int(CV), N, (f32x4*)out);
  } else if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(density_adjoint_kernel<double>, dim3(grid), dim3(256), 0, s, (const double*)adj, centers, E,
                       int(CV), N, (double*)out);
  } else {
    hipLaunchKernelGGL(density_adjoint_kernel<float>, dim3(grid), dim3(256), 0, s, (const float*)adj, centers, E,
                       int(CV), N, (float*)out);
  }
  return check_launch("density_adjoint_kernel");
}

}  // extern "C"
