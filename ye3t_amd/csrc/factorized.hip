// factorized_angular on gfx950: the reference's general factorized-angular DAG
// executor (schema execution_plan_torch.cpp:7586-7594, CPU core
// ye3t_runtime_core.cpp:5667-5769, adjoint :6481-6643, linear :7144-7399)
// for real and complex data.
//
// One wave (64 lanes) runs up to 64 samples, lane = sample.  The DAG tables are
// wave-uniform: they are read through the scalar cache (the plan's device
// copy, validated on the host at plan creation, so the kernels index without
// checks).  The per-sample workspace, and in reverse mode its adjoint, live in
// LDS as [slot][lanes]: nothing goes to global memory but the inputs and
// outputs (the reference's CUDA executor keeps its workspace in global memory,
// execution_plan_cuda.cu:11584-11589).  Workspaces too wide for 64 samples run
// with fewer samples per wave.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.h"

struct ye3t_hip_factorized_angular_plan {
  int dtype;
  int device;
  int64_t node_count, coef_count, root_count;
  int64_t source_dimension, input_dimension, workspace_dimension, output_dimension, projection_dimension;
  int64_t root_dimension;
  // int32 device tables (read as scalars)
  int32_t* node_offsets;
  int32_t* node_dims;
  int32_t* node_leaf;
  int32_t* node_left;
  int32_t* node_right;
  int32_t* node_coef_off;
  int32_t* coef_left;   // node_offsets[left] + row / right_dim
  int32_t* coef_right;  // node_offsets[right] + row % right_dim
  int32_t* coef_col;    // node_offsets[node] + column
  int32_t* roots;
  void* coef_values;
  void* projection;
};

namespace ye3t {
namespace {

template <typename R>
struct cpx {
  R re, im;
};

// arithmetic of the four scalar types
template <typename T>
struct Ops {
  __device__ static T zero() { return T(0); }
  __device__ static T conj(T x) { return x; }
  __device__ static T mul(T a, T b) { return a * b; }
  __device__ static T add(T a, T b) { return a + b; }
};
template <typename R>
struct Ops<cpx<R>> {
  typedef cpx<R> T;
  __device__ static T zero() { return T{R(0), R(0)}; }
  __device__ static T conj(T x) { return T{x.re, -x.im}; }
  __device__ static T mul(T a, T b) { return T{a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re}; }
  __device__ static T add(T a, T b) { return T{a.re + b.re, a.im + b.im}; }
};

typedef const __attribute__((address_space(4))) int32_t* sgpr_i32;

struct FATables {
  const int32_t* node_offsets;
  const int32_t* node_dims;
  const int32_t* node_leaf;
  const int32_t* node_coef_off;
  const int32_t* coef_left;
  const int32_t* coef_right;
  const int32_t* coef_col;
  const int32_t* roots;
  int node_count, root_count, source_dim, input_dim, ws_dim, out_dim, proj_dim, root_dim;
};

// a wave-uniform table entry, read through the constant address space (a
// scalar load: the tables are read-only for the kernel's lifetime)
__device__ inline int at(const int32_t* table, int i) { return ((sgpr_i32)(const void*)table)[i]; }

// Forward replay of one source of this lane's sample into ws ([slot][spw]).
template <typename T>
__device__ inline void fa_replay(const FATables& t, const T* __restrict__ coef, const T* __restrict__ in,
                                 T* ws, int spw) {
  typedef Ops<T> O;
  for (int q = 0; q < t.ws_dim; ++q) ws[q * spw] = O::zero();
  for (int n = 0; n < t.node_count; ++n) {
    const int off = at(t.node_offsets, n);
    const int leaf = at(t.node_leaf, n);
    if (leaf >= 0) {
      const int d = at(t.node_dims, n);
      for (int i = 0; i < d; ++i) ws[(off + i) * spw] = in[leaf + i];
      continue;
    }
    const int e1 = at(t.node_coef_off, n + 1);
    for (int e = at(t.node_coef_off, n); e < e1; ++e) {
      const int c = at(t.coef_col, e);
      ws[c * spw] = O::add(ws[c * spw], O::mul(O::mul(O::conj(coef[e]), ws[at(t.coef_left, e) * spw]),
                                               ws[at(t.coef_right, e) * spw]));
    }
  }
}

template <typename T>
__global__ __launch_bounds__(64) void fa_forward_kernel(FATables t, const T* __restrict__ coef,
                                                        const T* __restrict__ proj, const T* __restrict__ packed,
                                                        int64_t batch, int spw, T* __restrict__ out) {
  typedef Ops<T> O;
  extern __shared__ __align__(16) unsigned char fa_smem[];
  const int lane = threadIdx.x;
  if (lane >= spw) return;
  const int64_t b = int64_t(blockIdx.x) * spw + lane;
  if (b >= batch) return;
  T* ws = reinterpret_cast<T*>(fa_smem) + lane;
  T* orow = out + b * t.out_dim;
  for (int k = 0; k < t.out_dim; ++k) orow[k] = O::zero();
  for (int s = 0; s < t.source_dim; ++s) {
    const T* in = packed + (b * t.source_dim + s) * t.input_dim;
    fa_replay(t, coef, in, ws, spw);
    for (int r = 0; r < t.root_count; ++r) {
      const int roff = at(t.node_offsets, at(t.roots, r));
      for (int p = 0; p < t.proj_dim; ++p) {
        const T pv = proj[s * t.proj_dim + p];
        T* blk = orow + (r * t.proj_dim + p) * t.root_dim;
        for (int m = 0; m < t.root_dim; ++m) blk[m] = O::add(blk[m], O::mul(ws[(roff + m) * spw], pv));
      }
    }
  }
}

// Reverse mode.  LINEAR: the output adjoint of feature k of sample b is
// g[b] * conj(weight[k]) (the linear readout's adjoint), else gout[b, k].
template <typename T, bool LINEAR>
__global__ __launch_bounds__(64) void fa_adjoint_kernel(FATables t, const T* __restrict__ coef,
                                                        const T* __restrict__ proj, const T* __restrict__ packed,
                                                        const T* __restrict__ gout, const T* __restrict__ weight,
                                                        int64_t batch, int spw, T* __restrict__ gpacked) {
  typedef Ops<T> O;
  extern __shared__ __align__(16) unsigned char fa_smem[];
  const int lane = threadIdx.x;
  if (lane >= spw) return;
  const int64_t b = int64_t(blockIdx.x) * spw + lane;
  if (b >= batch) return;
  T* ws = reinterpret_cast<T*>(fa_smem) + lane;
  T* wa = reinterpret_cast<T*>(fa_smem) + int64_t(t.ws_dim) * spw + lane;
  T* grow = gpacked + b * int64_t(t.source_dim) * t.input_dim;
  for (int k = 0; k < t.source_dim * t.input_dim; ++k) grow[k] = O::zero();
  const T gl = LINEAR ? gout[b] : O::zero();
  for (int s = 0; s < t.source_dim; ++s) {
    const T* in = packed + (b * t.source_dim + s) * t.input_dim;
    fa_replay(t, coef, in, ws, spw);
    for (int q = 0; q < t.ws_dim; ++q) wa[q * spw] = O::zero();
    for (int r = 0; r < t.root_count; ++r) {
      const int roff = at(t.node_offsets, at(t.roots, r));
      for (int p = 0; p < t.proj_dim; ++p) {
        const T cpv = O::conj(proj[s * t.proj_dim + p]);
        const int f0 = (r * t.proj_dim + p) * t.root_dim;
        for (int m = 0; m < t.root_dim; ++m) {
          const T g = LINEAR ? O::mul(gl, O::conj(weight[f0 + m])) : gout[b * t.out_dim + f0 + m];
          wa[(roff + m) * spw] = O::add(wa[(roff + m) * spw], O::mul(g, cpv));
        }
      }
    }
    for (int n = t.node_count - 1; n >= 0; --n) {
      if (at(t.node_leaf, n) >= 0) continue;
      const int e1 = at(t.node_coef_off, n + 1);
      for (int e = at(t.node_coef_off, n); e < e1; ++e) {
        const int li = at(t.coef_left, e), ri = at(t.coef_right, e);
        const T gc = O::mul(wa[at(t.coef_col, e) * spw], coef[e]);
        wa[li * spw] = O::add(wa[li * spw], O::mul(gc, O::conj(ws[ri * spw])));
        wa[ri * spw] = O::add(wa[ri * spw], O::mul(gc, O::conj(ws[li * spw])));
      }
    }
    T* gin = grow + s * t.input_dim;
    for (int n = 0; n < t.node_count; ++n) {
      const int leaf = at(t.node_leaf, n);
      if (leaf < 0) continue;
      const int off = at(t.node_offsets, n), d = at(t.node_dims, n);
      for (int i = 0; i < d; ++i) gin[leaf + i] = O::add(gin[leaf + i], wa[(off + i) * spw]);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(64) void fa_linear_kernel(FATables t, const T* __restrict__ coef,
                                                       const T* __restrict__ proj, const T* __restrict__ packed,
                                                       const T* __restrict__ weight, T bias, int64_t batch, int spw,
                                                       T* __restrict__ out) {
  typedef Ops<T> O;
  extern __shared__ __align__(16) unsigned char fa_smem[];
  const int lane = threadIdx.x;
  if (lane >= spw) return;
  const int64_t b = int64_t(blockIdx.x) * spw + lane;
  if (b >= batch) return;
  T* ws = reinterpret_cast<T*>(fa_smem) + lane;
  T value = bias;
  for (int s = 0; s < t.source_dim; ++s) {
    const T* in = packed + (b * t.source_dim + s) * t.input_dim;
    fa_replay(t, coef, in, ws, spw);
    for (int r = 0; r < t.root_count; ++r) {
      const int roff = at(t.node_offsets, at(t.roots, r));
      for (int p = 0; p < t.proj_dim; ++p) {
        const T pv = proj[s * t.proj_dim + p];
        const int f0 = (r * t.proj_dim + p) * t.root_dim;
        for (int m = 0; m < t.root_dim; ++m)
          value = O::add(value, O::mul(O::mul(ws[(roff + m) * spw], pv), weight[f0 + m]));
      }
    }
  }
  out[b] = value;
}

// gw[k] = sum_b g[b] conj(F[b, k]) for k < K and gb = sum_b g[b] (thread K):
// the readout's parameter adjoints, each summed over the batch in order.
template <typename T>
__global__ __launch_bounds__(64) void fa_readout_params_kernel(const T* __restrict__ F, const T* __restrict__ g,
                                                               int64_t batch, int64_t K, T* __restrict__ gw,
                                                               T* __restrict__ gb) {
  typedef Ops<T> O;
  const int64_t k = int64_t(blockIdx.x) * 64 + threadIdx.x;
  if (k > K) return;
  T acc = O::zero();
  if (k < K) {
    for (int64_t b = 0; b < batch; ++b) acc = O::add(acc, O::mul(g[b], O::conj(F[b * K + k])));
    gw[k] = acc;
  } else {
    for (int64_t b = 0; b < batch; ++b) acc = O::add(acc, g[b]);
    *gb = acc;
  }
}

size_t fa_elem(int dtype) {
  switch (dtype) {
    case YE3T_F32: return 4;
    case YE3T_F64: return 8;
    case YE3T_C64: return 8;
    case YE3T_C128: return 16;
    default: return 0;
  }
}

// samples per wave whose workspace (copies of it) fits 64 KB of LDS
int fa_samples_per_wave(const ye3t_hip_factorized_angular_plan* p, int copies) {
  const size_t per = size_t(p->workspace_dimension) * fa_elem(p->dtype) * size_t(copies);
  for (int spw = 64; spw >= 1; spw /= 2)
    if (per * size_t(spw) <= 64 * 1024) return spw;
  return 0;
}

FATables fa_tables(const ye3t_hip_factorized_angular_plan* p) {
  FATables t;
  t.node_offsets = p->node_offsets;
  t.node_dims = p->node_dims;
  t.node_leaf = p->node_leaf;
  t.node_coef_off = p->node_coef_off;
  t.coef_left = p->coef_left;
  t.coef_right = p->coef_right;
  t.coef_col = p->coef_col;
  t.roots = p->roots;
  t.node_count = int(p->node_count);
  t.root_count = int(p->root_count);
  t.source_dim = int(p->source_dimension);
  t.input_dim = int(p->input_dimension);
  t.ws_dim = int(p->workspace_dimension);
  t.out_dim = int(p->output_dimension);
  t.proj_dim = int(p->projection_dimension);
  t.root_dim = int(p->root_dimension);
  return t;
}

template <typename T>
int fa_upload(T** dst, const T* src, int64_t n) {
  *dst = nullptr;
  if (n <= 0) return YE3T_OK;
  YE3T_CHECK_HIP(hipMalloc(reinterpret_cast<void**>(dst), size_t(n) * sizeof(T)));
  YE3T_CHECK_HIP(hipMemcpy(*dst, src, size_t(n) * sizeof(T), hipMemcpyHostToDevice));
  return YE3T_OK;
}

}  // namespace
}  // namespace ye3t

using namespace ye3t;

extern "C" {

void ye3t_hip_factorized_angular_plan_destroy(ye3t_hip_factorized_angular_plan* p) {
  if (!p) return;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(p->device);
  for (void* q : {(void*)p->node_offsets, (void*)p->node_dims, (void*)p->node_leaf, (void*)p->node_left,
                  (void*)p->node_right, (void*)p->node_coef_off, (void*)p->coef_left, (void*)p->coef_right,
                  (void*)p->coef_col, (void*)p->roots, p->coef_values, p->projection})
    if (q) (void)hipFree(q);
  (void)hipSetDevice(prev);
  delete p;
}

int ye3t_hip_factorized_angular_plan_create(const ye3t_factorized_angular_desc* d,
                                            ye3t_hip_factorized_angular_plan** out) {
  clear_error();
  YE3T_REQUIRE(d && out, "NULL description or output");
  *out = nullptr;
  const size_t elem = fa_elem(d->dtype);
  YE3T_REQUIRE(elem != 0, "unsupported dtype %d", d->dtype);
  const int64_t N = d->node_count, E = d->coefficient_count, R = d->root_count, S = d->source_dimension;
  // the Torch op's checks (execution_plan_torch.cpp:5910-5990, 177-250)
  YE3T_REQUIRE(N > 0, "factorized plan must contain nodes");
  YE3T_REQUIRE(R > 0, "factorized plan requires roots");
  YE3T_REQUIRE(S > 0, "source_dimension must be positive");
  YE3T_REQUIRE(d->projection_count > 0, "factorized plan requires projection weights");
  YE3T_REQUIRE(d->projection_count % S == 0, "projection weights must be divisible by source_dimension");
  YE3T_REQUIRE(d->input_dimension > 0, "input_dimension must be positive");
  YE3T_REQUIRE(E >= 0 && (E == 0 || (d->coefficient_rows && d->coefficient_columns && d->coefficient_values)),
               "factorized coefficient arrays must have equal length");
  YE3T_REQUIRE(d->node_offsets && d->node_dimensions && d->node_leaf_offsets && d->node_left && d->node_right &&
                   d->node_coefficient_offsets && d->root_nodes && d->projection_values,
               "NULL table");
  YE3T_REQUIRE(N < (int64_t(1) << 30) && E < (int64_t(1) << 30), "table too large");
  const int64_t W = d->node_offsets[N - 1] + d->node_dimensions[N - 1];
  YE3T_REQUIRE(W > 0 && d->workspace_dimension == W,
               "factorized workspace_dimension does not match compiler metadata");
  YE3T_REQUIRE(d->node_coefficient_offsets[0] == 0 && d->node_coefficient_offsets[N] == E,
               "node_coefficient_offsets must span the coefficient table");
  // everything the kernels index, checked here so the kernels need no checks
  for (int64_t n = 0; n < N; ++n) {
    const int64_t off = d->node_offsets[n], dim = d->node_dimensions[n];
    YE3T_REQUIRE(dim > 0 && off >= 0 && off + dim <= W, "node %lld lies outside the workspace", (long long)n);
    YE3T_REQUIRE(d->node_coefficient_offsets[n] <= d->node_coefficient_offsets[n + 1],
                 "node_coefficient_offsets must be nondecreasing");
    const int64_t leaf = d->node_leaf_offsets[n];
    if (leaf >= 0) {
      YE3T_REQUIRE(leaf + dim <= d->input_dimension, "leaf node %lld reads past the input slot", (long long)n);
      YE3T_REQUIRE(d->node_coefficient_offsets[n] == d->node_coefficient_offsets[n + 1],
                   "leaf node %lld has coefficients", (long long)n);
      continue;
    }
    const int64_t l = d->node_left[n], r = d->node_right[n];
    YE3T_REQUIRE(l >= 0 && l < N && r >= 0 && r < N, "node %lld has an out-of-range child", (long long)n);
    const int64_t ld = d->node_dimensions[l], rd = d->node_dimensions[r];
    for (int64_t e = d->node_coefficient_offsets[n]; e < d->node_coefficient_offsets[n + 1]; ++e) {
      YE3T_REQUIRE(d->coefficient_rows[e] >= 0 && d->coefficient_rows[e] < ld * rd,
                   "coefficient row %lld out of range", (long long)e);
      YE3T_REQUIRE(d->coefficient_columns[e] >= 0 && d->coefficient_columns[e] < dim,
                   "coefficient column %lld out of range", (long long)e);
    }
  }
  const int64_t P = d->projection_count / S;
  YE3T_REQUIRE(d->root_nodes[0] >= 0 && d->root_nodes[0] < N, "factorized root index is out of bounds");
  const int64_t rdim = d->node_dimensions[d->root_nodes[0]];
  for (int64_t r = 0; r < R; ++r) {
    YE3T_REQUIRE(d->root_nodes[r] >= 0 && d->root_nodes[r] < N, "factorized root index is out of bounds");
    YE3T_REQUIRE(d->node_dimensions[d->root_nodes[r]] == rdim, "uniform factorized roots must have identical dimensions");
  }
  YE3T_REQUIRE(d->output_dimension == R * P * rdim, "output width does not match uniform factorized root metadata");
  YE3T_REQUIRE(S * d->input_dimension < (int64_t(1) << 31) && d->output_dimension < (int64_t(1) << 31),
               "packed rows too wide");

  std::vector<int32_t> noff(N), ndim(N), nleaf(N), nl(N), nr(N), ncoef(N + 1), cl(E), cr(E), cc(E), roots(R);
  for (int64_t n = 0; n < N; ++n) {
    noff[n] = int32_t(d->node_offsets[n]);
    ndim[n] = int32_t(d->node_dimensions[n]);
    nleaf[n] = int32_t(d->node_leaf_offsets[n] >= 0 ? d->node_leaf_offsets[n] : -1);
    nl[n] = int32_t(d->node_left[n]);
    nr[n] = int32_t(d->node_right[n]);
    ncoef[n] = int32_t(d->node_coefficient_offsets[n]);
    if (nleaf[n] >= 0) continue;
    const int64_t rd = d->node_dimensions[d->node_right[n]];
    for (int64_t e = d->node_coefficient_offsets[n]; e < d->node_coefficient_offsets[n + 1]; ++e) {
      cl[e] = int32_t(d->node_offsets[d->node_left[n]] + d->coefficient_rows[e] / rd);
      cr[e] = int32_t(d->node_offsets[d->node_right[n]] + d->coefficient_rows[e] % rd);
      cc[e] = int32_t(d->node_offsets[n] + d->coefficient_columns[e]);
    }
  }
  ncoef[N] = int32_t(E);
  for (int64_t r = 0; r < R; ++r) roots[r] = int32_t(d->root_nodes[r]);

  auto* p = new ye3t_hip_factorized_angular_plan();
  std::memset(p, 0, sizeof(*p));
  p->dtype = d->dtype;
  (void)hipGetDevice(&p->device);
  p->node_count = N;
  p->coef_count = E;
  p->root_count = R;
  p->source_dimension = S;
  p->input_dimension = d->input_dimension;
  p->workspace_dimension = W;
  p->output_dimension = d->output_dimension;
  p->projection_dimension = P;
  p->root_dimension = rdim;
  int rc = YE3T_OK;
  if ((rc = fa_upload(&p->node_offsets, noff.data(), N)) != YE3T_OK ||
      (rc = fa_upload(&p->node_dims, ndim.data(), N)) != YE3T_OK ||
      (rc = fa_upload(&p->node_leaf, nleaf.data(), N)) != YE3T_OK ||
      (rc = fa_upload(&p->node_left, nl.data(), N)) != YE3T_OK ||
      (rc = fa_upload(&p->node_right, nr.data(), N)) != YE3T_OK ||
      (rc = fa_upload(&p->node_coef_off, ncoef.data(), N + 1)) != YE3T_OK ||
      (rc = fa_upload(&p->coef_left, cl.data(), E)) != YE3T_OK ||
      (rc = fa_upload(&p->coef_right, cr.data(), E)) != YE3T_OK ||
      (rc = fa_upload(&p->coef_col, cc.data(), E)) != YE3T_OK ||
      (rc = fa_upload(&p->roots, roots.data(), R)) != YE3T_OK ||
      (rc = fa_upload(reinterpret_cast<unsigned char**>(&p->coef_values),
                      static_cast<const unsigned char*>(d->coefficient_values), E * int64_t(elem))) != YE3T_OK ||
      (rc = fa_upload(reinterpret_cast<unsigned char**>(&p->projection),
                      static_cast<const unsigned char*>(d->projection_values),
                      d->projection_count * int64_t(elem))) != YE3T_OK) {
    ye3t_hip_factorized_angular_plan_destroy(p);
    return rc;
  }
  *out = p;
  return YE3T_OK;
}

int ye3t_hip_factorized_angular_plan_info(const ye3t_hip_factorized_angular_plan* p, int64_t* info) {
  clear_error();
  YE3T_REQUIRE(p && info, "NULL argument");
  const int64_t v[7] = {p->dtype, p->source_dimension, p->input_dimension, p->workspace_dimension,
                        p->output_dimension, p->projection_dimension, p->root_dimension};
  std::memcpy(info, v, sizeof(v));
  return YE3T_OK;
}

}  // extern "C"

namespace ye3t {
namespace {

template <typename T>
int fa_launch(const ye3t_hip_factorized_angular_plan* p, int op, const void* packed, const void* gout,
              const void* weight, const void* bias, int64_t batch, void* out, hipStream_t s) {
  const FATables t = fa_tables(p);
  const int copies = op == 1 || op == 3 ? 2 : 1;
  const int spw = fa_samples_per_wave(p, copies);
  if (spw == 0)
    return set_error(YE3T_EUNSUPPORTED, "a workspace of %lld values does not fit 64 KB of LDS for one sample",
                     (long long)p->workspace_dimension);
  const int64_t grid = (batch + spw - 1) / spw;
  YE3T_REQUIRE(grid <= int64_t(0x7FFFFFFF), "batch too large for one launch");
  const size_t lds = size_t(p->workspace_dimension) * sizeof(T) * size_t(copies) * size_t(spw);
  const T* coef = static_cast<const T*>(p->coef_values);
  const T* proj = static_cast<const T*>(p->projection);
  if (op == 0) {
    hipLaunchKernelGGL(fa_forward_kernel<T>, dim3(unsigned(grid)), dim3(64), lds, s, t, coef, proj,
                       static_cast<const T*>(packed), batch, spw, static_cast<T*>(out));
  } else if (op == 1) {
    hipLaunchKernelGGL((fa_adjoint_kernel<T, false>), dim3(unsigned(grid)), dim3(64), lds, s, t, coef, proj,
                       static_cast<const T*>(packed), static_cast<const T*>(gout), static_cast<const T*>(nullptr),
                       batch, spw, static_cast<T*>(out));
  } else if (op == 2) {
    hipLaunchKernelGGL(fa_linear_kernel<T>, dim3(unsigned(grid)), dim3(64), lds, s, t, coef, proj,
                       static_cast<const T*>(packed), static_cast<const T*>(weight), *static_cast<const T*>(bias),
                       batch, spw, static_cast<T*>(out));
  } else {
    hipLaunchKernelGGL((fa_adjoint_kernel<T, true>), dim3(unsigned(grid)), dim3(64), lds, s, t, coef, proj,
                       static_cast<const T*>(packed), static_cast<const T*>(gout), static_cast<const T*>(weight),
                       batch, spw, static_cast<T*>(out));
  }
  return check_launch("factorized_angular");
}

int fa_dispatch(const ye3t_hip_factorized_angular_plan* p, int op, const void* packed, const void* gout,
                const void* weight, const void* bias, int64_t batch, void* out, ye3t_stream_t stream) {
  int dev = 0;
  YE3T_CHECK_HIP(hipGetDevice(&dev));
  YE3T_REQUIRE(dev == p->device, "call on the plan's device");
  const hipStream_t s = as_stream(stream);
  switch (p->dtype) {
    case YE3T_F32: return fa_launch<float>(p, op, packed, gout, weight, bias, batch, out, s);
    case YE3T_F64: return fa_launch<double>(p, op, packed, gout, weight, bias, batch, out, s);
    case YE3T_C64: return fa_launch<cpx<float>>(p, op, packed, gout, weight, bias, batch, out, s);
    case YE3T_C128: return fa_launch<cpx<double>>(p, op, packed, gout, weight, bias, batch, out, s);
    default: return set_error(YE3T_EDTYPE, "unsupported dtype %d", p->dtype);
  }
}

template <typename T>
void fa_params(const void* F, const void* g, int64_t batch, int64_t K, void* gw, void* gb, hipStream_t s) {
  hipLaunchKernelGGL(fa_readout_params_kernel<T>, dim3(unsigned((K + 1 + 63) / 64)), dim3(64), 0, s,
                     static_cast<const T*>(F), static_cast<const T*>(g), batch, K, static_cast<T*>(gw),
                     static_cast<T*>(gb));
}

}  // namespace
}  // namespace ye3t

extern "C" {

int ye3t_hip_factorized_angular_forward(const ye3t_hip_factorized_angular_plan* p, const void* packed_slots,
                                        int64_t batch, void* output, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(batch >= 0, "negative batch");
  if (batch == 0) return YE3T_OK;
  YE3T_REQUIRE(packed_slots && output, "NULL input or output");
  return fa_dispatch(p, 0, packed_slots, nullptr, nullptr, nullptr, batch, output, stream);
}

int ye3t_hip_factorized_angular_adjoint(const ye3t_hip_factorized_angular_plan* p, const void* output_adjoint,
                                        const void* packed_slots, int64_t batch, void* packed_slots_adjoint,
                                        ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(batch >= 0, "negative batch");
  if (batch == 0) return YE3T_OK;
  YE3T_REQUIRE(output_adjoint && packed_slots && packed_slots_adjoint, "NULL argument");
  return fa_dispatch(p, 1, packed_slots, output_adjoint, nullptr, nullptr, batch, packed_slots_adjoint, stream);
}

int ye3t_hip_factorized_angular_linear_forward(const ye3t_hip_factorized_angular_plan* p, const void* packed_slots,
                                               int64_t batch, const void* weight, const void* bias, void* output,
                                               ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(batch >= 0, "negative batch");
  if (batch == 0) return YE3T_OK;
  YE3T_REQUIRE(packed_slots && weight && bias && output, "NULL argument");
  return fa_dispatch(p, 2, packed_slots, nullptr, weight, bias, batch, output, stream);
}

int ye3t_hip_factorized_angular_linear_adjoint(const ye3t_hip_factorized_angular_plan* p,
                                               const void* output_adjoint, const void* packed_slots, int64_t batch,
                                               const void* weight, void* features, void* packed_slots_adjoint,
                                               void* weight_adjoint, void* bias_adjoint, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(batch >= 0, "negative batch");
  YE3T_REQUIRE(output_adjoint || batch == 0, "NULL output adjoint");
  YE3T_REQUIRE(packed_slots_adjoint || batch == 0, "NULL slot adjoint");
  YE3T_REQUIRE(weight && weight_adjoint && bias_adjoint && (features || batch == 0), "NULL argument");
  int rc = YE3T_OK;
  if (batch > 0) {
    if ((rc = fa_dispatch(p, 3, packed_slots, output_adjoint, weight, nullptr, batch, packed_slots_adjoint,
                          stream)) != YE3T_OK)
      return rc;
    if ((rc = fa_dispatch(p, 0, packed_slots, nullptr, nullptr, nullptr, batch, features, stream)) != YE3T_OK)
      return rc;
  }
  const hipStream_t s = as_stream(stream);
  const int64_t K = p->output_dimension;
  switch (p->dtype) {
    case YE3T_F32: fa_params<float>(features, output_adjoint, batch, K, weight_adjoint, bias_adjoint, s); break;
    case YE3T_F64: fa_params<double>(features, output_adjoint, batch, K, weight_adjoint, bias_adjoint, s); break;
    case YE3T_C64: fa_params<cpx<float>>(features, output_adjoint, batch, K, weight_adjoint, bias_adjoint, s); break;
    case YE3T_C128:
      fa_params<cpx<double>>(features, output_adjoint, batch, K, weight_adjoint, bias_adjoint, s);
      break;
    default: return set_error(YE3T_EDTYPE, "unsupported dtype %d", p->dtype);
  }
  return check_launch("fa_readout_params_kernel");
}

}  // extern "C"
