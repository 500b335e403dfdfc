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

// One or more DAGs ("segments") over disjoint column ranges of the packed
// input and of the output row.  The single-DAG op is the one-segment case.
struct ye3t_hip_factorized_angular_plan {
  int dtype;
  int device;
  int64_t segment_count;
  int64_t node_count, coef_count, root_count;
  // the single-DAG op's dimensions (segment 0 for a segmented plan)
  int64_t source_dimension, input_dimension, workspace_dimension, output_dimension, projection_dimension;
  int64_t root_dimension;
  // segmented: packed row width, output row width, total sources, sum of S * W
  int64_t packed_dimension, total_output_dimension, total_source_count, total_workspace;
  int64_t max_workspace;  // widest segment workspace (sets samples per wave)
  int32_t* ints;          // every int32 device table, one allocation
  void* coef_values;
  void* projection;
  void* tables;           // device FATables[segment_count]
};

struct ye3t_hip_factorized_angular_segmented_plan {
  ye3t_hip_factorized_angular_plan base;
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

// The tables of one DAG (segment) as the kernels read them: node and root
// slices of the concatenated int32 tables, and where the DAG's columns sit in
// the packed input row, the output row and the projection values.
struct FATables {
  const int32_t* node_offsets;   // workspace slot of each node (segment-local)
  const int32_t* node_dims;
  const int32_t* node_leaf;      // input column of a leaf within one source, -1 for merges
  const int32_t* node_coef_off;  // coefficient range of node n: [node_coef_off[n], node_coef_off[n + 1])
  const int32_t* coef_left;      // per coefficient: workspace slot of the left factor
  const int32_t* coef_right;     // ... of the right factor
  const int32_t* coef_col;       // ... of the destination
  const int32_t* roots;          // root node indices (segment-local)
  const int32_t* root_ps;        // per root: first projection column
  const int32_t* root_pd;        // per root: projection column count
  const int32_t* root_oo;        // per root: offset of its block in the segment's output
  int node_count, root_count, source_dim, input_dim, ws_dim;
  int proj_dim, proj_off;        // this DAG's [source_dim x proj_dim] block of the projection values
  int in_off, in_stride;         // packed row: this DAG's first column, row width
  int out_off, out_stride, out_dim;  // output row: first column, row width, this DAG's width
};

// a wave-uniform table entry, read through the constant address space (a
// scalar load: the tables are read-only for the kernel's lifetime)
__device__ inline int at(const int32_t* table, int i) { return ((sgpr_i32)(const void*)table)[i]; }

// the block's segment: blockIdx.y indexes the plan's device table array (a
// read-only kernel argument at a wave-uniform index: scalar loads)
__device__ inline FATables segment_tables(const FATables* __restrict__ tabs) { return tabs[blockIdx.y]; }

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
__global__ __launch_bounds__(64) void fa_forward_kernel(const FATables* __restrict__ tabs,
                                                        const T* __restrict__ coef, const T* __restrict__ proj_all,
                                                        const T* __restrict__ packed, int64_t batch, int spw,
                                                        T* __restrict__ out) {
  typedef Ops<T> O;
  extern __shared__ __align__(16) unsigned char fa_smem[];
  const FATables t = segment_tables(tabs);
  const int lane = threadIdx.x;
  if (lane >= spw) return;
  const int64_t b = int64_t(blockIdx.x) * spw + lane;
  if (b >= batch) return;
  const T* proj = proj_all + t.proj_off;
  T* ws = reinterpret_cast<T*>(fa_smem) + lane;
  T* orow = out + b * t.out_stride + t.out_off;
  for (int k = 0; k < t.out_dim; ++k) orow[k] = O::zero();
  for (int s = 0; s < t.source_dim; ++s) {
    const T* in = packed + b * t.in_stride + t.in_off + s * t.input_dim;
    fa_replay(t, coef, in, ws, spw);
    for (int r = 0; r < t.root_count; ++r) {
      const int rn = at(t.roots, r);
      const int roff = at(t.node_offsets, rn), rd = at(t.node_dims, rn);
      const int ps = at(t.root_ps, r), pd = at(t.root_pd, r);
      T* blk0 = orow + at(t.root_oo, r);
      for (int p = 0; p < pd; ++p) {
        const T pv = proj[s * t.proj_dim + ps + p];
        T* blk = blk0 + p * rd;
        for (int m = 0; m < rd; ++m) blk[m] = O::add(blk[m], O::mul(ws[(roff + m) * spw], pv));
      }
    }
  }
}

// Reverse mode.  LINEAR: the output adjoint of feature k of sample b is
// g[b] * conj(weight[k]) (the linear readout's adjoint), else gout[b, k].
template <typename T, bool LINEAR>
__global__ __launch_bounds__(64) void fa_adjoint_kernel(const FATables* __restrict__ tabs,
                                                        const T* __restrict__ coef, const T* __restrict__ proj_all,
                                                        const T* __restrict__ packed, const T* __restrict__ gout,
                                                        const T* __restrict__ weight, int64_t batch, int spw,
                                                        T* __restrict__ gpacked) {
  typedef Ops<T> O;
  extern __shared__ __align__(16) unsigned char fa_smem[];
  const FATables t = segment_tables(tabs);
  const int lane = threadIdx.x;
  if (lane >= spw) return;
  const int64_t b = int64_t(blockIdx.x) * spw + lane;
  if (b >= batch) return;
  const T* proj = proj_all + t.proj_off;
  T* ws = reinterpret_cast<T*>(fa_smem) + lane;
  T* wa = reinterpret_cast<T*>(fa_smem) + int64_t(t.ws_dim) * spw + lane;
  T* grow = gpacked + b * t.in_stride + t.in_off;
  for (int k = 0; k < t.source_dim * t.input_dim; ++k) grow[k] = O::zero();
  const T gl = LINEAR ? gout[b] : O::zero();
  const T* grow_out = LINEAR ? nullptr : gout + b * t.out_stride + t.out_off;
  for (int s = 0; s < t.source_dim; ++s) {
    const T* in = packed + b * t.in_stride + t.in_off + s * t.input_dim;
    fa_replay(t, coef, in, ws, spw);
    for (int q = 0; q < t.ws_dim; ++q) wa[q * spw] = O::zero();
    for (int r = 0; r < t.root_count; ++r) {
      const int rn = at(t.roots, r);
      const int roff = at(t.node_offsets, rn), rd = at(t.node_dims, rn);
      const int ps = at(t.root_ps, r), pd = at(t.root_pd, r), oo = at(t.root_oo, r);
      for (int p = 0; p < pd; ++p) {
        const T cpv = O::conj(proj[s * t.proj_dim + ps + p]);
        const int f0 = oo + p * rd;
        for (int m = 0; m < rd; ++m) {
          const T g = LINEAR ? O::mul(gl, O::conj(weight[f0 + m])) : grow_out[f0 + m];
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
__global__ __launch_bounds__(64) void fa_linear_kernel(const FATables* __restrict__ tabs, const T* __restrict__ coef,
                                                       const T* __restrict__ proj_all, const T* __restrict__ packed,
                                                       const T* __restrict__ weight, T bias, int64_t batch, int spw,
                                                       T* __restrict__ out) {
  typedef Ops<T> O;
  extern __shared__ __align__(16) unsigned char fa_smem[];
  const FATables t = segment_tables(tabs);
  const int lane = threadIdx.x;
  if (lane >= spw) return;
  const int64_t b = int64_t(blockIdx.x) * spw + lane;
  if (b >= batch) return;
  const T* proj = proj_all + t.proj_off;
  T* ws = reinterpret_cast<T*>(fa_smem) + lane;
  T value = bias;
  for (int s = 0; s < t.source_dim; ++s) {
    const T* in = packed + b * t.in_stride + t.in_off + s * t.input_dim;
    fa_replay(t, coef, in, ws, spw);
    for (int r = 0; r < t.root_count; ++r) {
      const int rn = at(t.roots, r);
      const int roff = at(t.node_offsets, rn), rd = at(t.node_dims, rn);
      const int ps = at(t.root_ps, r), pd = at(t.root_pd, r), oo = at(t.root_oo, r);
      for (int p = 0; p < pd; ++p) {
        const T pv = proj[s * t.proj_dim + ps + p];
        const int f0 = oo + p * rd;
        for (int m = 0; m < rd; ++m)
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
  const size_t per = size_t(p->max_workspace) * fa_elem(p->dtype) * size_t(copies);
  for (int spw = 64; spw >= 1; spw /= 2)
    if (per * size_t(spw) <= 64 * 1024) return spw;
  return 0;
}

// Host view of one or more DAGs in the reference segmented op's layout:
// node and root indices local to their segment, coefficient ranges global.
struct FASegView {
  int64_t segment_count;
  const int64_t *seg_src_off, *seg_in_off, *seg_in_dim, *seg_ws_off, *seg_ws_dim, *seg_node_off, *seg_root_off;
  const int64_t *seg_proj_off, *seg_proj_dim, *seg_out_off;
  int64_t node_count;
  const int64_t *node_offsets, *node_dims, *node_leaf, *node_left, *node_right, *node_coef_off;
  int64_t coef_count;
  const int64_t *rows, *cols;
  int64_t root_count;
  const int64_t *roots, *root_ps, *root_pd, *root_oo;
  int64_t proj_count;
  int64_t packed_dim, total_sources, workspace, out_dim;
};

// The reference segmented op's checks (execution_plan_torch.cpp:434-726) and
// every index the kernels use, so the kernels index without checks.  The
// single-DAG op does not require children to precede their parent (its
// reference checks, execution_plan_torch.cpp:5930-5990, do not), only that
// they are nodes of the DAG.
int fa_validate(const FASegView& v, bool children_precede) {
  const int64_t K = v.segment_count, N = v.node_count, E = v.coef_count, R = v.root_count;
  YE3T_REQUIRE(K > 0, "segmented plan requires segments");
  YE3T_REQUIRE(K <= 65535, "at most 65535 segments in one launch");
  YE3T_REQUIRE(N > 0, "segmented plan requires nodes");
  YE3T_REQUIRE(R > 0, "segmented plan requires roots");
  YE3T_REQUIRE(E >= 0 && v.proj_count > 0, "segmented plan requires coefficients and projection values");
  YE3T_REQUIRE(N < (int64_t(1) << 30) && E < (int64_t(1) << 30) && R < (int64_t(1) << 30), "table too large");
  YE3T_REQUIRE(v.seg_src_off[0] == 0 && v.seg_node_off[0] == 0 && v.seg_root_off[0] == 0 && v.seg_out_off[0] == 0,
               "segmented boundary offsets must start at zero");
  YE3T_REQUIRE(v.node_coef_off[0] >= 0, "segmented coefficient interval is invalid");
  int64_t in_cursor = 0, ws_cursor = 0, proj_cursor = 0;
  std::vector<std::pair<int64_t, int64_t>> intervals;
  for (int64_t k = 0; k < K; ++k) {
    const int64_t S = v.seg_src_off[k + 1] - v.seg_src_off[k], D = v.seg_in_dim[k], W = v.seg_ws_dim[k];
    const int64_t P = v.seg_proj_dim[k];
    const int64_t n0 = v.seg_node_off[k], nk = v.seg_node_off[k + 1] - n0;
    const int64_t r0 = v.seg_root_off[k], rk = v.seg_root_off[k + 1] - r0;
    const int64_t out_k = v.seg_out_off[k + 1] - v.seg_out_off[k];
    YE3T_REQUIRE(S > 0 && D > 0 && W > 0 && P > 0 && nk > 0 && rk > 0 && out_k > 0,
                 "segmented plan dimensions must be positive");
    YE3T_REQUIRE(n0 + nk <= N && r0 + rk <= R, "segmented node/root offsets do not cover metadata");
    YE3T_REQUIRE(v.seg_in_off[k] == in_cursor, "segmented input intervals must exactly partition packed input");
    YE3T_REQUIRE(v.seg_ws_off[k] == ws_cursor, "segmented workspace intervals must exactly partition workspace");
    YE3T_REQUIRE(v.seg_proj_off[k] == proj_cursor,
                 "segmented projection intervals must exactly partition coefficients");
    in_cursor += S * D;
    ws_cursor += S * W;
    proj_cursor += S * P;
    for (int64_t j = 0; j < nk; ++j) {
      const int64_t n = n0 + j, off = v.node_offsets[n], dim = v.node_dims[n];
      YE3T_REQUIRE(dim > 0 && off >= 0 && off + dim <= W, "segmented node interval is outside its workspace");
      YE3T_REQUIRE(v.node_coef_off[n] <= v.node_coef_off[n + 1] && v.node_coef_off[n + 1] <= E,
                   "segmented coefficient interval is invalid");
      const int64_t leaf = v.node_leaf[n];
      if (leaf >= 0) {
        YE3T_REQUIRE(leaf + dim <= D, "segmented leaf interval is outside its input");
        continue;
      }
      const int64_t l = v.node_left[n], r = v.node_right[n];
      if (children_precede)
        YE3T_REQUIRE(l >= 0 && l < j && r >= 0 && r < j, "segmented merge children must precede their parent");
      else
        YE3T_REQUIRE(l >= 0 && l < nk && r >= 0 && r < nk, "node %lld has an out-of-range child", (long long)n);
      const int64_t ld = v.node_dims[n0 + l], rd = v.node_dims[n0 + r];
      for (int64_t e = v.node_coef_off[n]; e < v.node_coef_off[n + 1]; ++e) {
        YE3T_REQUIRE(v.rows[e] >= 0 && v.rows[e] < ld * rd, "coefficient row %lld out of range", (long long)e);
        YE3T_REQUIRE(v.cols[e] >= 0 && v.cols[e] < dim, "coefficient column %lld out of range", (long long)e);
      }
    }
    intervals.clear();
    for (int64_t j = 0; j < rk; ++j) {
      const int64_t r = r0 + j;
      YE3T_REQUIRE(v.roots[r] >= 0 && v.roots[r] < nk, "segmented root index is outside its local node range");
      YE3T_REQUIRE(v.root_ps[r] >= 0 && v.root_pd[r] > 0 && v.root_ps[r] + v.root_pd[r] <= P,
                   "segmented root projection interval is invalid");
      const int64_t block = v.root_pd[r] * v.node_dims[n0 + v.roots[r]];
      YE3T_REQUIRE(v.root_oo[r] >= 0 && v.root_oo[r] + block <= out_k, "segmented root output interval is invalid");
      intervals.emplace_back(v.root_oo[r], v.root_oo[r] + block);
    }
    std::sort(intervals.begin(), intervals.end());
    int64_t cursor = 0;
    for (const auto& iv : intervals) {
      YE3T_REQUIRE(iv.first == cursor, "segmented root outputs must exactly partition each destination");
      cursor = iv.second;
    }
    YE3T_REQUIRE(cursor == out_k, "segmented root outputs must cover each destination");
  }
  YE3T_REQUIRE(v.seg_src_off[K] == v.total_sources, "total_source_count does not match segmented source offsets");
  YE3T_REQUIRE(v.seg_node_off[K] == N && v.seg_root_off[K] == R, "segmented node/root offsets do not cover metadata");
  YE3T_REQUIRE(in_cursor == v.packed_dim, "segmented input intervals do not cover packed input");
  YE3T_REQUIRE(ws_cursor == v.workspace, "segmented workspace intervals do not match workspace dimension");
  YE3T_REQUIRE(proj_cursor == v.proj_count, "segmented projection intervals do not cover projection values");
  YE3T_REQUIRE(v.seg_out_off[K] == v.out_dim, "segmented output intervals do not match output dimension");
  YE3T_REQUIRE(v.node_coef_off[N] == E, "segmented coefficient offsets do not cover coefficients");
  YE3T_REQUIRE(v.packed_dim < (int64_t(1) << 31) && v.out_dim < (int64_t(1) << 31) &&
                   v.proj_count < (int64_t(1) << 31),
               "packed rows too wide");
  return YE3T_OK;
}

template <typename T>
int fa_upload(T** dst, const T* src, int64_t n) {
  *dst = nullptr;
  if (n <= 0) return YE3T_OK;
  YE3T_CHECK_HIP(hipMalloc(reinterpret_cast<void**>(dst), size_t(n) * sizeof(T)));
  YE3T_CHECK_HIP(hipMemcpy(*dst, src, size_t(n) * sizeof(T), hipMemcpyHostToDevice));
  return YE3T_OK;
}

// frees a plan's device tables (not the plan object)
void fa_release(ye3t_hip_factorized_angular_plan* p) {
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(p->device);
  for (void* q : {(void*)p->ints, p->coef_values, p->projection, p->tables})
    if (q) (void)hipFree(q);
  (void)hipSetDevice(prev);
  p->ints = nullptr;
  p->coef_values = p->projection = p->tables = nullptr;
}

// Device tables of a validated view into *p: one int32 allocation holding
// [node_offsets | node_dims | node_leaf | node_coef_off (N + 1) | coef_left |
//  coef_right | coef_col | roots | root_ps | root_pd | root_oo], the values,
// and one FATables per segment pointing into it.  On failure p holds no
// device memory.
int fa_build(const FASegView& v, int dtype, const void* coef_values, const void* projection_values,
             ye3t_hip_factorized_angular_plan* p) {
  const size_t elem = fa_elem(dtype);
  const int64_t N = v.node_count, E = v.coef_count, R = v.root_count;
  const int64_t o_noff = 0, o_ndim = N, o_leaf = 2 * N, o_coef = 3 * N, o_cl = 4 * N + 1, o_cr = o_cl + E,
                o_cc = o_cr + E, o_roots = o_cc + E, o_ps = o_roots + R, o_pd = o_ps + R, o_oo = o_pd + R,
                total = o_oo + R;
  std::vector<int32_t> h(size_t(total), 0);
  for (int64_t n = 0; n < N; ++n) {
    h[o_noff + n] = int32_t(v.node_offsets[n]);
    h[o_ndim + n] = int32_t(v.node_dims[n]);
    h[o_leaf + n] = int32_t(v.node_leaf[n] >= 0 ? v.node_leaf[n] : -1);
    h[o_coef + n] = int32_t(v.node_coef_off[n]);
  }
  h[o_coef + N] = int32_t(v.node_coef_off[N]);
  for (int64_t k = 0; k < v.segment_count; ++k) {
    const int64_t n0 = v.seg_node_off[k];
    for (int64_t n = n0; n < v.seg_node_off[k + 1]; ++n) {
      if (v.node_leaf[n] >= 0) continue;
      const int64_t l = n0 + v.node_left[n], r = n0 + v.node_right[n], rd = v.node_dims[r];
      for (int64_t e = v.node_coef_off[n]; e < v.node_coef_off[n + 1]; ++e) {
        h[o_cl + e] = int32_t(v.node_offsets[l] + v.rows[e] / rd);
        h[o_cr + e] = int32_t(v.node_offsets[r] + v.rows[e] % rd);
        h[o_cc + e] = int32_t(v.node_offsets[n] + v.cols[e]);
      }
    }
  }
  for (int64_t r = 0; r < R; ++r) {
    h[o_roots + r] = int32_t(v.roots[r]);
    h[o_ps + r] = int32_t(v.root_ps[r]);
    h[o_pd + r] = int32_t(v.root_pd[r]);
    h[o_oo + r] = int32_t(v.root_oo[r]);
  }
  std::memset(p, 0, sizeof(*p));
  p->dtype = dtype;
  (void)hipGetDevice(&p->device);
  p->segment_count = v.segment_count;
  p->node_count = N;
  p->coef_count = E;
  p->root_count = R;
  p->packed_dimension = v.packed_dim;
  p->total_output_dimension = v.out_dim;
  p->total_source_count = v.total_sources;
  p->total_workspace = v.workspace;
  int rc = YE3T_OK;
  if ((rc = fa_upload(&p->ints, h.data(), total)) != YE3T_OK ||
      (rc = fa_upload(reinterpret_cast<unsigned char**>(&p->coef_values),
                      static_cast<const unsigned char*>(coef_values), E * int64_t(elem))) != YE3T_OK ||
      (rc = fa_upload(reinterpret_cast<unsigned char**>(&p->projection),
                      static_cast<const unsigned char*>(projection_values), v.proj_count * int64_t(elem))) !=
          YE3T_OK) {
    fa_release(p);
    return rc;
  }
  std::vector<FATables> tabs(size_t(v.segment_count));
  for (int64_t k = 0; k < v.segment_count; ++k) {
    const int64_t n0 = v.seg_node_off[k], r0 = v.seg_root_off[k];
    FATables& t = tabs[size_t(k)];
    t.node_offsets = p->ints + o_noff + n0;
    t.node_dims = p->ints + o_ndim + n0;
    t.node_leaf = p->ints + o_leaf + n0;
    t.node_coef_off = p->ints + o_coef + n0;
    t.coef_left = p->ints + o_cl;
    t.coef_right = p->ints + o_cr;
    t.coef_col = p->ints + o_cc;
    t.roots = p->ints + o_roots + r0;
    t.root_ps = p->ints + o_ps + r0;
    t.root_pd = p->ints + o_pd + r0;
    t.root_oo = p->ints + o_oo + r0;
    t.node_count = int(v.seg_node_off[k + 1] - n0);
    t.root_count = int(v.seg_root_off[k + 1] - r0);
    t.source_dim = int(v.seg_src_off[k + 1] - v.seg_src_off[k]);
    t.input_dim = int(v.seg_in_dim[k]);
    t.ws_dim = int(v.seg_ws_dim[k]);
    t.proj_dim = int(v.seg_proj_dim[k]);
    t.proj_off = int(v.seg_proj_off[k]);
    t.in_off = int(v.seg_in_off[k]);
    t.in_stride = int(v.packed_dim);
    t.out_off = int(v.seg_out_off[k]);
    t.out_stride = int(v.out_dim);
    t.out_dim = int(v.seg_out_off[k + 1] - v.seg_out_off[k]);
    p->max_workspace = std::max<int64_t>(p->max_workspace, t.ws_dim);
  }
  if ((rc = fa_upload(reinterpret_cast<FATables**>(&p->tables), tabs.data(), v.segment_count)) != YE3T_OK) {
    fa_release(p);
    return rc;
  }
  return YE3T_OK;
}

}  // namespace
}  // namespace ye3t

using namespace ye3t;

extern "C" {

void ye3t_hip_factorized_angular_plan_destroy(ye3t_hip_factorized_angular_plan* p) {
  if (!p) return;
  fa_release(p);
  delete p;
}

int ye3t_hip_factorized_angular_plan_create(const ye3t_factorized_angular_desc* d,
                                            ye3t_hip_factorized_angular_plan** out) {
  clear_error();
  YE3T_REQUIRE(d && out, "NULL description or output");
  *out = nullptr;
  YE3T_REQUIRE(fa_elem(d->dtype) != 0, "unsupported dtype %d", d->dtype);
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
  // one segment with the uniform root metadata (execution_plan_torch.cpp:205-250)
  std::vector<int64_t> ps(static_cast<size_t>(R), 0), pd(static_cast<size_t>(R), P), oo(static_cast<size_t>(R), 0);
  for (int64_t r = 0; r < R; ++r) oo[size_t(r)] = r * P * rdim;
  const int64_t src_off[2] = {0, S}, in_off[1] = {0}, in_dim[1] = {d->input_dimension}, ws_off[1] = {0},
                ws_dim[1] = {W}, node_off[2] = {0, N}, root_off[2] = {0, R}, proj_off[1] = {0}, proj_dim[1] = {P},
                out_off[2] = {0, d->output_dimension};
  FASegView v;
  v.segment_count = 1;
  v.seg_src_off = src_off;
  v.seg_in_off = in_off;
  v.seg_in_dim = in_dim;
  v.seg_ws_off = ws_off;
  v.seg_ws_dim = ws_dim;
  v.seg_node_off = node_off;
  v.seg_root_off = root_off;
  v.seg_proj_off = proj_off;
  v.seg_proj_dim = proj_dim;
  v.seg_out_off = out_off;
  v.node_count = N;
  v.node_offsets = d->node_offsets;
  v.node_dims = d->node_dimensions;
  v.node_leaf = d->node_leaf_offsets;
  v.node_left = d->node_left;
  v.node_right = d->node_right;
  v.node_coef_off = d->node_coefficient_offsets;
  v.coef_count = E;
  v.rows = d->coefficient_rows;
  v.cols = d->coefficient_columns;
  v.root_count = R;
  v.roots = d->root_nodes;
  v.root_ps = ps.data();
  v.root_pd = pd.data();
  v.root_oo = oo.data();
  v.proj_count = d->projection_count;
  v.packed_dim = S * d->input_dimension;
  v.total_sources = S;
  v.workspace = W * S;
  v.out_dim = d->output_dimension;
  int rc = fa_validate(v, false);
  if (rc != YE3T_OK) return rc;
  auto* p = new ye3t_hip_factorized_angular_plan();
  if ((rc = fa_build(v, d->dtype, d->coefficient_values, d->projection_values, p)) != YE3T_OK) {
    delete p;
    return rc;
  }
  p->source_dimension = S;
  p->input_dimension = d->input_dimension;
  p->workspace_dimension = W;
  p->output_dimension = d->output_dimension;
  p->projection_dimension = P;
  p->root_dimension = rdim;
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
  const FATables* tabs = static_cast<const FATables*>(p->tables);
  const int copies = op == 1 || op == 3 ? 2 : 1;
  const int spw = fa_samples_per_wave(p, copies);
  if (spw == 0)
    return set_error(YE3T_EUNSUPPORTED, "a workspace of %lld values does not fit 64 KB of LDS for one sample",
                     (long long)p->max_workspace);
  const int64_t grid = (batch + spw - 1) / spw;
  YE3T_REQUIRE(grid <= int64_t(0x7FFFFFFF), "batch too large for one launch");
  const dim3 blocks(unsigned(grid), unsigned(p->segment_count));
  const size_t lds = size_t(p->max_workspace) * sizeof(T) * size_t(copies) * size_t(spw);
  const T* coef = static_cast<const T*>(p->coef_values);
  const T* proj = static_cast<const T*>(p->projection);
  if (op == 0) {
    hipLaunchKernelGGL(fa_forward_kernel<T>, blocks, dim3(64), lds, s, tabs, coef, proj,
                       static_cast<const T*>(packed), batch, spw, static_cast<T*>(out));
  } else if (op == 1) {
    hipLaunchKernelGGL((fa_adjoint_kernel<T, false>), blocks, dim3(64), lds, s, tabs, coef, proj,
                       static_cast<const T*>(packed), static_cast<const T*>(gout), static_cast<const T*>(nullptr),
                       batch, spw, static_cast<T*>(out));
  } else if (op == 2) {
    hipLaunchKernelGGL(fa_linear_kernel<T>, blocks, dim3(64), lds, s, tabs, coef, proj,
                       static_cast<const T*>(packed), static_cast<const T*>(weight), *static_cast<const T*>(bias),
                       batch, spw, static_cast<T*>(out));
  } else {
    hipLaunchKernelGGL((fa_adjoint_kernel<T, true>), blocks, dim3(64), lds, s, tabs, coef, proj,
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

extern "C" {

void ye3t_hip_factorized_angular_segmented_plan_destroy(ye3t_hip_factorized_angular_segmented_plan* p) {
  if (!p) return;
  fa_release(&p->base);
  delete p;
}

int ye3t_hip_factorized_angular_segmented_plan_create(const ye3t_factorized_angular_segmented_desc* d,
                                                      ye3t_hip_factorized_angular_segmented_plan** out) {
  clear_error();
  YE3T_REQUIRE(d && out, "NULL description or output");
  *out = nullptr;
  YE3T_REQUIRE(fa_elem(d->dtype) != 0, "unsupported dtype %d", d->dtype);
  YE3T_REQUIRE(d->segment_source_offsets && d->segment_input_offsets && d->segment_input_dimensions &&
                   d->segment_workspace_offsets && d->segment_workspace_dimensions && d->segment_node_offsets &&
                   d->segment_root_offsets && d->segment_projection_offsets && d->segment_projection_dimensions &&
                   d->segment_output_offsets && d->node_offsets && d->node_dimensions && d->node_leaf_offsets &&
                   d->node_left && d->node_right && d->node_coefficient_offsets && d->root_nodes &&
                   d->root_projection_starts && d->root_projection_dimensions && d->root_output_offsets &&
                   d->projection_values,
               "NULL table");
  YE3T_REQUIRE(d->coefficient_count >= 0 &&
                   (d->coefficient_count == 0 ||
                    (d->coefficient_rows && d->coefficient_columns && d->coefficient_values)),
               "segmented coefficient arrays must have equal length");
  FASegView v;
  v.segment_count = d->segment_count;
  v.seg_src_off = d->segment_source_offsets;
  v.seg_in_off = d->segment_input_offsets;
  v.seg_in_dim = d->segment_input_dimensions;
  v.seg_ws_off = d->segment_workspace_offsets;
  v.seg_ws_dim = d->segment_workspace_dimensions;
  v.seg_node_off = d->segment_node_offsets;
  v.seg_root_off = d->segment_root_offsets;
  v.seg_proj_off = d->segment_projection_offsets;
  v.seg_proj_dim = d->segment_projection_dimensions;
  v.seg_out_off = d->segment_output_offsets;
  v.node_count = d->node_count;
  v.node_offsets = d->node_offsets;
  v.node_dims = d->node_dimensions;
  v.node_leaf = d->node_leaf_offsets;
  v.node_left = d->node_left;
  v.node_right = d->node_right;
  v.node_coef_off = d->node_coefficient_offsets;
  v.coef_count = d->coefficient_count;
  v.rows = d->coefficient_rows;
  v.cols = d->coefficient_columns;
  v.root_count = d->root_count;
  v.roots = d->root_nodes;
  v.root_ps = d->root_projection_starts;
  v.root_pd = d->root_projection_dimensions;
  v.root_oo = d->root_output_offsets;
  v.proj_count = d->projection_count;
  v.packed_dim = d->packed_input_dimension;
  v.total_sources = d->total_source_count;
  v.workspace = d->workspace_dimension;
  v.out_dim = d->output_dimension;
  int rc = fa_validate(v, true);
  if (rc != YE3T_OK) return rc;
  auto* sp = new ye3t_hip_factorized_angular_segmented_plan();
  if ((rc = fa_build(v, d->dtype, d->coefficient_values, d->projection_values, &sp->base)) != YE3T_OK) {
    delete sp;
    return rc;
  }
  *out = sp;
  return YE3T_OK;
}

int ye3t_hip_factorized_angular_segmented_forward(const ye3t_hip_factorized_angular_segmented_plan* p,
                                                  const void* packed_slots, int64_t batch, void* output,
                                                  ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(batch >= 0, "negative batch");
  if (batch == 0) return YE3T_OK;
  YE3T_REQUIRE(packed_slots && output, "NULL input or output");
  return fa_dispatch(&p->base, 0, packed_slots, nullptr, nullptr, nullptr, batch, output, stream);
}

int ye3t_hip_factorized_angular_segmented_adjoint(const ye3t_hip_factorized_angular_segmented_plan* p,
                                                  const void* output_adjoint, const void* packed_slots, int64_t batch,
                                                  void* packed_slots_adjoint, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(batch >= 0, "negative batch");
  if (batch == 0) return YE3T_OK;
  YE3T_REQUIRE(output_adjoint && packed_slots && packed_slots_adjoint, "NULL argument");
  return fa_dispatch(&p->base, 1, packed_slots, output_adjoint, nullptr, nullptr, batch, packed_slots_adjoint,
                     stream);
}

int ye3t_hip_factorized_angular_segmented_plan_info(const ye3t_hip_factorized_angular_segmented_plan* p,
                                                    int64_t* info) {
  clear_error();
  YE3T_REQUIRE(p && info, "NULL argument");
  const ye3t_hip_factorized_angular_plan& b = p->base;
  const int64_t v[6] = {b.dtype, b.segment_count, b.total_source_count, b.packed_dimension, b.total_workspace,
                        b.total_output_dimension};
  std::memcpy(info, v, sizeof(v));
  return YE3T_OK;
}

}  // extern "C"
