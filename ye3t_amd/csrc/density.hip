// Stage 1 -- fused neighbour-density accumulation on gfx950.
//
//   A[i, c, r, lm] = sum_{e in row i} w_c(e) R_r(|v_e|) Y_lm(v_e / |v_e|)
//
// A workgroup of 256 threads owns `apb` consecutive atoms (apb ~ 256 / degree),
// so the segment reduction over their CSR edge ranges needs no atomics and the
// result is bit-reproducible.  Edges of those atoms are processed in tiles of
// up to 256 (one edge per thread):
//   phase 1  each thread evaluates the radial basis and real SH of its edge in
//            registers (fp64 for both storage types) and stages them in LDS;
//   phase 1b (node-feature weights) HW[j][c] = h[nbr_j, c] * sum_n mix[c, n] R_n(j);
//   phase 2  each thread owns output elements (atom, c, r, lm) and sums over
//            that atom's edges of the tile; consecutive threads take
//            consecutive lm, so the A row store is coalesced.
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "sph.h"

namespace ye3t {

constexpr int kDensityThreads = 256;
constexpr int kEdgeTile = 256;

// Real: accumulation and A storage type; In: storage type of the inputs.
template <typename Real, typename In>
struct DensityParams {
  int64_t N;
  const int64_t* __restrict__ offsets;
  const int64_t* __restrict__ nbr;
  const In* __restrict__ vec;
  const int32_t* __restrict__ species;
  const In* __restrict__ feats;
  const In* __restrict__ mix;
  int C;
  int n_max;
  int lmax;
  int apb;   // atoms per block
  int tile;  // edges per LDS tile (<= kEdgeTile)
  double cutoff;
  double lambda;
  double eps;
  Real* __restrict__ A;
};

// LDS row stride (elements) of the SH tile: a multiple of the vector width,
// odd in vector units so per-lane row writes spread over the banks.
template <typename Real>
inline __host__ __device__ int ys_stride(int LW) {
  constexpr int VN = 16 / int(sizeof(Real));
  int vecs = (LW + VN - 1) / VN;
  if (vecs % 2 == 0) vecs += 1;
  return vecs * VN;
}

template <typename Real>
struct Vec;
template <>
struct Vec<float> {
  using T = float4;
  static constexpr int N = 4;
};
template <>
struct Vec<double> {
  using T = double2;
  static constexpr int N = 2;
};

// MODE 0: one channel, weight 1.  MODE 1: one-hot species channels.
// MODE 2: node-feature weights with per-channel radial mix (one radial row).
template <typename Real, int MODE, typename BasisT, typename In>
__global__ __launch_bounds__(kDensityThreads) void ace_density_kernel(DensityParams<Real, In> p, NormTable nt) {
  using V = typename Vec<Real>::T;
  constexpr int VN = Vec<Real>::N;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int LW = (p.lmax + 1) * (p.lmax + 1);
  const int LWp = (LW + VN - 1) / VN * VN;  // lm values per SH row, padded to a 16-byte multiple
  const int YS = ys_stride<Real>(LW);        // LDS row stride of the SH tile (bank spread)
  const int HC = p.C | 1;                    // odd row stride of the feature tile
  const int NR = p.n_max + 1;
  const int rows = (MODE == 2) ? 1 : NR;
  const int RS = (MODE == 2) ? p.C : NR;
  const int T = p.tile;
  Real* Ys = reinterpret_cast<Real*>(smem_raw);  // [T][YS]
  Real* Rs = Ys + T * YS;                        // [T][RS]
  Real* Rt = Rs + T * RS;                        // [T][NR] raw radials (MODE 2)
  int* Sp = reinterpret_cast<int*>(Rt + (MODE == 2 ? T * NR : 0));  // [T] species (MODE 1)
  Real* Hs = Rt + (MODE == 2 ? T * NR : 0);                          // [T][HC] neighbour features (MODE 2)
  Real* Mx = Hs + (MODE == 2 ? T * HC : 0);                          // [C][NR] radial mix (MODE 2)
  __shared__ int64_t atom_lo[64 + 1];

  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int row_elems = p.C * rows * LW;
  const int groups = LWp / VN;
  const int ipa = p.C * rows * groups;  // vector items per atom
  const int64_t a0 = int64_t(blockIdx.x) * p.apb;
  if (a0 >= p.N) return;
  const int na = int((p.N - a0) < p.apb ? (p.N - a0) : p.apb);
  if (tid <= na) atom_lo[tid] = p.offsets[a0 + tid];
  if (MODE == 2) {
    for (int q = tid; q < p.C * NR; q += nthreads) Mx[q] = Real(p.mix[q]);
  }
  __syncthreads();
  const int64_t e_begin = atom_lo[0], e_end = atom_lo[na];
  Real* Ablk = p.A + a0 * int64_t(row_elems);

  // atoms without any edge still get their zero row
  for (int a = 0; a < na; ++a) {
    if (atom_lo[a + 1] == atom_lo[a]) {
      for (int k = tid; k < row_elems; k += nthreads) Ablk[int64_t(a) * row_elems + k] = Real(0);
    }
  }

  for (int64_t t0 = e_begin; t0 < e_end; t0 += T) {
    const int cnt = int((e_end - t0) < T ? (e_end - t0) : T);
    if (tid < cnt) {
      const int j = tid;
      const int64_t e = t0 + j;
      const BasisT x = BasisT(p.vec[3 * e]), y = BasisT(p.vec[3 * e + 1]), z = BasisT(p.vec[3 * e + 2]);
      const BasisT r = d_sqrt(x * x + y * y + z * z);
      const BasisT sr = r > BasisT(p.eps) ? r : BasisT(p.eps);
      const BasisT inv = BasisT(1) / sr;
      real_sph_row<BasisT, Real>(x * inv, y * inv, z * inv, p.lmax, nt, Ys + j * YS, 1);
      for (int k = LW; k < LWp; ++k) Ys[j * YS + k] = Real(0);
      // the radial basis is always evaluated in fp64: the Chebyshev recurrence
      // amplifies rounding of the warped variable by ~n^2
      if (MODE == 2) {
        cheb_exp_cos_row<double, false, Real>(double(r), p.cutoff, p.lambda, p.n_max, Rt + j * NR, nullptr);
      } else {
        cheb_exp_cos_row<double, false, Real>(double(r), p.cutoff, p.lambda, p.n_max, Rs + j * NR, nullptr);
      }
      if (MODE == 1) Sp[j] = p.species[p.nbr[e]];
      if (MODE == 2) {
        // gather the neighbour's feature row once (independent loads, one latency)
        const In* hrow = p.feats + p.nbr[e] * p.C;
        Real* hdst = Hs + j * HC;
        for (int c = 0; c < p.C; ++c) hdst[c] = Real(hrow[c]);
      }
    }
    __syncthreads();
    if (MODE == 2) {
      // HW[j][c] = h[nbr_j, c] * sum_n mix[c, n] R_n(j)
      if (nthreads % p.C == 0) {
        const int c = tid % p.C;
        const int jstep = nthreads / p.C;
        const Real* mrow = Mx + c * NR;
        for (int j = tid / p.C; j < cnt; j += jstep) {
          const Real h = Hs[j * HC + c];
          const Real* rrow = Rt + j * NR;
          Real r0 = Real(0), r1 = Real(0);
          int n = 0;
          for (; n + 2 <= NR; n += 2) {
            r0 = d_fma(mrow[n], rrow[n], r0);
            r1 = d_fma(mrow[n + 1], rrow[n + 1], r1);
          }
          if (n < NR) r0 = d_fma(mrow[n], rrow[n], r0);
          Rs[j * p.C + c] = h * (r0 + r1);
        }
      } else {
        for (int q = tid; q < cnt * p.C; q += nthreads) {
          const int j = q / p.C, c = q - (q / p.C) * p.C;
          const Real h = Hs[j * HC + c];
          Real rc = Real(0);
          for (int n = 0; n < NR; ++n) rc = d_fma(Mx[c * NR + n], Rt[j * NR + n], rc);
          Rs[j * p.C + c] = h * rc;
        }
      }
      __syncthreads();
    }
    // phase 2: vector item = (atom, c, r, group of VN consecutive lm).  When the
    // per-atom item count divides the workgroup, each thread keeps one
    // (c, r, group) and strides over atoms (decoded once).
    const bool fixed_rem = (nthreads % ipa) == 0;
    const int a_first = fixed_rem ? tid / ipa : 0;
    const int a_step = fixed_rem ? nthreads / ipa : 1;
    for (int it = fixed_rem ? tid % ipa : tid; it < (fixed_rem ? ipa : na * ipa);
         it += fixed_rem ? ipa : nthreads) {
      const int a_gen = fixed_rem ? 0 : it / ipa;
      const int rem = fixed_rem ? it : it - a_gen * ipa;
      const int g = rem % groups;
      const int cr = rem / groups;  // c * rows + r
      const int c = cr / rows;
      const int rr = cr - c * rows;
      const Real* rcol = (MODE == 2) ? (Rs + c) : (Rs + rr);
      const V* ycol = reinterpret_cast<const V*>(Ys + g * VN);
      const int ystride = YS / VN;
      const int valid = (LW - g * VN) < VN ? (LW - g * VN) : VN;
      for (int a = fixed_rem ? a_first : a_gen; a < na; a += fixed_rem ? a_step : na) {
        const int64_t lo = atom_lo[a], hi = atom_lo[a + 1];
        const int64_t j0 = lo > t0 ? lo : t0;
        const int64_t j1 = hi < t0 + cnt ? hi : t0 + cnt;
        if (j0 >= j1) continue;  // this atom has no edge in the tile
        const int jb = int(j0 - t0), je = int(j1 - t0);
        Real acc[VN], acc2[VN];
        for (int v = 0; v < VN; ++v) {
          acc[v] = Real(0);
          acc2[v] = Real(0);
        }
        int j = jb;
        for (; j + 2 <= je; j += 2) {
          const V y0 = ycol[j * ystride];
          const V y1 = ycol[(j + 1) * ystride];
          Real w0 = rcol[j * RS], w1 = rcol[(j + 1) * RS];
          if (MODE == 1) {
            w0 = Sp[j] == c ? w0 : Real(0);
            w1 = Sp[j + 1] == c ? w1 : Real(0);
          }
          const Real* y0p = reinterpret_cast<const Real*>(&y0);
          const Real* y1p = reinterpret_cast<const Real*>(&y1);
          for (int v = 0; v < VN; ++v) {
            acc[v] = d_fma(w0, y0p[v], acc[v]);
            acc2[v] = d_fma(w1, y1p[v], acc2[v]);
          }
        }
        if (j < je) {
          const V y0 = ycol[j * ystride];
          Real w0 = rcol[j * RS];
          if (MODE == 1) w0 = Sp[j] == c ? w0 : Real(0);
          const Real* y0p = reinterpret_cast<const Real*>(&y0);
          for (int v = 0; v < VN; ++v) acc[v] = d_fma(w0, y0p[v], acc[v]);
        }
        Real* dst = Ablk + int64_t(a) * row_elems + int64_t(cr) * LW + g * VN;
        for (int v = 0; v < VN; ++v) {
          if (v < valid) {
            const Real part = acc[v] + acc2[v];
            // the first tile holding this atom's edges starts from zero
            if (lo >= t0) {
              dst[v] = part;
            } else {
              dst[v] = dst[v] + part;
            }
          }
        }
      }
    }
    __syncthreads();
  }
}

template <typename Real, int MODE, typename BasisT, typename In>
int launch_density(const ye3t_density_args* a, void* A, hipStream_t stream, int nthreads) {
  DensityParams<Real, In> p;
  p.N = a->atom_count;
  p.offsets = a->row_offsets;
  p.nbr = a->neighbors;
  p.vec = static_cast<const In*>(a->edge_vectors);
  p.species = a->species;
  p.feats = static_cast<const In*>(a->node_features);
  p.mix = static_cast<const In*>(a->radial_mix);
  p.C = int(a->channel_count);
  p.n_max = int(a->max_radial_index);
  p.lmax = int(a->max_angular);
  p.cutoff = a->cutoff;
  p.lambda = a->lambda;
  p.eps = a->epsilon;
  p.A = static_cast<Real*>(A);
  const int LW = (p.lmax + 1) * (p.lmax + 1);
  const int NR = p.n_max + 1;
  const int RS = (MODE == 2) ? p.C : NR;
  // edge tile: as many edges as fit in 60 KiB of LDS, a multiple of 64, <= 256
  const int YS = ys_stride<Real>(LW);
  const size_t per_edge = sizeof(Real) * size_t(YS + RS + (MODE == 2 ? NR + (p.C | 1) : 0)) + (MODE == 1 ? sizeof(int) : 0);
  const size_t fixed = (MODE == 2) ? sizeof(Real) * size_t(p.C) * NR : 0;
  if (fixed > 16 * 1024) return set_error(YE3T_EUNSUPPORTED, "radial mix table too large for LDS");
  int tile = int((60 * 1024 - fixed) / per_edge) / 64 * 64;
  if (tile > nthreads) tile = nthreads;
  if (tile < 64) return set_error(YE3T_EUNSUPPORTED, "density row too wide for one LDS tile (%zu B/edge)", per_edge);
  p.tile = tile;
  // atoms per block from the mean degree: about one edge tile per block
  const double mean_degree = a->atom_count ? double(a->edge_count) / double(a->atom_count) : 1.0;
  int apb = int(double(tile) / (mean_degree > 1.0 ? mean_degree : 1.0));
  if (apb < 1) apb = 1;
  if (apb > 64) apb = 64;
  p.apb = apb;
  const size_t lds = per_edge * size_t(tile) + (MODE == 2 ? sizeof(Real) * size_t(p.C) * NR : 0);
  const int64_t grid = (p.N + apb - 1) / apb;
  if (grid > 0x7FFFFFFF) return set_error(YE3T_EUNSUPPORTED, "too many atoms for one launch");
  hipLaunchKernelGGL((ace_density_kernel<Real, MODE, BasisT, In>), dim3(unsigned(grid)), dim3(nthreads), lds, stream,
                     p, norm_table());
  set_density_kernel("ace_density_kernel");
  return check_launch("ace_density_kernel");
}

// Launch knobs (tuning, like the reference's YE3T_* policy variables):
//   YE3T_DENSITY_THREADS  workgroup size, 64..256 in steps of 64 (default 256)
//   YE3T_DENSITY_SH_FP32  1: evaluate the real SH of fp32 runs in fp32 (default: fp64)
inline int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return (v && *v) ? std::atoi(v) : fallback;
}

template <typename Real, int MODE, typename In>
int launch_mode(const ye3t_density_args* a, void* A, hipStream_t s) {
  int threads = env_int("YE3T_DENSITY_THREADS", 256);
  if (threads < 64 || threads > 256 || threads % 64) threads = 256;
  if (std::is_same<Real, float>::value && env_int("YE3T_DENSITY_SH_FP32", 0) == 1) {
    return launch_density<Real, MODE, float, In>(a, A, s, threads);
  }
  return launch_density<Real, MODE, double, In>(a, A, s, threads);
}

int launch_density_mfma(const ye3t_density_args* a, void* A, hipStream_t stream);
template <typename In, typename Out>
int launch_density_mfma64(const ye3t_density_args* a, void* A, hipStream_t stream);
template <typename In, typename Out>
int launch_density_species(const ye3t_density_args* a, void* A, hipStream_t stream);

template <typename Real, typename In>
int dispatch_density(const ye3t_density_args* a, void* A, hipStream_t s) {
  // one-hot species: each (atom, species) group of edges on the fp64 matrix
  // cores (YE3T_DENSITY_SPECIES_MFMA=0 selects the VALU kernel)
  if (a->species && env_int("YE3T_DENSITY_SPECIES_MFMA", 1) != 0) {
    const int rc = launch_density_species<In, Real>(a, A, s);
    if (rc != YE3T_EUNSUPPORTED) return rc;
    clear_error();
  }
  if (std::is_same<Real, float>::value) {
    // fp32 single-channel and node-feature densities run on the matrix cores
    const int rc = launch_density_mfma(a, A, s);
    if (rc != YE3T_EUNSUPPORTED) return rc;
    clear_error();
  } else {
    // so do fp64 densities of the compiled shapes (fp64 MFMA)
    const int rc = launch_density_mfma64<In, double>(a, A, s);
    if (rc != YE3T_EUNSUPPORTED) return rc;
    clear_error();
  }
  if (a->node_features) return launch_mode<Real, 2, In>(a, A, s);
  if (a->species) return launch_mode<Real, 1, In>(a, A, s);
  return launch_mode<Real, 0, In>(a, A, s);
}

}  // namespace ye3t

using namespace ye3t;

extern "C" int ye3t_hip_ace_density_forward(const ye3t_density_args* a, void* A, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(a != nullptr, "NULL args");
  YE3T_REQUIRE(a->atom_count >= 0 && a->edge_count >= 0, "negative size");
  YE3T_REQUIRE(a->channel_count >= 1, "channel_count must be >= 1");
  YE3T_REQUIRE(a->max_radial_index >= 0 && a->max_radial_index < 16, "max_radial_index must be in [0, 15]");
  YE3T_REQUIRE(a->max_angular >= 0 && a->max_angular <= 8, "max_angular must be in [0, 8]");
  YE3T_REQUIRE(!(a->species && a->node_features), "species and node_features are exclusive");
  YE3T_REQUIRE(a->node_features == nullptr || a->radial_mix != nullptr, "node_features need radial_mix");
  YE3T_REQUIRE(a->species != nullptr || a->node_features != nullptr || a->channel_count == 1,
               "channel_count > 1 needs species or node_features");
  YE3T_REQUIRE(!a->species || a->channel_count <= 64, "at most 64 species channels");
  if (a->atom_count == 0) return YE3T_OK;
  YE3T_REQUIRE(a->row_offsets && A, "NULL row_offsets or output");
  YE3T_REQUIRE(a->edge_count == 0 || (a->edge_vectors && (a->neighbors || (!a->species && !a->node_features))),
               "NULL edge arrays");
  const int out_dtype = a->out_dtype < 0 ? a->dtype : a->out_dtype;
  const int acc_dtype = a->accumulate_dtype < 0 ? out_dtype : a->accumulate_dtype;
  if (acc_dtype == out_dtype) {
    if (a->dtype == YE3T_F64 && out_dtype == YE3T_F64) return dispatch_density<double, double>(a, A, as_stream(stream));
    if (a->dtype == YE3T_F32 && out_dtype == YE3T_F32) return dispatch_density<float, float>(a, A, as_stream(stream));
    if (a->dtype == YE3T_F32 && out_dtype == YE3T_F64) return dispatch_density<double, float>(a, A, as_stream(stream));
  } else if (a->dtype == YE3T_F32 && out_dtype == YE3T_F32 && acc_dtype == YE3T_F64) {
    // fp64 accumulation rounded once to an fp32 density: the fp64 matrix-core kernels
    const int rc = a->species ? launch_density_species<float, float>(a, A, as_stream(stream))
                              : launch_density_mfma64<float, float>(a, A, as_stream(stream));
    if (rc != YE3T_EUNSUPPORTED) return rc;
    return set_error(YE3T_EUNSUPPORTED,
                     "an fp32 density accumulated in fp64 is built for the fp64 matrix-core shapes only "
                     "(node features at 16 channels, n_max 8, l_max 3; single channel at (3, 8), (4, 10), (6, 12); "
                     "up to 16 species with n_max <= 15, l_max <= 8)");
  }
  return set_error(YE3T_EDTYPE, "unsupported dtype combination (inputs %d, density %d, accumulation %d)", a->dtype,
                   out_dtype, acc_dtype);
}
