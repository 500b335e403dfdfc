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
#include "common.h"
#include "sph.h"

namespace ye3t {

constexpr int kDensityThreads = 256;
constexpr int kEdgeTile = 256;

template <typename Real>
struct DensityParams {
  int64_t N;
  const int64_t* __restrict__ offsets;
  const int64_t* __restrict__ nbr;
  const Real* __restrict__ vec;
  const int32_t* __restrict__ species;
  const Real* __restrict__ feats;
  const Real* __restrict__ mix;
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

// MODE 0: one channel, weight 1.  MODE 1: one-hot species channels.
// MODE 2: node-feature weights with per-channel radial mix (one radial row).
template <typename Real, int MODE>
__global__ __launch_bounds__(kDensityThreads) void ace_density_kernel(DensityParams<Real> p, NormTable nt) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int LW = (p.lmax + 1) * (p.lmax + 1);
  const int NR = p.n_max + 1;
  const int rows = (MODE == 2) ? 1 : NR;
  const int RS = (MODE == 2) ? p.C : NR;
  const int T = p.tile;
  Real* Ys = reinterpret_cast<Real*>(smem_raw);  // [T][LW]
  Real* Rs = Ys + T * LW;                        // [T][RS]
  Real* Rt = Rs + T * RS;                        // [T][NR] raw radials (MODE 2)
  int* Sp = reinterpret_cast<int*>(Rt + (MODE == 2 ? T * NR : 0));  // [T] species (MODE 1)
  __shared__ int64_t atom_lo[64 + 1];

  const int tid = threadIdx.x;
  const int row_elems = p.C * rows * LW;
  const int64_t a0 = int64_t(blockIdx.x) * p.apb;
  if (a0 >= p.N) return;
  const int na = int((p.N - a0) < p.apb ? (p.N - a0) : p.apb);
  if (tid <= na) atom_lo[tid] = p.offsets[a0 + tid];
  __syncthreads();
  const int64_t e_begin = atom_lo[0], e_end = atom_lo[na];
  const int items = na * row_elems;
  Real* Ablk = p.A + a0 * int64_t(row_elems);

  // atoms without any edge still get their zero row
  for (int k = tid; k < items; k += kDensityThreads) {
    const int a = k / row_elems;
    if (atom_lo[a + 1] == atom_lo[a]) Ablk[k] = Real(0);
  }

  for (int64_t t0 = e_begin; t0 < e_end; t0 += T) {
    const int cnt = int((e_end - t0) < T ? (e_end - t0) : T);
    if (tid < cnt) {
      const int j = tid;
      const int64_t e = t0 + j;
      const double x = double(p.vec[3 * e]), y = double(p.vec[3 * e + 1]), z = double(p.vec[3 * e + 2]);
      const double r = sqrt(x * x + y * y + z * z);
      const double sr = r > p.eps ? r : p.eps;
      const double inv = 1.0 / sr;
      real_sph_row<double, Real>(x * inv, y * inv, z * inv, p.lmax, nt, Ys + j * LW, 1);
      if (MODE == 2) {
        cheb_exp_cos_row<double, false, Real>(r, p.cutoff, p.lambda, p.n_max, Rt + j * NR, nullptr);
      } else {
        cheb_exp_cos_row<double, false, Real>(r, p.cutoff, p.lambda, p.n_max, Rs + j * NR, nullptr);
      }
      if (MODE == 1) Sp[j] = p.species[p.nbr[e]];
    }
    __syncthreads();
    if (MODE == 2) {
      for (int q = tid; q < cnt * p.C; q += kDensityThreads) {
        const int j = q / p.C, c = q - (q / p.C) * p.C;
        const int64_t nb = p.nbr[t0 + j];
        Real rc = Real(0);
        for (int n = 0; n < NR; ++n) rc = d_fma(p.mix[c * NR + n], Rt[j * NR + n], rc);
        Rs[j * p.C + c] = p.feats[nb * p.C + c] * rc;
      }
      __syncthreads();
    }
    for (int k = tid; k < items; k += kDensityThreads) {
      const int a = k / row_elems;
      const int64_t lo = atom_lo[a], hi = atom_lo[a + 1];
      const int64_t j0 = lo > t0 ? lo : t0;
      const int64_t j1 = hi < t0 + cnt ? hi : t0 + cnt;
      if (j0 >= j1) continue;  // this atom has no edge in the tile
      const int rem = k - a * row_elems;
      const int lm = rem % LW;
      const int cr = rem / LW;  // c * rows + r
      const int c = cr / rows;
      const int rr = cr - c * rows;
      Real acc = (lo >= t0) ? Real(0) : Ablk[k];  // first tile of this atom starts from zero
      const int jb = int(j0 - t0), je = int(j1 - t0);
      if (MODE == 0) {
        for (int j = jb; j < je; ++j) acc = d_fma(Rs[j * NR + rr], Ys[j * LW + lm], acc);
      } else if (MODE == 1) {
        for (int j = jb; j < je; ++j) {
          if (Sp[j] == c) acc = d_fma(Rs[j * NR + rr], Ys[j * LW + lm], acc);
        }
      } else {
        for (int j = jb; j < je; ++j) acc = d_fma(Rs[j * p.C + c], Ys[j * LW + lm], acc);
      }
      Ablk[k] = acc;
    }
    __syncthreads();
  }
}

template <typename Real, int MODE>
int launch_density(const ye3t_density_args* a, void* A, hipStream_t stream) {
  DensityParams<Real> p;
  p.N = a->atom_count;
  p.offsets = a->row_offsets;
  p.nbr = a->neighbors;
  p.vec = static_cast<const Real*>(a->edge_vectors);
  p.species = a->species;
  p.feats = static_cast<const Real*>(a->node_features);
  p.mix = static_cast<const Real*>(a->radial_mix);
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
  const size_t per_edge = sizeof(Real) * size_t(LW + RS + (MODE == 2 ? NR : 0)) + (MODE == 1 ? sizeof(int) : 0);
  int tile = int((60 * 1024) / per_edge) / 64 * 64;
  if (tile > kEdgeTile) tile = kEdgeTile;
  if (tile < 64) return set_error(YE3T_EUNSUPPORTED, "density row too wide for one LDS tile (%zu B/edge)", per_edge);
  p.tile = tile;
  // atoms per block from the mean degree: about one edge tile per block
  const double mean_degree = a->atom_count ? double(a->edge_count) / double(a->atom_count) : 1.0;
  int apb = int(double(tile) / (mean_degree > 1.0 ? mean_degree : 1.0));
  if (apb < 1) apb = 1;
  if (apb > 64) apb = 64;
  p.apb = apb;
  const size_t lds = per_edge * size_t(tile);
  const int64_t grid = (p.N + apb - 1) / apb;
  if (grid > 0x7FFFFFFF) return set_error(YE3T_EUNSUPPORTED, "too many atoms for one launch");
  hipLaunchKernelGGL((ace_density_kernel<Real, MODE>), dim3(unsigned(grid)), dim3(kDensityThreads), lds, stream, p,
                     norm_table());
  return check_launch("ace_density_kernel");
}

template <typename Real>
int dispatch_density(const ye3t_density_args* a, void* A, hipStream_t s) {
  if (a->node_features) return launch_density<Real, 2>(a, A, s);
  if (a->species) return launch_density<Real, 1>(a, A, s);
  return launch_density<Real, 0>(a, A, s);
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
  if (a->dtype == YE3T_F64) return dispatch_density<double>(a, A, as_stream(stream));
  if (a->dtype == YE3T_F32) return dispatch_density<float>(a, A, as_stream(stream));
  return set_error(YE3T_EDTYPE, "unsupported dtype %d", a->dtype);
}
