// Stage 1 -- fused neighbour-density accumulation on gfx950.
//
//   A[i, c, r, lm] = sum_{e in row i} w_c(e) R_r(|v_e|) Y_lm(v_e / |v_e|)
//
// One workgroup (256 threads = 4 waves) owns one atom at a time, so the
// segment reduction over its CSR edge range needs no atomics and the result is
// bit-reproducible.  Per tile of up to 64 edges:
//   phase 1  wave 0 computes radial basis and real SH of each edge in
//            registers and stages them in LDS (Y[j][lm], R[j][r]); for one-hot
//            species it also builds per-species edge lists with ballots;
//   phase 1b (node-feature weights) all threads form HW[j][c] = h[nbr_j, c] * R_c(j);
//   phase 2  every thread owns output elements (c, r, lm) -- consecutive
//            threads take consecutive lm, so the A row store is coalesced.
#include "common.h"
#include "sph.h"

namespace ye3t {

constexpr int kTile = 64;
constexpr int kDensityThreads = 256;

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
  Real cutoff;
  Real lambda;
  Real eps;
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
  const int RS = (MODE == 2) ? p.C : NR;  // radial/weight stride per edge in LDS
  Real* Ys = reinterpret_cast<Real*>(smem_raw);  // [kTile][LW]
  Real* Rs = Ys + kTile * LW;                    // [kTile][RS]
  Real* Rt = Rs + kTile * RS;                    // [kTile][NR] raw radials (MODE 2)
  int* lists = reinterpret_cast<int*>(Rt + (MODE == 2 ? kTile * NR : 0));  // [C][kTile] (MODE 1)
  int* counts = lists + (MODE == 1 ? p.C * kTile : 0);                    // [C]
  const int tid = threadIdx.x;
  const int row_elems = p.C * rows * LW;

  for (int64_t atom = blockIdx.x; atom < p.N; atom += gridDim.x) {
    const int64_t e0 = p.offsets[atom], e1 = p.offsets[atom + 1];
    Real* Arow = p.A + atom * int64_t(row_elems);
    if (e1 <= e0) {
      for (int k = tid; k < row_elems; k += kDensityThreads) Arow[k] = Real(0);
      continue;
    }
    bool first = true;
    for (int64_t t0 = e0; t0 < e1; t0 += kTile) {
      const int cnt = int((e1 - t0) < kTile ? (e1 - t0) : kTile);
      if (tid < kTile) {
        const int j = tid;
        int sp = -1;
        if (j < cnt) {
          const int64_t e = t0 + j;
          const Real x = p.vec[3 * e], y = p.vec[3 * e + 1], z = p.vec[3 * e + 2];
          const Real r = d_sqrt(x * x + y * y + z * z);
          const Real sr = r > p.eps ? r : p.eps;
          real_sph_row<Real>(x / sr, y / sr, z / sr, p.lmax, nt, Ys + j * LW, 1);
          Real rad[16];
          cheb_exp_cos_row<Real, false>(r, p.cutoff, p.lambda, p.n_max, rad, nullptr);
          if (MODE == 2) {
            for (int n = 0; n < NR; ++n) Rt[j * NR + n] = rad[n];
          } else {
            for (int n = 0; n < NR; ++n) Rs[j * NR + n] = rad[n];
          }
          if (MODE == 1) sp = p.species[p.nbr[e]];
        }
        if (MODE == 1) {
          // stable per-species edge lists (tile = one wave of 64 lanes)
          const uint64_t lt = (j == 0) ? 0ull : (~0ull >> (64 - j));
          for (int c = 0; c < p.C; ++c) {
            const uint64_t mask = __ballot(sp == c);
            if (sp == c) lists[c * kTile + __popcll(mask & lt)] = j;
            if (j == 0) counts[c] = __popcll(mask);
          }
        }
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
      for (int k = tid; k < row_elems; k += kDensityThreads) {
        const int lm = k % LW;
        const int cr = k / LW;  // c * rows + r
        const int c = cr / rows;
        const int r = cr - c * rows;
        Real acc = first ? Real(0) : Arow[k];
        if (MODE == 0) {
          for (int j = 0; j < cnt; ++j) acc = d_fma(Rs[j * NR + r], Ys[j * LW + lm], acc);
        } else if (MODE == 1) {
          const int n_c = counts[c];
          for (int q = 0; q < n_c; ++q) {
            const int j = lists[c * kTile + q];
            acc = d_fma(Rs[j * NR + r], Ys[j * LW + lm], acc);
          }
        } else {
          for (int j = 0; j < cnt; ++j) acc = d_fma(Rs[j * p.C + c], Ys[j * LW + lm], acc);
        }
        Arow[k] = acc;
      }
      first = false;
      __syncthreads();
    }
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
  p.cutoff = Real(a->cutoff);
  p.lambda = Real(a->lambda);
  p.eps = Real(a->epsilon);
  p.A = static_cast<Real*>(A);
  const int LW = (p.lmax + 1) * (p.lmax + 1);
  const int NR = p.n_max + 1;
  const int RS = (MODE == 2) ? p.C : NR;
  size_t lds = sizeof(Real) * size_t(kTile) * (LW + RS + (MODE == 2 ? NR : 0));
  if (MODE == 1) lds += sizeof(int) * size_t(p.C) * (kTile + 1);
  if (lds > 64 * 1024) {
    return set_error(YE3T_EUNSUPPORTED, "density tile needs %zu bytes of LDS (limit 65536)", lds);
  }
  int64_t grid = p.N;
  if (grid > (1 << 20)) grid = 1 << 20;
  if (grid < 1) grid = 1;
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
