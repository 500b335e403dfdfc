// Stage 1 on the matrix cores (fp32): the two dense channel-mixing products of
// the density,
//   radial mix  R_c(e)  = sum_n mix[c, n] g_n(e)            [edges x n]  x [n x C]
//   density     A[c,lm] = sum_{e in atom} w_c(e) Y_lm(e)     [C x edges]  x [edges x lm]
// run as v_mfma_f32_16x16x4f32 tiles (full fp32 products, fp32 accumulation).
//
// Operand layout of v_mfma_f32_16x16x4f32 (64 lanes, l = lane):
//   A[i][k]: lane l supplies A[l % 16][l / 16]
//   B[k][j]: lane l supplies B[l / 16][l % 16]
//   D[i][j]: lane l holds D[4 (l / 16) + v][l % 16], v = 0..3
//
// A workgroup (4 waves) owns `apb` consecutive atoms; their edges are staged in
// tiles of up to 256 (one per thread for the per-edge basis).  Rows of the
// output are r = c (node-feature weights with radial mix, one radial row) or
// r = n (single channel, one row per radial index).
#include <cstdlib>

#include "common.h"
#include "sph.h"

namespace ye3t {

typedef float mfma_f4 __attribute__((ext_vector_type(4)));

constexpr int kMfmaThreads = 256;

struct MfmaDensityParams {
  int64_t N;
  const int64_t* __restrict__ offsets;
  const int64_t* __restrict__ nbr;
  const float* __restrict__ vec;
  const float* __restrict__ feats;  // [N, C] (weighted mode) or NULL
  const float* __restrict__ mix;    // [C, NR] (weighted mode) or NULL
  int C;                            // channels (weighted mode) or 1
  int n_max;
  int lmax;
  int apb;
  int tile;
  // padded extents / LDS strides (floats)
  int NRp, gs;    // radial columns padded to 4; G row stride
  int LWp, ys;    // SH columns padded to 16; Y row stride
  int Cp, ws;     // output rows padded to 16; weight row stride
  int hs;         // feature row stride
  double cutoff, lambda, eps;
  float* __restrict__ A;
};

// WEIGHTED: rows are channels c with w_c(e) = h[nbr_e, c] * sum_n mix[c,n] g_n(e).
// otherwise: single channel, rows are radial indices n with w_n(e) = g_n(e).
template <bool WEIGHTED>
__global__ __launch_bounds__(kMfmaThreads) void ace_density_mfma_kernel(MfmaDensityParams p, NormTable nt) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int T = p.tile;
  const int NR = p.n_max + 1;
  const int LW = (p.lmax + 1) * (p.lmax + 1);
  const int R = WEIGHTED ? p.C : NR;  // output rows
  float* G = reinterpret_cast<float*>(smem_raw);  // [T][gs]   radial basis g_n
  float* Y = G + T * p.gs;                        // [T][ys]   real SH
  float* Wt = Y + T * p.ys;                       // [T][ws]   weights w_r (WEIGHTED)
  float* H = Wt + (WEIGHTED ? T * p.ws : 0);      // [T][hs]   neighbour features (WEIGHTED)
  float* M = H + (WEIGHTED ? T * p.hs : 0);       // [NRp][Cp] mix transposed (WEIGHTED)
  __shared__ int64_t atom_lo[64 + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15, lk = lane >> 4;
  const int row_elems = R * LW;
  const int64_t a0 = int64_t(blockIdx.x) * p.apb;
  if (a0 >= p.N) return;
  const int na = int((p.N - a0) < p.apb ? (p.N - a0) : p.apb);
  if (tid <= na) atom_lo[tid] = p.offsets[a0 + tid];
  if (WEIGHTED) {
    for (int q = tid; q < p.NRp * p.Cp; q += kMfmaThreads) {
      const int n = q / p.Cp, c = q - n * p.Cp;
      M[q] = (n < NR && c < p.C) ? p.mix[c * NR + n] : 0.f;
    }
  }
  __syncthreads();
  const int64_t e_begin = atom_lo[0], e_end = atom_lo[na];
  float* Ablk = p.A + a0 * int64_t(row_elems);
  for (int a = 0; a < na; ++a) {
    if (atom_lo[a + 1] == atom_lo[a]) {
      for (int k = tid; k < row_elems; k += kMfmaThreads) Ablk[int64_t(a) * row_elems + k] = 0.f;
    }
  }
  const int rtiles = p.Cp / 16;
  const int ltiles = p.LWp / 16;

  for (int64_t t0 = e_begin; t0 < e_end; t0 += T) {
    const int cnt = int((e_end - t0) < T ? (e_end - t0) : T);
    // ---- phase 1: per-edge basis (one edge per thread), zero padding ----
    if (tid < T) {
      const int j = tid;
      float* grow = G + j * p.gs;
      float* yrow = Y + j * p.ys;
      if (j < cnt) {
        const int64_t e = t0 + j;
        // per-edge basis in fp64 (stored fp32): B is cubic in A, so the 2e-5
        // fp32 budget on B leaves no room for fp32 SH / radial rounding
        const double x = double(p.vec[3 * e]), y = double(p.vec[3 * e + 1]), z = double(p.vec[3 * e + 2]);
        const double r = sqrt(x * x + y * y + z * z);
        const double sr = r > p.eps ? r : p.eps;
        const double inv = 1.0 / sr;
        real_sph_row<double, float>(x * inv, y * inv, z * inv, p.lmax, nt, yrow, 1);
        cheb_exp_cos_row<double, false, float>(r, p.cutoff, p.lambda, p.n_max, grow, nullptr);
        if (WEIGHTED) {
          const float* hrow = p.feats + p.nbr[e] * p.C;
          float* hdst = H + j * p.hs;
          for (int c = 0; c < p.C; ++c) hdst[c] = hrow[c];
        }
      } else {
        for (int k = 0; k < LW; ++k) yrow[k] = 0.f;
        for (int n = 0; n < NR; ++n) grow[n] = 0.f;
      }
      for (int k = LW; k < p.LWp; ++k) yrow[k] = 0.f;
      for (int n = NR; n < p.NRp; ++n) grow[n] = 0.f;
    }
    __syncthreads();
    // ---- phase 1b: w_c(e) = h_c * (g(e) . mix_c) as [16 edges x 16 c] MFMA tiles ----
    if (WEIGHTED) {
      const int etiles = (cnt + 15) / 16;
      for (int t = wave; t < etiles * rtiles; t += kMfmaThreads / 64) {
        const int et = t / rtiles, ct = t - (t / rtiles) * rtiles;
        mfma_f4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int kb = 0; kb < p.NRp; kb += 16) {
          float av[4], bv[4];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int k = kb + 4 * s + lk;
            av[s] = (k < p.NRp) ? G[(et * 16 + li) * p.gs + k] : 0.f;
            bv[s] = (k < p.NRp) ? M[k * p.Cp + ct * 16 + li] : 0.f;
          }
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            if (kb + 4 * s < p.NRp) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s], bv[s], acc, 0, 0, 0);
          }
        }
        const int c = ct * 16 + li;
        for (int v = 0; v < 4; ++v) {
          const int j = et * 16 + 4 * lk + v;
          const float h = (j < cnt && c < p.C) ? H[j * p.hs + c] : 0.f;
          Wt[j * p.ws + c] = h * acc[v];
        }
      }
      // rows j in [cnt, 16*etiles) were written above with weight 0
      __syncthreads();
    }
    // ---- phase 2: per atom, A[r, lm] = sum_e w_r(e) Y_lm(e) as [16 r x 16 lm] tiles ----
    const int tasks = na * rtiles * ltiles;
    for (int t = wave; t < tasks; t += kMfmaThreads / 64) {
      const int a = t / (rtiles * ltiles);
      const int rem = t - a * (rtiles * ltiles);
      const int rt = rem / ltiles, lt = rem - (rem / ltiles) * ltiles;
      const int64_t lo = atom_lo[a], hi = atom_lo[a + 1];
      const int64_t j0 = lo > t0 ? lo : t0;
      const int64_t j1 = hi < t0 + cnt ? hi : t0 + cnt;
      if (j0 >= j1) continue;
      const int jb = int(j0 - t0), je = int(j1 - t0);
      mfma_f4 acc = {0.f, 0.f, 0.f, 0.f};
      const int r_op = rt * 16 + li;
      const int y_op = lt * 16 + li;
      // operands of up to 8 k-steps (32 edges) are loaded before the MFMA chain
      for (int kb = jb; kb < je; kb += 32) {
        float av[8], bv[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int j = kb + 4 * s + lk;
          const bool in = j < je;
          av[s] = in ? (WEIGHTED ? Wt[j * p.ws + r_op] : ((r_op < NR) ? G[j * p.gs + r_op] : 0.f)) : 0.f;
          bv[s] = in ? Y[j * p.ys + y_op] : 0.f;
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          if (kb + 4 * s < je) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s], bv[s], acc, 0, 0, 0);
        }
      }
      const int lm = lt * 16 + li;
      for (int v = 0; v < 4; ++v) {
        const int r = rt * 16 + 4 * lk + v;
        if (r < R && lm < LW) {
          float* dst = Ablk + int64_t(a) * row_elems + int64_t(r) * LW + lm;
          if (lo >= t0) {
            *dst = acc[v];
          } else {
            *dst = *dst + acc[v];
          }
        }
      }
    }
    __syncthreads();
  }
}

static int env_flag_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return (v && *v) ? std::atoi(v) : fallback;
}

// Returns YE3T_EUNSUPPORTED (without launching) when the MFMA path does not
// apply, so the caller can use the VALU kernel.
int launch_density_mfma(const ye3t_density_args* a, void* A, hipStream_t stream) {
  if (a->dtype != YE3T_F32 || a->species) return YE3T_EUNSUPPORTED;
  if (env_flag_int("YE3T_DENSITY_MFMA", 1) == 0) return YE3T_EUNSUPPORTED;
  const bool weighted = a->node_features != nullptr;
  MfmaDensityParams p;
  p.N = a->atom_count;
  p.offsets = a->row_offsets;
  p.nbr = a->neighbors;
  p.vec = static_cast<const float*>(a->edge_vectors);
  p.feats = static_cast<const float*>(a->node_features);
  p.mix = static_cast<const float*>(a->radial_mix);
  p.C = weighted ? int(a->channel_count) : 1;
  if (!weighted && a->channel_count != 1) return YE3T_EUNSUPPORTED;
  p.n_max = int(a->max_radial_index);
  p.lmax = int(a->max_angular);
  const int NR = p.n_max + 1;
  const int LW = (p.lmax + 1) * (p.lmax + 1);
  const int R = weighted ? p.C : NR;
  p.NRp = (NR + 3) / 4 * 4;
  p.gs = p.NRp + 1;                      // odd: per-lane row writes spread over banks
  p.LWp = (LW + 15) / 16 * 16;
  p.ys = p.LWp + ((17 - p.LWp % 64) + 64) % 64;  // == 17 mod 64: per-lane row writes and
                                                 // 4-row operand reads both spread over banks
  p.Cp = (R + 15) / 16 * 16;
  p.ws = (p.Cp % 64 == 0) ? p.Cp + 16 : p.Cp;
  p.hs = p.C | 1;
  p.cutoff = a->cutoff;
  p.lambda = a->lambda;
  p.eps = a->epsilon;
  p.A = static_cast<float*>(A);
  const size_t fixed = weighted ? sizeof(float) * size_t(p.NRp) * p.Cp : 0;
  const size_t per_edge = sizeof(float) * size_t(p.gs + p.ys + (weighted ? p.ws + p.hs : 0));
  // about 40 KiB of LDS per workgroup: four workgroups (16 waves) per CU
  int tile = int((40 * 1024 - fixed) / per_edge) / 64 * 64;
  if (tile > kMfmaThreads) tile = kMfmaThreads;
  if (tile < 64) return YE3T_EUNSUPPORTED;
  p.tile = tile;
  const double mean_degree = a->atom_count ? double(a->edge_count) / double(a->atom_count) : 1.0;
  int apb = int(double(tile) / (mean_degree > 1.0 ? mean_degree : 1.0));
  if (apb < 1) apb = 1;
  if (apb > 64) apb = 64;
  p.apb = apb;
  const size_t lds = per_edge * size_t(tile) + fixed;
  const int64_t grid = (p.N + apb - 1) / apb;
  if (grid > 0x7FFFFFFF) return set_error(YE3T_EUNSUPPORTED, "too many atoms for one launch");
  if (weighted) {
    hipLaunchKernelGGL(ace_density_mfma_kernel<true>, dim3(unsigned(grid)), dim3(kMfmaThreads), lds, stream, p,
                       norm_table());
  } else {
    hipLaunchKernelGGL(ace_density_mfma_kernel<false>, dim3(unsigned(grid)), dim3(kMfmaThreads), lds, stream, p,
                       norm_table());
  }
  set_density_kernel("ace_density_mfma_kernel");
  return check_launch("ace_density_mfma_kernel");
}

}  // namespace ye3t
