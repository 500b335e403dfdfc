// Stage 1 with an fp64 density on the matrix cores:
//
//   A[i, r, lm] = sum_{e in row i} w_r(e) Y_lm(e)
//
// computed as per-atom [rows x edges] x [edges x lm] products with
// v_mfma_f64_16x16x4f64 (fp64 products and accumulation), so the density is
// exact to fp64 rounding whatever the input storage type.
//
// One wave (one 64-thread workgroup, no block barriers between waves) owns a
// contiguous range of atoms (as many waves as the device holds at once) and streams
// their CSR edge range in chunks of 64, one edge per lane:
//   phase 1  each lane evaluates the radial basis, the real SH and the row
//            weights of its edge in fp64 registers and writes them to LDS
//            transposed ([row][edge], [lm][edge]);
//   phase 2  the wave walks the chunk in k-blocks of 4 edges; each k-block is
//            one MFMA per (row tile, lm tile) for the atom that owns those
//            edges (edges of other atoms masked to zero), alternating between
//            two accumulator sets, and an atom's 16x16 tiles go straight from
//            registers to A when its last edge has been consumed.
// Global loads run one chunk ahead (edge vectors, neighbour feature rows) and
// two chunks ahead (neighbour indices), so no chunk waits on a fresh request.
//
// Operand layout of v_mfma_f64_16x16x4f64 (l = lane):
//   A[i][k]: lane l supplies A[l % 16][l / 16]
//   B[k][j]: lane l supplies B[l / 16][l % 16]
//   D[i][j]: lane l holds D[l / 16 + 4 v][l % 16], v = 0..3
//
// Rows: MODE 0 -- one channel, rows are radial indices n, w_n(e) = g_n(e);
//       MODE 2 -- node features with a per-channel radial mix, rows are
//                 channels c, w_c(e) = h[nbr_e, c] * sum_n mix[c, n] g_n(e).
// MODE 2 at 16 channels, n_max = 8, l_max = 3 runs on its own kernel
// (ace_density_channel16_kernel) that also puts the radial mix on the matrix
// cores and keeps W in registers.
#include <cmath>
#include <cstdlib>

#include "common.h"

// Issue priority of the channel kernel's MFMA phase (phase 1 runs at 0): with
// two waves per SIMD, the wave feeding the matrix core goes first while the
// other fills the gaps with its VALU basis math.
#ifndef YE3T_DENSITY_SETPRIO
#define YE3T_DENSITY_SETPRIO 1
#endif
#include "sph.h"

namespace ye3t {

typedef double mfma_d4 __attribute__((ext_vector_type(4)));

// LDS row pitch (doubles) of the transposed tiles: k-block reads of a partial
// chunk reach edge column cnt + 2 <= 65, and columns 64.. stay zero; 67 is odd,
// so 16 lanes reading one column of 16 rows hit 16 distinct bank pairs
constexpr int kPitch64 = 67;

template <typename In, typename Out>
struct Density64Params {
  int64_t N;
  const int64_t* __restrict__ offsets;
  const int64_t* __restrict__ nbr;
  const In* __restrict__ vec;
  const In* __restrict__ feats;  // [N, C] (MODE 2)
  const In* __restrict__ mix;    // [C, NR] (MODE 2)
  int64_t waves;                 // wave w owns atoms [w N / waves, (w + 1) N / waves)
  double cutoff;                 // max(cutoff, eps of double)
  double lambda;
  double den;                    // expm1(lambda)
  double eps;
  Out* __restrict__ A;           // fp64, or fp32 rounded once from the fp64 accumulators
  // host-side reciprocals of the channel kernel
  double inv_cutoff;             // 1 / cutoff
  double two_over_den;           // 2 / expm1(lambda)
  double inv_eps;                // 1 / eps
  double cutoff_tie;             // 8 ulp(cutoff): distances this close decide liveness exactly
};

// offsets[i] through the constant address space: a scalar load (the CSR
// offsets are read-only for the kernel's lifetime), so it is counted by
// lgkmcnt and never waits for the vector stores of A
__device__ inline int64_t offset_at(const int64_t* offsets, int64_t i) {
  return ((const __attribute__((address_space(4))) int64_t*)(offsets))[i];
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima)
__device__ inline void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ inline int64_t uniform64(int64_t v) {
  const int lo = __builtin_amdgcn_readfirstlane(int(uint32_t(uint64_t(v))));
  const int hi = __builtin_amdgcn_readfirstlane(int(uint32_t(uint64_t(v) >> 32)));
  return int64_t((uint64_t(uint32_t(hi)) << 32) | uint64_t(uint32_t(lo)));
}

__device__ inline int64_t readlane64(int64_t v, int idx) {
  const int lo = __builtin_amdgcn_readlane(int(uint32_t(uint64_t(v))), idx);
  const int hi = __builtin_amdgcn_readlane(int(uint32_t(uint64_t(v) >> 32)), idx);
  return int64_t((uint64_t(uint32_t(hi)) << 32) | uint64_t(uint32_t(lo)));
}

// ChebExpCos radial values g_0..g_NMAX of one distance (the algebra of
// cheb_exp_cos_row with the per-launch constants hoisted), g_n to out[n * stride].
template <int NMAX, typename P>
__device__ inline void radial_row64(double r, const P& p, double* out, int stride) {
  const double s = r / p.cutoff;
  if (s > 1.0) {
#pragma unroll
    for (int n = 0; n <= NMAX; ++n) out[n * stride] = 0.0;
    return;
  }
  const double env = 1.0 + cospi(s);
  out[0] = 1.0;
  if (NMAX >= 1) out[stride] = 0.5 * env;
  if (NMAX >= 2) {
    const double x = 1.0 - 2.0 * expm1(-p.lambda * (s - 1.0)) / p.den;
    double t0 = 1.0, t1 = x;
#pragma unroll
    for (int n = 2; n <= NMAX; ++n) {
      const double t2 = 2.0 * x * t1 - t0;
      out[n * stride] = 0.25 * (1.0 - t2) * env;
      t0 = t1;
      t1 = t2;
    }
  }
}

template <int MODE, typename In, typename Out, int LMAX, int NMAX, int C>
__global__ __launch_bounds__(64) void ace_density_mfma64_kernel(Density64Params<In, Out> p, NormTable nt) {
  constexpr int NR = NMAX + 1;
  constexpr int LW = (LMAX + 1) * (LMAX + 1);
  constexpr int ROWS = MODE == 2 ? C : NR;
  constexpr int RT = (ROWS + 15) / 16;
  constexpr int CT = (LW + 15) / 16;
  constexpr int HC = MODE == 2 ? C : 1;
  __shared__ double Wt[RT * 16 * kPitch64];
  __shared__ double Yt[CT * 16 * kPitch64];
  __shared__ double Mx[MODE == 2 ? C * NR : 1];

  const int lane = threadIdx.x;
  const int kq = lane >> 4, cc = lane & 15;
  const int64_t a_begin = int64_t(blockIdx.x) * p.N / p.waves;
  const int64_t a_end = (int64_t(blockIdx.x) + 1) * p.N / p.waves;
  if (a_begin >= a_end) return;
  // padding rows / columns of the tiles stay zero
  for (int q = lane; q < RT * 16 * kPitch64; q += 64) Wt[q] = 0.0;
  for (int q = lane; q < CT * 16 * kPitch64; q += 64) Yt[q] = 0.0;
  if (MODE == 2) {
    for (int q = lane; q < C * NR; q += 64) Mx[q] = double(p.mix[q]);
  }
  __syncthreads();
  const int64_t e_begin = offset_at(p.offsets, a_begin), e_end = offset_at(p.offsets, a_end);
  Out* __restrict__ Aw = p.A;

  // k-blocks whose operands are read from LDS in one batch
  constexpr int KB = (RT + CT <= 2) ? 16 : ((RT + CT <= 5) ? 8 : 4);
  mfma_d4 acc[2][RT][CT];
  auto zero_acc = [&]() {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[s2][rt][ct] = mfma_d4{0.0, 0.0, 0.0, 0.0};
  };
  zero_acc();
  int64_t a = a_begin;  // current atom (wave-uniform)
  int64_t lo = e_begin, hi = offset_at(p.offsets, a_begin + 1);

  auto store_atom = [&](int64_t atom) {
    Out* __restrict__ dst = Aw + atom * (ROWS * LW);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = rt * 16 + kq + 4 * v, col = ct * 16 + cc;
          if ((ROWS % 16 == 0 || row < ROWS) && (LW % 16 == 0 || col < LW))
            dst[row * LW + col] = Out(acc[0][rt][ct][v] + acc[1][rt][ct][v]);
        }
  };
  auto in_chunk = [&](int64_t t) { return t < e_end && lane < e_end - t; };

  // Software pipeline over 64-edge chunks i: on entry to chunk i the lane holds
  // its edge vector and feature row of chunk i and its neighbour index of
  // chunk i + 1; chunk i + 1's vector and feature row and chunk i + 2's
  // neighbour index are requested before chunk i is computed.
  In vx = In(0), vy = In(0), vz = In(0);
  In h[HC];
  int64_t nb1 = 0;  // neighbour index of chunk i + 1
#pragma unroll
  for (int c = 0; c < HC; ++c) h[c] = In(0);
  if (in_chunk(e_begin)) {
    const int64_t e = e_begin + lane;
    vx = p.vec[3 * e];
    vy = p.vec[3 * e + 1];
    vz = p.vec[3 * e + 2];
    if (MODE == 2) {
      const int64_t nb = p.nbr[e];
#pragma unroll
      for (int c = 0; c < HC; ++c) h[c] = p.feats[nb * C + c];
    }
  }
  if (MODE == 2 && e_begin < e_end) nb1 = p.nbr[(e_begin + 64 + lane) < e_end ? (e_begin + 64 + lane) : (e_end - 1)];

  for (int64_t t0 = e_begin; t0 < e_end; t0 += 64) {
    const int cnt = int((e_end - t0) < 64 ? (e_end - t0) : 64);
    // requests for the following chunks; lanes past the wave's last edge
    // re-read that edge (unconditional loads keep the requests in flight)
    const int64_t e2 = (t0 + 128 + lane) < e_end ? (t0 + 128 + lane) : (e_end - 1);
    const int64_t nb2 = MODE == 2 ? p.nbr[e2] : 0;
    const int64_t e1 = (t0 + 64 + lane) < e_end ? (t0 + 64 + lane) : (e_end - 1);
    const In nvx = p.vec[3 * e1], nvy = p.vec[3 * e1 + 1], nvz = p.vec[3 * e1 + 2];
    In nh[HC];
#pragma unroll
    for (int c = 0; c < HC; ++c) nh[c] = MODE == 2 ? p.feats[nb1 * C + c] : In(0);

    // ---- phase 1: basis and row weights of this lane's edge, in fp64
    if (lane < cnt) {
      const double x = double(vx), y = double(vy), z = double(vz);
      const double r = sqrt(x * x + y * y + z * z);
      const double sr = r > p.eps ? r : p.eps;
      const double inv = 1.0 / sr;
      real_sph_row<double, double>(x * inv, y * inv, z * inv, LMAX, nt, Yt + lane, kPitch64);
      if (MODE == 0) {
        radial_row64<NMAX>(r, p, Wt + lane, kPitch64);
      } else {
        double g[NR];
        radial_row64<NMAX>(r, p, g, 1);
#pragma unroll
        for (int c = 0; c < C; ++c) {
          double s0 = 0.0, s1 = 0.0;
#pragma unroll
          for (int n = 0; n + 1 < NR; n += 2) {
            s0 = fma(Mx[c * NR + n], g[n], s0);
            s1 = fma(Mx[c * NR + n + 1], g[n + 1], s1);
          }
          if (NR % 2) s0 = fma(Mx[c * NR + NR - 1], g[NR - 1], s0);
          Wt[c * kPitch64 + lane] = double(h[c]) * (s0 + s1);
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < LW; ++q) Yt[q * kPitch64 + lane] = 0.0;
#pragma unroll
      for (int q = 0; q < ROWS; ++q) Wt[q * kPitch64 + lane] = 0.0;
    }
    // The next chunk's loads were issued before this chunk's phase 1: wait for
    // them here, before phase 2 issues this chunk's stores.  Loads and stores
    // share one in-order counter, so a wait placed after the stores (where the
    // compiler would put it) also waits for the stores to drain.
    wait_vmem_all();
    __syncthreads();  // one wave: orders the LDS tile writes before the operand reads

    // ---- phase 2: per-atom MFMA accumulation over k-blocks of 4 edges.  The
    // operands of KB k-blocks are read from LDS in one batch; consecutive
    // k-blocks alternate between two accumulator sets (independent MFMAs)
    const int nkb = (cnt + 3) >> 2;
    for (int j0 = 0; j0 < nkb; j0 += KB) {
      double wv[KB][RT], yv[KB][CT];
#pragma unroll
      for (int jj = 0; jj < KB; ++jj) {
        const int el = 4 * (j0 + jj) + kq;  // <= 63: columns cnt..63 hold zeros
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) wv[jj][rt] = Wt[(rt * 16 + cc) * kPitch64 + el];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) yv[jj][ct] = Yt[(ct * 16 + cc) * kPitch64 + el];
      }
#pragma unroll
      for (int jj = 0; jj < KB; ++jj) {
        const int j = j0 + jj;
        const int64_t e = t0 + 4 * j + kq;
        const int64_t kend = t0 + 4 * j + 4;
        bool more = j < nkb;
        while (more) {
          const bool in = e >= lo && e < hi;
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const double w = in ? wv[jj][rt] : 0.0;
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
              acc[jj & 1][rt][ct] =
                  __builtin_amdgcn_mfma_f64_16x16x4f64(w, yv[jj][ct], acc[jj & 1][rt][ct], 0, 0, 0);
          }
          // the atom continues in a later k-block, or it ends here
          more = hi <= kend;
          if (more) {
            store_atom(a);
            zero_acc();
            ++a;
            more = a < a_end;
            if (more) {
              lo = hi;
              hi = offset_at(p.offsets, a + 1);
              more = lo < kend;  // the next atom has edges in this k-block
            }
          }
        }
      }
    }
    __syncthreads();  // operand reads done before the next chunk's tile writes

    vx = nvx;
    vy = nvy;
    vz = nvz;
#pragma unroll
    for (int c = 0; c < HC; ++c) h[c] = nh[c];
    nb1 = nb2;
  }
  // atoms after the last edge (no edges of their own) get zero rows
  for (; a < a_end; ++a) store_atom(a);
}

// ---------------------------------------------------------------------------
// Channel kernel: MODE 2 at C = 16 channels, n_max = 8, l_max = 3 (one 16 x 16
// density tile per atom), both products on the matrix cores.
//
// Per chunk of 64 edges (lane = edge in phase 1):
//   phase 1  the distance, the radial values g_1..g_8 -> LDS ([n - 1][edge]),
//            the neighbour feature row -> LDS ([c][perm(edge)], zero for
//            padding lanes and for edges beyond the cutoff, whose g_n are all
//            zero);
//   mix      R[e][c] = mix[c][0] + sum_{n=1..8} g_n(e) mix[c][n] as two MFMAs
//            per 16-edge tile (the constant g_0 = 1 enters as the initial
//            accumulator); lane l then holds R[16 t + 4 v + l / 16][l % 16],
//            which times h[e][c] is the A operand W[c][e] of k-block 4 t + v;
//            the harmonics are computed next, over the radial rows (LDS keeps
//            one wave's reads and writes in order, so the MFMA operand reads
//            see g), which keeps the wave at 12.6 KB of LDS;
//   phase 2  one MFMA per k-block of four edges.  A full chunk whose atom ends
//            all fall on k-block boundaries, with every atom holding at least
//            one k-block and at most P (4, or 2 for an fp64 density) atoms
//            ending in it, runs as 16 unmasked MFMAs with a scalar test for an
//            atom end after each; the rows of those atoms wait in registers
//            and are stored at the start of the next chunk.  Any other chunk
//            masks each k-block per lane by atom, splits the k-blocks that
//            straddle an atom boundary and stores rows as atoms end.
// On gfx950 the fp64 MFMAs and the fp64 VALU instructions of one SIMD take
// turns on the same fp64 pipe (a wave of MFMAs and a wave of FMAs sharing a
// SIMD take the sum of their separate times), so the basis math is not hidden
// under the matrix-core phase: the kernel's bound is the sum of the two.
// Atom ends come from a vector window of 64 CSR offsets (v_readlane), so the
// MFMA loop issues no scalar loads.  The next chunk's loads (two register
// sets, alternating) are issued after one wait for everything issued a chunk
// earlier, so the basis math never waits on loads still in flight; edge
// vectors, neighbour indices and the density are streamed non-temporally.
// The basis math is written for this shape: closed-form real harmonics of
// degree <= 3 (the reference's polynomials, not simplified with |u| = 1),
// 1/sqrt by v_rsq_f64 and two Newton steps, cos(pi s) and expm1 by Taylor
// polynomials truncated below 1e-17; liveness at the cutoff is decided
// exactly as the reference does (sqrt, then a division) for the distances
// within a few ulps of it.
namespace chan16 {
// sqrt2 N_lm Q_l^m(z) prefactors, N_lm = sqrt((2l+1)/(4 pi) (l-m)!/(l+m)!)
constexpr double kC00 = 0.28209479177387814;   // N_00
constexpr double kC1 = 0.4886025119029199;     // N_10 = sqrt2 N_11
constexpr double kN20 = 0.63078313050504;      // N_20
constexpr double kK21 = 1.0925484305920792;    // sqrt2 N_21 * 3
constexpr double kK22 = 0.5462742152960396;    // sqrt2 N_22 * 3
constexpr double kN30 = 0.7463526651802308;    // N_30
constexpr double kK31 = 0.30469719964297715;   // sqrt2 N_31
constexpr double kK32 = 1.4453057213202771;    // sqrt2 N_32 * 15
constexpr double kK33 = 0.5900435899266435;    // sqrt2 N_33 * 15
// sin(pi u) / u = sum_k (-1)^k pi^(2k+1) / (2k+1)! u^(2k), |u| <= 1/2
constexpr double kSinPi[11] = {3.141592653589793,       -5.16771278004997,       2.5501640398773455,
                               -0.5992645293207921,     0.08214588661112823,     -0.0073704309457143504,
                               0.00046630280576761255,  -2.1915353447830217e-05, 7.952054001475513e-07,
                               -2.2948428997269873e-08, 5.392664662608129e-10};
// expm1(r) / r = sum_k r^k / (k+1)!, |r| <= ln2 / 2
constexpr double kExpm1[13] = {1.0,
                               0.5,
                               0.16666666666666666,
                               0.041666666666666664,
                               0.008333333333333333,
                               0.001388888888888889,
                               0.0001984126984126984,
                               2.48015873015873e-05,
                               2.7557319223985893e-06,
                               2.755731922398589e-07,
                               2.505210838544172e-08,
                               2.08767569878681e-09,
                               1.6059043836821613e-10};
constexpr double kLn2Hi = 0.6931471805599453, kLn2Lo = 2.3190468138462996e-17, kLog2e = 1.4426950408889634;

// Both polynomials read their coefficients from an LDS copy of the tables
// (kCoef: kSinPi then kExpm1): fetched where they are used, they do not sit in
// registers for the whole kernel as hoisted 64-bit constants would.
constexpr int kCoef = 11 + 13;

// cos(pi s) for s in [0, 1] as -sin(pi (s - 1/2))
__device__ inline double cospi01(double s, const double* coef) {
  const double u = s - 0.5, u2 = u * u;
  double q = coef[10];
#pragma unroll
  for (int i = 9; i >= 0; --i) q = fma(q, u2, coef[i]);
  return -u * q;
}

// expm1(t) = 2^k expm1(r) + (2^k - 1), t = k ln2 + r (Cody-Waite)
__device__ inline double expm1_reduced(double t, const double* coef) {
  const double k = rint(t * kLog2e);
  double r = fma(-k, kLn2Hi, t);
  r = fma(-k, kLn2Lo, r);
  double q = coef[11 + 12];
#pragma unroll
  for (int i = 11; i >= 0; --i) q = fma(q, r, coef[11 + i]);
  const double scale = ldexp(1.0, int(k));
  return fma(scale, q * r, scale - 1.0);
}

// the 16 real harmonics of degree <= 3 (column-major in Y: Y[lm * YP])
template <int YP>
__device__ inline void sph3(double x, double y, double z, double* Y) {
  const double zz = z * z, xy = x * y, d2 = fma(x, x, -y * y);  // Re, Im/2 of (x+iy)^2
  Y[0] = kC00;
  Y[1 * YP] = -kC1 * y;
  Y[2 * YP] = kC1 * z;
  Y[3 * YP] = kC1 * x;
  Y[4 * YP] = -2.0 * kK22 * xy;
  Y[5 * YP] = -kK21 * z * y;
  Y[6 * YP] = kN20 * fma(1.5, zz, -0.5);
  Y[7 * YP] = kK21 * z * x;
  Y[8 * YP] = kK22 * d2;
  const double q31 = kK31 * fma(7.5, zz, -1.5);
  Y[9 * YP] = -kK33 * y * fma(3.0 * x, x, -y * y);
  Y[10 * YP] = -2.0 * kK32 * z * xy;
  Y[11 * YP] = -q31 * y;
  Y[12 * YP] = kN30 * z * fma(2.5, zz, -1.5);
  Y[13 * YP] = q31 * x;
  Y[14 * YP] = kK32 * z * d2;
  Y[15 * YP] = kK33 * x * fma(x, x, -3.0 * y * y);
}
}  // namespace chan16

template <typename In, typename Out>
__global__ __launch_bounds__(64) void ace_density_channel16_kernel(Density64Params<In, Out> p) {
  using namespace chan16;
  constexpr int C = 16, NR = 9, LW = 16;
  constexpr int YP = 65;                         // pitch (doubles) of Yt and Gt, odd
  constexpr int HP = sizeof(In) == 4 ? 68 : 66;  // pitch (elements) of Ht: rows 16-byte aligned
  typedef In in4 __attribute__((ext_vector_type(4)));
  // harmonics [lm][edge]; rows 0..7 first hold the radial values g_1..g_8
  // [n - 1][edge] until the mix MFMAs have read them (LDS keeps one wave's
  // reads and writes in order)
  __shared__ double Yt[LW * YP];
  double* const Gt = Yt;
  __shared__ __attribute__((aligned(16))) In Ht[C * HP];    // feature rows [c][perm(edge)]
  __shared__ double coef[kCoef];

  const int lane = threadIdx.x;
  const int kq = lane >> 4, cc = lane & 15;
  // edge 16 t + 4 v + k of a chunk sits at column 16 t + 4 k + v of Ht, so
  // lane (k = kq, c = cc) reads its four feature values of tile t as one word
  const int hcol = (lane & ~15) | ((lane & 3) << 2) | ((lane >> 2) & 3);
  const int64_t a_begin = uniform64(int64_t(blockIdx.x) * p.N / p.waves);
  const int64_t a_end = uniform64((int64_t(blockIdx.x) + 1) * p.N / p.waves);
  if (a_begin >= a_end) return;
  for (int q = lane; q < LW * YP; q += 64) Yt[q] = 0.0;
  for (int q = lane; q < C * HP; q += 64) Ht[q] = In(0);
  if (lane < 11) coef[lane] = kSinPi[lane];
  if (lane < 13) coef[11 + lane] = kExpm1[lane];
  const double mix0 = double(p.mix[cc * NR]);
  const double mixB0 = double(p.mix[cc * NR + 1 + kq]);
  const double mixB1 = double(p.mix[cc * NR + 5 + kq]);
  __syncthreads();
  const int64_t e_begin = offset_at(p.offsets, a_begin), e_end = offset_at(p.offsets, a_end);
  const int span = int(e_end - e_begin);  // edges of this wave (< 2^31, checked by the host)
  const int na = int(a_end - a_begin);

  // end offsets (wave-relative) of atoms wb + lane, clamped to the wave's last
  // atom: the low words of the CSR offsets suffice (the host keeps E < 2^31),
  // and a one-word load leaves no dead half-register for a later write to wait on
  const int* const off32 = reinterpret_cast<const int*>(p.offsets);
  const int e_begin32 = int(e_begin);
  auto window = [&](int wb) {
    const int64_t i = a_begin + wb + 1 + lane;
    return off32[2 * (i < a_end ? i : a_end)] - e_begin32;
  };
  int wb = 0;
  int offw = window(0);

  mfma_d4 acc = mfma_d4{0.0, 0.0, 0.0, 0.0};
  int a = 0, lo = 0;
  int hi = int(offset_at(p.offsets, a_begin + 1) - e_begin);
  Out* __restrict__ Aw = p.A + a_begin * (C * LW) + lane;
  auto store_atom = [&](int atom) {
    Out* __restrict__ dst = Aw + int64_t(atom) * (C * LW);
#pragma unroll
    for (int v = 0; v < 4; ++v) __builtin_nontemporal_store(Out(acc[v]), dst + 64 * v);  // row kq + 4v, column cc
  };
  auto next_atom = [&]() {
    store_atom(a);
    acc = mfma_d4{0.0, 0.0, 0.0, 0.0};
    ++a;
    lo = hi;
    if (a >= na) {
      hi = 0x7fffffff;
    } else if (a - wb < 64) {
      hi = __builtin_amdgcn_readlane(offw, a - wb);
    } else {
      hi = int(offset_at(p.offsets, a_begin + a + 1) - e_begin);
    }
  };
  auto clamp_edge = [&](int64_t e) { return e < e_end ? e : e_end - 1; };
  // Rows of the atoms a fast chunk completes are held in registers and stored
  // at the start of the next chunk, after its wait and ahead of its loads: the
  // next wait then finds those stores issued a whole chunk earlier (loads and
  // stores share one in-order counter).
  constexpr int P = sizeof(Out) == 4 ? 4 : 2;
  Out held[P][4];
  int held_atom[P];
  int nheld = 0;
#pragma unroll
  for (int s = 0; s < P; ++s) held_atom[s] = 0;
  auto hold_atom = [&]() {
#pragma unroll
    for (int s = 0; s < P; ++s)
      if (s == nheld) {
#pragma unroll
        for (int v = 0; v < 4; ++v) held[s][v] = Out(acc[v]);
        held_atom[s] = a;
      }
    ++nheld;
    acc = mfma_d4{0.0, 0.0, 0.0, 0.0};
    ++a;
    lo = hi;
    if (a >= na) {
      hi = 0x7fffffff;
    } else if (a - wb < 64) {
      hi = __builtin_amdgcn_readlane(offw, a - wb);
    } else {
      hi = int(offset_at(p.offsets, a_begin + a + 1) - e_begin);
    }
  };
  auto flush = [&]() {
#pragma unroll
    for (int s = 0; s < P; ++s)
      if (s < nheld) {
        Out* __restrict__ dst = Aw + int64_t(held_atom[s]) * (C * LW);
#pragma unroll
        for (int v = 0; v < 4; ++v) __builtin_nontemporal_store(held[s][v], dst + 64 * v);
      }
    nheld = 0;
  };

  // Software pipeline, two chunks per trip with two register sets: on entry
  // to a chunk the lane holds the vector and the feature row of its edge of
  // that chunk and the neighbour index of its edge of the next chunk.
  In vxA = In(0), vyA = In(0), vzA = In(0), vxB = In(0), vyB = In(0), vzB = In(0);
  in4 hA[4], hB[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) hA[t] = hB[t] = in4{In(0), In(0), In(0), In(0)};
  int64_t nb = 0;
  if (span > 0) {
    const int64_t e = clamp_edge(e_begin + lane);
    vxA = __builtin_nontemporal_load(p.vec + 3 * e);
    vyA = __builtin_nontemporal_load(p.vec + 3 * e + 1);
    vzA = __builtin_nontemporal_load(p.vec + 3 * e + 2);
    const in4* row = reinterpret_cast<const in4*>(p.feats + __builtin_nontemporal_load(p.nbr + e) * C);
#pragma unroll
    for (int t = 0; t < 4; ++t) hA[t] = row[t];
    nb = __builtin_nontemporal_load(p.nbr + clamp_edge(e_begin + 64 + lane));
  }

  auto chunk = [&](const int c0, const In vx, const In vy, const In vz, const in4* h4, In& nvx, In& nvy, In& nvz,
                   in4* nh4) {
    const int cnt = span - c0 < 64 ? span - c0 : 64;
    const int64_t t0 = e_begin + c0;
    // Everything issued before this point (this chunk's operands, loaded one
    // chunk ago, and the previous chunk's stores) is complete by now: one wait
    // here, before the next loads go out, spares the basis math below the
    // waits for loads that are still in flight (the in-order counter cannot
    // tell them apart once a variable number of stores sits in between).
    wait_vmem_all();
    flush();
    // the next chunk's vector and feature row, the neighbour index one further,
    // and the offsets window from the current atom on
    {
      const int64_t e1 = clamp_edge(t0 + 64 + lane);
      nvx = __builtin_nontemporal_load(p.vec + 3 * e1);
      nvy = __builtin_nontemporal_load(p.vec + 3 * e1 + 1);
      nvz = __builtin_nontemporal_load(p.vec + 3 * e1 + 2);
      const in4* row = reinterpret_cast<const in4*>(p.feats + nb * C);
#pragma unroll
      for (int t = 0; t < 4; ++t) nh4[t] = row[t];
      nb = __builtin_nontemporal_load(p.nbr + clamp_edge(t0 + 128 + lane));
    }
    const int wb_next = a;
    const int offw_next = window(a);

    // ---- phase 1 (lane = edge): radial rows -> Gt and feature row -> Ht, then
    // the mix MFMAs, then the harmonics over the radial rows
#if YE3T_DENSITY_SETPRIO
    __builtin_amdgcn_s_setprio(0);
#endif
    const double x = double(vx), y = double(vy), z = double(vz);
    double inv;
    {
      const double r2 = x * x + y * y + z * z;
      const double r2c = r2 > 2.2250738585072014e-308 ? r2 : 2.2250738585072014e-308;
      const double hr = 0.5 * r2c;
      double rs = __builtin_amdgcn_rsq(r2c);
      rs = rs * fma(-hr * rs, rs, 1.5);
      rs = rs * fma(-hr * rs, rs, 1.5);
      const double r = r2 * rs;  // sqrt(r2) within an ulp
      inv = r >= p.eps ? rs : p.inv_eps;
      bool over = r > p.cutoff;
      // liveness exactly as the reference decides it (sqrt(r2) / cutoff > 1)
      // for the rare distances within a few ulps of the cutoff
      const bool tie = fabs(r - p.cutoff) <= p.cutoff_tie;
      if (__ballot(tie) != 0) {
        asm volatile("" ::: "memory");
        if (tie) over = sqrt(r2) / p.cutoff > 1.0;
      }
      const bool live = lane < cnt && !over;
      const double s = r * p.inv_cutoff;
      const double sc = over ? 1.0 : (s < 1.0 ? s : 1.0);
      const double env = 1.0 + cospi01(sc, coef);
      const double xc = 1.0 - expm1_reduced(p.lambda * (1.0 - sc), coef) * p.two_over_den;
      Gt[lane] = 0.5 * env;
      const double q = 0.25 * env, x2 = xc + xc;
      double tm = 1.0, tn = xc;
#pragma unroll
      for (int n = 2; n < NR; ++n) {
        const double t2 = fma(x2, tn, -tm);
        Gt[(n - 1) * YP + lane] = fma(-q, t2, q);
        tm = tn;
        tn = t2;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) Ht[(4 * t + u) * HP + hcol] = live ? h4[t][u] : In(0);
    }
    __syncthreads();

    // ---- radial mix on the matrix cores: lane l holds R[16 t + 4 v + l / 16][l % 16]
    mfma_d4 R[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      R[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(Gt[kq * YP + 16 * t + cc], mixB0,
                                                  mfma_d4{mix0, mix0, mix0, mix0}, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      R[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(Gt[(4 + kq) * YP + 16 * t + cc], mixB1, R[t], 0, 0, 0);
    sph3<YP>(x * inv, y * inv, z * inv, Yt + lane);
    __syncthreads();
    // operands of the chunk's 16 k-blocks: B from Yt, A = W[c][e] = R[e][c] h[e][c]
    double wv[16];
    {
      in4 hk[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) hk[t] = *reinterpret_cast<const in4*>(Ht + cc * HP + 16 * t + 4 * kq);
#pragma unroll
      for (int j = 0; j < 16; ++j) wv[j] = R[j >> 2][j & 3] * double(hk[j >> 2][j & 3]);
    }

    // ---- phase 2: one MFMA per k-block of four edges
#if YE3T_DENSITY_SETPRIO
    __builtin_amdgcn_s_setprio(YE3T_DENSITY_SETPRIO);
#endif
    // atoms without edges that end where this chunk starts
    while (hi <= c0 && a < na) next_atom();
    // fast form: a full chunk whose atom ends all fall on k-block boundaries,
    // every atom inside it holding at least one k-block, all within the window
    bool fast = false;
    if (cnt == 64 && a - wb < 64 && __builtin_amdgcn_readlane(offw, 63) >= c0 + 64) {
      const int d = a - wb;
      const int prev = __shfl_up(offw, 1);
      const int start = lane == d ? lo : prev;
      const bool inside = lane >= d && wb + lane < na && offw > c0;
      const bool bad = inside && offw < c0 + 64 && ((offw & 3) != 0 || offw - start < 4);
      const bool ends = inside && offw <= c0 + 64;
      fast = __ballot(bad) == 0 && __popcll(__ballot(ends)) <= P;
    }
    // B operands are read from Yt one tile (four k-blocks) ahead of their MFMAs
    double yq[2][4];
#pragma unroll
    for (int v = 0; v < 4; ++v) yq[0][v] = Yt[cc * YP + 4 * v + kq];
    if (fast) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if ((j & 3) == 0 && j < 12) {
#pragma unroll
          for (int v = 0; v < 4; ++v) yq[((j >> 2) + 1) & 1][v] = Yt[cc * YP + 4 * (j + 4 + v) + kq];
        }
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(wv[j], yq[(j >> 2) & 1][j & 3], acc, 0, 0, 0);
        if (hi == c0 + 4 * j + 4) hold_atom();
      }
    } else {
      const int nkb = (cnt + 3) >> 2;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (j < nkb) {
          const int ke = c0 + 4 * j + 4, er = ke - 4 + kq;
          const double yv = Yt[cc * YP + 4 * j + kq];
          for (;;) {
            const double wm = unsigned(er - lo) < unsigned(hi - lo) ? wv[j] : 0.0;
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(wm, yv, acc, 0, 0, 0);
            if (hi > ke) break;  // the atom continues in a later k-block
            next_atom();
            if (a >= na || lo >= ke) break;  // the next atom starts in a later k-block
          }
        }
      }
    }
    __syncthreads();  // operand reads done before the next chunk's tile writes
    wb = wb_next;
    offw = offw_next;
  };

  for (int c0 = 0; c0 < span; c0 += 128) {
    chunk(c0, vxA, vyA, vzA, hA, vxB, vyB, vzB, hB);
    if (c0 + 64 >= span) break;
    chunk(c0 + 64, vxB, vyB, vzB, hB, vxA, vyA, vzA, hA);
  }
  flush();
  // atoms after the last edge (no edges of their own) get zero rows
  for (; a < na; ++a) store_atom(a);
}

static int env_int64(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return (v && *v) ? std::atoi(v) : fallback;
}

// Waves (64-thread workgroups) of one launch: as many as the device holds at
// once for `kernel` (one round, no tail), each walking a contiguous atom range
// (YE3T_DENSITY_WAVES overrides).
static int64_t density_waves(int64_t atoms, const void* kernel) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    cus = 256;
  }
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64, 0) != hipSuccess || per_cu <= 0) per_cu = 4;
  int64_t waves = env_int64("YE3T_DENSITY_WAVES", int(int64_t(cus) * per_cu));
  if (waves < 1) waves = 1;
  if (waves > 0x7FFFFFFF) waves = 0x7FFFFFFF;
  return atoms < waves ? (atoms > 0 ? atoms : 1) : waves;
}


template <int MODE, typename In, typename Out, int LMAX, int NMAX, int C>
int launch64(const ye3t_density_args* a, void* A, hipStream_t stream) {
  Density64Params<In, Out> p;
  p.N = a->atom_count;
  p.offsets = a->row_offsets;
  p.nbr = a->neighbors;
  p.vec = static_cast<const In*>(a->edge_vectors);
  p.feats = static_cast<const In*>(a->node_features);
  p.mix = static_cast<const In*>(a->radial_mix);
  p.cutoff = a->cutoff > 2.220446049250313e-16 ? a->cutoff : 2.220446049250313e-16;
  p.lambda = a->lambda;
  p.den = std::expm1(a->lambda);
  p.eps = a->epsilon;
  p.A = static_cast<Out*>(A);
  // about three 64-edge chunks per wave
  const int64_t grid =
      density_waves(p.N, reinterpret_cast<const void*>(&ace_density_mfma64_kernel<MODE, In, Out, LMAX, NMAX, C>));
  p.waves = grid;
  hipLaunchKernelGGL((ace_density_mfma64_kernel<MODE, In, Out, LMAX, NMAX, C>), dim3(unsigned(grid)), dim3(64), 0,
                     stream, p, norm_table());
  set_density_kernel("ace_density_mfma64_kernel");
  return check_launch("ace_density_mfma64_kernel");
}


template <typename In, typename Out>
int launch64_channel(const ye3t_density_args* a, void* A, hipStream_t stream) {
  Density64Params<In, Out> p;
  p.N = a->atom_count;
  p.offsets = a->row_offsets;
  p.nbr = a->neighbors;
  p.vec = static_cast<const In*>(a->edge_vectors);
  p.feats = static_cast<const In*>(a->node_features);
  p.mix = static_cast<const In*>(a->radial_mix);
  p.cutoff = a->cutoff > 2.220446049250313e-16 ? a->cutoff : 2.220446049250313e-16;
  p.lambda = a->lambda;
  p.den = std::expm1(a->lambda);
  p.eps = a->epsilon;
  p.A = static_cast<Out*>(A);
  p.inv_cutoff = 1.0 / p.cutoff;
  p.two_over_den = 2.0 / p.den;
  p.inv_eps = 1.0 / p.eps;
  p.cutoff_tie = 8.0 * (std::nextafter(p.cutoff, 2.0 * p.cutoff) - p.cutoff);
  const int64_t grid = density_waves(p.N, reinterpret_cast<const void*>(&ace_density_channel16_kernel<In, Out>));
  p.waves = grid;
  hipLaunchKernelGGL((ace_density_channel16_kernel<In, Out>), dim3(unsigned(grid)), dim3(64), 0, stream, p);
  set_density_kernel("ace_density_channel16_kernel");
  return check_launch("ace_density_channel16_kernel");
}


// Densities accumulated in fp64 for the compiled shapes, stored as Out (fp64,
// or fp32 rounded once from the fp64 accumulators); YE3T_EUNSUPPORTED (nothing
// launched) for the others, which run on the VALU kernel.
template <typename In, typename Out>
int launch_density_mfma64(const ye3t_density_args* a, void* A, hipStream_t stream) {
  if (a->species) return YE3T_EUNSUPPORTED;
  if (env_int64("YE3T_DENSITY_MFMA64", 1) == 0) return YE3T_EUNSUPPORTED;
  const int64_t L = a->max_angular, Nm = a->max_radial_index;
  if (a->node_features) {
    // neighbour indices are read as 32-bit values by the mix kernel
    if (L == 3 && Nm == 8 && a->channel_count == 16 && a->atom_count < (int64_t(1) << 31)) {
      // both products on the matrix cores with W in registers (wave-relative
      // edge indices need E < 2^31); YE3T_DENSITY_MIX_MFMA=0 selects the
      // generic kernel with the radial mix on the VALU
      if (env_int64("YE3T_DENSITY_MIX_MFMA", 1) != 0 && a->edge_count < (int64_t(1) << 31))
        return launch64_channel<In, Out>(a, A, stream);
      return launch64<2, In, Out, 3, 8, 16>(a, A, stream);
    }
    return YE3T_EUNSUPPORTED;
  }
  if (a->channel_count != 1) return YE3T_EUNSUPPORTED;
  if (L == 3 && Nm == 8) return launch64<0, In, Out, 3, 8, 1>(a, A, stream);
  if (L == 4 && Nm == 10) return launch64<0, In, Out, 4, 10, 1>(a, A, stream);
  if (L == 6 && Nm == 12) return launch64<0, In, Out, 6, 12, 1>(a, A, stream);
  return YE3T_EUNSUPPORTED;
}

template int launch_density_mfma64<float, double>(const ye3t_density_args*, void*, hipStream_t);
template int launch_density_mfma64<double, double>(const ye3t_density_args*, void*, hipStream_t);
template int launch_density_mfma64<float, float>(const ye3t_density_args*, void*, hipStream_t);

}  // namespace ye3t
