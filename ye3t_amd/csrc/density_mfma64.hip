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
// (ace_density_mfma64_channel_kernel) that also puts the radial mix on the
// matrix cores and keeps W in registers.
#include <cmath>
#include <cstdlib>

#include "common.h"

// Issue priority of the channel kernel's MFMA phase (phase 1 runs at 0).  With
// two waves per SIMD, the wave feeding the matrix core goes first while the
// other fills the gaps with its VALU basis math: 57.4 -> 55.7 us at config 4.
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

// MODE 2 at C = 16 channels, n_max = 8, l_max = 3 (one 16 x 16 density tile
// per atom) with both products on the matrix cores and W never stored:
//   phase 1  lane = edge, branch-free: real SH Y_lm (16) and the radial values
//            g_1..g_8 in fp64 -> LDS ([lm][edge], [n - 1][edge]); the
//            neighbour feature row -> LDS ([c][perm(edge)]), zero for padding
//            lanes and for edges beyond the cutoff (whose g_n are all zero).
//   phase 2  per 16-edge tile t: R[e][c] = mix[c][0] + sum_{n=1..8} g_n(e) mix[c][n]
//            is two MFMAs, the constant g_0 = 1 entering as the accumulator's
//            initial value.  Lane l then holds R[16 t + 4 v + l / 16][l % 16],
//            which times h[e][c] is the A operand W[c][e] of k-block 4 t + v
//            of the density product.  Atoms are walked with wave-relative
//            32-bit edge indices and scalar compares; only a k-block that
//            straddles an atom boundary is masked per lane.
template <typename In, typename Out>
__global__ __launch_bounds__(64) void ace_density_mfma64_channel_kernel(Density64Params<In, Out> p, NormTable nt) {
  constexpr int C = 16, NR = 9, LMAX = 3, LW = 16;
  constexpr int YP = 65;                         // pitch (doubles) of Yt and Gt, odd
  constexpr int HP = sizeof(In) == 4 ? 68 : 66;  // pitch (elements) of Ht: rows 16-byte aligned
  typedef In in4 __attribute__((ext_vector_type(4)));
  __shared__ double Yt[LW * YP];
  __shared__ double Gt[8 * YP];
  __shared__ __attribute__((aligned(16))) In Ht[C * HP];

  const int lane = threadIdx.x;
  const int kq = lane >> 4, cc = lane & 15;
  // edge 16 t + 4 v + k of a chunk sits at column 16 t + 4 k + v of Ht, so
  // lane (k = kq, c = cc) reads its four feature values of tile t as one word
  const int hcol = (lane & ~15) | ((lane & 3) << 2) | ((lane >> 2) & 3);
  // wave-uniform atom range (kept in scalar registers)
  const int64_t a_begin = uniform64(int64_t(blockIdx.x) * p.N / p.waves);
  const int64_t a_end = uniform64((int64_t(blockIdx.x) + 1) * p.N / p.waves);
  if (a_begin >= a_end) return;
  // stale tile entries must stay finite (they meet zero weights)
  for (int q = lane; q < LW * YP; q += 64) Yt[q] = 0.0;
  for (int q = lane; q < 8 * YP; q += 64) Gt[q] = 0.0;
  for (int q = lane; q < C * HP; q += 64) Ht[q] = In(0);
  // B operands of the mix: mix^T[n = 1 + 4 s + kq][c = cc]; g_0 = 1 adds mix[c][0]
  const double mix0 = double(p.mix[cc * NR]);
  const double mixB0 = double(p.mix[cc * NR + 1 + kq]);
  const double mixB1 = double(p.mix[cc * NR + 5 + kq]);
  __syncthreads();
  const int64_t e_begin = offset_at(p.offsets, a_begin), e_end = offset_at(p.offsets, a_end);
  const int span = int(e_end - e_begin);  // edges of this wave (< 2^31, checked by the host)

  // one accumulator: a dependent fp64 MFMA issues as soon as the matrix core
  // is free (its latency equals its issue interval)
  mfma_d4 acc = mfma_d4{0.0, 0.0, 0.0, 0.0};
  // current atom a_begin + a and its edges [lo, hi), all wave-relative (32-bit
  // scalar compares; the host keeps the edge count below 2^31)
  const int na = int(a_end - a_begin);
  int a = 0;
  int lo = 0, hi = int(offset_at(p.offsets, a_begin + 1) - e_begin);
  Out* __restrict__ Aw = p.A + a_begin * (C * LW) + lane;
  auto store_atom = [&](int atom) {
    Out* __restrict__ dst = Aw + int64_t(atom) * (C * LW);
#pragma unroll
    for (int v = 0; v < 4; ++v) dst[64 * v] = Out(acc[v]);  // row c = kq + 4 v, column lm = cc
  };
  // next atom: its edge range, or an empty range past the wave's edges
  auto next_atom = [&]() {
    store_atom(a);
    acc = mfma_d4{0.0, 0.0, 0.0, 0.0};
    ++a;
    lo = hi;
    hi = a < na ? int(offset_at(p.offsets, a_begin + a + 1) - e_begin) : 0x7fffffff;
  };
  auto clamp_edge = [&](int64_t e) { return e < e_end ? e : e_end - 1; };

  // Software pipeline: on entry to chunk i the lane holds the vector and the
  // feature row of its edge of chunk i and the neighbour index of its edge of
  // chunk i + 1 (lanes past the last edge re-read that edge).
  In vx = In(0), vy = In(0), vz = In(0);
  In h[C];
#pragma unroll
  for (int c = 0; c < C; ++c) h[c] = In(0);
  int64_t nb1 = 0;
  if (span > 0) {
    const int64_t e = clamp_edge(e_begin + lane);
    vx = p.vec[3 * e];
    vy = p.vec[3 * e + 1];
    vz = p.vec[3 * e + 2];
    const int64_t nb = p.nbr[e];
#pragma unroll
    for (int c = 0; c < C; ++c) h[c] = p.feats[nb * C + c];
    nb1 = p.nbr[clamp_edge(e_begin + 64 + lane)];
  }

  for (int c0 = 0; c0 < span; c0 += 64) {
    const int cnt = span - c0 < 64 ? span - c0 : 64;
    const int64_t t0 = e_begin + c0;
    const int64_t nb2 = p.nbr[clamp_edge(t0 + 128 + lane)];
    const int64_t e1 = clamp_edge(t0 + 64 + lane);
    const In nvx = p.vec[3 * e1], nvy = p.vec[3 * e1 + 1], nvz = p.vec[3 * e1 + 2];
    In nh[C];
#pragma unroll
    for (int c = 0; c < C; ++c) nh[c] = p.feats[nb1 * C + c];

    // ---- phase 1 (every lane; padding lanes hold a copy of the last edge)
#if YE3T_DENSITY_SETPRIO
    __builtin_amdgcn_s_setprio(0);
#endif
    {
      const double x = double(vx), y = double(vy), z = double(vz);
      const double r = sqrt(x * x + y * y + z * z);
      const double sr = r > p.eps ? r : p.eps;
      const double inv = 1.0 / sr;
      real_sph_row<double, double>(x * inv, y * inv, z * inv, LMAX, nt, Yt + lane, YP);
      const double s = r / p.cutoff;
      const bool live = lane < cnt && !(s > 1.0);
      const double sc = s > 1.0 ? 1.0 : s;
      const double env = 1.0 + cospi(sc);
      const double xc = 1.0 - 2.0 * expm1(-p.lambda * (sc - 1.0)) / p.den;
      Gt[lane] = 0.5 * env;
      double tm = 1.0, tn = xc;
#pragma unroll
      for (int n = 2; n < NR; ++n) {
        const double t2 = 2.0 * xc * tn - tm;
        Gt[(n - 1) * YP + lane] = 0.25 * (1.0 - t2) * env;
        tm = tn;
        tn = t2;
      }
#pragma unroll
      for (int c = 0; c < C; ++c) Ht[c * HP + hcol] = live ? h[c] : In(0);
    }
    // The next chunk's loads were issued before phase 1: wait for them here,
    // before phase 2 issues stores (loads and stores share one in-order counter).
    wait_vmem_all();
    __syncthreads();  // one wave: orders the LDS tile writes before the operand reads

    // ---- phase 2.  All operands of the chunk are read at once (columns past
    // cnt hold finite stale values that are never used) and the four tiles'
    // mix products are issued before the density MFMAs that consume them.
#if YE3T_DENSITY_SETPRIO
    __builtin_amdgcn_s_setprio(YE3T_DENSITY_SETPRIO);
#endif
    const int nkb = (cnt + 3) >> 2;
    double yv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) yv[j] = Yt[cc * YP + 4 * j + kq];
    mfma_d4 R[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      R[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(Gt[kq * YP + 16 * t + cc], mixB0,
                                                  mfma_d4{mix0, mix0, mix0, mix0}, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      R[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(Gt[(4 + kq) * YP + 16 * t + cc], mixB1, R[t], 0, 0, 0);
    in4 h4[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) h4[t] = *reinterpret_cast<const in4*>(Ht + cc * HP + 16 * t + 4 * kq);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (j < nkb) {
        const double w = R[j >> 2][j & 3] * double(h4[j >> 2][j & 3]);
        const int ke = c0 + 4 * j + 4, er = ke - 4 + kq;
        for (;;) {
          // this lane's edge belongs to the current atom
          const double wm = unsigned(er - lo) < unsigned(hi - lo) ? w : 0.0;
          acc = __builtin_amdgcn_mfma_f64_16x16x4f64(wm, yv[j], acc, 0, 0, 0);
          if (hi > ke) break;  // the atom continues in a later k-block
          next_atom();
          if (a >= na || lo >= ke) break;  // the next atom starts in a later k-block
        }
      }
    }
    __syncthreads();  // operand reads done before the next chunk's tile writes

    vx = nvx;
    vy = nvy;
    vz = nvz;
#pragma unroll
    for (int c = 0; c < C; ++c) h[c] = nh[c];
    nb1 = nb2;
  }
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
  const int64_t grid =
      density_waves(p.N, reinterpret_cast<const void*>(&ace_density_mfma64_channel_kernel<In, Out>));
  p.waves = grid;
  hipLaunchKernelGGL((ace_density_mfma64_channel_kernel<In, Out>), dim3(unsigned(grid)), dim3(64), 0, stream, p,
                     norm_table());
  set_density_kernel("ace_density_mfma64_channel_kernel");
  return check_launch("ace_density_mfma64_channel_kernel");
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
