// Stage 1 with one-hot species channels (and single-channel densities):
//
//   A[i, s, n, lm] = sum_{e in row i, species(nbr_e) = s} R_n(|v_e|) Y_lm(v_e / |v_e|)
//
// (the reference's radial table, real harmonics, scheduled_radial_angular
// channel product and density_accumulate, ye3t_runtime_core.cpp:214-423,
// 1550-1604, 1684-1702, fused).  Each (atom, species) pair is a small
// [NR x edges] x [edges x LW] product; an edge contributes to exactly one of
// them, so the kernel groups the edges of every atom by neighbour species and
// accumulates each group alone -- no work on edges of other species.
//
// One wave (a 64-thread workgroup; no barriers between waves) owns a
// contiguous atom range (as many waves as the device holds at once) and walks
// it in chunks of up to 16 (4 for l_max >= 5) consecutive whole atoms with at most 64 edges
// together:
//   sort     lane = edge; the neighbour's species is gathered, one ballot per
//            species gives every (atom, species) group's lanes, and each lane
//            computes its column of the chunk's tile: its atom's first column, plus
//            the sizes of the atom's groups of smaller species, plus its rank
//            within its own group (a stable counting sort);
//   phase 1  lane = edge; the radial values and real harmonics in fp64
//            registers, written to LDS transposed at the sorted column
//            (R[n][col], Y[lm][col]);
//   phase 2  per (atom, species) group, the k-blocks of four columns it
//            covers, one v_mfma_f64_16x16x4f64 per 16-component harmonic
//            tile (columns of neighbouring groups weigh zero), accumulating
//            in fp64; the group's [NR x LW] block then goes from the
//            accumulators to A (species absent from an atom get zero
//            blocks).  The MFMA moves each operand through LDS once per
//            k-block, where a lane-per-component VALU product would read the
//            radial values as LDS broadcasts once per edge and lane.
// Loads run two chunks ahead: chunk i + 2's edges and chunk i + 1's species
// gather are issued right after chunk i's one wait (which follows its basis
// math), so they hide behind chunk i's accumulation and stores and chunk
// i + 1's basis.  An atom with more than 64 edges is taken alone,
// species by species: each of its 64-edge windows in turn places its edges of
// that species in the tile and adds them to the same accumulators, so every
// block is accumulated in registers and stored once.
// The density is accumulated in fp64 and stored as Out (fp64, or fp32
// rounded once).  Lane layouts of the fp64 MFMA (l = lane):
//   A[i][k] from lane i + 16 k; B[k][j] from lane j + 16 k;
//   D[i][j] in lane j + 16 (i mod 4), element i div 4.
#include <cmath>

#include "common.h"
#include "sph.h"

namespace ye3t {
namespace {

// whole atoms per chunk: 16, or 4 for l_max >= 5 (sp_max_atoms), whose
// one-wave kernels would otherwise keep the chunk bounds in VGPRs for want of
// SGPRs and select them with a VALU chain per atom
template <int LMAX>
constexpr int sp_max_atoms() { return LMAX >= 5 ? 4 : 16; }
constexpr int kSpMaxSpecies = 16;
constexpr int kSpPitch = 67;  // LDS row pitch (doubles) of the transposed tile: odd, so 16 rows of a column spread over the banks

typedef double sp_d4 __attribute__((ext_vector_type(4)));

struct SpeciesParams {
  int64_t N;
  const int64_t* __restrict__ offsets;
  const int64_t* __restrict__ nbr;
  const void* __restrict__ vec;
  const int32_t* __restrict__ species;  // null: one channel, every edge in it
  int S;                                // channels
  int NR;                               // radial rows, n_max + 1 (<= 16)
  int64_t waves;
  double cutoff;
  double lambda;
  double den;  // expm1(lambda)
  double eps;
  void* __restrict__ A;
};

__device__ inline int64_t sp_offset(const int64_t* offsets, int64_t i) {
  return ((const __attribute__((address_space(4))) int64_t*)(offsets))[i];
}

__device__ inline uint64_t sp_ballot(bool v) { return __builtin_amdgcn_ballot_w64(v); }

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima)
__device__ inline void sp_wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// bits [lo, hi) of a 64-bit mask (0 <= lo <= hi <= 64)
__device__ inline uint64_t sp_range(int lo, int hi) {
  const uint64_t below_hi = hi >= 64 ? ~uint64_t(0) : ((uint64_t(1) << hi) - 1);
  const uint64_t below_lo = lo >= 64 ? ~uint64_t(0) : ((uint64_t(1) << lo) - 1);
  return below_hi & ~below_lo;
}

// Compile-time layout of one (l_max, radial rows) shape: the tile holds NRC
// radial rows and LW harmonic rows of 64 columns; the product covers them in
// 16-component tiles (CT of them over the harmonics).
template <int LMAX, int NRC>
struct SpShape {
  static constexpr int LW = (LMAX + 1) * (LMAX + 1);
  static constexpr int CT = (LW + 15) / 16;
  static constexpr int ROWS = NRC + LW;
};

// Radial values g_0..g_{NRC-1} and harmonics of one edge vector, fp64, in registers.
template <int LMAX, int NRC>
__device__ inline void sp_basis(double vx, double vy, double vz, const SpeciesParams& p, const NormTable& nt,
                                double (&Y)[(LMAX + 1) * (LMAX + 1)], double (&R)[NRC]) {
  const double r = sqrt(vx * vx + vy * vy + vz * vz);
  const double sr = r > p.eps ? r : p.eps;
  const double inv = 1.0 / sr;
  real_sph_row_fixed<LMAX, double, double>(vx * inv, vy * inv, vz * inv, nt, Y);
  const double s = r / p.cutoff;
  const bool live = s <= 1.0;
  const double env = 1.0 + cospi(s);
  R[0] = live ? 1.0 : 0.0;
  if (NRC > 1) R[1] = live ? 0.5 * env : 0.0;
  if (NRC > 2) {
    const double x = 1.0 - 2.0 * expm1(-p.lambda * (s - 1.0)) / p.den;
    double t0 = 1.0, t1 = x;
#pragma unroll
    for (int n = 2; n < NRC; ++n) {
      const double t2 = 2.0 * x * t1 - t0;
      R[n] = live ? 0.25 * (1.0 - t2) * env : 0.0;
      t0 = t1;
      t1 = t2;
    }
  }
}

// The basis of one edge into tile column `col`.
template <int LMAX, int NRC>
__device__ inline void sp_basis_to_tile(double vx, double vy, double vz, const SpeciesParams& p, const NormTable& nt,
                                        double* Wt, double* Yt, int col) {
  using Sh = SpShape<LMAX, NRC>;
  double Y[Sh::LW], R[NRC];
  sp_basis<LMAX, NRC>(vx, vy, vz, p, nt, Y, R);
#pragma unroll
  for (int n = 0; n < NRC; ++n) Wt[n * kSpPitch + col] = R[n];
#pragma unroll
  for (int k = 0; k < Sh::LW; ++k) Yt[k * kSpPitch + col] = Y[k];
}

// Adds the product of tile columns [base, base + c), c >= 1, to the
// accumulators (FRESH: sets them to it, the first k-block's MFMAs taking a
// zero accumulator): the k-blocks of four columns covering them, columns
// outside weighing zero (they read column `base`, which holds finite values).
// Rows past the tile (i >= NRC, components >= LW) read its last row: their
// accumulators are never stored.
template <int LMAX, int NRC, bool FRESH>
__device__ inline void sp_group_product(const double* Wt, const double* Yt, int base, int c, int kq, int cc,
                                        sp_d4 (&acc)[SpShape<LMAX, NRC>::CT]) {
  using Sh = SpShape<LMAX, NRC>;
  const double* const wrow = Wt + (cc < NRC ? cc : NRC - 1) * kSpPitch;
  const double* yrow[Sh::CT];
#pragma unroll
  for (int ct = 0; ct < Sh::CT; ++ct) {
    const int k = ct * 16 + cc;
    yrow[ct] = Yt + (k < Sh::LW ? k : Sh::LW - 1) * kSpPitch;
  }
  const int kb0 = base >> 2, kb1 = (base + c - 1) >> 2;
  for (int kb = kb0; kb <= kb1; ++kb) {
    const int col = 4 * kb + kq;
    const bool in = col >= base && col < base + c;
    const int rc = in ? col : base;
    const double w = wrow[rc];
    double y[Sh::CT];
#pragma unroll
    for (int ct = 0; ct < Sh::CT; ++ct) y[ct] = yrow[ct][rc];
    const double wm = in ? w : 0.0;
    if (FRESH && kb == kb0) {
#pragma unroll
      for (int ct = 0; ct < Sh::CT; ++ct)
        acc[ct] = __builtin_amdgcn_mfma_f64_16x16x4f64(wm, y[ct], sp_d4{0.0, 0.0, 0.0, 0.0}, 0, 0, 0);
    } else {
#pragma unroll
      for (int ct = 0; ct < Sh::CT; ++ct) acc[ct] = __builtin_amdgcn_mfma_f64_16x16x4f64(wm, y[ct], acc[ct], 0, 0, 0);
    }
  }
}

template <int CT>
__device__ inline void sp_zero(sp_d4 (&acc)[CT]) {
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) acc[ct] = sp_d4{0.0, 0.0, 0.0, 0.0};
}

typedef unsigned sp_u2 __attribute__((ext_vector_type(2)));
// per-lane byte offsets of the CT x 4 accumulator elements (see sp_store_offsets)
template <int CT>
struct SpOffsets {
  unsigned o[CT][4];
};

// Byte offsets of the lane's accumulator elements (row n = 4 v + kq,
// component lm = 16 ct + cc) in an (atom, species) block [NR x LW] of Out,
// and past the block for elements outside it: a buffer store there is
// dropped, so the stores need no lane masks.
template <int LMAX, int NRC, typename Out>
__device__ inline void sp_store_offsets(SpOffsets<SpShape<LMAX, NRC>::CT>& off, int NR, int kq, int cc) {
  using Sh = SpShape<LMAX, NRC>;
#pragma unroll
  for (int ct = 0; ct < Sh::CT; ++ct)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int n = 4 * v + kq, lm = ct * 16 + cc;
      off.o[ct][v] = (n < NR && lm < Sh::LW) ? unsigned(n * Sh::LW + lm) * unsigned(sizeof(Out)) : 0x7ffffff0u;
    }
}

template <typename Out>
__device__ inline void sp_put(__amdgpu_buffer_rsrc_t rb, unsigned off, double x) {
  if constexpr (sizeof(Out) == 8) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(sp_u2, x), rb, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, float(x)), rb, off, 0, 0);
  }
}

// One (atom, species) block [NR x LW] from the accumulators (rounded once to
// Out), through a buffer resource spanning the block.
template <int LMAX, int NRC, typename Out>
__device__ inline void sp_store(Out* __restrict__ dst, const sp_d4 (&acc)[SpShape<LMAX, NRC>::CT], int NR,
                                const SpOffsets<SpShape<LMAX, NRC>::CT>& off) {
  using Sh = SpShape<LMAX, NRC>;
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(dst, (short)0, NR * Sh::LW * int(sizeof(Out)), 0x00020000);
#pragma unroll
  for (int ct = 0; ct < Sh::CT; ++ct)
#pragma unroll
    for (int v = 0; v < 4; ++v) sp_put<Out>(rb, off.o[ct][v], acc[ct][v]);
}

// A zero block (a species absent from the atom).
template <int LMAX, int NRC, typename Out>
__device__ inline void sp_store_zero(Out* __restrict__ dst, int NR, const SpOffsets<SpShape<LMAX, NRC>::CT>& off) {
  using Sh = SpShape<LMAX, NRC>;
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(dst, (short)0, NR * Sh::LW * int(sizeof(Out)), 0x00020000);
#pragma unroll
  for (int ct = 0; ct < Sh::CT; ++ct)
#pragma unroll
    for (int v = 0; v < 4; ++v) sp_put<Out>(rb, off.o[ct][v], 0.0);
}

// The chunk starting at atom a: up to 16 whole atoms with at most 64 edges,
// read through the scalar cache (so nothing waits on the vector stores still
// draining); rel[j] = first edge of atom a + j relative to e0, cnt = edges.
// na == 0: atom a alone has more than 64 edges, or a == a_end (past the
// wave's range).
template <int MAXA>
struct SpChunk {
  int64_t a, e0;
  int na, cnt;
  int rel[MAXA + 1];
};

template <int MAXA>
__device__ inline SpChunk<MAXA> sp_form(const SpeciesParams& p, int64_t a, int64_t a_end) {
  SpChunk<MAXA> c;
  a = a < a_end ? a : a_end;  // past the end: an empty chunk at a_end
  c.a = a;
  c.e0 = sp_offset(p.offsets, a);
  int64_t ends[MAXA];
#pragma unroll
  for (int j = 1; j <= MAXA; ++j) ends[j - 1] = sp_offset(p.offsets, (a + j) <= a_end ? (a + j) : a_end);
  c.na = 0;
  c.rel[0] = 0;
  bool open = true;
#pragma unroll
  for (int j = 1; j <= MAXA; ++j) {
    open = open && (a + j) <= a_end && ends[j - 1] - c.e0 <= 64;
    c.rel[j] = open ? int(ends[j - 1] - c.e0) : 64 + 1;
    c.na += open ? 1 : 0;
  }
  c.cnt = 0;
#pragma unroll
  for (int j = 1; j <= MAXA; ++j) c.cnt = (j == c.na) ? c.rel[j] : c.cnt;
  return c;
}

// First atom after chunk c (a chunk with na == 0 is one atom).
template <int MAXA>
__device__ inline int64_t sp_after(const SpChunk<MAXA>& c) { return c.a + (c.na > 0 ? c.na : 1); }

// One lane's edge of a chunk: its vector and neighbour (zeros past the chunk's
// edges, and for a single-atom chunk of more than 64 edges, which loads its
// own).
template <typename In>
struct SpEdges {
  In x, y, z;
  int64_t nb;
};

template <typename In, int MAXA>
__device__ inline SpEdges<In> sp_load(const SpeciesParams& p, const In* __restrict__ vec, const SpChunk<MAXA>& c,
                                      int lane) {
  SpEdges<In> r{In(0), In(0), In(0), 0};
  if (c.na > 0 && lane < c.cnt) {
    const int64_t e = c.e0 + lane;
    r.x = vec[3 * e];
    r.y = vec[3 * e + 1];
    r.z = vec[3 * e + 2];
    r.nb = p.nbr[e];
  }
  return r;
}

// The species channel of the lane's neighbour (-1 past the chunk's edges).
template <int MAXA>
__device__ inline int sp_gather(const SpeciesParams& p, const SpChunk<MAXA>& c, int64_t nb, int lane) {
  if (c.na == 0 || lane >= c.cnt) return -1;
  return p.species ? int(p.species[nb]) : 0;
}

// l_max >= 5 tiles take more than 32 KB of LDS per wave, so one wave per SIMD
// runs anyway: let those kernels use every VGPR (the basis of a chunk is held
// in registers across its loads)
template <typename In, typename Out, int LMAX, int NRC>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, LMAX >= 5 ? 1 : 4))) void
ace_density_species_kernel(SpeciesParams p, NormTable nt) {
  using Sh = SpShape<LMAX, NRC>;
  constexpr int LW = Sh::LW, CT = Sh::CT;
  extern __shared__ __align__(16) double sp_smem[];
  double* const Wt = sp_smem;                    // [NRC][P]
  double* const Yt = sp_smem + NRC * kSpPitch;  // [LW][P]

  const int lane = threadIdx.x;
  const int kq = lane >> 4, cc = lane & 15;
  // the exact-shape instantiations (NRC < 16) run only with NR == NRC
  const int NR = NRC < 16 ? NRC : p.NR, S = p.S;
  const int64_t a_begin = int64_t(blockIdx.x) * p.N / p.waves;
  const int64_t a_end = (int64_t(blockIdx.x) + 1) * p.N / p.waves;
  if (a_begin >= a_end) return;
  const In* __restrict__ vec = static_cast<const In*>(p.vec);
  Out* __restrict__ Aout = static_cast<Out*>(p.A);
  const int64_t block = int64_t(NR) * LW;  // one (atom, species) block
  const uint64_t lt = sp_range(0, lane);   // lanes below this one
  SpOffsets<CT> soff;
  sp_store_offsets<LMAX, NRC, Out>(soff, NR, kq, cc);

  sp_d4 acc[CT];
  // Software pipeline over chunks.  On entry to chunk i (with at most 64
  // edges) the lane holds chunk i's edge vector, the gather of its neighbour's
  // species is in flight, and so are chunk i + 1's loads: the one wait, after
  // chunk i's basis, finds them (and chunk i - 1's stores) done, and chunk
  // i + 1's gather and chunk i + 2's loads then go out behind chunk i's
  // accumulation and stores and chunk i + 1's basis.
  constexpr int MAXA = sp_max_atoms<LMAX>();
  SpChunk<MAXA> cur = sp_form<MAXA>(p, a_begin, a_end);
  SpEdges<In> E = sp_load(p, vec, cur, lane);
  int sp = sp_gather(p, cur, E.nb, lane);
  SpChunk<MAXA> nxt = sp_form<MAXA>(p, sp_after(cur), a_end);
  SpEdges<In> NE = sp_load(p, vec, nxt, lane);
  while (cur.a < a_end) {
    if (cur.na == 0) {
      // ---- atom a has more than 64 edges: per species, every 64-edge window
      // of the atom in turn, accumulating in registers; each block is stored once
      const int64_t a = cur.a;
      const int64_t hi = sp_offset(p.offsets, a + 1);
      for (int s = 0; s < S; ++s) {
        sp_zero<CT>(acc);
        for (int64_t t0 = cur.e0; t0 < hi; t0 += 64) {
          const int64_t e = t0 + lane;
          const bool in_s = e < hi && (p.species ? int(p.species[p.nbr[e]]) : 0) == s;
          const uint64_t m = sp_ballot(in_s);
          const int c = __builtin_popcountll(m);
          if (c == 0) continue;
          if (in_s)
            sp_basis_to_tile<LMAX, NRC>(double(vec[3 * e]), double(vec[3 * e + 1]), double(vec[3 * e + 2]), p, nt,
                                        Wt, Yt, __builtin_popcountll(m & lt));
          __syncthreads();
          sp_group_product<LMAX, NRC, false>(Wt, Yt, 0, c, kq, cc, acc);
          __syncthreads();  // operand reads done before the next window's writes
        }
        sp_store<LMAX, NRC, Out>(Aout + (a * S + s) * block, acc, NR, soff);
      }
      // refill the pipeline from the chunk after the atom (its loads are out)
      cur = nxt;
      E = NE;
      sp = sp_gather(p, cur, E.nb, lane);
      nxt = sp_form<MAXA>(p, sp_after(cur), a_end);
      NE = sp_load(p, vec, nxt, lane);
      continue;
    }

    // ---- chunk i: basis in registers, the one wait, the next loads out
    const bool valid = lane < cur.cnt;
    double Y[LW], R[NRC];
    sp_basis<LMAX, NRC>(double(E.x), double(E.y), double(E.z), p, nt, Y, R);
    sp_wait_vmem();
    const int nsp = sp_gather(p, nxt, NE.nb, lane);
    const SpChunk<MAXA> nn = sp_form<MAXA>(p, sp_after(nxt), a_end);
    const SpEdges<In> NNE = sp_load(p, vec, nn, lane);

    // ---- sort: (atom, species) groups in column order
    int la = 0;  // the lane's atom within the chunk
#pragma unroll
    for (int j = 1; j < MAXA; ++j) la += (j < cur.na && lane >= cur.rel[j]) ? 1 : 0;
    int lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < MAXA; ++j) {
      lo = la == j ? cur.rel[j] : lo;
      hi = la == j ? cur.rel[j + 1] : hi;
    }
    const uint64_t amask = sp_range(lo, hi);
    int col = lo;
#pragma unroll
    for (int s = 0; s < kSpMaxSpecies; ++s) {
      if (s >= S) break;
      const uint64_t m = sp_ballot(valid && sp == s) & amask;
      col += s < sp ? __builtin_popcountll(m) : (s == sp ? __builtin_popcountll(m & lt) : 0);
    }
    if (valid) {
#pragma unroll
      for (int n = 0; n < NRC; ++n) Wt[n * kSpPitch + col] = R[n];
#pragma unroll
      for (int k = 0; k < LW; ++k) Yt[k * kSpPitch + col] = Y[k];
    }
    __syncthreads();

    // ---- phase 2: one product per (atom, species) group
    for (int j = 0; j < cur.na; ++j) {
      int rj = 0, rj1 = 0;  // chunk-relative columns of atom j
#pragma unroll
      for (int k = 0; k < MAXA; ++k) {
        rj = k == j ? cur.rel[k] : rj;
        rj1 = k == j ? cur.rel[k + 1] : rj1;
      }
      const uint64_t am = sp_range(rj, rj1);
      int base = rj;
      for (int s = 0; s < S; ++s) {
        const int c = __builtin_popcountll(sp_ballot(valid && sp == s) & am);
        Out* __restrict__ dst = Aout + ((cur.a + j) * S + s) * block;
        if (c > 0) {
          sp_d4 g[CT];  // the group's own accumulators, set by its first k-block
          sp_group_product<LMAX, NRC, true>(Wt, Yt, base, c, kq, cc, g);
          sp_store<LMAX, NRC, Out>(dst, g, NR, soff);
        } else {
          sp_store_zero<LMAX, NRC, Out>(dst, NR, soff);
        }
        base += c;
      }
    }
    __syncthreads();  // tile reads done before the next chunk's writes
    cur = nxt;
    E = NE;
    sp = nsp;
    nxt = nn;
    NE = NNE;
  }
}

template <typename In, typename Out, int LMAX, int NRC>
int launch_species(const ye3t_density_args* a, void* A, hipStream_t stream) {
  using Sh = SpShape<LMAX, NRC>;
  SpeciesParams p;
  p.N = a->atom_count;
  p.offsets = a->row_offsets;
  p.nbr = a->neighbors;
  p.vec = a->edge_vectors;
  p.species = a->species;
  p.S = int(a->channel_count);
  p.NR = int(a->max_radial_index) + 1;
  p.cutoff = a->cutoff > 2.220446049250313e-16 ? a->cutoff : 2.220446049250313e-16;
  p.lambda = a->lambda;
  p.den = std::expm1(a->lambda);
  p.eps = a->epsilon;
  p.A = A;
  const size_t lds = sizeof(double) * size_t(Sh::ROWS) * kSpPitch;
  const void* kernel = reinterpret_cast<const void*>(&ace_density_species_kernel<In, Out, LMAX, NRC>);
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64, lds) != hipSuccess || per_cu <= 0) per_cu = 2;
  const char* env = std::getenv("YE3T_DENSITY_WAVES");  // tuning
  int64_t waves = (env && *env) ? std::atoll(env) : int64_t(cus) * per_cu;
  if (waves < 1) waves = 1;
  if (waves > p.N) waves = p.N;
  p.waves = waves;
  hipLaunchKernelGGL((ace_density_species_kernel<In, Out, LMAX, NRC>), dim3(unsigned(waves)), dim3(64), lds, stream,
                     p, norm_table());
  set_density_kernel("ace_density_species_kernel");
  return check_launch("ace_density_species_kernel");
}

// The benchmark shapes get their exact radial row count; every other n_max
// runs with 16 rows computed and the unused ones not stored.
template <typename In, typename Out, int LMAX>
int launch_species_l(const ye3t_density_args* a, void* A, hipStream_t stream) {
  const int64_t nr = a->max_radial_index + 1;
  if (LMAX == 3 && nr == 9) return launch_species<In, Out, LMAX, 9>(a, A, stream);
  if (LMAX == 4 && nr == 11) return launch_species<In, Out, LMAX, 11>(a, A, stream);
  if (LMAX == 6 && nr == 13) return launch_species<In, Out, LMAX, 13>(a, A, stream);
  return launch_species<In, Out, LMAX, 16>(a, A, stream);
}

}  // namespace

// One-hot species densities (and single-channel densities without species)
// with n_max <= 15 and l_max <= 8, accumulated in fp64 and stored as Out;
// YE3T_EUNSUPPORTED (nothing launched) otherwise.
template <typename In, typename Out>
int launch_density_species(const ye3t_density_args* a, void* A, hipStream_t stream) {
  if (a->node_features) return YE3T_EUNSUPPORTED;
  if (a->max_radial_index > 15 || a->max_angular > 8) return YE3T_EUNSUPPORTED;
  if (a->channel_count > kSpMaxSpecies || (!a->species && a->channel_count != 1)) return YE3T_EUNSUPPORTED;
  if (a->atom_count == 0) return YE3T_OK;
  switch (a->max_angular) {
    case 0: return launch_species_l<In, Out, 0>(a, A, stream);
    case 1: return launch_species_l<In, Out, 1>(a, A, stream);
    case 2: return launch_species_l<In, Out, 2>(a, A, stream);
    case 3: return launch_species_l<In, Out, 3>(a, A, stream);
    case 4: return launch_species_l<In, Out, 4>(a, A, stream);
    case 5: return launch_species_l<In, Out, 5>(a, A, stream);
    case 6: return launch_species_l<In, Out, 6>(a, A, stream);
    case 7: return launch_species_l<In, Out, 7>(a, A, stream);
    default: return launch_species_l<In, Out, 8>(a, A, stream);
  }
}

template int launch_density_species<float, double>(const ye3t_density_args*, void*, hipStream_t);
template int launch_density_species<double, double>(const ye3t_density_args*, void*, hipStream_t);
template int launch_density_species<float, float>(const ye3t_density_args*, void*, hipStream_t);

}  // namespace ye3t
