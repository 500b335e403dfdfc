// Stage 1 with one-hot species channels on the matrix cores:
//
//   A[i, s, n, lm] = sum_{e in row i, species(nbr_e) = s} R_n(|v_e|) Y_lm(v_e / |v_e|)
//
// (the reference's radial table, real harmonics, scheduled_radial_angular
// channel product and density_accumulate, ye3t_runtime_core.cpp:214-423,
// 1550-1604, 1684-1702, fused).  Each (atom, species) pair is a small
// [NR x edges] x [edges x LW] product; an edge contributes to exactly one of
// them, so the kernel groups the edges of every atom by neighbour species and
// multiplies each group alone -- no work on edges of other species.
//
// One wave (a 64-thread workgroup; no barriers between waves) owns a
// contiguous atom range (as many waves as the device holds at once) and walks
// it in chunks of up to 16 consecutive whole atoms with at most 64 edges
// together:
//   sort     lane = edge; the neighbour's species is gathered, one ballot per
//            species gives every (atom, species) group's lanes, and each lane
//            computes its column in the chunk's tile: its atom's first
//            column, plus the sizes of the atom's groups of smaller species,
//            plus its rank within its own group (a stable counting sort);
//   phase 1  lane = edge; the radial values and real harmonics in fp64
//            registers, written to LDS transposed at the sorted column
//            ([n][col], [lm][col]);
//   phase 2  per (atom, species) group, the k-blocks of four columns it
//            covers, one v_mfma_f64_16x16x4f64 per 16-column harmonic tile
//            (columns of neighbouring groups masked to zero), alternating
//            between two accumulator sets; the group's [NR x LW] block then
//            goes from registers to A (species absent from an atom get zero
//            blocks).
// An atom with more than 64 edges is taken alone, species by species: each of
// its 64-edge windows in turn places its edges of that species in the tile
// and adds their product to the same accumulators, so every block is still
// accumulated in registers and stored once.
// The density is accumulated in fp64 and stored as Out (fp64, or fp32
// rounded once).  Lane layouts of the fp64 MFMA (l = lane):
//   A[i][k] from lane i + 16 k; B[k][j] from lane j + 16 k;
//   D[i][j] in lane j + 16 (i mod 4), element i div 4.
#include <cmath>

#include "common.h"
#include "sph.h"

namespace ye3t {
namespace {

constexpr int kSpPitch = 67;     // LDS row pitch (doubles): odd, so 16 rows of one column spread over the banks
constexpr int kSpMaxAtoms = 16;  // whole atoms per chunk
constexpr int kSpMaxSpecies = 16;

typedef double sp_d4 __attribute__((ext_vector_type(4)));

struct SpeciesParams {
  int64_t N;
  const int64_t* __restrict__ offsets;
  const int64_t* __restrict__ nbr;
  const void* __restrict__ vec;
  const int32_t* __restrict__ species;  // null: one channel, every edge in it
  int S;                                // channels
  int NR;                               // radial rows, n_max + 1 (<= 16)
  int LW;                               // (l_max + 1)^2
  int lmax;
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

// bits [lo, hi) of a 64-bit mask (0 <= lo <= hi <= 64)
__device__ inline uint64_t sp_range(int lo, int hi) {
  const uint64_t below_hi = hi >= 64 ? ~uint64_t(0) : ((uint64_t(1) << hi) - 1);
  const uint64_t below_lo = lo >= 64 ? ~uint64_t(0) : ((uint64_t(1) << lo) - 1);
  return below_hi & ~below_lo;
}

// ChebExpCos radial values g_0..g_{nr-1} of one distance (fp64), to out[n * stride]
__device__ inline void sp_radial(double r, const SpeciesParams& p, double* out, int stride) {
  const double s = r / p.cutoff;
  if (s > 1.0) {
    for (int n = 0; n < p.NR; ++n) out[n * stride] = 0.0;
    return;
  }
  const double env = 1.0 + cospi(s);
  out[0] = 1.0;
  if (p.NR > 1) out[stride] = 0.5 * env;
  if (p.NR > 2) {
    const double x = 1.0 - 2.0 * expm1(-p.lambda * (s - 1.0)) / p.den;
    double t0 = 1.0, t1 = x;
    for (int n = 2; n < p.NR; ++n) {
      const double t2 = 2.0 * x * t1 - t0;
      out[n * stride] = 0.25 * (1.0 - t2) * env;
      t0 = t1;
      t1 = t2;
    }
  }
}

// Radial values and harmonics of one edge vector, fp64, into tile column `col`.
__device__ inline void sp_basis_to_tile(double vx, double vy, double vz, const SpeciesParams& p, const NormTable& nt,
                                        double* Wt, double* Yt, int col) {
  const double r = sqrt(vx * vx + vy * vy + vz * vz);
  const double sr = r > p.eps ? r : p.eps;
  const double inv = 1.0 / sr;
  real_sph_row<double, double>(vx * inv, vy * inv, vz * inv, p.lmax, nt, Yt + col, kSpPitch);
  sp_radial(r, p, Wt + col, kSpPitch);
}

// Adds the product of tile columns [base, base + c) to the accumulators: the
// k-blocks of four columns covering them, columns outside masked to zero
// (they read column 0, which holds finite values, and weigh zero), two
// accumulator sets alternating over consecutive k-blocks.
template <int CT>
__device__ inline void sp_group_product(const double* Wt, const double* Yt, int LW, int base, int c, int kq, int cc,
                                        sp_d4 (&acc0)[CT], sp_d4 (&acc1)[CT]) {
  const int kb0 = base >> 2, kb1 = (base + c - 1) >> 2;
  for (int kb = kb0; kb <= kb1; kb += 2) {
    double w[2], y[2][CT];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int cl = 4 * (kb + h) + kq;
      const bool in = cl >= base && cl < base + c;
      const int rc = in ? cl : 0;
      w[h] = in ? Wt[cc * kSpPitch + rc] : 0.0;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const int row = ct * 16 + cc;
        y[h][ct] = row < LW ? Yt[row * kSpPitch + rc] : 0.0;
      }
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc0[ct] = __builtin_amdgcn_mfma_f64_16x16x4f64(w[0], y[0][ct], acc0[ct], 0, 0, 0);
    if (kb + 1 <= kb1) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        acc1[ct] = __builtin_amdgcn_mfma_f64_16x16x4f64(w[1], y[1][ct], acc1[ct], 0, 0, 0);
    }
  }
}

template <int CT>
__device__ inline void sp_zero(sp_d4 (&acc0)[CT], sp_d4 (&acc1)[CT]) {
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    acc0[ct] = sp_d4{0.0, 0.0, 0.0, 0.0};
    acc1[ct] = sp_d4{0.0, 0.0, 0.0, 0.0};
  }
}

// One (atom, species) block [NR x LW] from the accumulators (rounded once to Out).
template <typename Out, int CT>
__device__ inline void sp_store(Out* __restrict__ dst, const sp_d4 (&acc0)[CT], const sp_d4 (&acc1)[CT], int NR,
                                int LW, int kq, int cc) {
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int n = 4 * v + kq, lm = ct * 16 + cc;
      if (n < NR && lm < LW) dst[n * LW + lm] = Out(acc0[ct][v] + acc1[ct][v]);
    }
}

template <typename In, typename Out, int CT>
__global__ __launch_bounds__(64) void ace_density_species_kernel(SpeciesParams p, NormTable nt) {
  extern __shared__ __align__(16) double sp_smem[];
  double* const Wt = sp_smem;                  // [16][P]: rows >= NR stay zero
  double* const Yt = sp_smem + 16 * kSpPitch;  // [LW][P]
  __shared__ int rel[kSpMaxAtoms + 1];         // chunk-relative atom starts

  const int lane = threadIdx.x;
  const int kq = lane >> 4, cc = lane & 15;
  const int NR = p.NR, LW = p.LW, S = p.S;
  const int64_t a_begin = int64_t(blockIdx.x) * p.N / p.waves;
  const int64_t a_end = (int64_t(blockIdx.x) + 1) * p.N / p.waves;
  if (a_begin >= a_end) return;
  for (int q = lane; q < (16 + LW) * kSpPitch; q += 64) sp_smem[q] = 0.0;
  const In* __restrict__ vec = static_cast<const In*>(p.vec);
  Out* __restrict__ Aout = static_cast<Out*>(p.A);
  const int64_t block = int64_t(NR) * LW;  // one (atom, species) block
  const uint64_t lt = sp_range(0, lane);   // lanes below this one
  __syncthreads();

  sp_d4 acc0[CT], acc1[CT];
  int64_t a = a_begin;
  while (a < a_end) {
    // ---- the chunk: whole atoms [a, a + na) within 64 edges
    const int64_t e0 = sp_offset(p.offsets, a);
    // lane l (1..16) tests whether atoms a .. a + l - 1 fit in 64 edges; the
    // fitting lanes are a prefix 1..na (offsets do not decrease)
    const int64_t al = a + lane;
    const int64_t endl = (lane >= 1 && lane <= kSpMaxAtoms && al <= a_end) ? sp_offset(p.offsets, al) : e0 + 65;
    const int na = __builtin_popcountll(sp_ballot(lane >= 1 && endl - e0 <= 64));

    if (na == 0) {
      // ---- atom a has more than 64 edges: per species, every 64-edge window
      // of the atom in turn, accumulating in registers; each block is stored
      // once, whatever the number of windows
      const int64_t hi = sp_offset(p.offsets, a + 1);
      for (int s = 0; s < S; ++s) {
        sp_zero<CT>(acc0, acc1);
        for (int64_t t0 = e0; t0 < hi; t0 += 64) {
          const int64_t e = t0 + lane;
          const bool in_s = e < hi && (p.species ? int(p.species[p.nbr[e]]) : 0) == s;
          const uint64_t m = sp_ballot(in_s);
          const int c = __builtin_popcountll(m);
          if (c == 0) continue;
          if (in_s) sp_basis_to_tile(double(vec[3 * e]), double(vec[3 * e + 1]), double(vec[3 * e + 2]), p, nt, Wt,
                                     Yt, __builtin_popcountll(m & lt));
          __syncthreads();
          sp_group_product<CT>(Wt, Yt, LW, 0, c, kq, cc, acc0, acc1);
          __syncthreads();  // operand reads done before the next window's writes
        }
        sp_store<Out, CT>(Aout + (a * S + s) * block, acc0, acc1, NR, LW, kq, cc);
      }
      a += 1;
      continue;
    }

    if (lane <= na) rel[lane] = lane == 0 ? 0 : int(endl - e0);
    const int cnt = __builtin_amdgcn_readlane(int(endl - e0), na);
    __syncthreads();

    // ---- sort: (atom, species) groups in column order
    const bool valid = lane < cnt;
    const int64_t e = e0 + lane;
    double vx = 0.0, vy = 0.0, vz = 0.0;
    int sp = -1;
    if (valid) {
      vx = double(vec[3 * e]);
      vy = double(vec[3 * e + 1]);
      vz = double(vec[3 * e + 2]);
      sp = p.species ? int(p.species[p.nbr[e]]) : 0;
    }
    int la = 0;  // the lane's atom within the chunk
    for (int j = 1; j < na; ++j) la += (lane >= rel[j]) ? 1 : 0;
    const uint64_t amask = sp_range(rel[la], rel[la + 1]);
    int col = rel[la];
#pragma unroll
    for (int s = 0; s < kSpMaxSpecies; ++s) {
      if (s >= S) break;
      const uint64_t m = sp_ballot(valid && sp == s) & amask;
      col += s < sp ? __builtin_popcountll(m) : (s == sp ? __builtin_popcountll(m & lt) : 0);
    }

    // ---- phase 1: radial values and harmonics of this lane's edge at its column
    if (valid) sp_basis_to_tile(vx, vy, vz, p, nt, Wt, Yt, col);
    __syncthreads();

    // ---- phase 2: one product per (atom, species) group
    for (int j = 0; j < na; ++j) {
      const uint64_t am = sp_range(rel[j], rel[j + 1]);
      int base = rel[j];
      for (int s = 0; s < S; ++s) {
        const int c = __builtin_popcountll(sp_ballot(valid && sp == s) & am);
        Out* __restrict__ dst = Aout + ((a + j) * S + s) * block;
        if (c == 0) {
          for (int q = lane; q < block; q += 64) dst[q] = Out(0);
          continue;
        }
        sp_zero<CT>(acc0, acc1);
        sp_group_product<CT>(Wt, Yt, LW, base, c, kq, cc, acc0, acc1);
        sp_store<Out, CT>(dst, acc0, acc1, NR, LW, kq, cc);
        base += c;
      }
    }
    __syncthreads();  // tile reads done before the next chunk's writes
    a += na;
  }
}

template <typename In, typename Out, int CT>
int launch_species(const ye3t_density_args* a, void* A, hipStream_t stream) {
  SpeciesParams p;
  p.N = a->atom_count;
  p.offsets = a->row_offsets;
  p.nbr = a->neighbors;
  p.vec = a->edge_vectors;
  p.species = a->species;
  p.S = int(a->channel_count);
  p.NR = int(a->max_radial_index) + 1;
  p.LW = int((a->max_angular + 1) * (a->max_angular + 1));
  p.lmax = int(a->max_angular);
  p.cutoff = a->cutoff > 2.220446049250313e-16 ? a->cutoff : 2.220446049250313e-16;
  p.lambda = a->lambda;
  p.den = std::expm1(a->lambda);
  p.eps = a->epsilon;
  p.A = A;
  const size_t lds = sizeof(double) * size_t(16 + p.LW) * kSpPitch;
  const void* kernel = reinterpret_cast<const void*>(&ace_density_species_kernel<In, Out, CT>);
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
  hipLaunchKernelGGL((ace_density_species_kernel<In, Out, CT>), dim3(unsigned(waves)), dim3(64), lds, stream, p,
                     norm_table());
  set_density_kernel("ace_density_species_kernel");
  return check_launch("ace_density_species_kernel");
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
  const int LW = int((a->max_angular + 1) * (a->max_angular + 1));
  switch ((LW + 15) / 16) {
    case 1: return launch_species<In, Out, 1>(a, A, stream);
    case 2: return launch_species<In, Out, 2>(a, A, stream);
    case 3: return launch_species<In, Out, 3>(a, A, stream);
    case 4: return launch_species<In, Out, 4>(a, A, stream);
    case 5: return launch_species<In, Out, 5>(a, A, stream);
    default: return launch_species<In, Out, 6>(a, A, stream);
  }
}

template int launch_density_species<float, double>(const ye3t_density_args*, void*, hipStream_t);
template int launch_density_species<double, double>(const ye3t_density_args*, void*, hipStream_t);
template int launch_density_species<float, float>(const ye3t_density_args*, void*, hipStream_t);

}  // namespace ye3t
