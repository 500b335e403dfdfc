// On-device neighbour list in the CSR convention of the density inputs: for
// each centre i the neighbours j != i with |r_j - r_i| < cutoff, in ascending
// j, which is the stable (target, source) order that
// prepare_carrier_scatter_segments (execution_plan.py:9316-9434) gives edges
// keyed target*N + source; edge vectors r_j - r_i in the input type.
//
// Open boundaries.  count():
//   1. atoms are binned into a cell grid of edge >= cutoff by a counting sort
//      (per-cell atomic counters give each atom a slot, an inclusive scan of
//      the counts gives the cell starts, a scatter places the atoms and a
//      copy of their positions in cell order);
//   2. one wave per atom, atoms taken in cell order: the candidates are the
//      9 (x, y) columns of 3 z-cells around the atom's cell, each a contiguous
//      range of the cell-ordered copy; the 64 lanes test 64 candidates at a
//      time and a ballot counts the hits;
//   3. an inclusive scan of the counts gives the row offsets.
// fill() repeats the enumeration, collects the hits of a row in LDS and writes
// each at its rank among them (the number of smaller neighbour indices): the
// row comes out ascending without a sort.  Rows longer than the LDS buffer are
// built by one lane with an insertion in global memory.
// The within-cell order depends on the atomics, the rows do not: each row is
// a set ordered by a unique key.  The distance test is done in fp64 with every
// operation rounded on its own (no contraction), so rows do not depend on the
// compiler's fma choices and a scalar C loop reproduces them bit for bit.
#include <cstdint>

#include "common.h"

namespace ye3t {
namespace {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int64_t kScanTile = kScanThreads * kScanItems;
constexpr int kRowThreads = 256;  // 4 waves, one atom each
constexpr int kRowCap = 512;      // LDS entries per wave for a row

struct CellGrid {
  double origin[3];
  double inv_cell;  // 1 / cell edge
  int dims[3];
};

struct alignas(32) Pos4 {  // a position widened to fp64, padded to 32 bytes
  double x, y, z, pad;
};

// ---- device scan (inclusive, in place), three levels at most for n < 2^31 ---

template <typename T>
__global__ __launch_bounds__(kScanThreads) void scan_tile_kernel(T* __restrict__ data, int64_t n,
                                                                 T* __restrict__ tile_sums) {
  __shared__ T tile[kScanTile];
  __shared__ T wave_sums[kScanThreads / 64];
  const int64_t base = int64_t(blockIdx.x) * kScanTile;
  const int t = threadIdx.x;
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t x = base + k * kScanThreads + t;
    tile[k * kScanThreads + t] = x < n ? data[x] : T(0);
  }
  __syncthreads();
  T v[kScanItems];
  T run = 0;
  for (int k = 0; k < kScanItems; ++k) {
    run += tile[t * kScanItems + k];
    v[k] = run;
  }
  const int lane = t & 63;
  T incl = run;
  for (int d = 1; d < 64; d <<= 1) {
    const T o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wave_sums[t >> 6] = incl;
  __syncthreads();
  T before = 0;
  for (int w = 0; w < (t >> 6); ++w) before += wave_sums[w];
  const T excl = before + incl - run;
  for (int k = 0; k < kScanItems; ++k) tile[t * kScanItems + k] = v[k] + excl;
  __syncthreads();
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t x = base + k * kScanThreads + t;
    if (x < n) data[x] = tile[k * kScanThreads + t];
  }
  if (tile_sums != nullptr && t == kScanThreads - 1) tile_sums[blockIdx.x] = before + incl;
}

// adds the inclusive prefix of the tiles before each tile (tile_sums scanned)
template <typename T>
__global__ __launch_bounds__(kScanThreads) void scan_add_kernel(T* __restrict__ data, int64_t n,
                                                                const T* __restrict__ tile_sums) {
  if (blockIdx.x == 0) return;
  const T add = tile_sums[blockIdx.x - 1];
  const int64_t base = int64_t(blockIdx.x) * kScanTile;
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t x = base + k * kScanThreads + threadIdx.x;
    if (x < n) data[x] += add;
  }
}

int64_t round64(int64_t n) { return (n + 63) & ~int64_t(63); }

// elements of scratch the scan of n values needs for its tile sums
int64_t scan_partials(int64_t n) {
  int64_t total = 0;
  while (n > kScanTile) {
    n = (n + kScanTile - 1) / kScanTile;
    total += round64(n);
  }
  return total;
}

template <typename T>
int scan_inclusive(T* data, int64_t n, T* partials, hipStream_t s) {
  if (n <= 0) return YE3T_OK;
  const int64_t tiles = (n + kScanTile - 1) / kScanTile;
  if (tiles == 1) {
    hipLaunchKernelGGL(scan_tile_kernel<T>, dim3(1), dim3(kScanThreads), 0, s, data, n, (T*)nullptr);
    return check_launch("scan_tile_kernel");
  }
  hipLaunchKernelGGL(scan_tile_kernel<T>, dim3(unsigned(tiles)), dim3(kScanThreads), 0, s, data, n, partials);
  int rc = check_launch("scan_tile_kernel");
  if (rc != YE3T_OK) return rc;
  rc = scan_inclusive(partials, tiles, partials + round64(tiles), s);
  if (rc != YE3T_OK) return rc;
  hipLaunchKernelGGL(scan_add_kernel<T>, dim3(unsigned(tiles)), dim3(kScanThreads), 0, s, data, n,
                     (const T*)partials);
  return check_launch("scan_add_kernel");
}

// ---- binning ---------------------------------------------------------------

__global__ void clear_cells_kernel(int32_t* __restrict__ cell_start, int64_t cells, int64_t* __restrict__ row0) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; c <= cells; c += stride) cell_start[c] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0 && row0 != nullptr) row0[0] = 0;
}

__device__ inline int cell_coord(double x, double o, double inv, int n) {
  const double u = floor(__dmul_rn(__dsub_rn(x, o), inv));
  return !(u >= 0.0) ? 0 : (u >= double(n) ? n - 1 : int(u));  // NaN -> cell 0
}

__device__ inline int32_t cell_of_point(double x, double y, double z, const CellGrid& g) {
  const int cx = cell_coord(x, g.origin[0], g.inv_cell, g.dims[0]);
  const int cy = cell_coord(y, g.origin[1], g.inv_cell, g.dims[1]);
  const int cz = cell_coord(z, g.origin[2], g.inv_cell, g.dims[2]);
  return (cx * g.dims[1] + cy) * g.dims[2] + cz;
}

template <typename T>
__global__ __launch_bounds__(256) void bin_atoms_kernel(const T* __restrict__ pos, int32_t N, CellGrid g,
                                                        int32_t* __restrict__ cell_start,
                                                        int32_t* __restrict__ cell_of, int32_t* __restrict__ slot) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= N) return;
  const int32_t i = int32_t(t);
  const int32_t c = cell_of_point(double(pos[3 * t]), double(pos[3 * t + 1]), double(pos[3 * t + 2]), g);
  cell_of[i] = c;
  slot[i] = atomicAdd(cell_start + c + 1, 1);
}

template <typename T>
__global__ __launch_bounds__(256) void place_atoms_kernel(const T* __restrict__ pos, int32_t N,
                                                          const int32_t* __restrict__ cell_start,
                                                          const int32_t* __restrict__ cell_of,
                                                          const int32_t* __restrict__ slot,
                                                          int32_t* __restrict__ order, Pos4* __restrict__ spos) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= N) return;
  const int32_t i = int32_t(t);
  const int32_t k = cell_start[cell_of[i]] + slot[i];
  order[k] = i;
  Pos4 p;
  p.x = double(pos[3 * t]);
  p.y = double(pos[3 * t + 1]);
  p.z = double(pos[3 * t + 2]);
  p.pad = 0.0;
  spos[k] = p;
}

// ---- rows ------------------------------------------------------------------

// |r_j - r_i|^2 < rc2, each fp64 operation rounded on its own
__device__ inline bool within(double xi, double yi, double zi, double xj, double yj, double zj, double rc2) {
  const double dx = __dsub_rn(xj, xi);
  const double dy = __dsub_rn(yj, yi);
  const double dz = __dsub_rn(zj, zi);
  return __dadd_rn(__dadd_rn(__dmul_rn(dx, dx), __dmul_rn(dy, dy)), __dmul_rn(dz, dz)) < rc2;
}

// The 9 (x, y) columns around cell c: column q covers the cell-ordered range
// [k0[q], k0[q] + pre[q + 1] - pre[q]) (its z-cells are adjacent in order[]);
// pre[] is the running candidate count.  Empty or clipped columns have length 0.
__device__ inline void cell_columns(int32_t c, const CellGrid& g, const int32_t* __restrict__ cell_start,
                                    int32_t* k0, int32_t* pre) {
  const int cz = c % g.dims[2];
  const int cy = (c / g.dims[2]) % g.dims[1];
  const int cx = c / (g.dims[1] * g.dims[2]);
  const int zlo = cz > 0 ? cz - 1 : 0;
  const int zend = cz + 2 < g.dims[2] ? cz + 2 : g.dims[2];
  pre[0] = 0;
#pragma unroll
  for (int q = 0; q < 9; ++q) {
    const int ax = cx + q / 3 - 1, ay = cy + q % 3 - 1;
    int32_t a = 0, b = 0;
    if (ax >= 0 && ax < g.dims[0] && ay >= 0 && ay < g.dims[1]) {
      const int32_t row = (ax * g.dims[1] + ay) * g.dims[2];
      a = cell_start[row + zlo];
      b = cell_start[row + zend];
    }
    k0[q] = a;
    pre[q + 1] = pre[q] + (b - a);
  }
}

// cell-ordered index of candidate v < pre[9]
__device__ inline int32_t candidate(int32_t v, const int32_t* k0, const int32_t* pre) {
  int32_t k = 0;
#pragma unroll
  for (int q = 0; q < 9; ++q)
    if (v >= pre[q] && v < pre[q + 1]) k = k0[q] + (v - pre[q]);
  return k;
}

template <typename T>
__device__ inline void write_edge(int64_t e, int32_t i, int32_t j, const Pos4& pj, const Pos4& pi,
                                  int64_t* __restrict__ centers, int64_t* __restrict__ nbr, T* __restrict__ vec) {
  centers[e] = i;
  nbr[e] = j;
  // widened positions narrow back exactly: r_j - r_i rounds once, in T
  vec[3 * e] = T(pj.x) - T(pi.x);
  vec[3 * e + 1] = T(pj.y) - T(pi.y);
  vec[3 * e + 2] = T(pj.z) - T(pi.z);
}

// Rows of kGroup consecutive cell-ordered atoms per wave: neighbouring atoms
// mostly share a cell, so the wave reuses the cell's column ranges and keeps
// the first kCached * 64 candidate positions in registers across them.
constexpr int kGroup = 4;
constexpr int kCached = 4;

// FILL = false: row_offsets[i + 1] = number of neighbours of i.
// FILL = true: row i at row_offsets[i], ascending; entries at or beyond
// edge_capacity are not written and a row cut by it holds its smallest
// neighbours.  Rows up to kRowCap entries are collected in LDS and each hit is
// written at its rank; longer rows are built by one lane in global memory.
template <bool FILL, typename T>
__global__ __launch_bounds__(kRowThreads) void neighbor_rows_kernel(
    const Pos4* __restrict__ spos, int32_t N, CellGrid g, const int32_t* __restrict__ cell_start,
    const int32_t* __restrict__ order, double rc2, int64_t* __restrict__ row_offsets, int64_t edge_capacity,
    int64_t* __restrict__ centers, int64_t* __restrict__ nbr, T* __restrict__ vec) {
  // per wave: the hits of a row as (j, k) in arrival order, then k at its rank
  __shared__ int32_t row_j[FILL ? kRowThreads / 64 : 1][FILL ? kRowCap : 1];
  __shared__ int32_t row_k[FILL ? kRowThreads / 64 : 1][FILL ? kRowCap : 1];
  __shared__ int32_t out_k[FILL ? kRowThreads / 64 : 1][FILL ? kRowCap : 1];
  const int64_t t0 = (int64_t(blockIdx.x) * (kRowThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) *
                     kGroup;
  if (t0 >= N) return;
  const int64_t t1 = t0 + kGroup < N ? t0 + kGroup : N;
  const int lane = threadIdx.x & 63;
  const int wave = FILL ? (threadIdx.x >> 6) : 0;
  const uint64_t below = (uint64_t(1) << lane) - 1;
  int32_t cell = -1;
  int32_t k0[9], pre[10];
  double cx[kCached], cy[kCached], cz[kCached];
  int32_t ck[kCached], cj[kCached];
  // the group's atoms and row bounds, loaded ahead of the per-atom work
  int32_t gi[kGroup];
  int64_t gb[kGroup], gs[kGroup];
#pragma unroll
  for (int a = 0; a < kGroup; ++a) {
    gi[a] = order[t0 + a < t1 ? t0 + a : t0];
    if (FILL) {
      gb[a] = row_offsets[gi[a]];
      gs[a] = row_offsets[gi[a] + 1];
    }
  }
#pragma unroll
  for (int a = 0; a < kGroup; ++a) {
    const int64_t t = t0 + a;
    if (t >= t1) break;
    const Pos4 pi = spos[t];
    const int32_t c = cell_of_point(pi.x, pi.y, pi.z, g);
    if (c != cell) {  // uniform: a new cell's columns and cached candidates
      cell = c;
      cell_columns(c, g, cell_start, k0, pre);
#pragma unroll
      for (int r = 0; r < kCached; ++r) {
        const int32_t v = r * 64 + lane;
        ck[r] = v < pre[9] ? candidate(v, k0, pre) : -1;
        const Pos4 pj = spos[ck[r] < 0 ? 0 : ck[r]];
        cx[r] = pj.x;
        cy[r] = pj.y;
        cz[r] = pj.z;
        if (FILL) cj[r] = order[ck[r] < 0 ? 0 : ck[r]];
      }
    }
    const int32_t i = gi[a];
    const int32_t total = pre[9];
    int64_t base = 0, len = 0;
    if (FILL) {
      base = gb[a];
      const int64_t stop = gs[a];
      const int64_t end = stop < edge_capacity ? stop : edge_capacity;
      len = (base >= 0 && end > base) ? end - base : 0;
      if (len == 0) continue;
      if (stop - base > kRowCap) {
        // a long row: lane 0 inserts each hit, keyed (j << 32) | k, into the
        // sorted prefix nbr[base, base + min(n, len)); the key orders by j
        if (lane == 0) {
          int64_t n = 0;
          int64_t* r = nbr + base;
          for (int32_t v = 0; v < total; ++v) {
            const int32_t k = candidate(v, k0, pre);
            if (k == t) continue;
            const Pos4 pj = spos[k];
            if (!within(pi.x, pi.y, pi.z, pj.x, pj.y, pj.z, rc2)) continue;
            const int64_t key = (int64_t(order[k]) << 32) | int64_t(k);
            int64_t b = (n < len ? n : len) - 1;
            if (n < len || key < r[len - 1]) {
              if (n >= len) --b;  // full: the largest entry drops out
              while (b >= 0 && r[b] > key) {
                r[b + 1] = r[b];
                --b;
              }
              r[b + 1] = key;
            }
            ++n;
          }
          const int64_t written = n < len ? n : len;
          for (int64_t a = 0; a < written; ++a) {
            const int64_t key = r[a];
            write_edge(base + a, i, int32_t(key >> 32), spos[int32_t(key & 0xffffffff)], pi, centers, nbr, vec);
          }
        }
        continue;
      }
    }
    int32_t n = 0;
    auto take = [&](bool hit, int32_t j, int32_t k) {
      const uint64_t mask = __ballot(hit);
      if (FILL) {
        const int32_t slot = n + __popcll(mask & below);
        if (hit && slot < kRowCap) {
          row_j[wave][slot] = j;
          row_k[wave][slot] = k;
        }
      }
      n += __popcll(mask);
    };
#pragma unroll
    for (int r = 0; r < kCached; ++r) {
      const bool hit = r * 64 < total && ck[r] >= 0 && ck[r] != t &&
                       within(pi.x, pi.y, pi.z, cx[r], cy[r], cz[r], rc2);
      take(hit, FILL ? cj[r] : 0, ck[r]);
    }
    for (int32_t v0 = kCached * 64; v0 < total; v0 += 64) {
      const int32_t v = v0 + lane;
      bool hit = false;
      int32_t k = 0;
      if (v < total) {
        k = candidate(v, k0, pre);
        if (k != t) {
          const Pos4 pj = spos[k];
          hit = within(pi.x, pi.y, pi.z, pj.x, pj.y, pj.z, rc2);
        }
      }
      take(hit, FILL && hit ? order[k] : 0, k);
    }
    if (!FILL) {
      if (lane == 0) row_offsets[i + 1] = n;
      continue;
    }
    // the row's LDS entries were written by other lanes of this wave
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // rank of each hit = number of smaller j (j is unique): a permutation of [0, held)
    const int32_t held = n < kRowCap ? n : kRowCap;
    for (int32_t e = lane; e < held; e += 64) {
      const int32_t j = row_j[wave][e];
      int32_t rank = 0;
      for (int32_t q = 0; q < held; ++q) rank += row_j[wave][q] < j;
      out_k[wave][rank] = row_k[wave][e];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the row in order: consecutive lanes write consecutive edges
    const int32_t count = held < len ? held : int32_t(len);
    for (int32_t e = lane; e < count; e += 64) {
      const uint32_t kk = uint32_t(out_k[wave][e]);
      const int32_t k = kk < uint32_t(N) ? int32_t(kk) : 0;  // always a permutation; clamped regardless
      write_edge(base + e, i, order[k], spos[k], pi, centers, nbr, vec);
    }
    // every lane has read the row before the next atom overwrites it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// ---- host side -------------------------------------------------------------

struct Workspace {
  int32_t* cell_start;  // [cells + 1]
  int32_t* cell_of;     // [N]
  int32_t* slot;        // [N]
  int32_t* order;       // [N] atom at each cell-ordered slot
  Pos4* spos;           // [N] positions in cell order
  int64_t* partials;    // scan scratch
  int64_t bytes;
};

int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }

int64_t cell_count(const ye3t_cell_grid* g) { return g->dims[0] * g->dims[1] * g->dims[2]; }

Workspace layout(void* base, int64_t N, int64_t cells) {
  Workspace w;
  char* p = static_cast<char*>(base);
  int64_t off = 0;
  w.cell_start = reinterpret_cast<int32_t*>(p + off);
  off += align256(4 * (cells + 1));
  w.cell_of = reinterpret_cast<int32_t*>(p + off);
  off += align256(4 * N);
  w.slot = reinterpret_cast<int32_t*>(p + off);
  off += align256(4 * N);
  w.order = reinterpret_cast<int32_t*>(p + off);
  off += align256(4 * N);
  w.spos = reinterpret_cast<Pos4*>(p + off);
  off += align256(int64_t(sizeof(Pos4)) * N);
  w.partials = reinterpret_cast<int64_t*>(p + off);
  off += align256(8 * scan_partials(N > cells ? N : cells));
  w.bytes = off;
  return w;
}

int check_args(int64_t N, const ye3t_cell_grid* grid, double cutoff) {
  YE3T_REQUIRE(N >= 0 && N < (int64_t(1) << 31) - 1, "atom count must be in [0, 2^31 - 1)");
  YE3T_REQUIRE(grid != nullptr, "NULL cell grid");
  for (int a = 0; a < 3; ++a)
    YE3T_REQUIRE(grid->dims[a] >= 1 && grid->dims[a] <= (int64_t(1) << 24), "cell grid dims must be in [1, 2^24]");
  YE3T_REQUIRE(cell_count(grid) < (int64_t(1) << 31) - 1, "cell grid has 2^31 - 1 or more cells");
  YE3T_REQUIRE(grid->cell_edge > 0.0, "cell edge must be positive");
  // cells wider than the cutoff by a margin far above the rounding of the
  // cell coordinates (|u| <= 2^24 cells), so every pair within the cutoff lies
  // in neighbouring cells
  YE3T_REQUIRE(cutoff > 0.0 && cutoff * (1.0 + 1e-9) <= grid->cell_edge,
               "cutoff must be positive and at most cell_edge / (1 + 1e-9)");
  return YE3T_OK;
}

CellGrid device_grid(const ye3t_cell_grid* grid) {
  CellGrid g;
  for (int a = 0; a < 3; ++a) {
    g.origin[a] = grid->origin[a];
    g.dims[a] = int(grid->dims[a]);
  }
  g.inv_cell = 1.0 / grid->cell_edge;
  return g;
}

// blocks of the row kernels: kRowThreads / 64 waves of kGroup atoms each
unsigned row_blocks(int64_t n) {
  const int64_t per = int64_t(kRowThreads / 64) * kGroup;
  const int64_t b = (n + per - 1) / per;
  return unsigned(b < 1 ? 1 : b);
}

unsigned blocks_for(int64_t n, int threads) {
  const int64_t b = (n + threads - 1) / threads;
  return unsigned(b < 1 ? 1 : b);
}

template <typename T>
int count_rows(const T* pos, int32_t N, const ye3t_cell_grid* grid, double cutoff, const Workspace& w,
               int64_t* row_offsets, hipStream_t s) {
  const CellGrid g = device_grid(grid);
  const int64_t cells = cell_count(grid);
  hipLaunchKernelGGL(clear_cells_kernel, dim3(blocks_for(cells + 1, 256) > 4096 ? 4096 : blocks_for(cells + 1, 256)),
                     dim3(256), 0, s, w.cell_start, cells, row_offsets);
  int rc = check_launch("clear_cells_kernel");
  if (rc != YE3T_OK || N == 0) return rc;
  hipLaunchKernelGGL(bin_atoms_kernel<T>, dim3(blocks_for(N, 256)), dim3(256), 0, s, pos, N, g, w.cell_start,
                     w.cell_of, w.slot);
  if ((rc = check_launch("bin_atoms_kernel")) != YE3T_OK) return rc;
  if ((rc = scan_inclusive<int32_t>(w.cell_start + 1, cells, reinterpret_cast<int32_t*>(w.partials), s)) != YE3T_OK)
    return rc;
  hipLaunchKernelGGL(place_atoms_kernel<T>, dim3(blocks_for(N, 256)), dim3(256), 0, s, pos, N,
                     (const int32_t*)w.cell_start, (const int32_t*)w.cell_of, (const int32_t*)w.slot, w.order, w.spos);
  if ((rc = check_launch("place_atoms_kernel")) != YE3T_OK) return rc;
  hipLaunchKernelGGL((neighbor_rows_kernel<false, T>), dim3(row_blocks(N)), dim3(kRowThreads), 0, s,
                     (const Pos4*)w.spos, N, g, (const int32_t*)w.cell_start, (const int32_t*)w.order,
                     cutoff * cutoff, row_offsets, int64_t(0), (int64_t*)nullptr, (int64_t*)nullptr, (T*)nullptr);
  if ((rc = check_launch("neighbor_rows_kernel")) != YE3T_OK) return rc;
  return scan_inclusive<int64_t>(row_offsets + 1, N, w.partials, s);
}

template <typename T>
int fill_rows(int32_t N, const ye3t_cell_grid* grid, double cutoff, const Workspace& w,
              const int64_t* row_offsets, int64_t edge_capacity, int64_t* centers, int64_t* neighbors, T* vec,
              hipStream_t s) {
  if (N == 0) return YE3T_OK;
  hipLaunchKernelGGL((neighbor_rows_kernel<true, T>), dim3(row_blocks(N)), dim3(kRowThreads), 0, s,
                     (const Pos4*)w.spos, N, device_grid(grid), (const int32_t*)w.cell_start,
                     (const int32_t*)w.order, cutoff * cutoff, const_cast<int64_t*>(row_offsets), edge_capacity,
                     centers, neighbors, vec);
  return check_launch("neighbor_rows_kernel");
}

}  // namespace
}  // namespace ye3t

using namespace ye3t;

extern "C" {

int64_t ye3t_hip_neighbor_workspace_bytes(int64_t atom_count, const ye3t_cell_grid* grid) {
  clear_error();
  if (atom_count < 0 || grid == nullptr || grid->dims[0] < 1 || grid->dims[1] < 1 || grid->dims[2] < 1) {
    set_error(YE3T_EINVAL, "invalid atom count or cell grid");
    return -1;
  }
  return layout(nullptr, atom_count, cell_count(grid)).bytes;
}

int ye3t_hip_neighbor_count(int dtype, const void* positions, int64_t atom_count, const ye3t_cell_grid* grid,
                            double cutoff, void* workspace, int64_t workspace_bytes, int64_t* row_offsets,
                            ye3t_stream_t stream) {
  clear_error();
  int rc = check_args(atom_count, grid, cutoff);
  if (rc != YE3T_OK) return rc;
  const Workspace w = layout(workspace, atom_count, cell_count(grid));
  YE3T_REQUIRE(workspace != nullptr && workspace_bytes >= w.bytes, "workspace of %lld bytes needed",
               (long long)w.bytes);
  YE3T_REQUIRE(row_offsets != nullptr, "NULL row_offsets");
  YE3T_REQUIRE(atom_count == 0 || positions != nullptr, "NULL positions");
  const hipStream_t s = as_stream(stream);
  if (dtype == YE3T_F64) return count_rows((const double*)positions, int32_t(atom_count), grid, cutoff, w, row_offsets, s);
  if (dtype == YE3T_F32) return count_rows((const float*)positions, int32_t(atom_count), grid, cutoff, w, row_offsets, s);
  return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
}

int ye3t_hip_neighbor_fill(int dtype, int64_t atom_count, const ye3t_cell_grid* grid, double cutoff,
                           const void* workspace, int64_t workspace_bytes, const int64_t* row_offsets,
                           int64_t edge_capacity, int64_t* centers, int64_t* neighbors, void* edge_vectors,
                           ye3t_stream_t stream) {
  clear_error();
  int rc = check_args(atom_count, grid, cutoff);
  if (rc != YE3T_OK) return rc;
  const Workspace w = layout(const_cast<void*>(workspace), atom_count, cell_count(grid));
  YE3T_REQUIRE(workspace != nullptr && workspace_bytes >= w.bytes, "workspace of %lld bytes needed",
               (long long)w.bytes);
  YE3T_REQUIRE(edge_capacity >= 0, "negative edge capacity");
  YE3T_REQUIRE(row_offsets != nullptr, "NULL row_offsets");
  YE3T_REQUIRE(edge_capacity == 0 || (centers && neighbors && edge_vectors), "NULL edge outputs");
  const hipStream_t s = as_stream(stream);
  if (dtype == YE3T_F64)
    return fill_rows<double>(int32_t(atom_count), grid, cutoff, w, row_offsets, edge_capacity,
                     centers, neighbors, (double*)edge_vectors, s);
  if (dtype == YE3T_F32)
    return fill_rows<float>(int32_t(atom_count), grid, cutoff, w, row_offsets, edge_capacity,
                     centers, neighbors, (float*)edge_vectors, s);
  return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
}

}  // extern "C"
