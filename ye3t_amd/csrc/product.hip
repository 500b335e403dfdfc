// Stage 2 -- ACE B-features from the density on gfx950.
//
// (a) product_stream_kernel (the default interpreter) and product_kernel (the
//     program-word interpreter it replaces where its workspace fits): execute
//     a compiled product plan.  The plan is a DAG of
//     leaf loads, symmetric-block monomials and real CG pair couplings, shared
//     across labels and contents (intermediate couplings computed once per
//     sample).  One wave (64 lanes) processes 64 samples, lane = sample; the
//     instruction stream and coefficients are wave-uniform (scalar loads), the
//     per-sample workspace lives in LDS as [slot][65] (lane-minor, padded so the
//     transposed output read is bank-conflict free).  Output columns of a chunk
//     are written through LDS so each store instruction covers contiguous
//     columns of one row.
// (b) evaluate_schedule_kernel: device version of the reference's flat
//     schedule evaluator (the symmetric-power contractions are in monomial.hip).
#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"

struct ye3t_hip_product_plan {
  int dtype;      // coefficients and arithmetic (and A unless in_dtype differs)
  int out_dtype;  // B
  int in_dtype;   // A (fp32 rows into fp64 arithmetic: generated kernels only)
  int64_t a_width;
  int64_t feature_count;
  int64_t chunk_count;
  int64_t slots;
  int device;
  uint32_t* words;
  void* coeffs;
  uint16_t* out_slots;
  int64_t* word_off;   // [chunks+1]
  int64_t* coeff_off;  // [chunks+1]
  int64_t* out_off;    // [chunks+1]
  int64_t* first_col;  // [chunks]
  // plan-specialised kernel (optional)
  hipModule_t module;
  hipFunction_t generated;
  int64_t generated_chunks;
  int64_t generated_rows;  // samples per workgroup tile of the generated kernel
  int generated_threads;   // threads per workgroup of the generated kernel
  int64_t generated_max_grid;  // persistent kernel: workgroups resident at once (0: not persistent)
  // plan-specialised kernel in parts (plans too large for one module): part i
  // computes part_chunks[i] consecutive chunks, one per grid row, 64-row tiles
  int64_t part_count;
  hipModule_t* part_modules;
  hipFunction_t* part_fns;
  int64_t* part_chunks;
  // the parts run concurrently on part_lanes streams of the plan, forked from
  // and joined back to the caller's stream with events (1: the caller's stream only)
  int part_lanes;
  hipStream_t part_streams[4];
  hipEvent_t part_fork;
  hipEvent_t part_join[4];
  // plan-specialised reverse mode in parts: part i writes partial density
  // gradients of adj_chunks[i] chunks as rows of P[adj_rows][ldp]; column k of gA
  // sums P rows adj_row_ids[adj_col_off[k] .. adj_col_off[k + 1]) in that order
  int64_t adj_count;
  hipModule_t* adj_modules;
  hipFunction_t* adj_fns;
  int64_t* adj_chunks;
  int64_t adj_rows;
  int64_t* adj_col_off;  // device [a_width + 1]
  int64_t* adj_row_ids;  // device [adj_col_off[a_width]]
  // fused linear readout in parts: part i writes the partial dot products of
  // ro_chunks[i] chunks as rows of P[ro_total][ldp]
  int64_t ro_count;
  hipModule_t* ro_modules;
  hipFunction_t* ro_fns;
  int64_t* ro_chunks;
  int64_t ro_total;
  int use_interpreter;
  // plan-specialised fused linear readout (optional)
  hipModule_t readout_module;
  hipFunction_t readout;
  int readout_threads;
  int64_t readout_max_grid;  // workgroups resident at once
  // plan-specialised adjoint (optional)
  hipModule_t adjoint_module;
  hipFunction_t adjoint;
  int adjoint_threads;
  int64_t adjoint_max_grid;
  // term stream of the interpreter (built from `words` at creation; absent when
  // the workspace's byte offsets do not fit 16 bits)
  uint4* recs;         // 16-byte records, each chunk padded to a multiple of 4
  uint32_t* flags;     // flag word of each record
  int64_t* rec_off;    // [chunks+1], in records
  uint2* loads;        // (LDS byte offset, density column), each chunk padded to a multiple of 8
  int64_t* load_off;   // [chunks+1], in loads
  int use_stream;
  uint32_t stream_layout[7];  // StreamLayout of the stream kernel (byte offsets in its LDS)
  int64_t stream_lds;         // LDS bytes of the stream kernel
  int64_t stream_tiles;  // tiles per workgroup of the stream kernel (0: by size; YE3T_STREAM_TILES)
};

namespace ye3t {

constexpr int kLanes = 64;
constexpr int kPad = 65;  // LDS row stride in elements

enum : uint32_t { OP_LOAD = 1, OP_ACC1 = 2, OP_ACC2 = 3, OP_ACC3 = 4, OP_ACC4 = 5 };

template <typename Real, typename Out>
__global__ __launch_bounds__(kLanes) void product_kernel(
    const Real* __restrict__ A, int64_t samples, int64_t a_width, Out* __restrict__ B, int64_t F,
    const uint32_t* __restrict__ words, const int64_t* __restrict__ word_off, const Real* __restrict__ coeffs,
    const int64_t* __restrict__ coeff_off, const uint16_t* __restrict__ out_slots,
    const int64_t* __restrict__ out_off, const int64_t* __restrict__ first_col, int64_t chunks) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Real* ws = reinterpret_cast<Real*>(smem_raw);
  const int lane = threadIdx.x;
  const int64_t tile = blockIdx.x / chunks;
  const int64_t chunk = blockIdx.x - tile * chunks;
  const int64_t s0 = tile * kLanes;
  const int64_t s = s0 + lane;
  const bool valid = s < samples;
  const Real* __restrict__ arow = A + (valid ? s : 0) * a_width;
  Real* __restrict__ wl = ws + lane;

  const uint32_t* __restrict__ w = words + word_off[chunk];
  const uint32_t* __restrict__ wend = words + word_off[chunk + 1];
  const Real* __restrict__ cf = coeffs + coeff_off[chunk];

  while (w < wend) {
    const uint32_t h = w[0];
    const uint32_t op = h >> 28;
    const uint32_t n = h & 0x00FFFFFFu;
    if (op == OP_LOAD) {
      for (uint32_t i = 0; i < n; ++i) {
        const uint32_t t = w[1 + i];
        wl[(t >> 16) * kPad] = valid ? arow[t & 0xFFFFu] : Real(0);
      }
      w += 1 + n;
      continue;
    }
    const uint32_t dst = w[1];
    w += 2;
    Real acc = Real(0);
    if (op == OP_ACC2) {
#pragma unroll 4
      for (uint32_t i = 0; i < n; ++i) {
        const uint32_t t = w[i];
        const Real a = wl[(t & 0xFFFFu) * kPad];
        const Real b = wl[(t >> 16) * kPad];
        acc = d_fma(cf[i], a * b, acc);
      }
      w += n;
    } else if (op == OP_ACC1) {
#pragma unroll 4
      for (uint32_t i = 0; i < n; ++i) acc = d_fma(cf[i], wl[(w[i] & 0xFFFFu) * kPad], acc);
      w += n;
    } else {
      // OP_ACC3 / OP_ACC4: two words per term
      const bool four = (op == OP_ACC4);
#pragma unroll 2
      for (uint32_t i = 0; i < n; ++i) {
        const uint32_t t0 = w[2 * i], t1 = w[2 * i + 1];
        Real m = wl[(t0 & 0xFFFFu) * kPad] * wl[(t0 >> 16) * kPad];
        m *= wl[(t1 & 0xFFFFu) * kPad];
        if (four) m *= wl[(t1 >> 16) * kPad];
        acc = d_fma(cf[i], m, acc);
      }
      w += 2 * n;
    }
    cf += n;
    wl[dst * kPad] = acc;
  }
  __syncthreads();
  // transposed write-out: element (row, col) of this chunk's [64, nf] block
  const int64_t o0 = out_off[chunk];
  const int nf = int(out_off[chunk + 1] - o0);
  const int64_t c0 = first_col[chunk];
  const int64_t rows = (samples - s0) < kLanes ? (samples - s0) : kLanes;
  const int total = int(rows) * nf;
  for (int idx = lane; idx < total; idx += kLanes) {
    const int r = idx / nf;
    const int c = idx - r * nf;
    B[(s0 + r) * F + c0 + c] = Out(ws[int(out_slots[o0 + c]) * kPad + r]);
  }
}

// Term-stream interpreter.  The program words of a chunk are decoded on the
// host into one 16-byte record per factor pair and a flag word beside it:
//   record = (LDS byte offset of factor a, of factor b, coefficient: fp64 as
//             low and high word, fp32 in the third word)
//   flag   = flags | LDS byte offset of the destination << 16
// A plain record accumulates acc += c * (a * b); kFlush then stores acc at the
// destination and restarts it.  Terms of three or four factors take two
// records: kChain keeps p = a * b, the next record (kChained) multiplies
// (p * a) * b.  One-factor terms read b from a slot holding 1.  Each chunk's
// records are padded to a multiple of kGroup with c = 0 terms, and its density
// loads to a multiple of 8 with loads into a sink slot, so the unrolled loops
// need no bounds tests.  No record of an aligned group of kGroup reads a slot
// that an earlier record of the group flushes (the encoder pads with c = 0
// terms to start a new group), so a group's factors are all read before its
// stores.
//
// A workgroup is one wave that runs one chunk over tiles_per_group
// consecutive 64-sample tiles (lane = sample).  The chunk's density-load list
// and output slots are staged in LDS once; its records and flags are
// wave-uniform and read with scalar loads, one group ahead, so the next
// group's records are in flight while the current group computes.  The workspace is
// [slot][64] values (slots + 2 for the constant 1 and the sink).  The next
// tile's density values are loaded into registers while the current tile's
// terms run.  The density is read row-major (A[s * lda + col]) or column-major
// (A[col * lda + s]: one contiguous 64-sample block per column).
#ifndef YE3T_STREAM_GROUP
#define YE3T_STREAM_GROUP 8
#endif
constexpr uint32_t kFlush = 1, kChain = 2, kChained = 4;
constexpr int kPrefetch = 32;  // density loads per tile held in registers ahead of time
constexpr int kGroup = YE3T_STREAM_GROUP;  // records per hazard-free group (a multiple of 4)

template <typename Real>
__device__ inline Real record_coeff(const uint4& r) {
  if constexpr (sizeof(Real) == 8) {
    return __hiloint2double(int(r.w), int(r.z));
  } else {
    return __uint_as_float(r.z);
  }
}

template <typename Real>
__device__ inline Real& lds_at(unsigned char* base, uint32_t off) {
  return *reinterpret_cast<Real*>(base + off);
}

// LDS[base + off] += v as an LDS atomic add without return (ds_add_f32 /
// ds_add_f64): the wave does not wait for a read-modify-write round trip
template <typename Real>
__device__ inline void lds_add(unsigned char* base, uint32_t off, Real v) {
  __hip_atomic_fetch_add(reinterpret_cast<Real*>(base + off), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// One group of the term stream (kGroup == 8 records): two 64-byte record
// blocks and one 32-byte flag block, each a single scalar load (a chunk's
// records start at a multiple of 8 records, so every block is aligned).
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef const __attribute__((address_space(4))) u32x16* StreamRec16;
typedef const __attribute__((address_space(4))) u32x8* StreamFlag8;
struct StreamGroup {
  u32x16 lo, hi;
  u32x8 f;
};
static_assert(kGroup == 8, "the wide scalar loads of a group assume 8 records");

__device__ inline StreamGroup fetch_group(StreamRec16 rec16, StreamFlag8 flag8, int q) {
  StreamGroup g;
  g.lo = rec16[q / 4];
  g.hi = rec16[q / 4 + 1];
  g.f = flag8[q / 8];
  return g;
}

// word k of record u of a group
__device__ inline uint32_t group_word(const StreamGroup& g, int u, int k) {
  return u < 4 ? g.lo[4 * u + k] : g.hi[4 * (u - 4) + k];
}

template <typename Real>
__device__ inline Real group_coeff(const StreamGroup& g, int u) {
  if constexpr (sizeof(Real) == 8) {
    return __hiloint2double(int(group_word(g, u, 3)), int(group_word(g, u, 2)));
  } else {
    return __uint_as_float(group_word(g, u, 2));
  }
}

// s_waitcnt lgkmcnt(0) (vmcnt and expcnt left at their maxima)
__device__ inline void wait_lgkm_all() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Hardware dispatch places workgroup b on XCD b % 8.  Renumbered this way,
// each XCD runs one contiguous range of logical blocks, in order: the chunks of
// one sample group then run on one XCD, so their partial output cache lines
// merge in one L2 and the density rows they share are read from it.
__device__ inline int64_t xcd_contiguous(int64_t b, int64_t n) {
  constexpr int64_t X = 8;
  const int64_t q = n / X, r = n % X, x = b % X, i = b / X;
  return x * q + (x < r ? x : r) + i;
}

struct StreamLayout {
  uint32_t ws_bytes;    // workspace: (slots + 2) * 64 * elem
  uint32_t rec_at;      // end of the LDS-resident part (records stay in global memory)
  uint32_t flag_at;     // == rec_at (flag words stay in global memory)
  uint32_t load_at;     // (dst offset, column) pairs
  uint32_t out_at;      // output slot byte offsets
  uint32_t one_off;     // workspace byte offset of the slot holding 1
  uint32_t sink_off;    // workspace byte offset of the sink slot (padding loads, unflushed stores)
};

template <typename Real, typename Out, bool COLUMNS>
__global__ __launch_bounds__(kLanes) void product_stream_kernel(
    const Real* __restrict__ A, int64_t lda, int64_t samples, Out* __restrict__ B, int64_t F,
    const uint4* __restrict__ recs, const uint32_t* __restrict__ flags, const int64_t* __restrict__ rec_off,
    const uint2* __restrict__ loads, const int64_t* __restrict__ load_off, const uint16_t* __restrict__ out_slots,
    const int64_t* __restrict__ out_off, const int64_t* __restrict__ first_col, int64_t chunks,
    StreamLayout lay, int64_t tiles_per_group) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int lane = threadIdx.x;
  const int64_t blk = xcd_contiguous(blockIdx.x, gridDim.x);
  const int64_t group = blk / chunks;
  const int64_t chunk = blk - group * chunks;
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  const int64_t tile0 = group * tiles_per_group;
  const int64_t tile_end = tile0 + tiles_per_group < tiles ? tile0 + tiles_per_group : tiles;
  unsigned char* wsb = smem_raw + lane * sizeof(Real);
  uint4* lload = reinterpret_cast<uint4*>(smem_raw + lay.load_at);
  uint32_t* lout = reinterpret_cast<uint32_t*>(smem_raw + lay.out_at);

  // stage the chunk's loads and output slots in LDS; its records and flags are
  // wave-uniform and are read through the scalar cache (no LDS for them)
  const int64_t r0 = rec_off[chunk];
  const int nr = int(rec_off[chunk + 1] - r0);
  const int64_t l0 = load_off[chunk];
  const int nl = int(load_off[chunk + 1] - l0);
  const int64_t o0 = out_off[chunk];
  const int nf = int(out_off[chunk + 1] - o0);
  const StreamRec16 grec16 = (StreamRec16)(const void*)(recs + r0);
  const StreamFlag8 gflag8 = (StreamFlag8)(const void*)(flags + r0);
  // load entry i: (dst byte offset, element offset of its column: col * lda
  // column-major, col row-major) so a tile's load address is one add
  for (int i = lane; i < nl; i += kLanes) {
    const uint2 e = loads[l0 + i];
    const uint64_t eo = COLUMNS ? uint64_t(e.y) * uint64_t(lda) : uint64_t(e.y);
    lload[i] = make_uint4(e.x, 0u, uint32_t(eo), uint32_t(eo >> 32));
  }
  for (int i = lane; i < nf; i += kLanes) lout[i] = uint32_t(out_slots[o0 + i]) * (kLanes * sizeof(Real));
  lds_at<Real>(wsb, lay.one_off) = Real(1);
  __syncthreads();
  const int64_t c0 = first_col[chunk];
  const float inv_nf = 1.0f / float(nf > 0 ? nf : 1);
  const int npre = nl < kPrefetch ? nl : kPrefetch;

  auto tile_src = [&](int64_t tile) {
    const int64_t s = tile * kLanes + lane;
    return COLUMNS ? A + s : A + (s < samples ? s : 0) * lda;
  };
  auto entry_off = [&](int i) {
    const uint4 e = lload[i];
    return int64_t((uint64_t(e.w) << 32) | e.z);
  };
  // density values of one tile for the first npre loads (into registers)
  auto fetch = [&](int64_t tile, Real* v) {
    const Real* __restrict__ src = tile_src(tile);
#pragma unroll
    for (int u = 0; u < kPrefetch; u += 8) {
      if (u < npre) {
#pragma unroll
        for (int w = 0; w < 8; ++w) v[u + w] = src[entry_off(u + w)];
      }
    }
  };
  Real pre[kPrefetch];
  if (tile0 < tile_end) fetch(tile0, pre);

  for (int64_t tile = tile0; tile < tile_end; ++tile) {
    const int64_t s0 = tile * kLanes;
    // the prefetched values, then any loads beyond them
#pragma unroll
    for (int u = 0; u < kPrefetch; u += 8) {
      if (u < npre) {
#pragma unroll
        for (int w = 0; w < 8; ++w) lds_at<Real>(wsb, lload[u + w].x) = pre[u + w];
      }
    }
    if (nl > kPrefetch) {
      const Real* __restrict__ src = tile_src(tile);
      for (int q = kPrefetch; q < nl; q += 8) {
        Real v[8];
#pragma unroll
        for (int w = 0; w < 8; ++w) v[w] = src[entry_off(q + w)];
#pragma unroll
        for (int w = 0; w < 8; ++w) lds_at<Real>(wsb, lload[q + w].x) = v[w];
      }
    }
    if (tile + 1 < tile_end) fetch(tile + 1, pre);

    // the term stream, one group of 8 records at a time.  A group's records
    // and flags are three wide scalar loads, issued right after the wait for
    // the previous group's LDS operands (scalar and LDS reads share one
    // counter, and scalar reads return out of order): they are in flight while
    // that group computes, and no LDS wait has to wait for them.
    Real acc = Real(0), p = Real(1);
    StreamGroup ga = fetch_group(grec16, gflag8, 0), gb;
    const int last = nr - kGroup;
    auto run_group = [&](const StreamGroup& g, int qnext, StreamGroup& gn) {
      Real a[kGroup], b[kGroup];
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        a[u] = lds_at<Real>(wsb, group_word(g, u, 0));
        b[u] = lds_at<Real>(wsb, group_word(g, u, 1));
      }
      wait_lgkm_all();
      // branch-free records (one basic block per group, so the scalar loads
      // above stay where they are): every record stores acc, to its
      // destination when it flushes and to the sink slot otherwise, and a
      // flush restarts acc by a multiply with 0
      uint32_t any = 0;
#pragma unroll
      for (int u = 0; u < kGroup; ++u) any |= g.f[u];
      // (the next group's loads are issued at the top of each branch: placed
      // before the branch, the compiler sinks them below it)
      if ((any & (kChain | kChained)) == 0) {
        __builtin_amdgcn_sched_barrier(0);
        gn = fetch_group(grec16, gflag8, qnext);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
          const uint32_t fw = g.f[u];
          acc = d_fma(group_coeff<Real>(g, u), a[u] * b[u], acc);
          lds_at<Real>(wsb, (fw & kFlush) ? (fw >> 16) : lay.sink_off) = acc;
          acc *= (fw & kFlush) ? Real(0) : Real(1);
        }
      } else {
        // a kChain record (coefficient 0) sets p = a b, its kChained partner
        // adds c (p a) b
        __builtin_amdgcn_sched_barrier(0);
        gn = fetch_group(grec16, gflag8, qnext);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
          const uint32_t fw = g.f[u];
          const Real ab = a[u] * b[u];
          const Real t = (fw & kChained) ? (p * a[u]) * b[u] : ab;
          acc = d_fma(group_coeff<Real>(g, u), t, acc);
          p = (fw & kChain) ? ab : p;
          lds_at<Real>(wsb, (fw & kFlush) ? (fw >> 16) : lay.sink_off) = acc;
          acc *= (fw & kFlush) ? Real(0) : Real(1);
        }
      }
    };
    for (int q = 0; q < nr; q += 2 * kGroup) {
      run_group(ga, q + kGroup < last ? q + kGroup : last, gb);
      if (q + kGroup >= nr) break;
      run_group(gb, q + 2 * kGroup < last ? q + 2 * kGroup : last, ga);
    }
    // transposed write-out of the chunk's [rows, nf] block: consecutive lanes
    // take consecutive columns of a row, so a store covers a few row segments
    // (a few cache lines) rather than one line per lane
    {
      const int rows = (samples - s0) < kLanes ? int(samples - s0) : kLanes;
      const int total = rows * nf;
      for (int idx = lane; idx < total; idx += kLanes) {
        // (idx + 1/2) / nf lies at least 1/(2 nf) from an integer: the float quotient truncates exactly
        const int r = int((float(idx) + 0.5f) * inv_nf);
        const int c = idx - r * nf;
        B[(s0 + r) * F + c0 + c] = Out(lds_at<Real>(smem_raw + r * sizeof(Real), lout[c]));
      }
    }
    // the next tile's values overwrite slots this write-out reads (one wave:
    // LDS operations complete in order; this keeps the compiler from moving them)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
}

// Reverse mode of the term stream: gA[s] = J(A[s])^T gB[s] for plans run by
// the stream interpreter.  Workgroup (tile, group) runs the chunks
// [group * chunks / groups, (group + 1) * chunks / groups) of one 64-sample
// tile.  Per chunk: stage the program, load the density values and replay
// the stream forward (every node value stays in its slot), seed a gradient
// workspace with the chunk's feature gradients, then sweep the records
// backwards:
//   plain record  acc += c a b:      G[a] += c g b,  G[b] += c g a
//   chained pair  p = a1 b1; acc += c (p a2) b2:
//                 G[a2] += c g p b2, G[b2] += c g p a2,
//                 G[a1] += c g a2 b2 b1, G[b1] += c g a2 b2 a1
// with g = G[destination], read when the sweep meets the record that flushed
// it (its last term).  The density gradients of the chunk's loads are added
// into this workgroup's own block of P[group][col][s]; gA is the sum of the
// groups in a fixed order (stream_adjoint_reduce_kernel), so no global atomics
// and the same bits every run (the sweep's LDS atomic adds touch only the
// adding lane's own column, in program order).
// global loads (density values, partial-block entries) in flight per batch
// (16 measured slower than 8 at configs 2 and 3)
constexpr int kAdjBatch = 8;

template <typename Real, typename G, bool COLUMNS>
__global__ __launch_bounds__(kLanes) void product_stream_adjoint_kernel(
    const Real* __restrict__ A, int64_t lda, int64_t samples, const G* __restrict__ gB, int64_t F,
    const uint4* __restrict__ recs, const uint32_t* __restrict__ flags, const int64_t* __restrict__ rec_off,
    const uint2* __restrict__ loads, const int64_t* __restrict__ load_off, const uint16_t* __restrict__ out_slots,
    const int64_t* __restrict__ out_off, const int64_t* __restrict__ first_col, int64_t chunks, int64_t groups,
    StreamLayout lay, Real* __restrict__ P, int64_t a_width, int64_t ldp) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int lane = threadIdx.x;
  const int64_t tile = blockIdx.x / groups;
  const int64_t group = blockIdx.x - tile * groups;
  const int64_t s = tile * kLanes + lane;
  const bool valid = s < samples;
  unsigned char* wsb = smem_raw + lane * sizeof(Real);                  // values
  unsigned char* gsb = smem_raw + lay.ws_bytes + lane * sizeof(Real);   // gradients
  unsigned char* prog = smem_raw + lay.ws_bytes;                        // program region, past the gradients
  uint2* lload = reinterpret_cast<uint2*>(prog + lay.load_at);
  uint32_t* lout = reinterpret_cast<uint32_t*>(prog + lay.out_at);
  const uint32_t pitch = kLanes * sizeof(Real);
  const uint32_t sink = lay.one_off + pitch;
  const uint32_t ws_slots = lay.one_off / pitch + 2;
  Real* __restrict__ Pg = P + group * a_width * ldp + s;
  const Real* __restrict__ src = COLUMNS ? A + s : A + (valid ? s : 0) * lda;
  const int64_t c_begin = group * chunks / groups, c_end = (group + 1) * chunks / groups;

  for (int64_t chunk = c_begin; chunk < c_end; ++chunk) {
    const int64_t r0 = rec_off[chunk];
    const int nr = int(rec_off[chunk + 1] - r0);
    const int64_t l0 = load_off[chunk];
    const int nl = int(load_off[chunk + 1] - l0);
    const int64_t o0 = out_off[chunk];
    const int nf = int(out_off[chunk + 1] - o0);
    __syncthreads();  // the previous chunk is done with the program region
    // records and flags are wave-uniform: read through the scalar cache
    typedef const __attribute__((address_space(4))) uint32_t* scalar_u32;
    const scalar_u32 grec = (scalar_u32)(const void*)(recs + r0);
    const scalar_u32 gflag = (scalar_u32)(const void*)(flags + r0);
    auto rec_at = [&](int q) { return make_uint4(grec[4 * q], grec[4 * q + 1], grec[4 * q + 2], grec[4 * q + 3]); };
    for (int i = lane; i < nl; i += kLanes) lload[i] = loads[l0 + i];
    for (int i = lane; i < nf; i += kLanes) lout[i] = uint32_t(out_slots[o0 + i]) * pitch;
    __syncthreads();
    lds_at<Real>(wsb, lay.one_off) = Real(1);
    // density values, kAdjBatch loads in flight (nl is a multiple of 8;
    // padding entries read a valid column into the sink slot)
    for (int q = 0; q < nl; q += kAdjBatch) {
      uint2 e[kAdjBatch];
      Real v[kAdjBatch];
#pragma unroll
      for (int w = 0; w < kAdjBatch; ++w) e[w] = q + w < nl ? lload[q + w] : make_uint2(sink, 0u);
#pragma unroll
      for (int w = 0; w < kAdjBatch; ++w) v[w] = COLUMNS ? src[int64_t(e[w].y) * lda] : src[e[w].y];
#pragma unroll
      for (int w = 0; w < kAdjBatch; ++w) lds_at<Real>(wsb, e[w].x) = v[w];
    }
    // forward replay, kGroup records at a time: no record of a group reads a
    // slot flushed earlier in the group, so all its factors are read first
    Real acc = Real(0), p = Real(1);
    for (int q0 = 0; q0 < nr; q0 += kGroup) {
      uint32_t f[kGroup];
      uint4 r[kGroup];
      Real a[kGroup], b[kGroup];
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        f[u] = gflag[q0 + u];
        r[u] = rec_at(q0 + u);
      }
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        a[u] = lds_at<Real>(wsb, r[u].x);
        b[u] = lds_at<Real>(wsb, r[u].y);
      }
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        if (f[u] & kChain) {
          p = a[u] * b[u];
          continue;
        }
        const Real t = (f[u] & kChained) ? (p * a[u]) * b[u] : a[u] * b[u];
        acc = d_fma(record_coeff<Real>(r[u]), t, acc);
        if (f[u] & kFlush) {
          lds_at<Real>(wsb, f[u] >> 16) = acc;
          acc = Real(0);
        }
      }
    }
    // gradient workspace: zero, then the chunk's feature gradients
    for (uint32_t k = 0; k < ws_slots; ++k) lds_at<Real>(gsb, k * pitch) = Real(0);
    const int64_t c0 = first_col[chunk];
    for (int c = 0; c < nf; c += 8) {
      Real gv[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) gv[w] = (valid && c + w < nf) ? Real(gB[s * F + c0 + c + w]) : Real(0);
#pragma unroll
      for (int w = 0; w < 8; ++w)
        if (c + w < nf) lds_add<Real>(gsb, lout[c + w], gv[w]);
    }
    // reverse sweep, a group at a time.  The node values are not written here,
    // so a group's factors are read at once; gradients are added by LDS atomic
    // adds without return (each lane owns its column, and one wave's LDS
    // operations take effect in order, so a later read of g sees every add
    // before it and the sums are the same every run).
    Real g = Real(0);
    for (int q0 = nr - kGroup; q0 >= 0; q0 -= kGroup) {
      uint32_t f[kGroup];
      uint4 r[kGroup];
      Real a[kGroup], b[kGroup];
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        f[u] = gflag[q0 + u];
        r[u] = rec_at(q0 + u);
      }
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        a[u] = lds_at<Real>(wsb, r[u].x);
        b[u] = lds_at<Real>(wsb, r[u].y);
      }
#pragma unroll
      for (int u = kGroup - 1; u >= 0; --u) {
        if (f[u] & kChain) continue;  // consumed with its chained partner
        if (f[u] & kFlush) g = lds_at<Real>(gsb, f[u] >> 16);
        const Real cg = record_coeff<Real>(r[u]) * g;
        if (f[u] & kChained) {
          // the chain record precedes its partner, in this group or at the
          // end of the previous one
          const uint4 rc = u > 0 ? r[u > 0 ? u - 1 : 0] : rec_at(q0 - 1);
          const Real a1 = u > 0 ? a[u > 0 ? u - 1 : 0] : lds_at<Real>(wsb, rc.x);
          const Real b1 = u > 0 ? b[u > 0 ? u - 1 : 0] : lds_at<Real>(wsb, rc.y);
          const Real pp = a1 * b1, ab = a[u] * b[u];
          lds_add<Real>(gsb, r[u].x, cg * pp * b[u]);
          lds_add<Real>(gsb, r[u].y, cg * pp * a[u]);
          lds_add<Real>(gsb, rc.x, cg * ab * b1);
          lds_add<Real>(gsb, rc.y, cg * ab * a1);
        } else {
          lds_add<Real>(gsb, r[u].x, cg * b[u]);
          lds_add<Real>(gsb, r[u].y, cg * a[u]);
        }
      }
    }
    // density gradients of this chunk into the group's block, eight at a
    // time (the encoder loads a column at most once per chunk, so the eight
    // read-modify-writes touch distinct entries)
    for (int q = 0; q < nl; q += kAdjBatch) {
      uint32_t slot[kAdjBatch], col[kAdjBatch];
      Real sum[kAdjBatch];
#pragma unroll
      for (int w = 0; w < kAdjBatch; ++w) {
        const uint2 e = q + w < nl ? lload[q + w] : make_uint2(sink, 0u);
        slot[w] = uint32_t(__builtin_amdgcn_readfirstlane(int(e.x)));
        col[w] = uint32_t(__builtin_amdgcn_readfirstlane(int(e.y)));
      }
      // padding entries read column 0 and the sink slot, and store nothing
#pragma unroll
      for (int w = 0; w < kAdjBatch; ++w) sum[w] = Pg[int64_t(col[w]) * ldp];
#pragma unroll
      for (int w = 0; w < kAdjBatch; ++w) sum[w] += lds_at<Real>(gsb, slot[w]);
#pragma unroll
      for (int w = 0; w < kAdjBatch; ++w)
        if (slot[w] != sink) Pg[int64_t(col[w]) * ldp] = sum[w];
    }
  }
}

// gA[s * a_width + col] = sum over groups g (in order) of P[g][col][s], through
// 64 x 64 LDS tiles (P is column-major, gA row-major).
template <typename Real>
__global__ __launch_bounds__(256) void stream_adjoint_reduce_kernel(const Real* __restrict__ P, int64_t groups,
                                                                    int64_t a_width, int64_t ldp, int64_t samples,
                                                                    Real* __restrict__ gA) {
  __shared__ Real t[64][65];
  const int64_t c0 = int64_t(blockIdx.x) * 64, s0 = int64_t(blockIdx.y) * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int k = ty; k < 64; k += 4) {
    const int64_t col = c0 + k, s = s0 + tx;
    Real v = Real(0);
    if (col < a_width && s < ldp) {
      // eight groups' loads in flight, added in group order
      const Real* __restrict__ src = P + col * ldp + s;
      const int64_t gstride = a_width * ldp;
      int64_t g = 0;
      for (; g + 8 <= groups; g += 8) {
        Real x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = src[(g + u) * gstride];
#pragma unroll
        for (int u = 0; u < 8; ++u) v += x[u];
      }
      for (; g < groups; ++g) v += src[g * gstride];
    }
    t[k][tx] = v;
  }
  __syncthreads();
  for (int k = ty; k < 64; k += 4) {
    const int64_t s = s0 + k, col = c0 + tx;
    if (s < samples && col < a_width) gA[s * a_width + col] = t[tx][k];
  }
}

template <typename Real>
__global__ __launch_bounds__(256) void fill_zero_kernel(Real* __restrict__ x, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    x[i] = Real(0);
}

// At[c * ld + r] = A[r * cols + c] through 64 x 64 LDS tiles.
template <typename Real>
__global__ __launch_bounds__(256) void transpose_kernel(const Real* __restrict__ A, int64_t rows, int64_t cols,
                                                        Real* __restrict__ At, int64_t ld) {
  __shared__ Real t[64][65];
  const int64_t r0 = int64_t(blockIdx.y) * 64, c0 = int64_t(blockIdx.x) * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int k = ty; k < 64; k += 4) {
    const int64_t r = r0 + k, c = c0 + tx;
    t[k][tx] = (r < rows && c < cols) ? A[r * cols + c] : Real(0);
  }
  __syncthreads();
  for (int k = ty; k < 64; k += 4) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (c < cols && r < ld) At[c * ld + r] = t[tx][k];
  }
}

// out[s] = bias + sum_k B[s, k] w[k]: one wave per row (grid-stride over rows),
// lanes stride over k with fp64 partial sums, then a fixed butterfly over the
// 64 lanes, so the result does not depend on timing.
template <typename Real>
__global__ __launch_bounds__(256) void rows_dot_kernel(const Real* __restrict__ B, int64_t samples, int64_t F,
                                                       const Real* __restrict__ w, double bias,
                                                       Real* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = int64_t(gridDim.x) * (blockDim.x >> 6);
  for (int64_t s = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6); s < samples; s += waves) {
    const Real* __restrict__ row = B + s * F;
    double acc = 0.0;
    for (int64_t k = lane; k < F; k += 64) acc = fma(double(row[k]), double(w[k]), acc);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) out[s] = Real(bias + acc);
  }
}

template <typename Real>
__global__ __launch_bounds__(256) void evaluate_schedule_kernel(
    const Real* __restrict__ bv, int64_t batch, int64_t basis, int64_t blocks, int64_t mdim,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ labels, const int64_t* __restrict__ midx,
    const Real* __restrict__ coeffs, int64_t K, Real* __restrict__ out) {
  const int64_t total = batch * K;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int64_t b = idx / K;
    const int64_t k = idx - b * K;
    const Real* __restrict__ base = bv + (b * basis + labels[k]) * blocks * mdim;
    Real acc = Real(0);
    for (int64_t t = offsets[k]; t < offsets[k + 1]; ++t) {
      Real v = coeffs[t];
      const int64_t* tm = midx + t * blocks;
      for (int64_t blk = 0; blk < blocks; ++blk) v *= base[blk * mdim + tm[blk]];
      acc += v;
    }
    out[idx] = acc;
  }
}

inline unsigned grid_1d(int64_t work, int threads) {
  int64_t g = (work + threads - 1) / threads;
  if (g < 1) g = 1;
  if (g > (1 << 20)) g = 1 << 20;
  return unsigned(g);
}

template <typename T>
int upload(T** dst, const T* src, int64_t count) {
  *dst = nullptr;
  if (count <= 0) return YE3T_OK;
  if (hipMalloc(reinterpret_cast<void**>(dst), sizeof(T) * size_t(count)) != hipSuccess) {
    *dst = nullptr;
    return set_error(YE3T_ENOMEM, "hipMalloc of %lld bytes failed", (long long)(sizeof(T) * count));
  }
  YE3T_CHECK_HIP(hipMemcpy(*dst, src, sizeof(T) * size_t(count), hipMemcpyHostToDevice));
  return YE3T_OK;
}

size_t product_lds_bytes(const ye3t_hip_product_plan* p) {
  const size_t elem = p->dtype == YE3T_F64 ? 8 : 4;
  return p->use_stream ? size_t(p->stream_layout[1]) : size_t(p->slots) * kPad * elem;
}

// Decode validated program words into the term stream of product_stream_kernel
// (workspace pitch 64 values; slots `slots` and `slots + 1` hold 1 and the
// padding loads) and lay out its LDS.  Returns false when the workspace's byte
// offsets do not fit the flag words' 16 bits or the LDS exceeds 64 KB.
bool build_stream(const ye3t_product_plan_desc* d, std::vector<uint4>& recs, std::vector<uint32_t>& flags,
                  std::vector<int64_t>& rec_off, std::vector<uint2>& loads, std::vector<int64_t>& load_off,
                  StreamLayout& lay, int64_t& lds_bytes) {
  const uint32_t elem = d->dtype == YE3T_F64 ? 8 : 4;
  const uint32_t pitch = uint32_t(kLanes) * elem;
  if ((uint64_t(d->workspace_slots) + 2) * pitch > 0x10000u) return false;
  const uint32_t one = uint32_t(d->workspace_slots) * pitch, sink = one + pitch;
  auto off = [&](uint32_t slot) { return slot * pitch; };
  auto record = [&](uint32_t a, uint32_t b, int64_t ci) {
    uint4 r = make_uint4(a, b, 0, 0);
    if (ci < 0) return r;
    if (elem == 8) {
      uint64_t bits;
      std::memcpy(&bits, static_cast<const double*>(d->coeffs) + ci, 8);
      r.z = uint32_t(bits);
      r.w = uint32_t(bits >> 32);
    } else {
      std::memcpy(&r.z, static_cast<const float*>(d->coeffs) + ci, 4);
    }
    return r;
  };
  rec_off.assign(1, 0);
  load_off.assign(1, 0);
  const uint4 nop = make_uint4(one, one, 0, 0);  // acc += 0 * 1 * 1
  uint32_t flushed[kGroup];  // destinations flushed so far in the current group
  int nflushed = 0;
  auto pad_group = [&]() {
    while ((int64_t(recs.size()) - rec_off.back()) % kGroup) {
      recs.push_back(nop);
      flags.push_back(0);
    }
  };
  // append a record; start a new group first if it reads a slot flushed earlier in this one
  auto emit = [&](const uint4& r, uint32_t flag) {
    bool hazard = false;
    for (int k = 0; k < nflushed; ++k) hazard |= (flushed[k] == r.x || flushed[k] == r.y);
    if (hazard) pad_group();
    if ((int64_t(recs.size()) - rec_off.back()) % kGroup == 0) nflushed = 0;
    recs.push_back(r);
    flags.push_back(flag);
    if (flag & kFlush) flushed[nflushed++] = flag >> 16;
  };
  int64_t max_recs = 0, max_loads = 0, max_out = 0;
  for (int64_t c = 0; c < d->chunk_count; ++c) {
    nflushed = 0;
    int64_t wpos = d->chunk_word_offsets[c];
    const int64_t wend = d->chunk_word_offsets[c + 1];
    int64_t cpos = d->chunk_coeff_offsets[c];
    while (wpos < wend) {
      const uint32_t h = d->words[wpos];
      const uint32_t op = h >> 28, n = h & 0x00FFFFFFu;
      if (op == OP_LOAD) {
        for (uint32_t i = 0; i < n; ++i) {
          const uint32_t t = d->words[wpos + 1 + i];
          loads.push_back(make_uint2(off(t >> 16), t & 0xFFFFu));
        }
        wpos += 1 + n;
        continue;
      }
      const uint32_t dst = off(d->words[wpos + 1]);
      const uint32_t* tw = d->words + wpos + 2;
      if (n == 0) emit(nop, kFlush | (dst << 16));  // an empty sum stores 0
      for (uint32_t i = 0; i < n; ++i) {
        const uint32_t flush = (i + 1 == n) ? (kFlush | (dst << 16)) : 0;
        if (op == OP_ACC1) {
          emit(record(off(tw[i] & 0xFFFFu), one, cpos + i), flush);
        } else if (op == OP_ACC2) {
          emit(record(off(tw[i] & 0xFFFFu), off(tw[i] >> 16), cpos + i), flush);
        } else {
          // the pair stays adjacent (the adjoint reads the chain record just
          // before its partner): any hazard padding goes before both
          const uint32_t t0 = tw[2 * i], t1 = tw[2 * i + 1];
          const uint4 rc = record(off(t0 & 0xFFFFu), off(t0 >> 16), -1);
          const uint4 rd = record(off(t1 & 0xFFFFu), op == OP_ACC4 ? off(t1 >> 16) : one, cpos + i);
          bool hazard = false;
          for (int k = 0; k < nflushed; ++k)
            hazard |= (flushed[k] == rc.x || flushed[k] == rc.y || flushed[k] == rd.x || flushed[k] == rd.y);
          if (hazard) pad_group();
          emit(rc, kChain);
          emit(rd, kChained | flush);
        }
      }
      wpos += 2 + int64_t((op == OP_ACC3 || op == OP_ACC4) ? 2 : 1) * n;
      cpos += n;
    }
    pad_group();
    {
      // the adjoint adds a chunk's density gradients eight loads at a time:
      // a density column is loaded at most once per chunk
      std::vector<uint32_t> cols;
      for (int64_t i = load_off.back(); i < int64_t(loads.size()); ++i) cols.push_back(loads[size_t(i)].y);
      std::sort(cols.begin(), cols.end());
      if (std::adjacent_find(cols.begin(), cols.end()) != cols.end()) return false;
    }
    while ((int64_t(loads.size()) - load_off.back()) % 8) loads.push_back(make_uint2(sink, 0));
    max_recs = std::max<int64_t>(max_recs, int64_t(recs.size()) - rec_off.back());
    max_loads = std::max<int64_t>(max_loads, int64_t(loads.size()) - load_off.back());
    max_out = std::max<int64_t>(max_out, d->chunk_out_offsets[c + 1] - d->chunk_out_offsets[c]);
    rec_off.push_back(int64_t(recs.size()));
    load_off.push_back(int64_t(loads.size()));
  }
  if (recs.empty()) {
    recs.push_back(nop);
    flags.push_back(0);
  }
  if (loads.empty()) loads.push_back(make_uint2(sink, 0));
  auto up16 = [](int64_t b) { return (b + 15) & ~int64_t(15); };
  int64_t at = up16((int64_t(d->workspace_slots) + 2) * pitch);
  lay.ws_bytes = uint32_t(at);
  lay.load_at = uint32_t(at);
  at = up16(at + 16 * max_loads);
  lay.out_at = uint32_t(at);
  at = up16(at + 4 * max_out);
  // records and flags stay in global memory (both kernels read them through
  // the scalar cache): rec_at and flag_at mark the end of the LDS a wave uses
  lay.rec_at = uint32_t(at);
  lay.flag_at = uint32_t(at);
  lay.one_off = one;
  lay.sink_off = sink;
  lds_bytes = at;
  (void)max_recs;
  return at <= 64 * 1024;
}

// tiles per workgroup of the stream kernel: the most (up to 16) that still
// leaves about 8 workgroups per workgroup slot of the device
int64_t stream_tiles_per_group(const ye3t_hip_product_plan* p, int64_t tiles) {
  int64_t per = p->stream_tiles;
  if (per <= 0) {
    per = 1;
    while (per < 16 && (tiles + 2 * per - 1) / (2 * per) * p->chunk_count >= 8 * 256 * 6) per *= 2;
  }
  return per;
}

template <bool COLUMNS>
int launch_stream(const ye3t_hip_product_plan* p, const void* A, int64_t lda, int64_t samples, void* B,
                  ye3t_stream_t stream) {
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  const int64_t per = stream_tiles_per_group(p, tiles);
  const int64_t groups = (tiles + per - 1) / per;
  const int64_t grid = groups * p->chunk_count;
  YE3T_REQUIRE(grid <= int64_t(0x7FFFFFFF), "too many samples for one launch");
  const size_t lds = size_t(p->stream_layout[1]);  // up to rec_at: records and flags stay in global memory
  StreamLayout lay;
  lay.ws_bytes = p->stream_layout[0];
  lay.rec_at = p->stream_layout[1];
  lay.flag_at = p->stream_layout[2];
  lay.load_at = p->stream_layout[3];
  lay.out_at = p->stream_layout[4];
  lay.one_off = p->stream_layout[5];
  lay.sink_off = p->stream_layout[6];
  const hipStream_t s = as_stream(stream);
  if (p->dtype == YE3T_F64 && p->out_dtype == YE3T_F64) {
    hipLaunchKernelGGL((product_stream_kernel<double, double, COLUMNS>), dim3(unsigned(grid)), dim3(kLanes), lds, s,
                       (const double*)A, lda, samples, (double*)B, p->feature_count, p->recs, p->flags, p->rec_off,
                       p->loads, p->load_off, p->out_slots, p->out_off, p->first_col, p->chunk_count, lay, per);
  } else if (p->dtype == YE3T_F64) {
    hipLaunchKernelGGL((product_stream_kernel<double, float, COLUMNS>), dim3(unsigned(grid)), dim3(kLanes), lds, s,
                       (const double*)A, lda, samples, (float*)B, p->feature_count, p->recs, p->flags, p->rec_off,
                       p->loads, p->load_off, p->out_slots, p->out_off, p->first_col, p->chunk_count, lay, per);
  } else {
    hipLaunchKernelGGL((product_stream_kernel<float, float, COLUMNS>), dim3(unsigned(grid)), dim3(kLanes), lds, s,
                       (const float*)A, lda, samples, (float*)B, p->feature_count, p->recs, p->flags, p->rec_off,
                       p->loads, p->load_off, p->out_slots, p->out_off, p->first_col, p->chunk_count, lay, per);
  }
  return check_launch("product_stream_kernel");
}

// Groups of chunks per tile for the stream adjoint (enough workgroups to fill
// the device, partial blocks within 4 GiB) and the partial blocks' bytes.
// `cap` bounds the partial blocks' bytes.  When one group alone exceeds it the
// result is one group, or 0 with `strict` (a cap that cannot grow).
int64_t stream_adjoint_groups(const ye3t_hip_product_plan* p, int64_t samples, int64_t* bytes,
                              int64_t cap = int64_t(4) << 30, bool strict = false) {
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  const int64_t ldp = tiles * kLanes;
  const int64_t per_group = p->a_width * ldp * (p->dtype == YE3T_F64 ? 8 : 4);
  const char* wg = std::getenv("YE3T_ADJOINT_WORKGROUPS");
  const int64_t target = (wg && *wg && std::atoll(wg) > 0) ? std::atoll(wg) : 8 * 256 * 6;
  int64_t groups = (target + tiles - 1) / tiles;
  if (groups > p->chunk_count) groups = p->chunk_count;
  if (groups * per_group > cap) groups = cap / per_group;
  if (groups < 1) groups = (strict && per_group > cap) ? 0 : 1;
  if (bytes) *bytes = groups * per_group;
  return groups;
}

template <bool COLUMNS>
int launch_stream_adjoint(const ye3t_hip_product_plan* p, const void* A, int64_t lda, const void* gB,
                          int64_t samples, void* P, int64_t groups, void* gA, hipStream_t s) {
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  const int64_t ldp = tiles * kLanes;
  const size_t elem = p->dtype == YE3T_F64 ? 8 : 4;
  const int64_t nP = groups * p->a_width * ldp;
  const unsigned fill_grid = unsigned(std::min<int64_t>((nP + 255) / 256, 65536));
  StreamLayout lay;
  lay.ws_bytes = p->stream_layout[0];
  lay.rec_at = p->stream_layout[1];
  lay.flag_at = p->stream_layout[2];
  lay.load_at = p->stream_layout[3];
  lay.out_at = p->stream_layout[4];
  lay.one_off = p->stream_layout[5];
  lay.sink_off = p->stream_layout[6];
  // values, gradients, loads and output slots (records and flags stay in global memory)
  const size_t lds = size_t(p->stream_layout[1]) + lay.ws_bytes;
  const int64_t grid = tiles * groups;
  YE3T_REQUIRE(grid <= int64_t(0x7FFFFFFF), "too many samples for one launch");
  const dim3 rgrid = dim3(unsigned((p->a_width + 63) / 64), unsigned((samples + 63) / 64), 1u);
  YE3T_REQUIRE((samples + 63) / 64 <= 65535, "too many samples for one launch");
  if (p->dtype == YE3T_F64) {
    hipLaunchKernelGGL(fill_zero_kernel<double>, dim3(fill_grid), dim3(256), 0, s, (double*)P, nP);
    if (p->out_dtype == YE3T_F64)
      hipLaunchKernelGGL((product_stream_adjoint_kernel<double, double, COLUMNS>), dim3(unsigned(grid)), dim3(kLanes),
                         lds, s, (const double*)A, lda, samples, (const double*)gB, p->feature_count, p->recs,
                         p->flags, p->rec_off, p->loads, p->load_off, p->out_slots, p->out_off, p->first_col,
                         p->chunk_count, groups, lay, (double*)P, p->a_width, ldp);
    else
      hipLaunchKernelGGL((product_stream_adjoint_kernel<double, float, COLUMNS>), dim3(unsigned(grid)), dim3(kLanes),
                         lds, s, (const double*)A, lda, samples, (const float*)gB, p->feature_count, p->recs,
                         p->flags, p->rec_off, p->loads, p->load_off, p->out_slots, p->out_off, p->first_col,
                         p->chunk_count, groups, lay, (double*)P, p->a_width, ldp);
    hipLaunchKernelGGL(stream_adjoint_reduce_kernel<double>, rgrid, dim3(256), 0, s, (const double*)P, groups,
                       p->a_width, ldp, samples, (double*)gA);
  } else {
    hipLaunchKernelGGL(fill_zero_kernel<float>, dim3(fill_grid), dim3(256), 0, s, (float*)P, nP);
    hipLaunchKernelGGL((product_stream_adjoint_kernel<float, float, COLUMNS>), dim3(unsigned(grid)), dim3(kLanes),
                       lds, s, (const float*)A, lda, samples, (const float*)gB, p->feature_count, p->recs,
                       p->flags, p->rec_off, p->loads, p->load_off, p->out_slots, p->out_off, p->first_col,
                       p->chunk_count, groups, lay, (float*)P, p->a_width, ldp);
    hipLaunchKernelGGL(stream_adjoint_reduce_kernel<float>, rgrid, dim3(256), 0, s, (const float*)P, groups,
                       p->a_width, ldp, samples, (float*)gA);
  }
  (void)elem;
  return check_launch("product_stream_adjoint_kernel");
}

// Host-side validation of every index a plan's kernels will use.
int validate_plan_desc(const ye3t_product_plan_desc* d) {
  YE3T_REQUIRE(d != nullptr, "NULL plan description");
  YE3T_REQUIRE(d->dtype == YE3T_F32 || d->dtype == YE3T_F64, "unsupported dtype %d", d->dtype);
  const int out_dtype = d->out_dtype < 0 ? d->dtype : d->out_dtype;
  YE3T_REQUIRE(out_dtype == d->dtype || (d->dtype == YE3T_F64 && out_dtype == YE3T_F32),
               "unsupported output dtype %d for a plan of dtype %d", d->out_dtype, d->dtype);
  const int in_dtype = d->in_dtype < 0 ? d->dtype : d->in_dtype;
  YE3T_REQUIRE(in_dtype == d->dtype || (d->dtype == YE3T_F64 && in_dtype == YE3T_F32),
               "unsupported density dtype %d for a plan of dtype %d", d->in_dtype, d->dtype);
  (void)out_dtype;
  (void)in_dtype;
  YE3T_REQUIRE(d->chunk_count >= 1 && d->a_width >= 1 && d->a_width <= 65536 && d->feature_count >= 1,
               "bad plan sizes");
  YE3T_REQUIRE(d->workspace_slots >= 1 && d->workspace_slots <= 65535, "bad workspace size");
  const size_t elem = d->dtype == YE3T_F64 ? 8 : 4;
  const size_t lds = size_t(d->workspace_slots) * kPad * elem;
  YE3T_REQUIRE(lds <= 64 * 1024, "plan workspace needs %zu bytes of LDS (limit 65536)", lds);
  // host-side validation of every index the kernel will use
  const int64_t C = d->chunk_count;
  YE3T_REQUIRE(d->chunk_word_offsets[0] == 0 && d->chunk_word_offsets[C] == d->word_count, "word offsets");
  YE3T_REQUIRE(d->chunk_coeff_offsets[0] == 0 && d->chunk_coeff_offsets[C] == d->coeff_count, "coeff offsets");
  YE3T_REQUIRE(d->chunk_out_offsets[0] == 0 && d->chunk_out_offsets[C] == d->out_slot_count, "out offsets");
  for (int64_t c = 0; c < C; ++c) {
    int64_t wpos = d->chunk_word_offsets[c];
    const int64_t wend = d->chunk_word_offsets[c + 1];
    int64_t cpos = d->chunk_coeff_offsets[c];
    YE3T_REQUIRE(wpos <= wend, "word offsets not monotone");
    while (wpos < wend) {
      const uint32_t h = d->words[wpos];
      const uint32_t op = h >> 28, n = h & 0x00FFFFFFu;
      if (op == OP_LOAD) {
        YE3T_REQUIRE(wpos + 1 + int64_t(n) <= wend, "chunk %lld: LOAD overruns", (long long)c);
        for (uint32_t i = 0; i < n; ++i) {
          const uint32_t t = d->words[wpos + 1 + i];
          YE3T_REQUIRE(int64_t(t >> 16) < d->workspace_slots && int64_t(t & 0xFFFFu) < d->a_width,
                       "chunk %lld: LOAD index out of range", (long long)c);
        }
        wpos += 1 + n;
        continue;
      }
      YE3T_REQUIRE(op >= OP_ACC1 && op <= OP_ACC4, "chunk %lld: bad opcode %u", (long long)c, op);
      const int per = (op == OP_ACC3 || op == OP_ACC4) ? 2 : 1;
      YE3T_REQUIRE(wpos + 2 + int64_t(per) * n <= wend, "chunk %lld: op overruns", (long long)c);
      YE3T_REQUIRE(int64_t(d->words[wpos + 1]) < d->workspace_slots, "chunk %lld: bad dst", (long long)c);
      for (uint32_t i = 0; i < per * n; ++i) {
        const uint32_t t = d->words[wpos + 2 + i];
        const bool hi_used = !(op == OP_ACC1) && !(op == OP_ACC3 && (i % 2) == 1);
        YE3T_REQUIRE(int64_t(t & 0xFFFFu) < d->workspace_slots, "chunk %lld: bad operand", (long long)c);
        if (hi_used) YE3T_REQUIRE(int64_t(t >> 16) < d->workspace_slots, "chunk %lld: bad operand", (long long)c);
      }
      wpos += 2 + int64_t(per) * n;
      cpos += n;
    }
    YE3T_REQUIRE(cpos == d->chunk_coeff_offsets[c + 1], "chunk %lld: coefficient count mismatch", (long long)c);
    const int64_t o0 = d->chunk_out_offsets[c], o1 = d->chunk_out_offsets[c + 1];
    YE3T_REQUIRE(d->chunk_first_column[c] >= 0 && d->chunk_first_column[c] + (o1 - o0) <= d->feature_count,
                 "chunk %lld: output columns out of range", (long long)c);
    for (int64_t o = o0; o < o1; ++o)
      YE3T_REQUIRE(int64_t(d->out_slots[o]) < d->workspace_slots, "chunk %lld: bad out slot", (long long)c);
  }
  return YE3T_OK;
}

// Scratch of ye3t_hip_product_adjoint_stream_noalloc: the per-group partial
// density gradients live in this file-scope device array instead of a
// caller's or the library's allocation.  Each device the library runs on
// holds its own copy until the process ends.  Host code never uses the
// array's name as an address: the device address comes from
// hipGetSymbolAddress, once per device, with that device current.
constexpr int64_t kNoAllocScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;  // held across each call's set-up and launches
void* g_scratch_address[kMaxScratchDevices] = {};
// Last eager use of each device's scratch: its stream and an event recorded
// after its kernels, so a call on another stream first waits for it.
hipEvent_t g_scratch_done[kMaxScratchDevices] = {};
hipStream_t g_scratch_stream[kMaxScratchDevices] = {};
bool g_scratch_used[kMaxScratchDevices] = {};

// Device address of `scratch` on device `dev` (the current device), and the
// event that orders its users.  Done once per device, at plan creation (never
// under stream capture), with the device current.  Caller holds
// g_scratch_mutex.
int scratch_setup_locked(int dev) {
  YE3T_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "device %d beyond the scratch table", dev);
  if (!g_scratch_address[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      return set_error(YE3T_ELAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                       hipGetErrorString(e));
    }
    g_scratch_address[dev] = ptr;
  }
  if (!g_scratch_done[dev]) {
    const hipError_t e = hipEventCreateWithFlags(&g_scratch_done[dev], hipEventDisableTiming);
    if (e != hipSuccess) {
      g_scratch_done[dev] = nullptr;
      return set_error(YE3T_ELAUNCH, "hipEventCreate for the scratch failed on device %d: %s", dev,
                       hipGetErrorString(e));
    }
  }
  return YE3T_OK;
}

int scratch_setup(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  return scratch_setup_locked(dev);
}

// ---- scratch of generated parts -------------------------------------------
// Kernel facts read from a gfx950 code object on the host: the AMDHSA kernel
// descriptor is the 64-byte object "<kernel>.kd" of the ELF symbol table, with
// the private (scratch) segment size per lane at byte 4 and the kernel code
// properties at byte 56 (bit 11: the kernel uses a dynamic stack).

template <typename T>
static bool elf_read(const unsigned char* base, uint64_t size, uint64_t off, T* out) {
  if (off > size || size - off < sizeof(T)) return false;
  std::memcpy(out, base + off, sizeof(T));
  return true;
}

static int kernel_descriptor_info(const void* code, int64_t size, const char* name, uint32_t* private_bytes,
                           uint32_t* group_bytes, int* dynamic_stack) {
  const auto* b = static_cast<const unsigned char*>(code);
  const uint64_t n = uint64_t(size);
  if (!code || size < 64 || !name) return set_error(YE3T_EINVAL, "NULL or short code object");
  if (!(b[0] == 0x7f && b[1] == 'E' && b[2] == 'L' && b[3] == 'F' && b[4] == 2))
    return set_error(YE3T_EINVAL, "not an ELF64 code object");
  uint64_t shoff = 0;
  uint16_t shentsize = 0, shnum = 0;
  if (!elf_read(b, n, 0x28, &shoff) || !elf_read(b, n, 0x3A, &shentsize) || !elf_read(b, n, 0x3C, &shnum) ||
      shentsize != 64)
    return set_error(YE3T_EINVAL, "bad ELF section table");
  const std::string want = std::string(name) + ".kd";
  for (uint16_t si = 0; si < shnum; ++si) {
    const uint64_t sh = shoff + uint64_t(si) * 64;
    uint32_t type = 0, link = 0;
    uint64_t off = 0, sz = 0, entsize = 0;
    if (!elf_read(b, n, sh + 4, &type) || !elf_read(b, n, sh + 24, &off) || !elf_read(b, n, sh + 32, &sz) ||
        !elf_read(b, n, sh + 40, &link) || !elf_read(b, n, sh + 56, &entsize))
      return set_error(YE3T_EINVAL, "bad ELF section header");
    if ((type != 2 && type != 11) || entsize != 24 || link >= shnum) continue;  // SHT_SYMTAB / SHT_DYNSYM
    uint64_t str_off = 0, str_size = 0;
    if (!elf_read(b, n, shoff + uint64_t(link) * 64 + 24, &str_off) ||
        !elf_read(b, n, shoff + uint64_t(link) * 64 + 32, &str_size) || str_off > n || n - str_off < str_size)
      return set_error(YE3T_EINVAL, "bad ELF string table");
    for (uint64_t k = 0; k + 24 <= sz; k += 24) {
      uint32_t st_name = 0;
      uint16_t shndx = 0;
      uint64_t value = 0;
      if (!elf_read(b, n, off + k, &st_name) || !elf_read(b, n, off + k + 6, &shndx) ||
          !elf_read(b, n, off + k + 8, &value))
        return set_error(YE3T_EINVAL, "bad ELF symbol");
      if (st_name >= str_size || str_size - st_name < want.size() + 1) continue;
      if (std::memcmp(b + str_off + st_name, want.c_str(), want.size() + 1) != 0) continue;
      if (shndx == 0 || shndx >= shnum) return set_error(YE3T_EINVAL, "kernel descriptor without a section");
      uint64_t saddr = 0, soff = 0;
      if (!elf_read(b, n, shoff + uint64_t(shndx) * 64 + 16, &saddr) ||
          !elf_read(b, n, shoff + uint64_t(shndx) * 64 + 24, &soff) || value < saddr)
        return set_error(YE3T_EINVAL, "bad kernel descriptor section");
      const uint64_t kd = soff + (value - saddr);
      uint32_t group = 0, priv = 0;
      uint16_t props = 0;
      if (!elf_read(b, n, kd, &group) || !elf_read(b, n, kd + 4, &priv) || !elf_read(b, n, kd + 56, &props))
        return set_error(YE3T_EINVAL, "kernel descriptor out of the code object");
      *private_bytes = priv;
      *group_bytes = group;
      *dynamic_stack = (props >> 11) & 1;
      return YE3T_OK;
    }
  }
  return set_error(YE3T_EINVAL, "kernel descriptor %s not found", want.c_str());
}

// hipRTC options of every generated kernel (after --offload-arch); they are
// part of the fingerprint that keys the on-disk code-object cache.
const char* const kRtcOptions[] = {"-O3", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};

// Largest private segment per lane a generated part may have.  Config 5's parts
// in 550-value chunks (2052 and 1260 bytes per lane) ended in a memory aperture
// violation on four part streams; 772 bytes (400-value chunks) ran clean.  Scratch
// is provisioned per queue for every wave slot of the device, so four streams of
// such parts asked for 4 x 2052 x 64 x (256 CUs x 32 slots) = 4.3 GB of it, against
// 1.6 GB at 772 bytes.  Parts above the bound, or using a dynamic stack (whose
// size the descriptor does not state), are refused before anything is loaded.
constexpr uint32_t kPartPrivateMax = 1024;
constexpr int64_t kPartScratchTotalMax = int64_t(2) << 30;  // all part streams together
constexpr int kPartStreamsMax = 4;

static int check_part_scratch(const void* code, int64_t size, const char* name, int device, const char* what, int64_t i) {
  uint32_t priv = 0, group = 0;
  int dyn = 0;
  const int rc = kernel_descriptor_info(code, size, name, &priv, &group, &dyn);
  if (rc != YE3T_OK) return rc;
  uint32_t limit = kPartPrivateMax;
  if (const char* e = std::getenv("YE3T_PART_PRIVATE_MAX")) {  // may only lower the bound
    const long v = std::atol(e);
    if (v >= 0 && uint32_t(v) < limit) limit = uint32_t(v);
  }
  if (dyn) return set_error(YE3T_EUNSUPPORTED, "%s %lld: kernel %s uses a dynamic stack", what, (long long)i, name);
  if (priv > limit)
    return set_error(YE3T_EUNSUPPORTED,
                     "%s %lld: kernel %s needs %u bytes of scratch per lane, above the %u this library runs "
                     "(use smaller chunks)",
                     what, (long long)i, name, priv, limit);
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) cus = 256;
  const int64_t total = int64_t(priv) * kLanes * int64_t(cus) * 32 * kPartStreamsMax;
  if (total > kPartScratchTotalMax)
    return set_error(YE3T_EUNSUPPORTED, "%s %lld: kernel %s would need %lld bytes of scratch on %d streams", what,
                     (long long)i, name, (long long)total, kPartStreamsMax);
  return YE3T_OK;
}

}  // namespace ye3t

using namespace ye3t;

extern "C" {

int ye3t_hip_product_stream_encode(const ye3t_product_plan_desc* d, int64_t* counts, uint32_t* recs,
                                   uint32_t* flags, int64_t* rec_off, uint32_t* loads, int64_t* load_off,
                                   int64_t* layout) {
  clear_error();
  YE3T_REQUIRE(counts != nullptr, "NULL counts");
  int rc = validate_plan_desc(d);
  if (rc != YE3T_OK) return rc;
  std::vector<uint4> r;
  std::vector<uint32_t> f;
  std::vector<uint2> l;
  std::vector<int64_t> ro, lo;
  StreamLayout lay{};
  int64_t lds = 0;
  if (!build_stream(d, r, f, ro, l, lo, lay, lds)) {
    counts[0] = counts[1] = counts[2] = 0;
    return YE3T_OK;  // no term stream for this plan
  }
  // the arrays keep one padding record / load when a plan has none
  const int64_t nrec = ro.back(), nload = lo.back();
  counts[0] = nrec;
  counts[1] = nload;
  counts[2] = d->chunk_count;
  if (recs) std::memcpy(recs, r.data(), sizeof(uint4) * size_t(nrec));
  if (flags) std::memcpy(flags, f.data(), sizeof(uint32_t) * size_t(nrec));
  if (rec_off) std::memcpy(rec_off, ro.data(), sizeof(int64_t) * ro.size());
  if (loads) std::memcpy(loads, l.data(), sizeof(uint2) * size_t(nload));
  if (load_off) std::memcpy(load_off, lo.data(), sizeof(int64_t) * lo.size());
  if (layout) {
    const int64_t v[8] = {lay.ws_bytes, lay.rec_at, lay.flag_at, lay.load_at, lay.out_at, lay.one_off, lds, kGroup};
    std::memcpy(layout, v, sizeof(v));
  }
  return YE3T_OK;
}

int64_t ye3t_hip_product_adjoint_workspace_bytes(const ye3t_hip_product_plan* p, int64_t samples) {
  clear_error();
  if (!p || samples < 0) {
    set_error(YE3T_EINVAL, "NULL plan or negative sample count");
    return -1;
  }
  if (!p->use_stream || samples == 0) return 0;
  int64_t bytes = 0;
  stream_adjoint_groups(p, samples, &bytes);
  return bytes;
}

int ye3t_hip_product_adjoint_stream(const ye3t_hip_product_plan* p, const void* A, int64_t lda, int columns,
                                    const void* gB, int64_t samples, void* workspace, int64_t workspace_bytes,
                                    void* gA, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(samples >= 0, "negative sample count");
  if (samples == 0) return YE3T_OK;
  YE3T_REQUIRE(p->use_stream, "this plan has no term stream (workspace too large)");
  if (p->in_dtype != p->dtype)
    return set_error(YE3T_EUNSUPPORTED, "the term stream reads densities of the plan's dtype only");
  YE3T_REQUIRE(A && gB && gA, "NULL input or output");
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  if (columns) {
    YE3T_REQUIRE(lda >= tiles * kLanes, "lda must cover whole 64-sample tiles");
  } else {
    YE3T_REQUIRE(lda == p->a_width, "a row-major density has lda == a_width");
  }
  int64_t need = 0;
  const int64_t groups = stream_adjoint_groups(p, samples, &need);
  YE3T_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace of %lld bytes needed", (long long)need);
  YE3T_REQUIRE(int64_t(p->stream_layout[1]) + int64_t(p->stream_layout[0]) <= 64 * 1024,
               "the adjoint's values, gradients, loads and output slots exceed 64 KB of LDS");
  const hipStream_t s = as_stream(stream);
  return columns ? launch_stream_adjoint<true>(p, A, lda, gB, samples, workspace, groups, gA, s)
                 : launch_stream_adjoint<false>(p, A, lda, gB, samples, workspace, groups, gA, s);
}

int ye3t_hip_product_adjoint_stream_noalloc(const ye3t_hip_product_plan* p, const void* A, int64_t lda,
                                            int columns, const void* gB, int64_t samples, void* gA,
                                            ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(samples >= 0, "negative sample count");
  if (samples == 0) return YE3T_OK;
  YE3T_REQUIRE(p->use_stream, "this plan has no term stream (workspace too large)");
  if (p->in_dtype != p->dtype)
    return set_error(YE3T_EUNSUPPORTED, "the term stream reads densities of the plan's dtype only");
  YE3T_REQUIRE(A && gB && gA, "NULL input or output");
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  if (columns) {
    YE3T_REQUIRE(lda >= tiles * kLanes, "lda must cover whole 64-sample tiles");
  } else {
    YE3T_REQUIRE(lda == p->a_width, "a row-major density has lda == a_width");
  }
  YE3T_REQUIRE(int64_t(p->stream_layout[1]) + int64_t(p->stream_layout[0]) <= 64 * 1024,
               "the adjoint's values, gradients, loads and output slots exceed 64 KB of LDS");
  int dev = 0;
  YE3T_CHECK_HIP(hipGetDevice(&dev));
  YE3T_REQUIRE(dev == p->device, "call on the plan's device");
  int64_t need = 0;
  const int64_t groups = stream_adjoint_groups(p, samples, &need, kNoAllocScratchBytes, true);
  if (groups < 1) {
    const int64_t one = p->a_width * tiles * kLanes * (p->dtype == YE3T_F64 ? 8 : 4);
    return set_error(YE3T_EUNSUPPORTED,
                     "%lld samples need %lld bytes of partial gradients; the static scratch holds %lld "
                     "(at most %lld samples of this plan)",
                     (long long)samples, (long long)one, (long long)kNoAllocScratchBytes,
                     (long long)(kNoAllocScratchBytes / (p->a_width * (p->dtype == YE3T_F64 ? 8 : 4)) / kLanes *
                                 kLanes));
  }
  const hipStream_t s = as_stream(stream);
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  YE3T_CHECK_HIP(hipStreamIsCapturing(s, &capture));
  // One call at a time per device: host threads queue on the mutex, and an
  // eager call on another stream than the last one waits on the GPU for the
  // last one's kernels.  Under capture no event is recorded or waited on: the
  // captured kernels are ordered by the stream the graph is launched on.
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_address[dev] || !g_scratch_done[dev]) {
    YE3T_REQUIRE(capture == hipStreamCaptureStatusNone,
                 "the scratch of device %d is set up by plan creation, not under stream capture", dev);
    const int rc = scratch_setup_locked(dev);
    if (rc != YE3T_OK) return rc;
  }
  void* const P = g_scratch_address[dev];
  const bool eager = capture == hipStreamCaptureStatusNone;
  if (eager && g_scratch_used[dev] && g_scratch_stream[dev] != s)
    YE3T_CHECK_HIP(hipStreamWaitEvent(s, g_scratch_done[dev], 0));
  const int rc = columns ? launch_stream_adjoint<true>(p, A, lda, gB, samples, P, groups, gA, s)
                         : launch_stream_adjoint<false>(p, A, lda, gB, samples, P, groups, gA, s);
  if (rc != YE3T_OK || !eager) return rc;
  YE3T_CHECK_HIP(hipEventRecord(g_scratch_done[dev], s));
  g_scratch_stream[dev] = s;
  g_scratch_used[dev] = true;
  return YE3T_OK;
}

int ye3t_hip_transpose(int dtype, const void* A, int64_t rows, int64_t cols, void* At, int64_t ld,
                       ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(rows >= 0 && cols >= 0 && ld >= rows, "bad transpose shape");
  if (cols == 0 || ld == 0) return YE3T_OK;
  YE3T_REQUIRE(A != nullptr || rows == 0, "NULL input");
  YE3T_REQUIRE(At != nullptr, "NULL output");
  const int64_t gx = (cols + 63) / 64, gy = (ld + 63) / 64;
  YE3T_REQUIRE(gx <= 0x7FFFFFFF && gy <= 65535, "transpose too large for one launch");
  const dim3 grid = dim3(unsigned(gx), unsigned(gy), 1u);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(transpose_kernel<double>, grid, dim3(256), 0, as_stream(stream), (const double*)A, rows, cols,
                       (double*)At, ld);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(transpose_kernel<float>, grid, dim3(256), 0, as_stream(stream), (const float*)A, rows, cols,
                       (float*)At, ld);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("transpose_kernel");
}

// Samples per block of part launches (tuning; off by default): with
// YE3T_PARTS_BLOCK_MB = m > 0 every part runs over one block of samples whose
// density rows take at most m MiB before any part starts the next block, so
// the parts after the first could re-read those rows from the device's
// last-level cache.  Measured at config 5 (28 parts, 200 000 samples): one
// block 113 ms, 192 MiB blocks 125 ms, 96 MiB 133 ms, 32 MiB 197 ms -- the
// smaller launches cost more than the reuse saves.  Blocks hold whole
// 64-sample tiles in multiples of 8 (one per XCD).
static int64_t part_block_samples(const ye3t_hip_product_plan* p, int64_t samples) {
  const char* env = std::getenv("YE3T_PARTS_BLOCK_MB");
  const int64_t mb = (env && *env) ? std::atoll(env) : 0;
  if (mb <= 0) return samples;
  const int64_t row = p->a_width * (p->in_dtype == YE3T_F64 ? 8 : 4);
  int64_t block = (mb << 20) / (row > 0 ? row : 1);
  block = block / (8 * kLanes) * (8 * kLanes);
  if (block < 8 * kLanes) block = 8 * kLanes;
  return block < samples ? block : samples;
}

// the generated kernel in parts, in order: density value (s, k) at A[s * row_stride + k * col_stride]
static int launch_parts(const ye3t_hip_product_plan* p, const void* A, int64_t row_stride, int64_t col_stride,
                        int64_t samples, void* B, hipStream_t stream) {
  const int64_t block = part_block_samples(p, samples);
  // a multiple of 8 tile columns: the parts deal tiles to XCDs by linear workgroup id
  const int64_t max_tiles = ((block + kLanes - 1) / kLanes + 7) & ~int64_t(7);
  YE3T_REQUIRE(max_tiles <= int64_t(0x7FFFFFF8), "too many samples for one launch");
  const size_t a_elem = p->in_dtype == YE3T_F64 ? 8 : 4, b_elem = p->out_dtype == YE3T_F64 ? 8 : 4;
  // the parts address a lane's density values and a tile of B with 32-bit byte offsets
  YE3T_REQUIRE(row_stride >= 0 && col_stride >= 0 && uint64_t(63 * row_stride) * a_elem < (uint64_t(1) << 32),
               "density rows too wide for the generated parts");
  YE3T_REQUIRE(uint64_t(64) * uint64_t(p->feature_count) * b_elem < (uint64_t(1) << 32),
               "feature rows too wide for the generated parts");
  long rs_arg = long(row_stride), cs_arg = long(col_stride);
  const int lanes = p->part_lanes;
  // launches every part over samples [s0, s0 + n)
  auto launch_block = [&](int64_t s0, int64_t n, bool on_lanes) -> int {
    const int64_t tiles = ((n + kLanes - 1) / kLanes + 7) & ~int64_t(7);
    long s_arg = long(n);
    const void* a_arg = static_cast<const unsigned char*>(A) + size_t(s0 * row_stride) * a_elem;
    void* b_arg = static_cast<unsigned char*>(B) + size_t(s0) * size_t(p->feature_count) * b_elem;
    void* args[] = {&a_arg, &s_arg, &b_arg, &rs_arg, &cs_arg};
    for (int64_t i = 0; i < p->part_count; ++i)
      YE3T_CHECK_HIP(hipModuleLaunchKernel(p->part_fns[i], unsigned(tiles), unsigned(p->part_chunks[i]), 1, kLanes,
                                           1, 1, 0, on_lanes ? p->part_streams[i % lanes] : stream, args, nullptr));
    return YE3T_OK;
  };
  if (lanes <= 1) {
    for (int64_t s0 = 0; s0 < samples; s0 += block) {
      const int rc = launch_block(s0, std::min(block, samples - s0), false);
      if (rc != YE3T_OK) return rc;
    }
    return YE3T_OK;
  }
  // fork: the plan's streams start after the caller's prior work; join: the
  // caller's stream continues after every part
  YE3T_CHECK_HIP(hipEventRecord(p->part_fork, stream));
  for (int k = 0; k < lanes; ++k) YE3T_CHECK_HIP(hipStreamWaitEvent(p->part_streams[k], p->part_fork, 0));
  for (int64_t s0 = 0; s0 < samples; s0 += block) {
    const int rc = launch_block(s0, std::min(block, samples - s0), true);
    if (rc != YE3T_OK) return rc;
  }
  for (int k = 0; k < lanes; ++k) {
    YE3T_CHECK_HIP(hipEventRecord(p->part_join[k], p->part_streams[k]));
    YE3T_CHECK_HIP(hipStreamWaitEvent(stream, p->part_join[k], 0));
  }
  return YE3T_OK;
}

int ye3t_hip_product_forward_columns(const ye3t_hip_product_plan* p, const void* At, int64_t ld, int64_t samples,
                                     void* B, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(samples >= 0, "negative sample count");
  if (samples == 0) return YE3T_OK;
  YE3T_REQUIRE(At && B, "NULL input or output");
  YE3T_REQUIRE(ld >= samples, "ld must cover the samples");
  if (p->part_count > 0 && !p->use_interpreter) return launch_parts(p, At, 1, ld, samples, B, as_stream(stream));
  YE3T_REQUIRE(p->use_stream, "this plan has no term stream (workspace too large); use ye3t_hip_product_forward");
  if (p->in_dtype != p->dtype)
    return set_error(YE3T_EUNSUPPORTED, "the term stream reads densities of the plan's dtype only");
  YE3T_REQUIRE(ld >= (samples + kLanes - 1) / kLanes * kLanes, "ld must cover whole 64-sample tiles");
  return launch_stream<true>(p, At, ld, samples, B, stream);
}

extern "C++" {
namespace ye3t {
// gA[s, k] = sum of P[row * ldp + s] over column k's partial rows, in their
// listed order: 256 threads per 64 samples x 64 columns, staged in LDS so the
// row-major gA block is written in row segments
template <typename Real, typename Out>
__global__ __launch_bounds__(256) void adjoint_parts_reduce_kernel(const Real* __restrict__ P, int64_t ldp,
                                                                   const int64_t* __restrict__ col_off,
                                                                   const int64_t* __restrict__ row_ids, int64_t W,
                                                                   int64_t samples, Out* __restrict__ gA) {
  __shared__ Real tile[64][65];
  const int lane = threadIdx.x & 63, cw = threadIdx.x >> 6;
  const int64_t s0 = int64_t(blockIdx.x) * 64, k0 = int64_t(blockIdx.y) * 64;
  const int rows = samples - s0 < 64 ? int(samples - s0) : 64;
  const int cols = W - k0 < 64 ? int(W - k0) : 64;
  // the map is wave-uniform: read through the scalar cache; eight partial rows
  // in flight per step, added in the listed order
  typedef const __attribute__((address_space(4))) int64_t* cptr;
  const cptr off = (cptr)(col_off);
  const cptr ids = (cptr)(row_ids);
  const Real* __restrict__ Ps = P + s0 + lane;
  for (int c = cw; c < cols; c += 4) {
    Real v = Real(0);
    int64_t q = off[k0 + c];
    const int64_t e = off[k0 + c + 1];
    for (; q + 8 <= e; q += 8) {
      Real t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = Ps[ids[q + u] * ldp];
#pragma unroll
      for (int u = 0; u < 8; ++u) v += t[u];
    }
    for (; q < e; ++q) v += Ps[ids[q] * ldp];
    tile[c][lane] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < rows * cols; i += 256) {
    const int r = i / cols, c = i - r * cols;
    gA[(s0 + r) * W + k0 + c] = Out(tile[c][r]);
  }
}
// out[s] = bias + sum over rows c < rows of P[c * ldp + s], in row order
template <typename Real, typename Out>
__global__ __launch_bounds__(256) void readout_parts_reduce_kernel(const Real* __restrict__ P, int64_t ldp,
                                                                   int64_t rows, Real bias, int64_t samples,
                                                                   Out* __restrict__ out) {
  const int64_t s = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (s >= samples) return;
  Real v = bias;
  int64_t c = 0;
  for (; c + 8 <= rows; c += 8) {
    Real t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = P[(c + u) * ldp + s];
#pragma unroll
    for (int u = 0; u < 8; ++u) v += t[u];
  }
  for (; c < rows; ++c) v += P[c * ldp + s];
  out[s] = Out(v);
}
}  // namespace ye3t
}  // extern "C++"

static void release_readout_parts(ye3t_hip_product_plan* p) {
  for (int64_t i = 0; i < p->ro_count; ++i)
    if (p->ro_modules[i]) (void)hipModuleUnload(p->ro_modules[i]);
  delete[] p->ro_modules;
  delete[] p->ro_fns;
  delete[] p->ro_chunks;
  p->ro_modules = nullptr;
  p->ro_fns = nullptr;
  p->ro_chunks = nullptr;
  p->ro_count = 0;
  p->ro_total = 0;
}

static void release_adjoint_parts(ye3t_hip_product_plan* p) {
  for (int64_t i = 0; i < p->adj_count; ++i)
    if (p->adj_modules[i]) (void)hipModuleUnload(p->adj_modules[i]);
  delete[] p->adj_modules;
  delete[] p->adj_fns;
  delete[] p->adj_chunks;
  (void)hipFree(p->adj_col_off);
  (void)hipFree(p->adj_row_ids);
  p->adj_modules = nullptr;
  p->adj_fns = nullptr;
  p->adj_chunks = nullptr;
  p->adj_col_off = nullptr;
  p->adj_row_ids = nullptr;
  p->adj_count = 0;
  p->adj_rows = 0;
}

static void release_parts(ye3t_hip_product_plan* p) {
  for (int k = 0; k < p->part_lanes; ++k) {
    (void)hipStreamDestroy(p->part_streams[k]);
    (void)hipEventDestroy(p->part_join[k]);
  }
  if (p->part_lanes > 0) (void)hipEventDestroy(p->part_fork);
  p->part_lanes = 0;
  for (int64_t i = 0; i < p->part_count; ++i)
    if (p->part_modules[i]) (void)hipModuleUnload(p->part_modules[i]);
  delete[] p->part_modules;
  delete[] p->part_fns;
  delete[] p->part_chunks;
  p->part_modules = nullptr;
  p->part_fns = nullptr;
  p->part_chunks = nullptr;
  p->part_count = 0;
}

void ye3t_hip_product_plan_destroy(ye3t_hip_product_plan* p) {
  if (!p) return;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(p->device);
  (void)hipFree(p->words);
  (void)hipFree(p->coeffs);
  (void)hipFree(p->out_slots);
  (void)hipFree(p->word_off);
  (void)hipFree(p->coeff_off);
  (void)hipFree(p->out_off);
  (void)hipFree(p->first_col);
  (void)hipFree(p->recs);
  (void)hipFree(p->flags);
  (void)hipFree(p->rec_off);
  (void)hipFree(p->loads);
  (void)hipFree(p->load_off);
  if (p->module) (void)hipModuleUnload(p->module);
  if (p->readout_module) (void)hipModuleUnload(p->readout_module);
  if (p->adjoint_module) (void)hipModuleUnload(p->adjoint_module);
  release_parts(p);
  release_adjoint_parts(p);
  release_readout_parts(p);
  (void)hipSetDevice(prev);
  delete p;
}

int ye3t_hip_product_plan_create(const ye3t_product_plan_desc* d, ye3t_hip_product_plan** out) {
  clear_error();
  YE3T_REQUIRE(d && out, "NULL plan description or output");
  *out = nullptr;
  {
    const int rc = validate_plan_desc(d);
    if (rc != YE3T_OK) return rc;
  }
  const int out_dtype = d->out_dtype < 0 ? d->dtype : d->out_dtype;
  const size_t elem = d->dtype == YE3T_F64 ? 8 : 4;
  const int64_t C = d->chunk_count;
  auto* p = new ye3t_hip_product_plan();
  p->dtype = d->dtype;
  p->out_dtype = out_dtype;
  p->in_dtype = d->in_dtype < 0 ? d->dtype : d->in_dtype;
  p->a_width = d->a_width;
  p->feature_count = d->feature_count;
  p->chunk_count = C;
  p->slots = d->workspace_slots;
  (void)hipGetDevice(&p->device);
  int rc = YE3T_OK;
  if ((rc = upload(&p->words, d->words, d->word_count)) != YE3T_OK ||
      (rc = upload(reinterpret_cast<unsigned char**>(&p->coeffs), static_cast<const unsigned char*>(d->coeffs),
                   d->coeff_count * int64_t(elem))) != YE3T_OK ||
      (rc = upload(&p->out_slots, d->out_slots, d->out_slot_count)) != YE3T_OK ||
      (rc = upload(&p->word_off, d->chunk_word_offsets, C + 1)) != YE3T_OK ||
      (rc = upload(&p->coeff_off, d->chunk_coeff_offsets, C + 1)) != YE3T_OK ||
      (rc = upload(&p->out_off, d->chunk_out_offsets, C + 1)) != YE3T_OK ||
      (rc = upload(&p->first_col, d->chunk_first_column, C)) != YE3T_OK) {
    ye3t_hip_product_plan_destroy(p);
    return rc;
  }
  // the term-stream interpreter; YE3T_PRODUCT_STREAM=0 keeps the word interpreter (comparisons)
  const char* env = std::getenv("YE3T_PRODUCT_STREAM");
  std::vector<uint4> recs;
  std::vector<uint32_t> flags;
  std::vector<uint2> loads;
  std::vector<int64_t> rec_off, load_off;
  StreamLayout lay{};
  int64_t stream_lds = 0;
  if (!(env && env[0] == '0') && build_stream(d, recs, flags, rec_off, loads, load_off, lay, stream_lds)) {
    if ((rc = upload(&p->recs, recs.data(), int64_t(recs.size()))) != YE3T_OK ||
        (rc = upload(&p->flags, flags.data(), int64_t(flags.size()))) != YE3T_OK ||
        (rc = upload(&p->rec_off, rec_off.data(), C + 1)) != YE3T_OK ||
        (rc = upload(&p->loads, loads.data(), int64_t(loads.size()))) != YE3T_OK ||
        (rc = upload(&p->load_off, load_off.data(), C + 1)) != YE3T_OK) {
      ye3t_hip_product_plan_destroy(p);
      return rc;
    }
    const uint32_t fields[7] = {lay.ws_bytes, lay.rec_at,  lay.flag_at, lay.load_at,
                                lay.out_at,   lay.one_off, lay.sink_off};
    std::memcpy(p->stream_layout, fields, sizeof(fields));
    p->stream_lds = stream_lds;
    p->use_stream = 1;
    const char* per = std::getenv("YE3T_STREAM_TILES");
    p->stream_tiles = per ? std::atoll(per) : 0;
    // the allocation-free adjoint's scratch address and ordering event, looked
    // up here so that entry point makes no set-up call (it may run under capture)
    if ((rc = scratch_setup(p->device)) != YE3T_OK) {
      ye3t_hip_product_plan_destroy(p);
      return rc;
    }
  }
  *out = p;
  return YE3T_OK;
}

int ye3t_hip_rtc_fingerprint(char* buf, int64_t capacity) {
  clear_error();
  YE3T_REQUIRE(buf && capacity > 0, "NULL argument");
  int major = 0, minor = 0;
  if (hiprtcVersion(&major, &minor) != HIPRTC_SUCCESS) return set_error(YE3T_ELAUNCH, "hiprtcVersion failed");
  std::string fp = "hiprtc " + std::to_string(major) + "." + std::to_string(minor) + " | options";
  for (const char* o : ye3t::kRtcOptions) fp += std::string(" ") + o;
  fp += " | abi " + std::to_string(YE3T_HIP_ABI_VERSION);
  YE3T_REQUIRE(int64_t(fp.size()) < capacity, "fingerprint buffer too small");
  std::memcpy(buf, fp.c_str(), fp.size() + 1);
  return YE3T_OK;
}

int ye3t_hip_rtc_compile(const char* source, const char* name, const char* arch, void** code, int64_t* size) {
  clear_error();
  YE3T_REQUIRE(source && code && size, "NULL argument");
  *code = nullptr;
  *size = 0;
  std::string arch_opt = std::string("--offload-arch=") + (arch && *arch ? arch : "gfx950");
  const char* opts[1 + sizeof(ye3t::kRtcOptions) / sizeof(ye3t::kRtcOptions[0])] = {arch_opt.c_str()};
  for (size_t i = 0; i < sizeof(ye3t::kRtcOptions) / sizeof(ye3t::kRtcOptions[0]); ++i) opts[i + 1] = ye3t::kRtcOptions[i];
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, source, name ? name : "ye3t_generated.hip", 0, nullptr, nullptr) !=
      HIPRTC_SUCCESS) {
    return set_error(YE3T_ELAUNCH, "hiprtcCreateProgram failed");
  }
  const hiprtcResult rc = hiprtcCompileProgram(prog, int(sizeof(opts) / sizeof(opts[0])), opts);
  if (rc != HIPRTC_SUCCESS) {
    size_t log_size = 0;
    hiprtcGetProgramLogSize(prog, &log_size);
    std::string log(log_size + 1, '\0');
    if (log_size) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    return set_error(YE3T_ELAUNCH, "hiprtc compile failed: %s", log.substr(0, 900).c_str());
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  void* buf = std::malloc(n ? n : 1);
  if (!buf) {
    hiprtcDestroyProgram(&prog);
    return set_error(YE3T_ENOMEM, "out of host memory");
  }
  hiprtcGetCode(prog, static_cast<char*>(buf));
  hiprtcDestroyProgram(&prog);
  *code = buf;
  *size = int64_t(n);
  return YE3T_OK;
}

void ye3t_hip_free(void* ptr) { std::free(ptr); }

int ye3t_hip_code_object_kernel_info(const void* code, int64_t size, const char* kernel_name,
                                     int64_t* private_segment_bytes, int64_t* group_segment_bytes,
                                     int* uses_dynamic_stack) {
  clear_error();
  YE3T_REQUIRE(private_segment_bytes && group_segment_bytes && uses_dynamic_stack, "NULL output");
  uint32_t priv = 0, group = 0;
  int dyn = 0;
  const int rc = kernel_descriptor_info(code, size, kernel_name, &priv, &group, &dyn);
  if (rc != YE3T_OK) return rc;
  *private_segment_bytes = priv;
  *group_segment_bytes = group;
  *uses_dynamic_stack = dyn;
  return YE3T_OK;
}

int64_t ye3t_hip_part_private_limit(void) { return kPartPrivateMax; }

int ye3t_hip_product_plan_attach_generated(ye3t_hip_product_plan* p, const void* code, int64_t size,
                                           const char* kernel_name, int64_t chunk_count, int64_t rows_per_tile,
                                           int persistent, int threads_per_block) {
  clear_error();
  YE3T_REQUIRE(p && code && size > 0 && kernel_name, "NULL argument");
  YE3T_REQUIRE(chunk_count >= 1 && chunk_count <= 65535, "bad generated chunk count");
  YE3T_REQUIRE(rows_per_tile >= 1 && rows_per_tile <= kLanes, "rows_per_tile must be in [1, 64]");
  YE3T_REQUIRE(threads_per_block >= kLanes && threads_per_block <= 1024 && threads_per_block % kLanes == 0,
               "threads_per_block must be a multiple of 64 in [64, 1024]");
  int prev = 0;
  YE3T_CHECK_HIP(hipGetDevice(&prev));
  YE3T_REQUIRE(prev == p->device, "attach on the plan's device");
  hipModule_t module;
  YE3T_CHECK_HIP(hipModuleLoadData(&module, code));
  hipFunction_t fn;
  if (hipModuleGetFunction(&fn, module, kernel_name) != hipSuccess) {
    (void)hipModuleUnload(module);
    return set_error(YE3T_EINVAL, "kernel %s not found in code object", kernel_name);
  }
  if (p->module) (void)hipModuleUnload(p->module);
  p->module = module;
  p->generated = fn;
  p->generated_chunks = chunk_count;
  p->generated_rows = rows_per_tile;
  p->generated_threads = threads_per_block;
  p->generated_max_grid = 0;
  if (persistent) {
    YE3T_REQUIRE(chunk_count == 1 && rows_per_tile == kLanes, "a persistent kernel has one chunk of 64-row tiles");
    int per_cu = 0, cus = 0;
    YE3T_CHECK_HIP(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads_per_block, 0));
    YE3T_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p->device));
    p->generated_max_grid = int64_t(per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    // YE3T_PRODUCT_GRID overrides the resident-workgroup count (tuning)
    const char* g = std::getenv("YE3T_PRODUCT_GRID");
    if (g && *g && std::atoll(g) > 0) p->generated_max_grid = std::atoll(g);
  }
  p->use_interpreter = 0;
  return YE3T_OK;
}

int ye3t_hip_product_plan_attach_generated_parts(ye3t_hip_product_plan* p, int64_t part_count,
                                                 const void* const* codes, const int64_t* sizes,
                                                 const char* const* kernel_names, const int64_t* chunk_counts) {
  clear_error();
  YE3T_REQUIRE(p && codes && sizes && kernel_names && chunk_counts, "NULL argument");
  YE3T_REQUIRE(part_count >= 1 && part_count <= (int64_t(1) << 20), "part_count must be in [1, 2^20]");
  int64_t total = 0;
  for (int64_t i = 0; i < part_count; ++i) {
    YE3T_REQUIRE(codes[i] && sizes[i] > 0 && kernel_names[i], "NULL or empty part %lld", (long long)i);
    YE3T_REQUIRE(chunk_counts[i] >= 1 && chunk_counts[i] <= 65535, "bad chunk count of part %lld", (long long)i);
    total += chunk_counts[i];
  }
  YE3T_REQUIRE(total <= (int64_t(1) << 31), "too many chunks");
  int prev = 0;
  YE3T_CHECK_HIP(hipGetDevice(&prev));
  YE3T_REQUIRE(prev == p->device, "attach on the plan's device");
  for (int64_t i = 0; i < part_count; ++i) {
    const int rc = check_part_scratch(codes[i], sizes[i], kernel_names[i], p->device, "part", i);
    if (rc != YE3T_OK) return rc;
  }
  auto* modules = new hipModule_t[size_t(part_count)]();
  auto* fns = new hipFunction_t[size_t(part_count)]();
  auto* chunks = new int64_t[size_t(part_count)];
  for (int64_t i = 0; i < part_count; ++i) {
    chunks[i] = chunk_counts[i];
    hipError_t e = hipModuleLoadData(&modules[i], codes[i]);
    if (e == hipSuccess && hipModuleGetFunction(&fns[i], modules[i], kernel_names[i]) != hipSuccess)
      e = hipErrorNotFound;
    if (e != hipSuccess) {
      for (int64_t j = 0; j <= i; ++j)
        if (modules[j]) (void)hipModuleUnload(modules[j]);
      delete[] modules;
      delete[] fns;
      delete[] chunks;
      return set_error(YE3T_EINVAL, "part %lld: code object not loadable or kernel %s not found", (long long)i,
                       kernel_names[i]);
    }
  }
  release_parts(p);
  p->part_modules = modules;
  p->part_fns = fns;
  p->part_chunks = chunks;
  p->part_count = part_count;
  // concurrent streams for the parts (YE3T_PARTS_STREAMS, 1..4, default 4), at the default priority
  int lanes = 4;
  if (const char* e = std::getenv("YE3T_PARTS_STREAMS")) lanes = std::atoi(e);
  lanes = lanes < 1 ? 1 : (lanes > 4 ? 4 : lanes);
  if (lanes > part_count) lanes = int(part_count);
  if (lanes > 1) {
    YE3T_CHECK_HIP(hipEventCreateWithFlags(&p->part_fork, hipEventDisableTiming));
    for (int k = 0; k < lanes; ++k) {
      YE3T_CHECK_HIP(hipStreamCreateWithFlags(&p->part_streams[k], hipStreamNonBlocking));
      YE3T_CHECK_HIP(hipEventCreateWithFlags(&p->part_join[k], hipEventDisableTiming));
      p->part_lanes = k + 1;
    }
  }
  p->use_interpreter = 0;
  return YE3T_OK;
}

int ye3t_hip_product_plan_attach_adjoint_parts(ye3t_hip_product_plan* p, int64_t part_count,
                                               const void* const* codes, const int64_t* sizes,
                                               const char* const* kernel_names, const int64_t* chunk_counts,
                                               int64_t partial_rows, const int64_t* col_off, const int64_t* row_ids) {
  clear_error();
  YE3T_REQUIRE(p && codes && sizes && kernel_names && chunk_counts && col_off, "NULL argument");
  YE3T_REQUIRE(part_count >= 1 && part_count <= (int64_t(1) << 20), "part_count must be in [1, 2^20]");
  YE3T_REQUIRE(partial_rows >= 0 && partial_rows < (int64_t(1) << 40), "bad partial row count");
  const int64_t W = p->a_width;
  YE3T_REQUIRE(col_off[0] == 0, "col_off[0] must be 0");
  for (int64_t k = 0; k < W; ++k) YE3T_REQUIRE(col_off[k + 1] >= col_off[k], "col_off must be non-decreasing");
  const int64_t nnz = col_off[W];
  YE3T_REQUIRE(nnz == 0 || row_ids != nullptr, "NULL row_ids");
  for (int64_t q = 0; q < nnz; ++q)
    YE3T_REQUIRE(row_ids[q] >= 0 && row_ids[q] < partial_rows, "row id %lld out of range", (long long)q);
  for (int64_t i = 0; i < part_count; ++i) {
    YE3T_REQUIRE(codes[i] && sizes[i] > 0 && kernel_names[i], "NULL or empty part %lld", (long long)i);
    YE3T_REQUIRE(chunk_counts[i] >= 1 && chunk_counts[i] <= 65535, "bad chunk count of part %lld", (long long)i);
  }
  int prev = 0;
  YE3T_CHECK_HIP(hipGetDevice(&prev));
  YE3T_REQUIRE(prev == p->device, "attach on the plan's device");
  for (int64_t i = 0; i < part_count; ++i) {
    const int rc = check_part_scratch(codes[i], sizes[i], kernel_names[i], p->device, "adjoint part", i);
    if (rc != YE3T_OK) return rc;
  }
  int64_t* d_off = nullptr;
  int64_t* d_ids = nullptr;
  YE3T_CHECK_HIP(hipMalloc(&d_off, size_t(W + 1) * sizeof(int64_t)));
  if (hipMalloc(&d_ids, size_t(nnz > 0 ? nnz : 1) * sizeof(int64_t)) != hipSuccess) {
    (void)hipFree(d_off);
    return set_error(YE3T_ENOMEM, "device allocation failed");
  }
  if (hipMemcpy(d_off, col_off, size_t(W + 1) * sizeof(int64_t), hipMemcpyHostToDevice) != hipSuccess ||
      (nnz > 0 && hipMemcpy(d_ids, row_ids, size_t(nnz) * sizeof(int64_t), hipMemcpyHostToDevice) != hipSuccess)) {
    (void)hipFree(d_off);
    (void)hipFree(d_ids);
    return set_error(YE3T_ELAUNCH, "copying the reduction map failed");
  }
  auto* modules = new hipModule_t[size_t(part_count)]();
  auto* fns = new hipFunction_t[size_t(part_count)]();
  auto* chunks = new int64_t[size_t(part_count)];
  for (int64_t i = 0; i < part_count; ++i) {
    chunks[i] = chunk_counts[i];
    hipError_t e = hipModuleLoadData(&modules[i], codes[i]);
    if (e == hipSuccess && hipModuleGetFunction(&fns[i], modules[i], kernel_names[i]) != hipSuccess)
      e = hipErrorNotFound;
    if (e != hipSuccess) {
      for (int64_t j = 0; j <= i; ++j)
        if (modules[j]) (void)hipModuleUnload(modules[j]);
      delete[] modules;
      delete[] fns;
      delete[] chunks;
      (void)hipFree(d_off);
      (void)hipFree(d_ids);
      return set_error(YE3T_EINVAL, "adjoint part %lld: code object not loadable or kernel %s not found",
                       (long long)i, kernel_names[i]);
    }
  }
  release_adjoint_parts(p);
  p->adj_modules = modules;
  p->adj_fns = fns;
  p->adj_chunks = chunks;
  p->adj_count = part_count;
  p->adj_rows = partial_rows;
  p->adj_col_off = d_off;
  p->adj_row_ids = d_ids;
  return YE3T_OK;
}

int64_t ye3t_hip_product_adjoint_parts_workspace_bytes(const ye3t_hip_product_plan* p, int64_t samples) {
  clear_error();
  if (!p || samples < 0) {
    set_error(YE3T_EINVAL, "NULL plan or negative sample count");
    return -1;
  }
  if (p->adj_count == 0 || samples == 0) return 0;
  const int64_t ldp = (samples + kLanes - 1) / kLanes * kLanes;
  return p->adj_rows * ldp * int64_t(p->dtype == YE3T_F64 ? 8 : 4);
}

int ye3t_hip_product_adjoint_parts(const ye3t_hip_product_plan* p, const void* A, int64_t lda, int columns,
                                   const void* gB, int64_t samples, void* workspace, int64_t workspace_bytes,
                                   void* gA, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(samples >= 0, "negative sample count");
  if (samples == 0) return YE3T_OK;
  YE3T_REQUIRE(p->adj_count > 0, "no adjoint parts attached");
  YE3T_REQUIRE(A && gB && gA, "NULL input or output");
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  if (columns) {
    YE3T_REQUIRE(lda >= samples, "lda must cover the samples");
  } else {
    YE3T_REQUIRE(lda == p->a_width, "a row-major density has lda == a_width");
  }
  const int64_t ldp = tiles * kLanes;
  const int64_t need = p->adj_rows * ldp * int64_t(p->dtype == YE3T_F64 ? 8 : 4);
  YE3T_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace of %lld bytes needed", (long long)need);
  const int64_t gx = (tiles + 7) & ~int64_t(7);  // the parts deal tiles to XCDs by linear workgroup id
  YE3T_REQUIRE(gx <= int64_t(0x7FFFFFF8), "too many samples for one launch");
  const hipStream_t s = as_stream(stream);
  long s_arg = long(samples), rs_arg = long(columns ? 1 : p->a_width), cs_arg = long(columns ? lda : 1);
  // the parts address a lane's density values and a tile of gB with 32-bit byte offsets
  YE3T_REQUIRE(uint64_t(63 * rs_arg) * (p->in_dtype == YE3T_F64 ? 8u : 4u) < (uint64_t(1) << 32),
               "density rows too wide for the adjoint parts");
  YE3T_REQUIRE(uint64_t(64) * uint64_t(p->feature_count) * (p->out_dtype == YE3T_F64 ? 8u : 4u) <
                   (uint64_t(1) << 32),
               "feature rows too wide for the adjoint parts");
  long ldp_arg = long(ldp);
  const void* a_arg = A;
  const void* g_arg = gB;
  void* w_arg = workspace;
  void* args[] = {&a_arg, &g_arg, &s_arg, &w_arg, &rs_arg, &cs_arg, &ldp_arg};
  const int lanes = p->part_lanes;
  if (lanes > 1) {
    YE3T_CHECK_HIP(hipEventRecord(p->part_fork, s));
    for (int k = 0; k < lanes; ++k) YE3T_CHECK_HIP(hipStreamWaitEvent(p->part_streams[k], p->part_fork, 0));
  }
  for (int64_t i = 0; i < p->adj_count; ++i)
    YE3T_CHECK_HIP(hipModuleLaunchKernel(p->adj_fns[i], unsigned(gx), unsigned(p->adj_chunks[i]), 1, kLanes, 1, 1, 0,
                                         lanes > 1 ? p->part_streams[i % lanes] : s, args, nullptr));
  if (lanes > 1) {
    for (int k = 0; k < lanes; ++k) {
      YE3T_CHECK_HIP(hipEventRecord(p->part_join[k], p->part_streams[k]));
      YE3T_CHECK_HIP(hipStreamWaitEvent(s, p->part_join[k], 0));
    }
  }
  const dim3 grid = dim3(unsigned(tiles), unsigned((p->a_width + 63) / 64)), block = dim3(256);
  if (p->dtype == YE3T_F64 && p->in_dtype == YE3T_F64) {
    hipLaunchKernelGGL((adjoint_parts_reduce_kernel<double, double>), grid, block, 0, s,
                       static_cast<const double*>(workspace), ldp, p->adj_col_off, p->adj_row_ids, p->a_width,
                       samples, static_cast<double*>(gA));
  } else if (p->dtype == YE3T_F64) {
    hipLaunchKernelGGL((adjoint_parts_reduce_kernel<double, float>), grid, block, 0, s,
                       static_cast<const double*>(workspace), ldp, p->adj_col_off, p->adj_row_ids, p->a_width,
                       samples, static_cast<float*>(gA));
  } else {
    hipLaunchKernelGGL((adjoint_parts_reduce_kernel<float, float>), grid, block, 0, s,
                       static_cast<const float*>(workspace), ldp, p->adj_col_off, p->adj_row_ids, p->a_width,
                       samples, static_cast<float*>(gA));
  }
  return check_launch("adjoint_parts_reduce_kernel");
}

int ye3t_hip_product_plan_attach_readout_parts(ye3t_hip_product_plan* p, int64_t part_count,
                                               const void* const* codes, const int64_t* sizes,
                                               const char* const* kernel_names, const int64_t* chunk_counts) {
  clear_error();
  YE3T_REQUIRE(p && codes && sizes && kernel_names && chunk_counts, "NULL argument");
  YE3T_REQUIRE(part_count >= 1 && part_count <= (int64_t(1) << 20), "part_count must be in [1, 2^20]");
  int64_t total = 0;
  for (int64_t i = 0; i < part_count; ++i) {
    YE3T_REQUIRE(codes[i] && sizes[i] > 0 && kernel_names[i], "NULL or empty part %lld", (long long)i);
    YE3T_REQUIRE(chunk_counts[i] >= 1 && chunk_counts[i] <= 65535, "bad chunk count of part %lld", (long long)i);
    total += chunk_counts[i];
  }
  int prev = 0;
  YE3T_CHECK_HIP(hipGetDevice(&prev));
  YE3T_REQUIRE(prev == p->device, "attach on the plan's device");
  for (int64_t i = 0; i < part_count; ++i) {
    const int rc = check_part_scratch(codes[i], sizes[i], kernel_names[i], p->device, "readout part", i);
    if (rc != YE3T_OK) return rc;
  }
  auto* modules = new hipModule_t[size_t(part_count)]();
  auto* fns = new hipFunction_t[size_t(part_count)]();
  auto* chunks = new int64_t[size_t(part_count)];
  for (int64_t i = 0; i < part_count; ++i) {
    chunks[i] = chunk_counts[i];
    hipError_t e = hipModuleLoadData(&modules[i], codes[i]);
    if (e == hipSuccess && hipModuleGetFunction(&fns[i], modules[i], kernel_names[i]) != hipSuccess)
      e = hipErrorNotFound;
    if (e != hipSuccess) {
      for (int64_t j = 0; j <= i; ++j)
        if (modules[j]) (void)hipModuleUnload(modules[j]);
      delete[] modules;
      delete[] fns;
      delete[] chunks;
      return set_error(YE3T_EINVAL, "readout part %lld: code object not loadable or kernel %s not found",
                       (long long)i, kernel_names[i]);
    }
  }
  release_readout_parts(p);
  p->ro_modules = modules;
  p->ro_fns = fns;
  p->ro_chunks = chunks;
  p->ro_count = part_count;
  p->ro_total = total;
  return YE3T_OK;
}

int64_t ye3t_hip_product_linear_parts_workspace_bytes(const ye3t_hip_product_plan* p, int64_t samples) {
  clear_error();
  if (!p || samples < 0) {
    set_error(YE3T_EINVAL, "NULL plan or negative sample count");
    return -1;
  }
  if (p->ro_count == 0 || samples == 0) return 0;
  return p->ro_total * ((samples + kLanes - 1) / kLanes * kLanes) * int64_t(p->dtype == YE3T_F64 ? 8 : 4);
}

int ye3t_hip_product_linear_forward_parts(const ye3t_hip_product_plan* p, const void* A, int64_t lda, int columns,
                                          int64_t samples, const void* weight, double bias, void* workspace,
                                          int64_t workspace_bytes, void* out, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(samples >= 0, "negative sample count");
  if (samples == 0) return YE3T_OK;
  YE3T_REQUIRE(p->ro_count > 0, "no readout parts attached");
  YE3T_REQUIRE(A && weight && out, "NULL input or output");
  if (columns) {
    YE3T_REQUIRE(lda >= samples, "lda must cover the samples");
  } else {
    YE3T_REQUIRE(lda == p->a_width, "a row-major density has lda == a_width");
  }
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  const int64_t ldp = tiles * kLanes;
  const int64_t need = p->ro_total * ldp * int64_t(p->dtype == YE3T_F64 ? 8 : 4);
  YE3T_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace of %lld bytes needed", (long long)need);
  const int64_t gx = (tiles + 7) & ~int64_t(7);  // the parts deal tiles to XCDs by linear workgroup id
  YE3T_REQUIRE(gx <= int64_t(0x7FFFFFF8), "too many samples for one launch");
  const hipStream_t s = as_stream(stream);
  long s_arg = long(samples), rs_arg = long(columns ? 1 : p->a_width), cs_arg = long(columns ? lda : 1);
  // the parts address a lane's density values with 32-bit byte offsets
  YE3T_REQUIRE(uint64_t(63 * rs_arg) * (p->in_dtype == YE3T_F64 ? 8u : 4u) < (uint64_t(1) << 32),
               "density rows too wide for the readout parts");
  long ldp_arg = long(ldp);
  const void* a_arg = A;
  void* w_arg = workspace;
  const void* wt_arg = weight;
  void* args[] = {&a_arg, &s_arg, &w_arg, &wt_arg, &rs_arg, &cs_arg, &ldp_arg};
  const int lanes = p->part_lanes;
  if (lanes > 1) {
    YE3T_CHECK_HIP(hipEventRecord(p->part_fork, s));
    for (int k = 0; k < lanes; ++k) YE3T_CHECK_HIP(hipStreamWaitEvent(p->part_streams[k], p->part_fork, 0));
  }
  for (int64_t i = 0; i < p->ro_count; ++i)
    YE3T_CHECK_HIP(hipModuleLaunchKernel(p->ro_fns[i], unsigned(gx), unsigned(p->ro_chunks[i]), 1, kLanes, 1, 1, 0,
                                         lanes > 1 ? p->part_streams[i % lanes] : s, args, nullptr));
  if (lanes > 1) {
    for (int k = 0; k < lanes; ++k) {
      YE3T_CHECK_HIP(hipEventRecord(p->part_join[k], p->part_streams[k]));
      YE3T_CHECK_HIP(hipStreamWaitEvent(s, p->part_join[k], 0));
    }
  }
  const unsigned grid = unsigned((samples + 255) / 256);
  if (p->dtype == YE3T_F64 && p->out_dtype == YE3T_F64) {
    hipLaunchKernelGGL((readout_parts_reduce_kernel<double, double>), dim3(grid), dim3(256), 0, s,
                       static_cast<const double*>(workspace), ldp, p->ro_total, bias, samples,
                       static_cast<double*>(out));
  } else if (p->dtype == YE3T_F64) {
    hipLaunchKernelGGL((readout_parts_reduce_kernel<double, float>), dim3(grid), dim3(256), 0, s,
                       static_cast<const double*>(workspace), ldp, p->ro_total, bias, samples,
                       static_cast<float*>(out));
  } else {
    hipLaunchKernelGGL((readout_parts_reduce_kernel<float, float>), dim3(grid), dim3(256), 0, s,
                       static_cast<const float*>(workspace), ldp, p->ro_total, float(bias), samples,
                       static_cast<float*>(out));
  }
  return check_launch("readout_parts_reduce_kernel");
}

int ye3t_hip_product_plan_select(ye3t_hip_product_plan* p, int use_interpreter) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(use_interpreter || p->generated || p->part_count > 0, "no generated kernel attached");
  p->use_interpreter = use_interpreter ? 1 : 0;
  return YE3T_OK;
}

int ye3t_hip_product_plan_uses_stream(const ye3t_hip_product_plan* p) { return p && p->use_stream ? 1 : 0; }

int ye3t_hip_product_launch_info(const ye3t_hip_product_plan* p, int64_t samples, int64_t* grid, int64_t* block,
                                 int64_t* lds) {
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  const int64_t per = p->use_stream ? stream_tiles_per_group(p, tiles) : 1;
  if (grid) *grid = (tiles + per - 1) / per * p->chunk_count;
  if (block) *block = kLanes;
  if (lds) *lds = int64_t(product_lds_bytes(p));
  return YE3T_OK;
}

int ye3t_hip_product_forward(const ye3t_hip_product_plan* p, const void* A, int64_t samples, void* B,
                             ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(samples >= 0, "negative sample count");
  if (samples == 0) return YE3T_OK;
  YE3T_REQUIRE(A && B, "NULL input or output");
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  // the persistent generated kernel stores 16-byte vectors: a misaligned B runs the generic kernel
  const bool generated_ok =
      p->generated && !p->use_interpreter && (p->generated_max_grid == 0 || reinterpret_cast<uintptr_t>(B) % 16 == 0);
  if (generated_ok) {
    int64_t gtiles = (samples + p->generated_rows - 1) / p->generated_rows;
    YE3T_REQUIRE(gtiles <= int64_t(0x7FFFFFFF), "too many samples for one launch");
    if (p->generated_max_grid > 0 && gtiles > p->generated_max_grid) gtiles = p->generated_max_grid;
    long s_arg = long(samples);
    const void* a_arg = A;
    void* b_arg = B;
    void* args[] = {&a_arg, &s_arg, &b_arg};
    YE3T_CHECK_HIP(hipModuleLaunchKernel(p->generated, unsigned(gtiles), unsigned(p->generated_chunks), 1,
                                         unsigned(p->generated_threads), 1,
                                         1, 0, as_stream(stream), args, nullptr));
    return YE3T_OK;
  }
  if (p->part_count > 0 && !p->use_interpreter)
    return launch_parts(p, A, p->a_width, 1, samples, B, as_stream(stream));
  if (p->in_dtype != p->dtype)
    return set_error(YE3T_EUNSUPPORTED,
                     "an fp32 density with fp64 arithmetic runs on an attached generated kernel only "
                     "(and, for a persistent one, a 16-byte aligned B)");
  const int64_t grid = tiles * p->chunk_count;
  YE3T_REQUIRE(grid <= int64_t(0x7FFFFFFF), "too many samples for one launch");
  const size_t lds = product_lds_bytes(p);
  if (p->use_stream) return launch_stream<false>(p, A, p->a_width, samples, B, stream);
  if (p->dtype == YE3T_F64 && p->out_dtype == YE3T_F64) {
    hipLaunchKernelGGL((product_kernel<double, double>), dim3(unsigned(grid)), dim3(kLanes), lds, as_stream(stream),
                       (const double*)A, samples, p->a_width, (double*)B, p->feature_count, p->words, p->word_off,
                       (const double*)p->coeffs, p->coeff_off, p->out_slots, p->out_off, p->first_col,
                       p->chunk_count);
  } else if (p->dtype == YE3T_F64) {
    hipLaunchKernelGGL((product_kernel<double, float>), dim3(unsigned(grid)), dim3(kLanes), lds, as_stream(stream),
                       (const double*)A, samples, p->a_width, (float*)B, p->feature_count, p->words, p->word_off,
                       (const double*)p->coeffs, p->coeff_off, p->out_slots, p->out_off, p->first_col,
                       p->chunk_count);
  } else {
    hipLaunchKernelGGL((product_kernel<float, float>), dim3(unsigned(grid)), dim3(kLanes), lds, as_stream(stream),
                       (const float*)A, samples, p->a_width, (float*)B, p->feature_count, p->words, p->word_off,
                       (const float*)p->coeffs, p->coeff_off, p->out_slots, p->out_off, p->first_col,
                       p->chunk_count);
  }
  return check_launch("product_kernel");
}

namespace {
// Load `kernel_name` from a code object for a persistent launch: the module,
// the function and the number of workgroups of `threads` the device holds at once.
int load_persistent(const ye3t_hip_product_plan* p, const void* code, const char* kernel_name, int threads,
                    hipModule_t* module, hipFunction_t* fn, int64_t* max_grid) {
  int prev = 0;
  YE3T_CHECK_HIP(hipGetDevice(&prev));
  YE3T_REQUIRE(prev == p->device, "attach on the plan's device");
  YE3T_CHECK_HIP(hipModuleLoadData(module, code));
  if (hipModuleGetFunction(fn, *module, kernel_name) != hipSuccess) {
    (void)hipModuleUnload(*module);
    return set_error(YE3T_EINVAL, "kernel %s not found in code object", kernel_name);
  }
  int per_cu = 0, cus = 0;
  if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, *fn, threads, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p->device) != hipSuccess) {
    (void)hipModuleUnload(*module);
    return set_error(YE3T_ELAUNCH, "occupancy query failed for %s", kernel_name);
  }
  *max_grid = int64_t(per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
  return YE3T_OK;
}
}  // namespace

int ye3t_hip_product_plan_attach_readout(ye3t_hip_product_plan* p, const void* code, int64_t size,
                                         const char* kernel_name, int threads_per_block) {
  clear_error();
  YE3T_REQUIRE(p && code && size > 0 && kernel_name, "NULL argument");
  YE3T_REQUIRE(threads_per_block >= kLanes && threads_per_block <= 1024 && threads_per_block % kLanes == 0,
               "threads_per_block must be a multiple of 64 in [64, 1024]");
  hipModule_t module;
  hipFunction_t fn;
  int64_t max_grid = 0;
  const int rc = load_persistent(p, code, kernel_name, threads_per_block, &module, &fn, &max_grid);
  if (rc != YE3T_OK) return rc;
  if (p->readout_module) (void)hipModuleUnload(p->readout_module);
  p->readout_module = module;
  p->readout = fn;
  p->readout_threads = threads_per_block;
  p->readout_max_grid = max_grid;
  return YE3T_OK;
}

int ye3t_hip_product_plan_attach_adjoint(ye3t_hip_product_plan* p, const void* code, int64_t size,
                                         const char* kernel_name, int threads_per_block) {
  clear_error();
  YE3T_REQUIRE(p && code && size > 0 && kernel_name, "NULL argument");
  YE3T_REQUIRE(threads_per_block >= kLanes && threads_per_block <= 1024 && threads_per_block % kLanes == 0,
               "threads_per_block must be a multiple of 64 in [64, 1024]");
  hipModule_t module;
  hipFunction_t fn;
  int64_t max_grid = 0;
  const int rc = load_persistent(p, code, kernel_name, threads_per_block, &module, &fn, &max_grid);
  if (rc != YE3T_OK) return rc;
  if (p->adjoint_module) (void)hipModuleUnload(p->adjoint_module);
  p->adjoint_module = module;
  p->adjoint = fn;
  p->adjoint_threads = threads_per_block;
  p->adjoint_max_grid = max_grid;
  return YE3T_OK;
}

int ye3t_hip_product_adjoint(const ye3t_hip_product_plan* p, const void* A, const void* gB, int64_t samples,
                             void* gA, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(samples >= 0, "negative sample count");
  if (!p->adjoint) return set_error(YE3T_EUNSUPPORTED, "no adjoint kernel attached to this plan");
  if (samples == 0) return YE3T_OK;
  YE3T_REQUIRE(A && gB && gA, "NULL input, gradient or output");
  YE3T_REQUIRE(reinterpret_cast<uintptr_t>(gB) % 16 == 0, "gB must be 16-byte aligned (tiles load 16-byte words)");
  int64_t grid = (samples + kLanes - 1) / kLanes;
  if (grid > p->adjoint_max_grid) grid = p->adjoint_max_grid;
  long s_arg = long(samples);
  const void* a_arg = A;
  const void* g_arg = gB;
  void* o_arg = gA;
  void* args[] = {&a_arg, &g_arg, &s_arg, &o_arg};
  YE3T_CHECK_HIP(hipModuleLaunchKernel(p->adjoint, unsigned(grid), 1, 1, unsigned(p->adjoint_threads), 1, 1, 0,
                                       as_stream(stream), args, nullptr));
  return YE3T_OK;
}

int ye3t_hip_product_linear_forward(const ye3t_hip_product_plan* p, const void* A, int64_t samples,
                                    const void* weight, double bias, void* out, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(samples >= 0, "negative sample count");
  if (!p->readout) return set_error(YE3T_EUNSUPPORTED, "no fused readout kernel attached to this plan");
  if (samples == 0) return YE3T_OK;
  YE3T_REQUIRE(A && weight && out, "NULL input, weight or output");
  int64_t grid = (samples + kLanes - 1) / kLanes;
  if (grid > p->readout_max_grid) grid = p->readout_max_grid;
  long s_arg = long(samples);
  const void* a_arg = A;
  void* o_arg = out;
  const void* w_arg = weight;
  double bias64 = bias;
  float bias32 = float(bias);
  void* args[] = {&a_arg, &s_arg, &o_arg, &w_arg,
                  p->dtype == YE3T_F64 ? static_cast<void*>(&bias64) : static_cast<void*>(&bias32)};
  YE3T_CHECK_HIP(hipModuleLaunchKernel(p->readout, unsigned(grid), 1, 1, unsigned(p->readout_threads), 1, 1, 0,
                                       as_stream(stream), args, nullptr));
  return YE3T_OK;
}

int ye3t_hip_rows_dot(int dtype, const void* B, int64_t samples, int64_t F, const void* weight, double bias,
                      void* out, ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(samples >= 0 && F >= 0, "negative size");
  if (samples == 0) return YE3T_OK;
  YE3T_REQUIRE(out && (F == 0 || (B && weight)), "NULL input, weight or output");
  int64_t grid = (samples + 3) / 4;  // four waves (rows) per 256-thread workgroup
  if (grid > (1 << 20)) grid = 1 << 20;
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(rows_dot_kernel<double>, dim3(unsigned(grid)), dim3(256), 0, as_stream(stream),
                       (const double*)B, samples, F, (const double*)weight, bias, (double*)out);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(rows_dot_kernel<float>, dim3(unsigned(grid)), dim3(256), 0, as_stream(stream),
                       (const float*)B, samples, F, (const float*)weight, bias, (float*)out);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("rows_dot_kernel");
}

int ye3t_hip_evaluate_factorized_schedule(int dtype, const void* bv, int64_t batch, int64_t basis, int64_t blocks,
                                          int64_t mdim, const int64_t* offsets, const int64_t* labels,
                                          const int64_t* midx, const void* coeffs, int64_t K, void* out,
                                          ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(batch >= 0 && basis >= 0 && blocks >= 0 && mdim >= 0 && K >= 0, "negative size");
  if (batch * K == 0) return YE3T_OK;
  YE3T_REQUIRE(bv && offsets && labels && out, "NULL argument");
  const unsigned grid = grid_1d(batch * K, 256);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(evaluate_schedule_kernel<double>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const double*)bv, batch, basis, blocks, mdim, offsets, labels, midx, (const double*)coeffs, K,
                       (double*)out);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(evaluate_schedule_kernel<float>, dim3(grid), dim3(256), 0, as_stream(stream),
                       (const float*)bv, batch, basis, blocks, mdim, offsets, labels, midx, (const float*)coeffs, K,
                       (float*)out);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("evaluate_schedule_kernel");
}

}  // extern "C"
