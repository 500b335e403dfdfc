// Stage 2 -- ACE B-features from the density on gfx950.
//
// (a) product_kernel: executes a compiled product plan.  The plan is a DAG of
//     leaf loads, symmetric-block monomials and real CG pair couplings, shared
//     across labels and contents (intermediate couplings computed once per
//     sample).  One wave (64 lanes) processes 64 samples, lane = sample; the
//     instruction stream and coefficients are wave-uniform (scalar loads), the
//     per-sample workspace lives in LDS as [slot][65] (lane-minor, padded so the
//     transposed output read is bank-conflict free).  Output columns of a chunk
//     are written through LDS so each store instruction covers contiguous
//     columns of one row.
// (b) evaluate_schedule_kernel / sym_monomial_kernel: device versions of the
//     reference's flat schedule evaluator and symmetric-power contraction.
#include <hip/hiprtc.h>

#include <cstdlib>
#include <cstring>
#include <vector>

#include "common.h"

struct ye3t_hip_product_plan {
  int dtype;      // A, coefficients and arithmetic
  int out_dtype;  // B
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

template <typename Real>
__device__ inline Real ipow(Real b, int64_t e) {
  Real v = Real(1);
  while (e > 0) {
    if (e & 1) v *= b;
    e >>= 1;
    if (e > 0) b *= b;
  }
  return v;
}

template <typename Real>
__global__ __launch_bounds__(256) void sym_monomial_kernel(const Real* __restrict__ x, int64_t batch, int64_t D,
                                                           const int64_t* __restrict__ counts,
                                                           const int64_t* __restrict__ offsets,
                                                           const Real* __restrict__ values, int64_t O,
                                                           Real* __restrict__ out) {
  const int64_t total = batch * O;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int64_t b = idx / O, o = idx - (idx / O) * O;
    const Real* row = x + b * D;
    Real acc = Real(0);
    for (int64_t t = offsets[o]; t < offsets[o + 1]; ++t) {
      Real m = values[t];
      for (int64_t c = 0; c < D; ++c) m *= ipow(row[c], counts[t * D + c]);
      acc += m;
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
  return size_t(p->slots) * kPad * elem;
}

}  // namespace ye3t

using namespace ye3t;

extern "C" {

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
  if (p->module) (void)hipModuleUnload(p->module);
  if (p->readout_module) (void)hipModuleUnload(p->readout_module);
  if (p->adjoint_module) (void)hipModuleUnload(p->adjoint_module);
  (void)hipSetDevice(prev);
  delete p;
}

int ye3t_hip_product_plan_create(const ye3t_product_plan_desc* d, ye3t_hip_product_plan** out) {
  clear_error();
  YE3T_REQUIRE(d && out, "NULL plan description or output");
  *out = nullptr;
  YE3T_REQUIRE(d->dtype == YE3T_F32 || d->dtype == YE3T_F64, "unsupported dtype %d", d->dtype);
  const int out_dtype = d->out_dtype < 0 ? d->dtype : d->out_dtype;
  YE3T_REQUIRE(out_dtype == d->dtype || (d->dtype == YE3T_F64 && out_dtype == YE3T_F32),
               "unsupported output dtype %d for a plan of dtype %d", d->out_dtype, d->dtype);
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
  auto* p = new ye3t_hip_product_plan();
  p->dtype = d->dtype;
  p->out_dtype = out_dtype;
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
  *out = p;
  return YE3T_OK;
}

int ye3t_hip_rtc_compile(const char* source, const char* name, const char* arch, void** code, int64_t* size) {
  clear_error();
  YE3T_REQUIRE(source && code && size, "NULL argument");
  *code = nullptr;
  *size = 0;
  std::string arch_opt = std::string("--offload-arch=") + (arch && *arch ? arch : "gfx950");
  const char* opts[] = {arch_opt.c_str(), "-O3", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
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

int ye3t_hip_product_plan_select(ye3t_hip_product_plan* p, int use_interpreter) {
  clear_error();
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  YE3T_REQUIRE(use_interpreter || p->generated, "no generated kernel attached");
  p->use_interpreter = use_interpreter ? 1 : 0;
  return YE3T_OK;
}

int ye3t_hip_product_launch_info(const ye3t_hip_product_plan* p, int64_t samples, int64_t* grid, int64_t* block,
                                 int64_t* lds) {
  YE3T_REQUIRE(p != nullptr, "NULL plan");
  const int64_t tiles = (samples + kLanes - 1) / kLanes;
  if (grid) *grid = tiles * p->chunk_count;
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
  const int64_t grid = tiles * p->chunk_count;
  YE3T_REQUIRE(grid <= int64_t(0x7FFFFFFF), "too many samples for one launch");
  const size_t lds = product_lds_bytes(p);
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

int ye3t_hip_symmetric_power_monomial(int dtype, const void* x, int64_t batch, int64_t D, const int64_t* counts,
                                      const int64_t* offsets, const void* values, int64_t O, void* out,
                                      ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(batch >= 0 && D >= 0 && O >= 0, "negative size");
  if (batch * O == 0) return YE3T_OK;
  YE3T_REQUIRE(x && offsets && out, "NULL argument");
  const unsigned grid = grid_1d(batch * O, 256);
  if (dtype == YE3T_F64) {
    hipLaunchKernelGGL(sym_monomial_kernel<double>, dim3(grid), dim3(256), 0, as_stream(stream), (const double*)x,
                       batch, D, counts, offsets, (const double*)values, O, (double*)out);
  } else if (dtype == YE3T_F32) {
    hipLaunchKernelGGL(sym_monomial_kernel<float>, dim3(grid), dim3(256), 0, as_stream(stream), (const float*)x,
                       batch, D, counts, offsets, (const float*)values, O, (float*)out);
  } else {
    return set_error(YE3T_EDTYPE, "unsupported dtype %d", dtype);
  }
  return check_launch("sym_monomial_kernel");
}

}  // extern "C"
