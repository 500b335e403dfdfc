/*
 * ye3t_hip -- C ABI of the MI355X (gfx950) HIP backend for the ACE
 * native-execution-plan hot path.
 *
 * Conventions
 *   - All array arguments are device pointers to contiguous row-major memory
 *     (host pointers only where a comment says "host").
 *   - `dtype` is YE3T_F32 or YE3T_F64; float arrays of one call share it.
 *   - Work is enqueued on `stream` (NULL = default stream); calls never
 *     synchronise the device except plan creation, which copies tables.
 *   - Return 0 on success, a negative ye3t_status on failure; the message of
 *     the last failure on the calling thread is ye3t_hip_last_error().
 *     Nothing throws across this boundary.
 */
#ifndef YE3T_HIP_H
#define YE3T_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define YE3T_HIP_ABI_VERSION 61 /* reference native ABI floor is 42 (execution_plan.py:35) */

typedef struct ihipStream_t* ye3t_stream_t; /* == hipStream_t */

enum ye3t_dtype { YE3T_F32 = 0, YE3T_F64 = 1, YE3T_C64 = 2, YE3T_C128 = 3 /* complex: (re, im) pairs */ };

enum ye3t_status {
  YE3T_OK = 0,
  YE3T_EINVAL = -1,      /* invalid argument / shape */
  YE3T_ELAUNCH = -2,     /* HIP launch or runtime failure */
  YE3T_EDTYPE = -3,      /* unsupported dtype */
  YE3T_ENOMEM = -4,      /* device allocation failed */
  YE3T_EUNSUPPORTED = -5 /* size outside the compiled kernel limits */
};

/* Library ABI version; replaces core_abi_version() of the reference's pybind
 * module (ye3t/runtime/csrc/execution_plan_torch.cpp:7924-7934). */
int ye3t_hip_abi_version(void);

/* 1 when a HIP device is visible to this process, else 0: the counterpart of
 * has_cuda() of the reference's pybind module (execution_plan_torch.cpp:7924-7934,
 * consumed by native_execution_plan_capabilities, execution_plan.py:6118). */
int ye3t_hip_has_hip(void);

/* 0: this library has no CPU kernels (the reference's CPU runtime serves CPU
 * tensors); counterpart of has_cpu() (execution_plan_torch.cpp:7924-7934). */
int ye3t_hip_has_cpu(void);

/* Thread-local message of the last failed call ("" if none). */
const char* ye3t_hip_last_error(void);

typedef struct {
  char arch[64];            /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int device;
  int cu_count;
  int wavefront_size;
  int lds_bytes_per_block;  /* max shared memory per block */
  int clock_khz;
  int64_t hbm_bytes;
  double hbm_peak_gbs;      /* nominal peak used for roofline fractions */
} ye3t_hip_caps;

/* Device facts for the capability report (has_cuda()/has_cpu() counterpart,
 * execution_plan_torch.cpp:7924-7934). */
int ye3t_hip_device_caps(int device, ye3t_hip_caps* out);

/* ChebExpCos radial table and d/dr, [E, n_max+1] each.
 * Replaces the CUDA branch of ye3t_runtime::cheb_exp_cos_radial_table_with_derivative
 * (schema execution_plan_torch.cpp:7237-7240; kernel execution_plan_cuda.cu:3386-3470).
 * `derivatives` may be NULL. */
int ye3t_hip_radial_table(int dtype, const void* radii, const void* cutoffs, const void* lambdas,
                          int64_t edge_count, int64_t max_radial_index, void* values, void* derivatives,
                          ye3t_stream_t stream);

/* Real spherical-harmonic table [E, (l_max+1)^2] and Cartesian gradient
 * [E, (l_max+1)^2, 3] of edge vectors [E, 3].  Replaces the CUDA branch of
 * ye3t_runtime::spherical_harmonics_table_with_derivative with real_output=true
 * (schema execution_plan_torch.cpp:7250-7253; kernel execution_plan_cuda.cu:4266-4365).
 * `gradients` may be NULL.  l_max <= 12. */
int ye3t_hip_real_sph_table(int dtype, const void* edge_vectors, int64_t edge_count, int64_t l_max,
                            double epsilon, void* values, void* gradients, ye3t_stream_t stream);

/* Scheduled radial-angular edge channels and their Cartesian derivatives:
 * edge_values[e, k] = channel_scales[k] * R[e, ri_k] * Y[e, ai_k] where
 * channel_types[k] is -1 or edge_types[e] (zero otherwise), and
 * edge_derivatives[e, k, :] = channel_scales[k] * (dR[e, ri_k] *
 * radial_directions[e, :] * Y[e, ai_k] + R[e, ri_k] * dY[e, ai_k, :]), from the
 * radial table R, dR [E, radial_width], the angular table Y [E, angular_width]
 * with dY [E, angular_width, 3] and unit directions [E, 3].  Rounded as the
 * reference core rounds (ye3t_runtime_core.cpp:1550-1604): bit-identical.
 * Channel indices must lie in their tables and types be >= -1 (checked by the
 * caller; the kernel clamps indices instead of faulting).  Replaces
 * ye3t_runtime::scheduled_radial_angular_channels_with_derivative (schema
 * execution_plan_torch.cpp:7268-7274, CPU execution_plan_torch.cpp:1230-1336,
 * CUDA kernel execution_plan_cuda.cu:4568, launcher :9946-10060). */
int ye3t_hip_scheduled_radial_angular_channels(int dtype, int64_t edge_count, int64_t radial_width,
                                               int64_t angular_width, int64_t channel_count,
                                               const void* radial_values, const void* radial_derivatives,
                                               const void* angular_values, const void* angular_derivatives,
                                               const void* radial_directions, const int64_t* edge_types,
                                               const int64_t* channel_radial_indices,
                                               const int64_t* channel_angular_indices,
                                               const int64_t* channel_types, const void* channel_scales,
                                               void* edge_values, void* edge_derivatives,
                                               ye3t_stream_t stream);

/* out[i, c] = sum over edges e in [row_offsets[i], row_offsets[i+1]) of
 * edge_values[e, c]; deterministic CSR segment reduction, no atomics.
 * Replaces ye3t_runtime::density_accumulate (schema execution_plan_torch.cpp:7284-7286,
 * CUDA atomics kernel execution_plan_cuda.cu:281-301) for centre-sorted edges. */
int ye3t_hip_density_accumulate_csr(int dtype, const void* edge_values, const int64_t* row_offsets,
                                    int64_t atom_count, int64_t channel_count, void* out,
                                    ye3t_stream_t stream);

/* edge_adjoint[e, c] = atomic_adjoint[centers[e], c] for e < edge_count, c <
 * channel_count: the adjoint of density accumulation (a gather of centre rows;
 * any edge order).  centers[e] must lie in [0, atom_count) (checked by the
 * caller; the kernel clamps out-of-range indices instead of faulting).
 * Replaces ye3t_runtime::density_accumulate_adjoint (schema
 * execution_plan_torch.cpp:7288, CUDA kernel execution_plan_cuda.cu:9241-9260,
 * launcher :13890-13921; CPU core ye3t_runtime_core.cpp:1704-1715). */
int ye3t_hip_density_accumulate_adjoint(int dtype, const void* atomic_adjoint, const int64_t* centers,
                                        int64_t edge_count, int64_t channel_count, int64_t atom_count,
                                        void* edge_adjoint, ye3t_stream_t stream);

/* Fused stage 1: A[i, c, r, lm] = sum_{e in row i} w_c(e) R_r(|v_e|) Y_lm(v_e/|v_e|).
 * One pass over edges: radial basis and real SH in registers, per-atom CSR
 * segment reduction, no atomics.  Fuses the reference chain
 * cheb_exp_cos_radial_table -> spherical_harmonics_table ->
 * scheduled_radial_angular_channels -> density_accumulate
 * (execution_plan.py:7298, 7479, 7675, 7913). */
typedef struct {
  int dtype;
  int64_t atom_count;
  int64_t edge_count;
  const int64_t* row_offsets;   /* [N+1] edges sorted by centre */
  const int64_t* neighbors;     /* [E] neighbour atom of each edge */
  const void* edge_vectors;     /* [E, 3] r_j - r_i */
  const int32_t* species;       /* [N] one-hot channel of each atom, or NULL */
  const void* node_features;    /* [N, C] channel weights h[j, c], or NULL */
  const void* radial_mix;       /* [C, n_max+1]: R_c = sum_n mix[c,n] R_n, or NULL */
  int64_t channel_count;        /* C (species count, feature channels, or 1) */
  int64_t max_radial_index;     /* n_max <= 15 */
  int64_t max_angular;          /* l_max <= 8 */
  double cutoff;
  double lambda;
  double epsilon;
  int out_dtype;                /* dtype of A and of the accumulation; -1 = dtype.  YE3T_F64 with
                                   dtype YE3T_F32 keeps fp32 inputs but an fp64 density */
  int accumulate_dtype;         /* arithmetic of the density; -1 = out_dtype.  YE3T_F64 with an
                                   fp32 out_dtype accumulates in fp64 (matrix cores) and rounds A
                                   once to fp32 at the store (fp64-MFMA shapes only, else
                                   YE3T_EUNSUPPORTED) */
} ye3t_density_args;

/* A has shape [N, C, R, (l_max+1)^2] with R = 1 when radial_mix is set, else n_max+1. */
int ye3t_hip_ace_density_forward(const ye3t_density_args* args, void* A, ye3t_stream_t stream);

/* Name of the kernel the last ye3t_hip_ace_density_forward call on this thread
 * launched ("" if none), for profiling.  No reference counterpart. */
const char* ye3t_hip_last_density_kernel(void);

/* Edge-vector gradient of the fused stage 1 (forces): edge_gradient[e, :] =
 * d <density_adjoint, A> / d edge_vectors[e, :] for density_adjoint shaped like
 * A ([N, C, R, (l_max+1)^2], dtype adjoint_dtype: YE3T_F64, or YE3T_F32 /
 * YE3T_F64 with fp32 edge vectors) and edge_gradient [E, 3] in args->dtype;
 * fp64 arithmetic, one lane per edge, no atomics.  The radial derivative's
 * direction is v / max(|v|, epsilon), the unit vector of the harmonics.
 * args->out_dtype and args->accumulate_dtype are ignored; n_max <= 15,
 * l_max <= 8.  Replaces the reference's force path
 * scheduled_radial_angular_channels_with_derivative (execution_plan.py:7675;
 * schema execution_plan_torch.cpp:7267; CPU core ye3t_runtime_core.cpp:1550-1604)
 * on the radial/harmonic derivative tables, followed by density_accumulate_adjoint
 * (execution_plan_torch.cpp:7288) and the contraction with the edge adjoint. */
int ye3t_hip_ace_density_edge_gradient(const ye3t_density_args* args, int adjoint_dtype, const void* density_adjoint,
                                       void* edge_gradient, ye3t_stream_t stream);

/* S[b, o] = sum_{t in [output_offsets[o], output_offsets[o+1])} monomial_values[t]
 *           * prod_c input[b, c]^monomial_counts[t, c]
 * for input[batch, input_dim], monomial_counts[T, input_dim], output_offsets[O+1]
 * and output_indices[T] (the output of each term, consistent with the offsets;
 * the adjoint's gather index).  Device tables, validated by the caller.
 * Replaces the CUDA branch of ye3t_runtime::symmetric_power_monomial
 * (schema execution_plan_torch.cpp:7528-7530; kernel execution_plan_cuda.cu:5229;
 * CPU ye3t_runtime_core.cpp:5279-5315). */
int ye3t_hip_symmetric_power_monomial(int dtype, const void* input, int64_t batch, int64_t input_dim,
                                      const int64_t* monomial_counts, const int64_t* output_offsets,
                                      const int64_t* output_indices, const void* monomial_values, int64_t term_count,
                                      int64_t output_dim, void* output, ye3t_stream_t stream);

/* input_adjoint[b, c] of output_adjoint[batch, output_dim] through the grouped
 * table: the reference's rule for zero factors (ye3t_runtime_core.cpp:5318-5389).
 * Replaces ye3t_runtime::symmetric_power_monomial_adjoint (schema
 * execution_plan_torch.cpp:7531-7534). */
int ye3t_hip_symmetric_power_monomial_adjoint(int dtype, const void* output_adjoint, const void* input,
                                              int64_t batch, int64_t input_dim, const int64_t* monomial_counts,
                                              const int64_t* output_indices, const void* monomial_values,
                                              int64_t term_count, int64_t output_dim, void* input_adjoint,
                                              ye3t_stream_t stream);

/* S[b, o] = sum_{k in [output_offsets[o], output_offsets[o+1])} coefficient_values[k]
 *           * prod_c input[b, c]^monomial_counts[coefficient_terms[k], c]:
 * outputs as sparse combinations of monomial_count unique monomials.
 * Replaces ye3t_runtime::symmetric_power_shared_monomial (schema
 * execution_plan_torch.cpp:7540-7544; CPU ye3t_runtime_core.cpp:5392-5440). */
int ye3t_hip_symmetric_power_shared_monomial(int dtype, const void* input, int64_t batch, int64_t input_dim,
                                             const int64_t* monomial_counts, int64_t monomial_count,
                                             const int64_t* output_offsets, const int64_t* coefficient_terms,
                                             const void* coefficient_values, int64_t coefficient_count,
                                             int64_t output_dim, void* output, ye3t_stream_t stream);

/* Adjoint of the shared form (ye3t_runtime_core.cpp:5442-5540).  Replaces
 * ye3t_runtime::symmetric_power_shared_monomial_adjoint. */
int ye3t_hip_symmetric_power_shared_monomial_adjoint(int dtype, const void* output_adjoint, const void* input,
                                                     int64_t batch, int64_t input_dim,
                                                     const int64_t* monomial_counts, int64_t monomial_count,
                                                     const int64_t* output_offsets,
                                                     const int64_t* coefficient_terms,
                                                     const void* coefficient_values, int64_t coefficient_count,
                                                     int64_t output_dim, void* input_adjoint, ye3t_stream_t stream);

/* Shared form with sparse monomial supports: monomial t is
 *   prod_{q in [term_offsets[t], term_offsets[t+1])} input[b, term_components[q]]^term_exponents[q]
 * (monomial_count = t range, support_count = q range), and
 * S[b, o] = sum_{k in [output_offsets[o], output_offsets[o+1])} coefficient_values[k] * monomial_{coefficient_terms[k]}.
 * Every table index must be in range and every exponent positive (checked on
 * the host by the Python layer).  dtype YE3T_F32, YE3T_F64, YE3T_C64 or
 * YE3T_C128 (input, coefficients and outputs alike; complex as (re, im)
 * pairs), as the reference dispatches floating and complex types.  Replaces
 * ye3t_runtime::symmetric_power_shared_sparse_monomial (schema
 * execution_plan_torch.cpp:7562-7567; CUDA execution_plan_cuda.cu:11012-11104). */
int ye3t_hip_symmetric_power_shared_sparse_monomial(int dtype, const void* input, int64_t batch, int64_t input_dim,
                                                    const int64_t* term_offsets, const int64_t* term_components,
                                                    const int64_t* term_exponents, int64_t monomial_count,
                                                    int64_t support_count, const int64_t* output_offsets,
                                                    const int64_t* coefficient_terms, const void* coefficient_values,
                                                    int64_t coefficient_count, int64_t output_dim, void* output,
                                                    ye3t_stream_t stream);

/* input_adjoint[b, c] of the sparse shared form: zero factors add their
 * exponents into a zero degree; degree one gives the cofactor, a higher degree
 * nothing (execution_plan_cuda.cu:5757-5813).  For complex data each
 * contribution is g * conj(coefficient) * conj(derivative), the reference's
 * conjugate-transpose rule (:6002-6033).  Replaces
 * ye3t_runtime::symmetric_power_shared_sparse_monomial_adjoint (schema
 * execution_plan_torch.cpp:7568-7573; CUDA :11106-11204). */
int ye3t_hip_symmetric_power_shared_sparse_monomial_adjoint(
    int dtype, const void* output_adjoint, const void* input, int64_t batch, int64_t input_dim,
    const int64_t* term_offsets, const int64_t* term_components, const int64_t* term_exponents,
    int64_t monomial_count, int64_t support_count, const int64_t* output_offsets, const int64_t* coefficient_terms,
    const void* coefficient_values, int64_t coefficient_count, int64_t output_dim, void* input_adjoint,
    ye3t_stream_t stream);

/* Second order of the sparse shared form along input_adjoint_tangent v:
 * output_tangent[b, o] = d S[b, o] . v, input_tangent[b, c] = sum over
 * coefficients of output_adjoint[b, o] value_k (Hessian of the monomial) v
 * (execution_plan_cuda.cu:5815-5955); for complex data
 * output_adjoint * conj(value_k) * conj(Hessian . v).  Replaces
 * ye3t_runtime::symmetric_power_shared_sparse_monomial_double_backward (schema
 * execution_plan_torch.cpp:7574-7580; CUDA :11206-11330). */
int ye3t_hip_symmetric_power_shared_sparse_monomial_double_backward(
    int dtype, const void* input_adjoint_tangent, const void* output_adjoint, const void* input, int64_t batch,
    int64_t input_dim, const int64_t* term_offsets, const int64_t* term_components, const int64_t* term_exponents,
    int64_t monomial_count, int64_t support_count, const int64_t* output_offsets, const int64_t* coefficient_terms,
    const void* coefficient_values, int64_t coefficient_count, int64_t output_dim, void* output_tangent,
    void* input_tangent, ye3t_stream_t stream);

/* out[b, k] = sum_{t in k} coeffs[t] prod_blk block_values[b, label_k, blk, block_m_indices[t, blk]].
 * Device counterpart of evaluate_factorized_schedule_cpu
 * (ye3t/core/csrc/factorized_runtime.cpp:426-548; evaluator core :251-285). */
int ye3t_hip_evaluate_factorized_schedule(int dtype, const void* block_values, int64_t batch,
                                          int64_t basis_count, int64_t block_count, int64_t magnetic_dim,
                                          const int64_t* component_offsets,
                                          const int64_t* component_label_index,
                                          const int64_t* block_m_indices, const void* coeffs,
                                          int64_t component_count, void* out, ye3t_stream_t stream);

/* ---- Fused stage 2: compiled product plan (DAG of shared CG couplings) ---- */

/* Host-side description of a compiled product plan (see ye3t_amd/ace/program.py).
 * The plan is split into `chunk_count` programs; each produces a contiguous
 * range of output columns from a [samples, a_width] density. */
typedef struct {
  int dtype;
  int64_t a_width;              /* values per density row */
  int64_t feature_count;        /* output columns */
  int64_t chunk_count;
  int64_t workspace_slots;      /* max slots of any chunk (LDS per wave = slots*65*elem) */
  const int64_t* chunk_word_offsets;   /* host [chunk_count+1] into words */
  const int64_t* chunk_coeff_offsets;  /* host [chunk_count+1] into coeffs */
  const int64_t* chunk_out_offsets;    /* host [chunk_count+1] into out_slots */
  const int64_t* chunk_first_column;   /* host [chunk_count] */
  const uint32_t* words;        /* host program words */
  int64_t word_count;
  const void* coeffs;           /* host coefficients (dtype) */
  int64_t coeff_count;
  const uint16_t* out_slots;    /* host workspace slot of each output column, chunk-major */
  int64_t out_slot_count;
  int out_dtype;                /* dtype of B; -1 = dtype.  A and the arithmetic use dtype, so an
                                   fp64 plan may write fp32 features (rounded once, at the store) */
  int in_dtype;                 /* dtype of the density A; -1 = dtype.  YE3T_F32 with an fp64 plan
                                   reads fp32 density rows into fp64 arithmetic; such plans run
                                   their attached generated kernels only (forward, readout,
                                   adjoint with an fp32 gA); the interpreters return
                                   YE3T_EUNSUPPORTED for them */
} ye3t_product_plan_desc;

typedef struct ye3t_hip_product_plan ye3t_hip_product_plan;

/* Copies the tables to the current device (synchronous). Counterpart of the
 * reference's plan buffers (execution_plan.py:12918-13151). */
int ye3t_hip_product_plan_create(const ye3t_product_plan_desc* desc, ye3t_hip_product_plan** out);
void ye3t_hip_product_plan_destroy(ye3t_hip_product_plan* plan);

/* B[samples, feature_count] (out_dtype) from A[samples, a_width] (dtype) for a
 * plan compiled by this backend (program words of ye3t_amd.ace.program).  It is
 * the ACE-product form of the reference's factorized-angular forward
 * (execution_plan_cuda.cu:6228-6358, launcher :11488-11672): one DAG for every
 * content and target L of a configuration.  Callers holding the reference op's
 * own DAG tables use ye3t_hip_factorized_angular_forward below. */
int ye3t_hip_product_forward(const ye3t_hip_product_plan* plan, const void* A, int64_t samples, void* B,
                             ye3t_stream_t stream);

/* Compile HIP source for the current device's architecture with hipRTC.
 * On success *code is a malloc'ed code object of *size bytes (free with
 * ye3t_hip_free).  Used for plan-specialised kernels; no reference counterpart
 * (the reference JIT-compiles its whole extension, execution_plan.py:253-292). */
int ye3t_hip_rtc_compile(const char* source, const char* name, const char* arch, void** code, int64_t* size);
void ye3t_hip_free(void* ptr);

/* What besides the source and the architecture decides ye3t_hip_rtc_compile's
 * output, as text: the hipRTC version, its options and this ABI version
 * ("hiprtc 7.2 | options -O3 ... | abi 61"), NUL-terminated into buf
 * (capacity bytes).  Callers caching code objects on disk key them by it.
 * No reference counterpart (the reference caches its whole extension build by
 * source and flags, execution_plan.py:253-292). */
int ye3t_hip_rtc_fingerprint(char* buf, int64_t capacity);

/* Facts of kernel `kernel_name` read from a gfx950 code object on the host
 * (its AMDHSA kernel descriptor): private (scratch) segment bytes per lane, LDS
 * bytes, and whether it uses a dynamic stack.  No GPU needed.  The
 * attach_*_parts entry points refuse a part whose private segment exceeds
 * ye3t_hip_part_private_limit() bytes per lane (1024; YE3T_PART_PRIVATE_MAX may
 * lower it), whose scratch over four part streams and every wave slot of the
 * device would exceed 2 GiB, or that uses a dynamic stack.  No reference
 * counterpart (the reference has no generated kernels). */
int ye3t_hip_code_object_kernel_info(const void* code, int64_t size, const char* kernel_name,
                                     int64_t* private_segment_bytes, int64_t* group_segment_bytes,
                                     int* uses_dynamic_stack);
int64_t ye3t_hip_part_private_limit(void);

/* Attach a plan-specialised kernel (code object from ye3t_hip_rtc_compile of
 * ye3t_amd/ace/codegen.py output) to `plan`; product_forward then launches it
 * with 64 threads per workgroup and grid (ceil(samples / rows_per_tile),
 * chunk_count), rows_per_tile in [1, 64] being the samples one workgroup
 * produces.  `persistent` != 0: a one-chunk kernel whose workgroups loop over
 * 64-row tiles; it is launched with at most as many workgroups as the device
 * holds at once and needs a 16-byte aligned B (else the generic kernel runs).
 * `threads_per_block` (a multiple of 64) is the workgroup size the kernel was
 * generated for.  The kernel signature is (const T* A, long samples, U* B),
 * T = the plan's dtype, U = its out_dtype. */
int ye3t_hip_product_plan_attach_generated(ye3t_hip_product_plan* plan, const void* code, int64_t size,
                                           const char* kernel_name, int64_t chunk_count, int64_t rows_per_tile,
                                           int persistent, int threads_per_block);

/* Attach a plan-specialised kernel in `part_count` parts, for plans whose
 * generated code is too large to compile as one kernel: part i is the code
 * object codes[i] (sizes[i] bytes, from ye3t_hip_rtc_compile of
 * ye3t_amd/ace/codegen.py:generate_parts output) with kernel kernel_names[i],
 * which computes chunk_counts[i] consecutive output chunks of the plan.
 * product_forward and product_forward_columns then launch the parts in order
 * on their stream, each with 64 threads per workgroup and grid (ceil(samples
 * / 64) rounded up to a multiple of 8, chunk_counts[i]) -- the kernel maps its
 * linear workgroup id to (tile, chunk) so that each XCD takes one eighth of the
 * tiles, and workgroups past the last tile return at once; the signature is
 * (const T* A, long samples, U* B, long row_stride, long col_stride), density
 * value (s, k) at A[s * row_stride + k * col_stride]: (a_width, 1) for the
 * row-major density, (1, ld) for its column-major copy.  Replaces earlier
 * parts; a kernel attached with ye3t_hip_product_plan_attach_generated takes
 * precedence in product_forward.  No
 * reference counterpart (the reference runs such plans on its generic DAG
 * executor, execution_plan_cuda.cu:11584-11589). */
int ye3t_hip_product_plan_attach_generated_parts(ye3t_hip_product_plan* plan, int64_t part_count,
                                                 const void* const* codes, const int64_t* sizes,
                                                 const char* const* kernel_names, const int64_t* chunk_counts);

/* Reverse mode of a plan in parts (code objects of
 * ye3t_amd/ace/codegen.py:generate_adjoint_parts, kernel signature
 * (const T* A, const G* gB, long samples, R* P, long row_stride,
 * long col_stride, long ldp), R = the plan's dtype, T = its density type, G =
 * its out_dtype).  Each part writes partial density gradients of its chunks as
 * rows of P [partial_rows, ldp]; column k of gA then sums P rows
 * row_ids[col_off[k] .. col_off[k + 1]) in that order (host arrays, copied to
 * the device; col_off has a_width + 1 entries).  No reference counterpart:
 * the plan-specialised form of the reference's factorized_angular_adjoint
 * (execution_plan_cuda.cu:6361) for the plans of
 * ye3t_hip_product_plan_attach_generated_parts. */
int ye3t_hip_product_plan_attach_adjoint_parts(ye3t_hip_product_plan* plan, int64_t part_count,
                                               const void* const* codes, const int64_t* sizes,
                                               const char* const* kernel_names, const int64_t* chunk_counts,
                                               int64_t partial_rows, const int64_t* col_off, const int64_t* row_ids);

/* Bytes of the partial buffer ye3t_hip_product_adjoint_parts needs for
 * `samples` (partial_rows x samples rounded up to 64 x the plan's element
 * size); 0 without adjoint parts, -1 on error. */
int64_t ye3t_hip_product_adjoint_parts_workspace_bytes(const ye3t_hip_product_plan* plan, int64_t samples);

/* gA[s] = J(A[s])^T gB[s] on the attached adjoint parts: A row-major
 * [samples, a_width] (lda == a_width) or, with `columns`, column-major
 * [a_width, lda] (lda >= samples); gB [samples, feature_count] of the plan's
 * out_dtype; gA row-major in the density's type.  The parts run on the plan's
 * streams (as the forward parts do), then one fixed-order reduction on
 * `stream`; results do not depend on the launch schedule.  Replaces the same
 * reference op as ye3t_hip_product_adjoint. */
int ye3t_hip_product_adjoint_parts(const ye3t_hip_product_plan* plan, const void* A, int64_t lda, int columns,
                                   const void* gB, int64_t samples, void* workspace, int64_t workspace_bytes,
                                   void* gA, ye3t_stream_t stream);

/* Fused linear readout of a plan in parts (code objects of
 * ye3t_amd/ace/codegen.py:generate_readout_parts, kernel signature
 * (const T* A, long samples, R* P, const R* W, long row_stride,
 * long col_stride, long ldp)): part i writes, for each of its chunk_counts[i]
 * chunks, the chunk's partial dot product sum_{k in chunk} W[k] B[s, k] as one
 * row of P.  No reference counterpart: the plan-specialised form of the
 * reference's factorized_angular_linear (execution_plan.py:13793-13850) for
 * the plans of ye3t_hip_product_plan_attach_generated_parts. */
int ye3t_hip_product_plan_attach_readout_parts(ye3t_hip_product_plan* plan, int64_t part_count,
                                               const void* const* codes, const int64_t* sizes,
                                               const char* const* kernel_names, const int64_t* chunk_counts);

/* Bytes of the partial buffer ye3t_hip_product_linear_forward_parts needs
 * (chunks x samples rounded up to 64 x the plan's element size); 0 without
 * readout parts, -1 on error. */
int64_t ye3t_hip_product_linear_parts_workspace_bytes(const ye3t_hip_product_plan* plan, int64_t samples);

/* out[s] = bias + sum_k B[s, k] weight[k] on the attached readout parts,
 * without materialising B: A row-major [samples, a_width] (lda == a_width) or,
 * with `columns`, column-major [a_width, lda] (lda >= samples); weight
 * [feature_count] of the plan's dtype; out of its out_dtype.  The parts run on
 * the plan's streams, then one reduction adds the bias and the chunks' rows in
 * chunk order.  Replaces the same reference op as
 * ye3t_hip_product_linear_forward. */
int ye3t_hip_product_linear_forward_parts(const ye3t_hip_product_plan* plan, const void* A, int64_t lda, int columns,
                                          int64_t samples, const void* weight, double bias, void* workspace,
                                          int64_t workspace_bytes, void* out, ye3t_stream_t stream);

/* Attach a plan-specialised fused linear readout kernel (code object of
 * ye3t_amd/ace/codegen.py:generate_readout compiled with ye3t_hip_rtc_compile).
 * Kernel signature (const T* A, long samples, U* out, const T* W, T bias), T =
 * the plan's dtype, U = its out_dtype; launched persistent with at most as many
 * workgroups of `threads_per_block` threads as the device holds at once. */
int ye3t_hip_product_plan_attach_readout(ye3t_hip_product_plan* plan, const void* code, int64_t size,
                                         const char* kernel_name, int threads_per_block);

/* out[s] = bias + sum_k B[s, k] weight[k] without materialising B (B = the
 * plan's features of A[s]); out has the plan's out_dtype, weight [feature_count]
 * the plan's dtype.  YE3T_EUNSUPPORTED when no readout kernel is attached (the
 * caller then materialises B and uses ye3t_hip_rows_dot).  Replaces
 * ye3t_runtime::factorized_angular_linear (schema execution_plan_torch.cpp:7713,
 * CUDA execution_plan_cuda.cu:8957; readout semantics execution_plan.py:13832-13850). */
int ye3t_hip_product_linear_forward(const ye3t_hip_product_plan* plan, const void* A, int64_t samples,
                                    const void* weight, double bias, void* out, ye3t_stream_t stream);

/* Attach a plan-specialised adjoint kernel (ye3t_amd/ace/codegen.py:
 * generate_adjoint compiled with ye3t_hip_rtc_compile), signature
 * (const T* A, const G* gB, long samples, T* gA), T = the plan's dtype, G = that
 * of the feature gradients (the plan's out_dtype). */
int ye3t_hip_product_plan_attach_adjoint(ye3t_hip_product_plan* plan, const void* code, int64_t size,
                                         const char* kernel_name, int threads_per_block);

/* gA[s] = J(A[s])^T gB[s]: the density gradient of a feature gradient gB
 * [samples, feature_count] (16-byte aligned) through the plan's product
 * (forward values recomputed).  YE3T_EUNSUPPORTED when no adjoint kernel is attached.
 * Replaces ye3t_runtime::factorized_angular_adjoint (execution_plan_cuda.cu:6361,
 * CPU core ye3t_runtime_core.h:1431-1456) for ACE plans. */
int ye3t_hip_product_adjoint(const ye3t_hip_product_plan* plan, const void* A, const void* gB, int64_t samples,
                             void* gA, ye3t_stream_t stream);

/* out[s] = bias + sum_k B[s, k] weight[k] for a materialised B[samples, F]
 * (fp64 accumulation, fixed reduction order).  The reference's materialised
 * readout `features @ weight + bias` (execution_plan.py:13838-13845). */
int ye3t_hip_rows_dot(int dtype, const void* B, int64_t samples, int64_t F, const void* weight, double bias,
                      void* out, ye3t_stream_t stream);

/* Cell grid of the neighbour-list builder: dims[a] cells of edge cell_edge per
 * axis from origin (1 <= dims[a] <= 2^24, fewer than 2^31 - 1 cells in all).
 * Atoms outside the grid are clamped into its border cells, which is correct
 * for any grid and fast when the grid covers the atoms. */
typedef struct {
  double origin[3];
  double cell_edge; /* >= cutoff * (1 + 1e-9) */
  int64_t dims[3];
} ye3t_cell_grid;

/* Device workspace bytes of a neighbour-list build (-1 on invalid input). */
int64_t ye3t_hip_neighbor_workspace_bytes(int64_t atom_count, const ye3t_cell_grid* grid);

/* Neighbour list, pass 1 of 2.  Bins positions[atom_count, 3] into the grid
 * (kept in the workspace) and writes row_offsets[atom_count + 1]: row i holds
 * the j != i with |r_j - r_i| < cutoff, decided in fp64 with each operation
 * rounded on its own; the edge count is row_offsets[atom_count].  Open
 * boundaries.  No neighbour builder exists in the reference: this produces the
 * CSR that its density inputs take (centers, execution_plan.py:7913-7984;
 * ye3t_runtime_core.h:294-301) in the order prepare_carrier_scatter_segments
 * gives edges keyed (target, source) (execution_plan.py:9316-9434). */
int ye3t_hip_neighbor_count(int dtype, const void* positions, int64_t atom_count, const ye3t_cell_grid* grid,
                            double cutoff, void* workspace, int64_t workspace_bytes, int64_t* row_offsets,
                            ye3t_stream_t stream);

/* Neighbour list, pass 2 of 2, with the dtype, grid, cutoff, workspace and
 * row_offsets of pass 1 (the workspace holds the positions in cell order):
 * edge e in [row_offsets[i], row_offsets[i + 1]) gets centers[e] = i,
 * neighbors[e] = j ascending within the row, edge_vectors[e] = r_j - r_i
 * (computed in dtype).  Edges at or beyond edge_capacity are not written; a
 * row cut by it holds its smallest neighbours. */
int ye3t_hip_neighbor_fill(int dtype, int64_t atom_count, const ye3t_cell_grid* grid, double cutoff,
                           const void* workspace, int64_t workspace_bytes, const int64_t* row_offsets,
                           int64_t edge_capacity, int64_t* centers, int64_t* neighbors, void* edge_vectors,
                           ye3t_stream_t stream);

/* At[c * ld + r] = A[r * cols + c] for r < rows, c < cols, and At[c * ld + r]
 * = 0 for rows <= r < ld: the column-major density of
 * ye3t_hip_product_forward_columns.  No reference counterpart (a layout step
 * of this backend). */
int ye3t_hip_transpose(int dtype, const void* A, int64_t rows, int64_t cols, void* At, int64_t ld,
                       ye3t_stream_t stream);

/* ye3t_hip_product_forward on a column-major density At [a_width, ld]
 * (element (s, col) at At[col * ld + s]; ld >= samples rounded up to 64):
 * the interpreter reads each density column of 64 samples as one contiguous
 * block.  For plans with generated parts attached, or run by the term-stream
 * interpreter (workspace byte offsets within 16 bits); YE3T_EINVAL otherwise.
 * Same results as
 * ye3t_hip_product_forward on the row-major density.  Replaces the same
 * reference ops as ye3t_hip_product_forward. */
int ye3t_hip_product_forward_columns(const ye3t_hip_product_plan* plan, const void* At, int64_t ld,
                                     int64_t samples, void* B, ye3t_stream_t stream);

/* Select which kernel product_forward launches: 0 = generated (if attached,
 * whole or in parts), 1 = generic interpreter. */
int ye3t_hip_product_plan_select(ye3t_hip_product_plan* plan, int use_interpreter);

/* Host only (no device work): the term stream a plan description would run.
 * counts[3] = (records, loads, chunks), all 0 when the plan gets no term
 * stream.  Called with NULL arrays first to size them, then with
 * recs[4 * records] (factor a LDS byte offset, factor b, coefficient words),
 * flags[records] (flags | destination byte offset << 16; flags 1 = flush,
 * 2 = chain, 4 = chained), rec_off[chunks + 1], loads[2 * loads] (LDS byte
 * offset, density column), load_off[chunks + 1] and layout[8] (workspace
 * bytes, record, flag, load and output-slot offsets, byte offset of the slot
 * holding 1, LDS bytes, records per group).  For inspection and tests; no
 * reference counterpart. */
int ye3t_hip_product_stream_encode(const ye3t_product_plan_desc* desc, int64_t* counts, uint32_t* recs,
                                   uint32_t* flags, int64_t* rec_off, uint32_t* loads, int64_t* load_off,
                                   int64_t* layout);

/* ---- General factorized-angular DAG (the reference's factorized_angular op) ---- */

/* Host tables of one factorized-angular DAG, exactly the arguments of the
 * reference op factorized_angular(packed_slots, node_offsets, node_dimensions,
 * node_leaf_offsets, node_left, node_right, node_coefficient_offsets,
 * coefficient_rows, coefficient_columns, coefficient_values, root_nodes,
 * projection_values, source_dimension, workspace_dimension, output_dimension)
 * (schema execution_plan_torch.cpp:7586-7594), with the counts of its vectors.
 * Nodes are in topological order; a leaf node copies node_dimensions values
 * of the input slot from node_leaf_offsets; a merge node accumulates
 * out[column] += conj(value) * left[row / dim(right)] * right[row % dim(right)]
 * over its coefficient range; every root is projected onto all P =
 * projection_count / source_dimension projection columns (the reference's
 * uniform root metadata, execution_plan_torch.cpp:205-250). */
typedef struct {
  int dtype;                               /* YE3T_F32, YE3T_F64, YE3T_C64 or YE3T_C128 */
  int64_t node_count;
  const int64_t* node_offsets;             /* host [node_count] */
  const int64_t* node_dimensions;          /* host [node_count] */
  const int64_t* node_leaf_offsets;        /* host [node_count], -1 for merge nodes */
  const int64_t* node_left;                /* host [node_count] */
  const int64_t* node_right;               /* host [node_count] */
  const int64_t* node_coefficient_offsets; /* host [node_count + 1] */
  int64_t coefficient_count;
  const int64_t* coefficient_rows;         /* host [coefficient_count] */
  const int64_t* coefficient_columns;      /* host [coefficient_count] */
  const void* coefficient_values;          /* host [coefficient_count] of dtype */
  int64_t root_count;
  const int64_t* root_nodes;               /* host [root_count] */
  int64_t projection_count;
  const void* projection_values;           /* host [source_dimension * P] of dtype */
  int64_t source_dimension;
  int64_t input_dimension;                 /* values per source slot (packed width / source_dimension) */
  int64_t workspace_dimension;             /* node_offsets[-1] + node_dimensions[-1] */
  int64_t output_dimension;                /* root_count * P * dim(root) */
} ye3t_factorized_angular_desc;

typedef struct ye3t_hip_factorized_angular_plan ye3t_hip_factorized_angular_plan;

/* Validates the tables on the host (the reference op's TORCH_CHECKs, plus every
 * index the kernels use) and copies them to the current device (synchronous).
 * Counterpart of the reference module's plan buffers (execution_plan.py:12918-13151). */
int ye3t_hip_factorized_angular_plan_create(const ye3t_factorized_angular_desc* desc,
                                            ye3t_hip_factorized_angular_plan** out);
void ye3t_hip_factorized_angular_plan_destroy(ye3t_hip_factorized_angular_plan* plan);

/* info[7] = (dtype, source_dimension, input_dimension, workspace_dimension,
 * output_dimension, projection columns P, root dimension). */
int ye3t_hip_factorized_angular_plan_info(const ye3t_hip_factorized_angular_plan* plan, int64_t* info);

/* output[batch, output_dimension] from packed_slots[batch, source_dimension *
 * input_dimension].  Replaces the CUDA branch of ye3t_runtime::factorized_angular
 * (kernel execution_plan_cuda.cu:6228-6358, launcher :11488-11672; CPU core
 * ye3t_runtime_core.cpp:5667-5769).  The per-sample workspace lives in LDS;
 * YE3T_EUNSUPPORTED when one sample's workspace exceeds 64 KB. */
int ye3t_hip_factorized_angular_forward(const ye3t_hip_factorized_angular_plan* plan, const void* packed_slots,
                                        int64_t batch, void* output, ye3t_stream_t stream);

/* packed_slots_adjoint[batch, S * input_dimension]: the conjugate-transpose
 * (analysis) adjoint of an output adjoint, forward values recomputed.
 * Replaces ye3t_runtime::factorized_angular_adjoint (execution_plan_cuda.cu:6361;
 * CPU core ye3t_runtime_core.cpp:6481-6643). */
int ye3t_hip_factorized_angular_adjoint(const ye3t_hip_factorized_angular_plan* plan, const void* output_adjoint,
                                        const void* packed_slots, int64_t batch, void* packed_slots_adjoint,
                                        ye3t_stream_t stream);

/* output[b] = bias + sum_k features[b, k] weight[k] without storing the
 * features (weight [output_dimension] on the device, bias one host value of
 * dtype).  Replaces ye3t_runtime::factorized_angular_linear (execution_plan_cuda.cu:8957;
 * CPU core ye3t_runtime_core.cpp:7144-7234). */
int ye3t_hip_factorized_angular_linear_forward(const ye3t_hip_factorized_angular_plan* plan, const void* packed_slots,
                                               int64_t batch, const void* weight, const void* bias, void* output,
                                               ye3t_stream_t stream);

/* Adjoint of the linear readout for output_adjoint[batch]: packed_slots_adjoint,
 * weight_adjoint[output_dimension] = sum_b g[b] conj(features[b]) and
 * bias_adjoint = sum_b g[b] (device, summed over the batch in order).
 * `features` is a caller-provided [batch, output_dimension] device buffer the
 * call fills with the forward features.  Replaces
 * ye3t_runtime::factorized_angular_linear_adjoint (CPU core
 * ye3t_runtime_core.cpp:7237-7399). */
int ye3t_hip_factorized_angular_linear_adjoint(const ye3t_hip_factorized_angular_plan* plan,
                                               const void* output_adjoint, const void* packed_slots, int64_t batch,
                                               const void* weight, void* features, void* packed_slots_adjoint,
                                               void* weight_adjoint, void* bias_adjoint, ye3t_stream_t stream);

/* ---- Segmented factorized-angular DAGs (several plans in one launch) ---- */

/* Host tables of the reference op factorized_angular_segmented(packed_slots,
 * segment_source_offsets, segment_input_offsets, segment_input_dimensions,
 * segment_workspace_offsets, segment_workspace_dimensions, segment_node_offsets,
 * segment_root_offsets, segment_projection_offsets, segment_projection_dimensions,
 * segment_output_offsets, node_offsets, node_dimensions, node_leaf_offsets,
 * node_left, node_right, node_coefficient_offsets, coefficient_rows,
 * coefficient_columns, coefficient_values, root_nodes, root_projection_starts,
 * root_projection_dimensions, root_output_offsets, projection_values,
 * total_source_count, workspace_dimension, output_dimension)
 * (schema execution_plan_torch.cpp:7666-7679), with the counts of its vectors
 * and packed_input_dimension = packed_slots.size(1).  Segment k is one DAG over
 * packed columns [segment_input_offsets[k], + S_k * segment_input_dimensions[k])
 * and output columns [segment_output_offsets[k], segment_output_offsets[k + 1]);
 * its node and root indices are local to its slices, node_coefficient_offsets
 * index the concatenated coefficients, and root r projects onto columns
 * [root_projection_starts[r], + root_projection_dimensions[r]) of the segment's
 * [S_k x segment_projection_dimensions[k]] projection block into output block
 * root_output_offsets[r] of the segment. */
typedef struct {
  int dtype; /* YE3T_F32, YE3T_F64, YE3T_C64 or YE3T_C128 */
  int64_t segment_count;
  const int64_t* segment_source_offsets;        /* [segment_count + 1] */
  const int64_t* segment_input_offsets;         /* [segment_count] */
  const int64_t* segment_input_dimensions;      /* [segment_count] */
  const int64_t* segment_workspace_offsets;     /* [segment_count] */
  const int64_t* segment_workspace_dimensions;  /* [segment_count] */
  const int64_t* segment_node_offsets;          /* [segment_count + 1] */
  const int64_t* segment_root_offsets;          /* [segment_count + 1] */
  const int64_t* segment_projection_offsets;    /* [segment_count] */
  const int64_t* segment_projection_dimensions; /* [segment_count] */
  const int64_t* segment_output_offsets;        /* [segment_count + 1] */
  int64_t node_count;
  const int64_t* node_offsets;
  const int64_t* node_dimensions;
  const int64_t* node_leaf_offsets;
  const int64_t* node_left;
  const int64_t* node_right;
  const int64_t* node_coefficient_offsets; /* [node_count + 1] */
  int64_t coefficient_count;
  const int64_t* coefficient_rows;
  const int64_t* coefficient_columns;
  const void* coefficient_values; /* [coefficient_count] of dtype */
  int64_t root_count;
  const int64_t* root_nodes;
  const int64_t* root_projection_starts;
  const int64_t* root_projection_dimensions;
  const int64_t* root_output_offsets;
  int64_t projection_count;
  const void* projection_values; /* [projection_count] of dtype */
  int64_t packed_input_dimension;
  int64_t total_source_count;
  int64_t workspace_dimension;
  int64_t output_dimension;
} ye3t_factorized_angular_segmented_desc;

typedef struct ye3t_hip_factorized_angular_segmented_plan ye3t_hip_factorized_angular_segmented_plan;

/* Validates the tables on the host (the reference op's checks,
 * execution_plan_torch.cpp:434-726, plus every index the kernels use) and
 * copies them to the current device (synchronous).  Counterpart of the
 * reference's segmented group buffers (execution_plan.py:16632-16890). */
int ye3t_hip_factorized_angular_segmented_plan_create(const ye3t_factorized_angular_segmented_desc* desc,
                                                      ye3t_hip_factorized_angular_segmented_plan** out);
void ye3t_hip_factorized_angular_segmented_plan_destroy(ye3t_hip_factorized_angular_segmented_plan* plan);

/* info[6] = (dtype, segment_count, total_source_count, packed_input_dimension,
 * workspace_dimension, output_dimension). */
int ye3t_hip_factorized_angular_segmented_plan_info(const ye3t_hip_factorized_angular_segmented_plan* plan,
                                                    int64_t* info);

/* output[batch, output_dimension] from packed_slots[batch, packed_input_dimension],
 * every segment in one launch (blocks of 64 samples by segment).  Replaces the
 * CUDA branch of ye3t_runtime::factorized_angular_segmented
 * (execution_plan_cuda.cu:13099; CPU core ye3t_runtime_core.cpp:6977-7021). */
int ye3t_hip_factorized_angular_segmented_forward(const ye3t_hip_factorized_angular_segmented_plan* plan,
                                                  const void* packed_slots, int64_t batch, void* output,
                                                  ye3t_stream_t stream);

/* packed_slots_adjoint[batch, packed_input_dimension] of an output adjoint
 * (conjugate-transpose convention, forward values recomputed).  Replaces
 * ye3t_runtime::factorized_angular_segmented_adjoint (schema
 * execution_plan_torch.cpp:7681-7695; CPU core ye3t_runtime_core.cpp:7023-7070). */
int ye3t_hip_factorized_angular_segmented_adjoint(const ye3t_hip_factorized_angular_segmented_plan* plan,
                                                  const void* output_adjoint, const void* packed_slots, int64_t batch,
                                                  void* packed_slots_adjoint, ye3t_stream_t stream);

/* Device workspace bytes of ye3t_hip_product_adjoint_stream for `samples`
 * samples (0 for plans without a term stream; -1 on invalid input). */
int64_t ye3t_hip_product_adjoint_workspace_bytes(const ye3t_hip_product_plan* plan, int64_t samples);

/* gA[s] = J(A[s])^T gB[s] (row-major gA [samples, a_width]) for plans run by
 * the term-stream interpreter: the product's reverse mode with forward values
 * recomputed, deterministic (per-group partial sums added in a fixed order,
 * no atomics).  A is row-major (columns = 0, lda = a_width) or column-major
 * (columns = 1, lda >= samples rounded up to 64); gB [samples, feature_count]
 * in the plan's output dtype.  The workspace (ye3t_hip_product_adjoint_
 * workspace_bytes) is cleared by the call.  Replaces
 * ye3t_runtime::factorized_angular_adjoint (execution_plan_cuda.cu:6361, CPU
 * core ye3t_runtime_core.h:1431-1456) for ACE plans too large for generated
 * code. */
int ye3t_hip_product_adjoint_stream(const ye3t_hip_product_plan* plan, const void* A, int64_t lda, int columns,
                                    const void* gB, int64_t samples, void* workspace, int64_t workspace_bytes,
                                    void* gA, ye3t_stream_t stream);

/* ye3t_hip_product_adjoint_stream without a workspace argument and without
 * any allocation: the per-group partial gradients live in a static device
 * array of 64 MiB (one per device the library runs on, held until the process
 * ends), cleared by the call with a fill kernel.  Its address and an ordering
 * event are looked up when a term-stream plan is created, so the call itself
 * makes no set-up call.  Fewer groups than the workspace form may be used, so
 * sums are grouped differently (same values to rounding).  YE3T_EUNSUPPORTED
 * when one group's partials exceed 64 MiB (a_width * samples rounded up to 64
 * * element size).  Calls on one device are serialised: host threads take a
 * lock, and an eager call on another stream than the previous call's waits on
 * the GPU (hipStreamWaitEvent) for the previous call's kernels.  Under stream
 * capture the call records its kernels only; a graph holding it must not run
 * concurrently with other users of the scratch on that device.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under stream capture, tight serving loops, allocation-free
 * harnesses). */
int ye3t_hip_product_adjoint_stream_noalloc(const ye3t_hip_product_plan* plan, const void* A, int64_t lda,
                                            int columns, const void* gB, int64_t samples, void* gA,
                                            ye3t_stream_t stream);

/* 1 if the plan's interpreter is the term stream (workspace in LDS, records
 * and flags read through the scalar cache, column loads and output slots
 * staged in LDS; the plan also accepts ye3t_hip_product_forward_columns), 0 for
 * the program-word interpreter (workspaces too wide for the stream's 16-bit
 * offsets or 64 KB of LDS).  No reference counterpart. */
int ye3t_hip_product_plan_uses_stream(const ye3t_hip_product_plan* plan);

/* Kernel name/launch geometry of the last product_forward (for profiling). */
int ye3t_hip_product_launch_info(const ye3t_hip_product_plan* plan, int64_t samples, int64_t* grid,
                                 int64_t* block, int64_t* lds_bytes);

#ifdef __cplusplus
}
#endif

#endif /* YE3T_HIP_H */
