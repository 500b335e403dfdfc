/*
 * CPU ORACLE -- test infrastructure only (see ye3t_oracle.c).
 *
 * Plain-C restatement of the reference's factorized-angular DAG executor and
 * of its symmetric-power monomial adjoint / shared-monomial operators:
 *   ye3t/runtime/csrc/ye3t_runtime_core.cpp
 *     factorized_angular_forward         :5667-5769
 *     factorized_angular_adjoint         :6481-6643
 *     factorized_angular_linear_forward  :7144-7234
 *     factorized_angular_linear_adjoint  :7237-7399
 *     symmetric_power_monomial_adjoint   :5318-5389
 *     symmetric_power_shared_monomial_forward / _adjoint :5392-5540
 * with the uniform root metadata the Torch op derives
 * (execution_plan_torch.cpp:205-250: every root projects onto all P
 * projection columns, root r's block starts at r * P * root_dim).
 *
 * Each operator exists for real (double) and complex (double complex) data;
 * the loops are the reference's, in its order, so sums round alike.
 */
#include <complex.h>
#include <stdint.h>
#include <string.h>

static inline double conj_r(double x) { return x; }
static inline double complex conj_c(double complex x) { return conj(x); }

static double ipow_r(double b, int64_t e) {
  double v = 1.0;
  while (e > 0) {
    if (e & 1) v *= b;
    e >>= 1;
    if (e > 0) b *= b;
  }
  return v;
}

/* ---- factorized angular DAG ------------------------------------------------ */

#define FA_FORWARD(NAME, T, CONJ)                                                                            \
  void NAME(const T* packed, int64_t batch, int64_t input_dim, int64_t source_dim, const int64_t* node_offsets, \
            const int64_t* node_dims, const int64_t* node_leaf, const int64_t* node_left,                     \
            const int64_t* node_right, const int64_t* node_coef_off, int64_t node_count, const int64_t* rows,  \
            const int64_t* cols, const T* coef, const int64_t* roots, int64_t root_count, const T* proj,        \
            int64_t proj_dim, int64_t out_dim, T* ws, T* out) {                                                \
    const int64_t W = node_offsets[node_count - 1] + node_dims[node_count - 1];                              \
    for (int64_t b = 0; b < batch; ++b) {                                                                     \
      T* orow = out + b * out_dim;                                                                            \
      for (int64_t k = 0; k < out_dim; ++k) orow[k] = 0;                                                      \
      for (int64_t s = 0; s < source_dim; ++s) {                                                              \
        for (int64_t q = 0; q < W; ++q) ws[q] = 0;                                                            \
        const T* in = packed + (b * source_dim + s) * input_dim;                                              \
        for (int64_t n = 0; n < node_count; ++n) {                                                            \
          T* o = ws + node_offsets[n];                                                                        \
          if (node_leaf[n] >= 0) {                                                                            \
            for (int64_t i = 0; i < node_dims[n]; ++i) o[i] = in[node_leaf[n] + i];                           \
            continue;                                                                                         \
          }                                                                                                   \
          const T* l = ws + node_offsets[node_left[n]];                                                       \
          const T* r = ws + node_offsets[node_right[n]];                                                      \
          const int64_t rd = node_dims[node_right[n]];                                                        \
          for (int64_t e = node_coef_off[n]; e < node_coef_off[n + 1]; ++e)                                   \
            o[cols[e]] += CONJ(coef[e]) * l[rows[e] / rd] * r[rows[e] % rd];                                  \
        }                                                                                                     \
        for (int64_t ri = 0; ri < root_count; ++ri) {                                                         \
          const int64_t rn = roots[ri], rdim = node_dims[rn];                                                 \
          const T* rv = ws + node_offsets[rn];                                                                \
          for (int64_t p = 0; p < proj_dim; ++p) {                                                            \
            T* blk = orow + ri * proj_dim * rdim + p * rdim;                                                  \
            const T pv = proj[s * proj_dim + p];                                                              \
            for (int64_t m = 0; m < rdim; ++m) blk[m] += rv[m] * pv;                                          \
          }                                                                                                   \
        }                                                                                                     \
      }                                                                                                       \
    }                                                                                                         \
  }

FA_FORWARD(oracle_factorized_angular_f64, double, conj_r)
FA_FORWARD(oracle_factorized_angular_c128, double complex, conj_c)

/* forward replay of one source into ws (the first half of the adjoint and of
 * the linear adjoint) */
#define FA_REPLAY(T, CONJ)                                                                                    \
  for (int64_t q = 0; q < W; ++q) {                                                                           \
    ws[q] = 0;                                                                                                \
    wa[q] = 0;                                                                                                \
  }                                                                                                           \
  for (int64_t n = 0; n < node_count; ++n) {                                                                  \
    T* o = ws + node_offsets[n];                                                                              \
    if (node_leaf[n] >= 0) {                                                                                  \
      for (int64_t i = 0; i < node_dims[n]; ++i) o[i] = in[node_leaf[n] + i];                                 \
      continue;                                                                                               \
    }                                                                                                         \
    const T* l = ws + node_offsets[node_left[n]];                                                             \
    const T* r = ws + node_offsets[node_right[n]];                                                            \
    const int64_t rd = node_dims[node_right[n]];                                                              \
    for (int64_t e = node_coef_off[n]; e < node_coef_off[n + 1]; ++e)                                         \
      o[cols[e]] += CONJ(coef[e]) * l[rows[e] / rd] * r[rows[e] % rd];                                        \
  }

/* reverse sweep of one source from the root adjoints in wa, then the leaf
 * adjoints added into gin */
#define FA_SWEEP(T, CONJ)                                                                                     \
  for (int64_t n = node_count; n-- > 0;) {                                                                    \
    if (node_leaf[n] >= 0) continue;                                                                          \
    const T* g = wa + node_offsets[n];                                                                        \
    const T* l = ws + node_offsets[node_left[n]];                                                             \
    const T* r = ws + node_offsets[node_right[n]];                                                            \
    T* la = wa + node_offsets[node_left[n]];                                                                  \
    T* ra = wa + node_offsets[node_right[n]];                                                                 \
    const int64_t rd = node_dims[node_right[n]];                                                              \
    for (int64_t e = node_coef_off[n]; e < node_coef_off[n + 1]; ++e) {                                       \
      const int64_t li = rows[e] / rd, rj = rows[e] % rd;                                                     \
      const T grad = g[cols[e]];                                                                              \
      la[li] += grad * coef[e] * CONJ(r[rj]);                                                                 \
      ra[rj] += grad * coef[e] * CONJ(l[li]);                                                                 \
    }                                                                                                         \
  }                                                                                                           \
  for (int64_t n = 0; n < node_count; ++n) {                                                                  \
    if (node_leaf[n] < 0) continue;                                                                           \
    const T* a = wa + node_offsets[n];                                                                        \
    for (int64_t i = 0; i < node_dims[n]; ++i) gin[node_leaf[n] + i] += a[i];                                 \
  }

#define FA_ADJOINT(NAME, T, CONJ)                                                                            \
  void NAME(const T* gout, const T* packed, int64_t batch, int64_t input_dim, int64_t source_dim,             \
            const int64_t* node_offsets, const int64_t* node_dims, const int64_t* node_leaf,                  \
            const int64_t* node_left, const int64_t* node_right, const int64_t* node_coef_off,                \
            int64_t node_count, const int64_t* rows, const int64_t* cols, const T* coef, const int64_t* roots, \
            int64_t root_count, const T* proj, int64_t proj_dim, int64_t out_dim, T* ws, T* wa, T* gpacked) { \
    const int64_t W = node_offsets[node_count - 1] + node_dims[node_count - 1];                              \
    for (int64_t b = 0; b < batch; ++b) {                                                                     \
      const T* orow = gout + b * out_dim;                                                                     \
      T* grow = gpacked + b * source_dim * input_dim;                                                         \
      for (int64_t k = 0; k < source_dim * input_dim; ++k) grow[k] = 0;                                       \
      for (int64_t s = 0; s < source_dim; ++s) {                                                              \
        const T* in = packed + (b * source_dim + s) * input_dim;                                              \
        FA_REPLAY(T, CONJ)                                                                                    \
        for (int64_t ri = 0; ri < root_count; ++ri) {                                                         \
          const int64_t rn = roots[ri], rdim = node_dims[rn];                                                 \
          T* ra = wa + node_offsets[rn];                                                                      \
          for (int64_t p = 0; p < proj_dim; ++p) {                                                            \
            const T* blk = orow + ri * proj_dim * rdim + p * rdim;                                            \
            const T pv = proj[s * proj_dim + p];                                                              \
            for (int64_t m = 0; m < rdim; ++m) ra[m] += blk[m] * CONJ(pv);                                    \
          }                                                                                                   \
        }                                                                                                     \
        T* gin = grow + s * input_dim;                                                                        \
        FA_SWEEP(T, CONJ)                                                                                     \
      }                                                                                                       \
    }                                                                                                         \
  }

FA_ADJOINT(oracle_factorized_angular_adjoint_f64, double, conj_r)
FA_ADJOINT(oracle_factorized_angular_adjoint_c128, double complex, conj_c)

#define FA_LINEAR(NAME, T, CONJ)                                                                             \
  void NAME(const T* packed, int64_t batch, int64_t input_dim, int64_t source_dim, const int64_t* node_offsets, \
            const int64_t* node_dims, const int64_t* node_leaf, const int64_t* node_left,                     \
            const int64_t* node_right, const int64_t* node_coef_off, int64_t node_count, const int64_t* rows,  \
            const int64_t* cols, const T* coef, const int64_t* roots, int64_t root_count, const T* proj,        \
            int64_t proj_dim, const T* weight, T bias, T* ws, T* out) {                                       \
    const int64_t W = node_offsets[node_count - 1] + node_dims[node_count - 1];                              \
    const int64_t rdim = node_dims[roots[0]];                                                                 \
    for (int64_t b = 0; b < batch; ++b) {                                                                     \
      T value = bias;                                                                                         \
      for (int64_t s = 0; s < source_dim; ++s) {                                                              \
        for (int64_t q = 0; q < W; ++q) ws[q] = 0;                                                            \
        const T* in = packed + (b * source_dim + s) * input_dim;                                              \
        for (int64_t n = 0; n < node_count; ++n) {                                                            \
          T* o = ws + node_offsets[n];                                                                        \
          if (node_leaf[n] >= 0) {                                                                            \
            for (int64_t i = 0; i < node_dims[n]; ++i) o[i] = in[node_leaf[n] + i];                           \
            continue;                                                                                         \
          }                                                                                                   \
          const T* l = ws + node_offsets[node_left[n]];                                                       \
          const T* r = ws + node_offsets[node_right[n]];                                                      \
          const int64_t rd = node_dims[node_right[n]];                                                        \
          for (int64_t e = node_coef_off[n]; e < node_coef_off[n + 1]; ++e)                                   \
            o[cols[e]] += CONJ(coef[e]) * l[rows[e] / rd] * r[rows[e] % rd];                                  \
        }                                                                                                     \
        for (int64_t ri = 0; ri < root_count; ++ri) {                                                         \
          const T* rv = ws + node_offsets[roots[ri]];                                                         \
          for (int64_t p = 0; p < proj_dim; ++p) {                                                            \
            const T pv = proj[s * proj_dim + p];                                                              \
            const int64_t f0 = (ri * proj_dim + p) * rdim;                                                    \
            for (int64_t m = 0; m < rdim; ++m) value += rv[m] * pv * weight[f0 + m];                          \
          }                                                                                                   \
        }                                                                                                     \
      }                                                                                                       \
      out[b] = value;                                                                                         \
    }                                                                                                         \
  }

FA_LINEAR(oracle_factorized_angular_linear_f64, double, conj_r)
FA_LINEAR(oracle_factorized_angular_linear_c128, double complex, conj_c)

#define FA_LINEAR_ADJOINT(NAME, T, CONJ)                                                                     \
  void NAME(const T* gout, const T* packed, int64_t batch, int64_t input_dim, int64_t source_dim,             \
            const int64_t* node_offsets, const int64_t* node_dims, const int64_t* node_leaf,                  \
            const int64_t* node_left, const int64_t* node_right, const int64_t* node_coef_off,                \
            int64_t node_count, const int64_t* rows, const int64_t* cols, const T* coef, const int64_t* roots, \
            int64_t root_count, const T* proj, int64_t proj_dim, const T* weight, T* ws, T* wa, T* gpacked,   \
            T* gweight, T* gbias) {                                                                           \
    const int64_t W = node_offsets[node_count - 1] + node_dims[node_count - 1];                              \
    const int64_t rdim = node_dims[roots[0]];                                                                 \
    for (int64_t k = 0; k < root_count * proj_dim * rdim; ++k) gweight[k] = 0;                                \
    *gbias = 0;                                                                                               \
    for (int64_t b = 0; b < batch; ++b) {                                                                     \
      const T gr = gout[b];                                                                                   \
      *gbias += gr;                                                                                           \
      T* grow = gpacked + b * source_dim * input_dim;                                                         \
      for (int64_t k = 0; k < source_dim * input_dim; ++k) grow[k] = 0;                                       \
      for (int64_t s = 0; s < source_dim; ++s) {                                                              \
        const T* in = packed + (b * source_dim + s) * input_dim;                                              \
        FA_REPLAY(T, CONJ)                                                                                    \
        for (int64_t ri = 0; ri < root_count; ++ri) {                                                         \
          const T* rv = ws + node_offsets[roots[ri]];                                                         \
          T* ra = wa + node_offsets[roots[ri]];                                                               \
          for (int64_t p = 0; p < proj_dim; ++p) {                                                            \
            const T pv = proj[s * proj_dim + p];                                                              \
            const int64_t f0 = (ri * proj_dim + p) * rdim;                                                    \
            for (int64_t m = 0; m < rdim; ++m) {                                                              \
              gweight[f0 + m] += gr * CONJ(rv[m] * pv);                                                       \
              ra[m] += gr * CONJ(weight[f0 + m]) * CONJ(pv);                                                  \
            }                                                                                                 \
          }                                                                                                   \
        }                                                                                                     \
        T* gin = grow + s * input_dim;                                                                        \
        FA_SWEEP(T, CONJ)                                                                                     \
      }                                                                                                       \
    }                                                                                                         \
  }

FA_LINEAR_ADJOINT(oracle_factorized_angular_linear_adjoint_f64, double, conj_r)
FA_LINEAR_ADJOINT(oracle_factorized_angular_linear_adjoint_c128, double complex, conj_c)

/* ---- segmented DAGs -------------------------------------------------------
 * factorized_angular_segmented_forward / _adjoint (ye3t_runtime_core.cpp:
 * 6977-7100): per sample, per segment, the general single-DAG forward (or
 * adjoint) with explicit root metadata (root r of a segment projects onto
 * projection columns [start, start + dim) of that segment's [S x P] block and
 * writes at segment output offset + root_output_offsets[r]).  Node, root and
 * root-metadata arrays are segment-local slices; node_coefficient_offsets
 * index the concatenated coefficient arrays. */

#define FA_SEG_ARGS(T)                                                                                        \
  int64_t batch, int64_t packed_dim, int64_t seg_count, const int64_t* seg_src_off, const int64_t* seg_in_off,  \
      const int64_t* seg_in_dim, const int64_t* seg_node_off, const int64_t* seg_root_off,                      \
      const int64_t* seg_proj_off, const int64_t* seg_proj_dim, const int64_t* seg_out_off, int64_t out_dim,    \
      const int64_t* all_node_offsets, const int64_t* all_node_dims, const int64_t* all_node_leaf,              \
      const int64_t* all_node_left, const int64_t* all_node_right, const int64_t* all_node_coef_off,            \
      const int64_t* rows, const int64_t* cols, const T* coef, const int64_t* all_roots,                        \
      const int64_t* all_root_ps, const int64_t* all_root_pd, const int64_t* all_root_oo, const T* all_proj

/* segment k's slices under the names FA_REPLAY / FA_SWEEP use */
#define FA_SEG_BIND                                                                                           \
  const int64_t n0 = seg_node_off[k], r0 = seg_root_off[k];                                                  \
  const int64_t source_dim = seg_src_off[k + 1] - seg_src_off[k], input_dim = seg_in_dim[k];                  \
  const int64_t node_count = seg_node_off[k + 1] - n0, root_count = seg_root_off[k + 1] - r0;               \
  const int64_t *node_offsets = all_node_offsets + n0, *node_dims = all_node_dims + n0;                       \
  const int64_t *node_leaf = all_node_leaf + n0, *node_left = all_node_left + n0;                             \
  const int64_t *node_right = all_node_right + n0, *node_coef_off = all_node_coef_off + n0;                   \
  const int64_t *roots = all_roots + r0, *root_ps = all_root_ps + r0, *root_pd = all_root_pd + r0;            \
  const int64_t* root_oo = all_root_oo + r0;                                                                  \
  const int64_t proj_dim = seg_proj_dim[k], seg_out = seg_out_off[k + 1] - seg_out_off[k];                    \
  const int64_t W = node_offsets[node_count - 1] + node_dims[node_count - 1];                                 \
  (void)W;

#define FA_SEG_FORWARD(NAME, T, CONJ)                                                                        \
  void NAME(const T* packed, FA_SEG_ARGS(T), T* ws, T* out) {                                                 \
    for (int64_t b = 0; b < batch; ++b) {                                                                     \
      for (int64_t k = 0; k < seg_count; ++k) {                                                               \
        FA_SEG_BIND                                                                                           \
        const T* proj = all_proj + seg_proj_off[k];                                                           \
        T* orow = out + b * out_dim + seg_out_off[k];                                                         \
        for (int64_t q = 0; q < seg_out; ++q) orow[q] = 0;                                                    \
        for (int64_t s = 0; s < source_dim; ++s) {                                                            \
          for (int64_t q = 0; q < W; ++q) ws[q] = 0;                                                          \
          const T* in = packed + b * packed_dim + seg_in_off[k] + s * input_dim;                              \
          for (int64_t n = 0; n < node_count; ++n) {                                                          \
            T* o = ws + node_offsets[n];                                                                      \
            if (node_leaf[n] >= 0) {                                                                          \
              for (int64_t i = 0; i < node_dims[n]; ++i) o[i] = in[node_leaf[n] + i];                         \
              continue;                                                                                       \
            }                                                                                                 \
            const T* l = ws + node_offsets[node_left[n]];                                                     \
            const T* r = ws + node_offsets[node_right[n]];                                                    \
            const int64_t rd = node_dims[node_right[n]];                                                      \
            for (int64_t e = node_coef_off[n]; e < node_coef_off[n + 1]; ++e)                                 \
              o[cols[e]] += CONJ(coef[e]) * l[rows[e] / rd] * r[rows[e] % rd];                                \
          }                                                                                                   \
          for (int64_t ri = 0; ri < root_count; ++ri) {                                                       \
            const int64_t rn = roots[ri], rdim = node_dims[rn];                                               \
            const T* rv = ws + node_offsets[rn];                                                              \
            for (int64_t p = 0; p < root_pd[ri]; ++p) {                                                       \
              T* blk = orow + root_oo[ri] + p * rdim;                                                         \
              const T pv = proj[s * proj_dim + root_ps[ri] + p];                                              \
              for (int64_t m = 0; m < rdim; ++m) blk[m] += rv[m] * pv;                                        \
            }                                                                                                 \
          }                                                                                                   \
        }                                                                                                     \
      }                                                                                                       \
    }                                                                                                         \
  }

FA_SEG_FORWARD(oracle_factorized_angular_segmented_f64, double, conj_r)
FA_SEG_FORWARD(oracle_factorized_angular_segmented_c128, double complex, conj_c)

#define FA_SEG_ADJOINT(NAME, T, CONJ)                                                                        \
  void NAME(const T* gout, const T* packed, FA_SEG_ARGS(T), T* ws, T* wa, T* gpacked) {                       \
    for (int64_t b = 0; b < batch; ++b) {                                                                     \
      for (int64_t k = 0; k < seg_count; ++k) {                                                               \
        FA_SEG_BIND                                                                                           \
        const T* proj = all_proj + seg_proj_off[k];                                                           \
        const T* orow = gout + b * out_dim + seg_out_off[k];                                                  \
        T* grow = gpacked + b * packed_dim + seg_in_off[k];                                                   \
        for (int64_t q = 0; q < source_dim * input_dim; ++q) grow[q] = 0;                                     \
        for (int64_t s = 0; s < source_dim; ++s) {                                                            \
          const T* in = packed + b * packed_dim + seg_in_off[k] + s * input_dim;                              \
          FA_REPLAY(T, CONJ)                                                                                  \
          for (int64_t ri = 0; ri < root_count; ++ri) {                                                       \
            const int64_t rn = roots[ri], rdim = node_dims[rn];                                               \
            T* ra = wa + node_offsets[rn];                                                                    \
            for (int64_t p = 0; p < root_pd[ri]; ++p) {                                                       \
              const T* blk = orow + root_oo[ri] + p * rdim;                                                   \
              const T pv = proj[s * proj_dim + root_ps[ri] + p];                                              \
              for (int64_t m = 0; m < rdim; ++m) ra[m] += blk[m] * CONJ(pv);                                  \
            }                                                                                                 \
          }                                                                                                   \
          T* gin = grow + s * input_dim;                                                                      \
          FA_SWEEP(T, CONJ)                                                                                   \
        }                                                                                                     \
      }                                                                                                       \
    }                                                                                                         \
  }

FA_SEG_ADJOINT(oracle_factorized_angular_segmented_adjoint_f64, double, conj_r)
FA_SEG_ADJOINT(oracle_factorized_angular_segmented_adjoint_c128, double complex, conj_c)

/* ---- symmetric-power monomials ------------------------------------------- */

/* symmetric_power_monomial_adjoint (ye3t_runtime_core.cpp:5318-5389): per term,
 * the monomial without its zero factors; two or more zero factors give no
 * gradient, one zero factor of exponent 1 gives the cofactor, otherwise each
 * factor gets e * monomial / x. */
void oracle_symmetric_power_monomial_adjoint(const double* gout, const double* input, int64_t batch,
                                             int64_t in_dim, const int64_t* counts, const int64_t* out_index,
                                             const double* values, int64_t terms, int64_t out_dim,
                                             double* gin) {
  for (int64_t b = 0; b < batch; ++b) {
    const double* x = input + b * in_dim;
    double* g = gin + b * in_dim;
    for (int64_t c = 0; c < in_dim; ++c) g[c] = 0.0;
    for (int64_t t = 0; t < terms; ++t) {
      double mono = values[t];
      int64_t zeros = 0, zc = -1;
      for (int64_t c = 0; c < in_dim; ++c) {
        const int64_t e = counts[t * in_dim + c];
        if (e == 0) continue;
        if (x[c] == 0.0) {
          ++zeros;
          zc = c;
          continue;
        }
        mono *= ipow_r(x[c], e);
      }
      if (zeros >= 2) continue;
      const double og = gout[b * out_dim + out_index[t]];
      if (zeros == 1) {
        if (counts[t * in_dim + zc] == 1) g[zc] += og * mono;
        continue;
      }
      for (int64_t c = 0; c < in_dim; ++c) {
        const int64_t e = counts[t * in_dim + c];
        if (e == 0) continue;
        g[c] += og * ((double)e * mono / x[c]);
      }
    }
  }
}

/* symmetric_power_shared_monomial_forward (ye3t_runtime_core.cpp:5392-5440):
 * every monomial once per row, then each output sums its coefficients times
 * the monomials they name. */
void oracle_symmetric_power_shared_monomial(const double* input, int64_t batch, int64_t in_dim,
                                            const int64_t* counts, int64_t monomials, const int64_t* out_off,
                                            const int64_t* coef_terms, const double* coef_values,
                                            int64_t out_dim, double* mono_ws, double* out) {
  for (int64_t b = 0; b < batch; ++b) {
    const double* x = input + b * in_dim;
    for (int64_t t = 0; t < monomials; ++t) {
      double v = 1.0;
      for (int64_t c = 0; c < in_dim; ++c) v *= ipow_r(x[c], counts[t * in_dim + c]);
      mono_ws[t] = v;
    }
    for (int64_t o = 0; o < out_dim; ++o) {
      double v = 0.0;
      for (int64_t k = out_off[o]; k < out_off[o + 1]; ++k) v += coef_values[k] * mono_ws[coef_terms[k]];
      out[b * out_dim + o] = v;
    }
  }
}

/* symmetric_power_shared_monomial_adjoint (ye3t_runtime_core.cpp:5442-5540):
 * monomial adjoints from the output adjoints, then the monomial_adjoint rule
 * per monomial. */
void oracle_symmetric_power_shared_monomial_adjoint(const double* gout, const double* input, int64_t batch,
                                                    int64_t in_dim, const int64_t* counts, int64_t monomials,
                                                    const int64_t* out_off, const int64_t* coef_terms,
                                                    const double* coef_values, int64_t out_dim, double* mono_ws,
                                                    double* gin) {
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t t = 0; t < monomials; ++t) mono_ws[t] = 0.0;
    for (int64_t o = 0; o < out_dim; ++o)
      for (int64_t k = out_off[o]; k < out_off[o + 1]; ++k)
        mono_ws[coef_terms[k]] += gout[b * out_dim + o] * coef_values[k];
    const double* x = input + b * in_dim;
    double* g = gin + b * in_dim;
    for (int64_t c = 0; c < in_dim; ++c) g[c] = 0.0;
    for (int64_t t = 0; t < monomials; ++t) {
      const double tg = mono_ws[t];
      double mono = 1.0;
      int64_t zeros = 0, zc = -1;
      for (int64_t c = 0; c < in_dim; ++c) {
        const int64_t e = counts[t * in_dim + c];
        if (e == 0) continue;
        if (x[c] == 0.0) {
          ++zeros;
          zc = c;
          continue;
        }
        mono *= ipow_r(x[c], e);
      }
      if (zeros >= 2) continue;
      if (zeros == 1) {
        if (counts[t * in_dim + zc] == 1) g[zc] += tg * mono;
        continue;
      }
      for (int64_t c = 0; c < in_dim; ++c) {
        const int64_t e = counts[t * in_dim + c];
        if (e == 0) continue;
        g[c] += tg * ((double)e * mono / x[c]);
      }
    }
  }
}

/* ---- sparse shared monomials -----------------------------------------------
 * symmetric_power_shared_sparse_monomial{,_adjoint,_double_backward}
 * (execution_plan_cuda.cu:5720-5955, host :11012-11330; the reference has no
 * CPU kernel for them).  Monomial t is the product over its support
 * q in [term_offsets[t], term_offsets[t+1]) of x[comp[q]]^exp[q]; outputs are
 * sparse combinations of monomials as in the dense shared form.  The device
 * code accumulates its adjoints with atomics; this restatement takes the
 * coefficients and supports in index order. */

static void sparse_monomial_values(const double* x, const int64_t* toff, const int64_t* comp, const int64_t* ex,
                                   int64_t monomials, double* ws) {
  for (int64_t t = 0; t < monomials; ++t) {
    double v = 1.0;
    for (int64_t q = toff[t]; q < toff[t + 1]; ++q) v *= ipow_r(x[comp[q]], ex[q]);
    ws[t] = v;
  }
}

static void sparse_term_adjoint(const double* gout_row, const int64_t* coef_terms, const int64_t* coef_outputs,
                                const double* coef_values, int64_t coefs, int64_t monomials, double* ws) {
  for (int64_t t = 0; t < monomials; ++t) ws[t] = 0.0;
  for (int64_t k = 0; k < coefs; ++k) ws[coef_terms[k]] += gout_row[coef_outputs[k]] * coef_values[k];
}

void oracle_symmetric_power_shared_sparse_monomial(const double* input, int64_t batch, int64_t in_dim,
                                                   const int64_t* toff, const int64_t* comp, const int64_t* ex,
                                                   int64_t monomials, const int64_t* out_off,
                                                   const int64_t* coef_terms, const double* coef_values,
                                                   int64_t out_dim, double* mono_ws, double* out) {
  for (int64_t b = 0; b < batch; ++b) {
    sparse_monomial_values(input + b * in_dim, toff, comp, ex, monomials, mono_ws);
    for (int64_t o = 0; o < out_dim; ++o) {
      double v = 0.0;
      for (int64_t k = out_off[o]; k < out_off[o + 1]; ++k) v += coef_values[k] * mono_ws[coef_terms[k]];
      out[b * out_dim + o] = v;
    }
  }
}

/* :5757-5813 -- zero factors accumulate their exponents ("zero degree"): degree
 * one gives the cofactor to the zero component, a higher degree nothing,
 * degree zero e m / x per support entry. */
void oracle_symmetric_power_shared_sparse_monomial_adjoint(const double* gout, const double* input, int64_t batch,
                                                           int64_t in_dim, const int64_t* toff, const int64_t* comp,
                                                           const int64_t* ex, int64_t monomials,
                                                           const int64_t* coef_terms, const int64_t* coef_outputs,
                                                           const double* coef_values, int64_t coefs,
                                                           int64_t out_dim, double* mono_ws, double* gin) {
  for (int64_t b = 0; b < batch; ++b) {
    const double* x = input + b * in_dim;
    double* g = gin + b * in_dim;
    for (int64_t c = 0; c < in_dim; ++c) g[c] = 0.0;
    sparse_term_adjoint(gout + b * out_dim, coef_terms, coef_outputs, coef_values, coefs, monomials, mono_ws);
    for (int64_t t = 0; t < monomials; ++t) {
      const double tg = mono_ws[t];
      double mono = 1.0;
      int64_t zdeg = 0, zc = -1;
      for (int64_t q = toff[t]; q < toff[t + 1]; ++q) {
        if (x[comp[q]] == 0.0) {
          zdeg += ex[q];
          zc = comp[q];
        } else {
          mono *= ipow_r(x[comp[q]], ex[q]);
        }
      }
      if (zdeg == 1) {
        g[zc] += tg * mono;
        continue;
      }
      if (zdeg != 0) continue;
      for (int64_t q = toff[t]; q < toff[t + 1]; ++q) g[comp[q]] += tg * ((double)ex[q] * mono / x[comp[q]]);
    }
  }
}

/* :5815-5955 and host :11206-11330: the monomial adjoints are replaced by the
 * directional derivatives of the monomials along the tangent (which the
 * output kernel turns into the output tangent), and each monomial adds its
 * Hessian along the tangent, weighted by its adjoint, to the input tangent. */
void oracle_symmetric_power_shared_sparse_monomial_double_backward(
    const double* tangent, const double* gout, const double* input, int64_t batch, int64_t in_dim,
    const int64_t* toff, const int64_t* comp, const int64_t* ex, int64_t monomials, const int64_t* out_off,
    const int64_t* coef_terms, const int64_t* coef_outputs, const double* coef_values, int64_t coefs,
    int64_t out_dim, double* mono_ws, double* out_tangent, double* in_tangent) {
  for (int64_t b = 0; b < batch; ++b) {
    const double* x = input + b * in_dim;
    const double* v = tangent + b * in_dim;
    double* it = in_tangent + b * in_dim;
    for (int64_t c = 0; c < in_dim; ++c) it[c] = 0.0;
    sparse_term_adjoint(gout + b * out_dim, coef_terms, coef_outputs, coef_values, coefs, monomials, mono_ws);
    for (int64_t t = 0; t < monomials; ++t) {
      const double tg = mono_ws[t];
      double mono = 1.0;
      int64_t zdeg = 0, z1 = -1, z2 = -1;
      for (int64_t q = toff[t]; q < toff[t + 1]; ++q) {
        if (x[comp[q]] == 0.0) {
          zdeg += ex[q];
          if (z1 < 0) z1 = comp[q];
          else if (z2 < 0) z2 = comp[q];
        } else {
          mono *= ipow_r(x[comp[q]], ex[q]);
        }
      }
      double dir = 0.0;
      if (zdeg == 0) {
        double logdir = 0.0;
        for (int64_t q = toff[t]; q < toff[t + 1]; ++q) logdir += (double)ex[q] * v[comp[q]] / x[comp[q]];
        dir = mono * logdir;
        for (int64_t q = toff[t]; q < toff[t + 1]; ++q) {
          const int64_t c = comp[q];
          it[c] += tg * ((double)ex[q] * mono / x[c] * (logdir - v[c] / x[c]));
        }
      } else if (zdeg == 1) {
        dir = v[z1] * mono;
        double zdir = 0.0;
        for (int64_t q = toff[t]; q < toff[t + 1]; ++q) {
          const int64_t c = comp[q];
          if (c == z1) continue;
          const double d = (double)ex[q] * mono / x[c];
          zdir += v[c] * d;
          it[c] += tg * (v[z1] * d);
        }
        it[z1] += tg * zdir;
      } else if (zdeg == 2) {
        if (z2 < 0) {
          it[z1] += tg * (2.0 * mono * v[z1]);
        } else {
          it[z1] += tg * (mono * v[z2]);
          it[z2] += tg * (mono * v[z1]);
        }
      }
      mono_ws[t] = dir;
    }
    for (int64_t o = 0; o < out_dim; ++o) {
      double s = 0.0;
      for (int64_t k = out_off[o]; k < out_off[o + 1]; ++k) s += coef_values[k] * mono_ws[coef_terms[k]];
      out_tangent[b * out_dim + o] = s;
    }
  }
}
