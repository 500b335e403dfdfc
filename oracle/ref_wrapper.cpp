// Test-only C shim over the reference's own CPU core (ye3t_runtime_core.cpp),
// compiled from the reference sources in place by oracle/Makefile into
// oracle/_ref/.  Used to validate the C restatement and as a CPU baseline in
// this container.  Never part of the product.
#include <complex>
#include <cstdint>
#include <vector>
#include "ye3t_runtime_core.h"

namespace {
// uniform root metadata of the Torch op (execution_plan_torch.cpp:205-250)
struct Roots {
  std::vector<int64_t> starts, dims, offsets;
  Roots(int64_t root_count, int64_t proj_dim, int64_t root_dim)
      : starts(root_count, 0), dims(root_count, proj_dim), offsets(root_count) {
    for (int64_t r = 0; r < root_count; ++r) offsets[r] = r * proj_dim * root_dim;
  }
};

template <typename T>
void fa_forward(const T* packed, int64_t batch, int64_t in_dim, int64_t src_dim, const int64_t* noff,
                const int64_t* ndim, const int64_t* nleaf, const int64_t* nl, const int64_t* nr, const int64_t* ncoef,
                int64_t nodes, const int64_t* rows, const int64_t* cols, const T* coef, const int64_t* roots,
                int64_t root_count, const T* proj, int64_t proj_dim, int64_t out_dim, T* out) {
  Roots m(root_count, proj_dim, ndim[roots[0]]);
  ye3t::runtime::factorized_angular_forward<T>(packed, batch, in_dim, src_dim, noff, ndim, nleaf, nl, nr, ncoef,
                                              nodes, rows, cols, coef, roots, root_count, m.starts.data(),
                                              m.dims.data(), m.offsets.data(), proj, proj_dim, out_dim, out);
}

template <typename T>
void fa_adjoint(const T* gout, const T* packed, int64_t batch, int64_t in_dim, int64_t src_dim, const int64_t* noff,
                const int64_t* ndim, const int64_t* nleaf, const int64_t* nl, const int64_t* nr, const int64_t* ncoef,
                int64_t nodes, const int64_t* rows, const int64_t* cols, const T* coef, const int64_t* roots,
                int64_t root_count, const T* proj, int64_t proj_dim, int64_t out_dim, T* gpacked) {
  Roots m(root_count, proj_dim, ndim[roots[0]]);
  ye3t::runtime::factorized_angular_adjoint<T>(gout, packed, batch, in_dim, src_dim, noff, ndim, nleaf, nl, nr, ncoef,
                                              nodes, rows, cols, coef, roots, root_count, m.starts.data(),
                                              m.dims.data(), m.offsets.data(), proj, proj_dim, out_dim, gpacked);
}
}  // namespace

extern "C" {
void ref_radial_table(const double* r, const double* c, const double* l, int64_t e, int64_t n,
                      double* v, double* d) {
  ye3t::runtime::cheb_exp_cos_radial_table_with_derivative<double>(r, c, l, e, n, v, d);
}
void ref_real_sph_table(const double* vec, int64_t e, int64_t lmax, double eps, double* v, double* d) {
  ye3t::runtime::real_spherical_harmonics_table_with_derivative<double>(vec, e, lmax, eps, v, d);
}
void ref_scheduled_channels(const double* rv, const double* rd, const double* av, const double* ad,
                            const double* dir, const int64_t* et, const int64_t* cri, const int64_t* cai,
                            const int64_t* ct, const double* cs, int64_t e, int64_t nr, int64_t na, int64_t k,
                            double* v, double* d) {
  ye3t::runtime::scheduled_radial_angular_channels_with_derivative<double>(rv, rd, av, ad, dir, et, cri, cai, ct, cs,
                                                                           e, nr, na, k, v, d);
}
void ref_density_accumulate(const double* ev, const int64_t* centers, int64_t e, int64_t c, int64_t n,
                            double* out) {
  ye3t::runtime::density_accumulate_forward<double>(ev, centers, e, c, n, out);
}
void ref_density_accumulate_adjoint(const double* adj, const int64_t* centers, int64_t e, int64_t c,
                                    double* out) {
  ye3t::runtime::density_accumulate_adjoint<double>(adj, centers, e, c, out);
}
void ref_symmetric_power_monomial(const double* in, int64_t batch, int64_t in_dim, const int64_t* counts,
                                  const int64_t* offsets, const double* values, int64_t terms,
                                  int64_t out_dim, double* out) {
  ye3t::runtime::symmetric_power_monomial_forward<double>(in, batch, in_dim, counts, offsets, values, terms,
                                                          out_dim, out);
}
void ref_symmetric_power_monomial_adjoint(const double* gout, const double* in, int64_t batch, int64_t in_dim,
                                          const int64_t* counts, const int64_t* out_index, const double* values,
                                          int64_t terms, int64_t out_dim, double* gin) {
  ye3t::runtime::symmetric_power_monomial_adjoint<double>(gout, in, batch, in_dim, counts, out_index, values, terms,
                                                          out_dim, gin);
}
void ref_symmetric_power_shared_monomial(const double* in, int64_t batch, int64_t in_dim, const int64_t* counts,
                                         int64_t monomials, const int64_t* out_off, const int64_t* terms,
                                         const double* values, int64_t coef_count, int64_t out_dim, double* out) {
  ye3t::runtime::symmetric_power_shared_monomial_forward<double>(in, batch, in_dim, counts, monomials, out_off,
                                                                 terms, values, coef_count, out_dim, out);
}
void ref_symmetric_power_shared_monomial_adjoint(const double* gout, const double* in, int64_t batch,
                                                 int64_t in_dim, const int64_t* counts, int64_t monomials,
                                                 const int64_t* out_off, const int64_t* terms, const double* values,
                                                 int64_t coef_count, int64_t out_dim, double* gin) {
  ye3t::runtime::symmetric_power_shared_monomial_adjoint<double>(gout, in, batch, in_dim, counts, monomials, out_off,
                                                                 terms, values, coef_count, out_dim, gin);
}
// factorized angular DAG: real (f64) and complex (c128, interleaved re/im)
#define YE3T_REF_FA(SUFFIX, T)                                                                                    \
  void ref_factorized_angular_##SUFFIX(const T* packed, int64_t batch, int64_t in_dim, int64_t src_dim,           \
                                       const int64_t* noff, const int64_t* ndim, const int64_t* nleaf,            \
                                       const int64_t* nl, const int64_t* nr, const int64_t* ncoef, int64_t nodes, \
                                       const int64_t* rows, const int64_t* cols, const T* coef,                   \
                                       const int64_t* roots, int64_t root_count, const T* proj, int64_t proj_dim, \
                                       int64_t out_dim, T* out) {                                                 \
    fa_forward<T>(packed, batch, in_dim, src_dim, noff, ndim, nleaf, nl, nr, ncoef, nodes, rows, cols, coef,     \
                  roots, root_count, proj, proj_dim, out_dim, out);                                              \
  }                                                                                                              \
  void ref_factorized_angular_adjoint_##SUFFIX(                                                                  \
      const T* gout, const T* packed, int64_t batch, int64_t in_dim, int64_t src_dim, const int64_t* noff,         \
      const int64_t* ndim, const int64_t* nleaf, const int64_t* nl, const int64_t* nr, const int64_t* ncoef,       \
      int64_t nodes, const int64_t* rows, const int64_t* cols, const T* coef, const int64_t* roots,              \
      int64_t root_count, const T* proj, int64_t proj_dim, int64_t out_dim, T* gpacked) {                         \
    fa_adjoint<T>(gout, packed, batch, in_dim, src_dim, noff, ndim, nleaf, nl, nr, ncoef, nodes, rows, cols, coef,\
                  roots, root_count, proj, proj_dim, out_dim, gpacked);                                          \
  }                                                                                                              \
  void ref_factorized_angular_linear_##SUFFIX(                                                                   \
      const T* packed, int64_t batch, int64_t in_dim, int64_t src_dim, const int64_t* noff, const int64_t* ndim,   \
      const int64_t* nleaf, const int64_t* nl, const int64_t* nr, const int64_t* ncoef, int64_t nodes,            \
      const int64_t* rows, const int64_t* cols, const T* coef, const int64_t* roots, int64_t root_count,          \
      const T* proj, int64_t proj_dim, const T* weight, const T* bias, T* out) {                                  \
    ye3t::runtime::factorized_angular_linear_forward<T>(packed, batch, in_dim, src_dim, noff, ndim, nleaf, nl, nr, \
                                                        ncoef, nodes, rows, cols, coef, roots, root_count, proj,  \
                                                        proj_dim, weight, *bias, out);                            \
  }                                                                                                              \
  void ref_factorized_angular_linear_adjoint_##SUFFIX(                                                           \
      const T* gout, const T* packed, int64_t batch, int64_t in_dim, int64_t src_dim, const int64_t* noff,         \
      const int64_t* ndim, const int64_t* nleaf, const int64_t* nl, const int64_t* nr, const int64_t* ncoef,       \
      int64_t nodes, const int64_t* rows, const int64_t* cols, const T* coef, const int64_t* roots,              \
      int64_t root_count, const T* proj, int64_t proj_dim, const T* weight, T* gpacked, T* gweight, T* gbias) {  \
    ye3t::runtime::factorized_angular_linear_adjoint<T>(gout, packed, batch, in_dim, src_dim, noff, ndim, nleaf,  \
                                                        nl, nr, ncoef, nodes, rows, cols, coef, roots,            \
                                                        root_count, proj, proj_dim, weight, gpacked, gweight,     \
                                                        gbias);                                                   \
  }
YE3T_REF_FA(f64, double)
YE3T_REF_FA(c128, std::complex<double>)
#undef YE3T_REF_FA

// segmented DAGs (factorized_angular_segmented_forward / _adjoint), with the
// argument order of the oracle's restatement (minus its scratch buffers)
#define YE3T_REF_FA_SEG_ARGS(T)                                                                                   \
  int64_t batch, int64_t packed_dim, int64_t seg_count, const int64_t *seg_src_off, const int64_t *seg_in_off,   \
      const int64_t *seg_in_dim, const int64_t *seg_node_off, const int64_t *seg_root_off,                       \
      const int64_t *seg_proj_off, const int64_t *seg_proj_dim, const int64_t *seg_out_off, int64_t out_dim,     \
      const int64_t *noff, const int64_t *ndim, const int64_t *nleaf, const int64_t *nl, const int64_t *nr,      \
      const int64_t *ncoef, const int64_t *rows, const int64_t *cols, const T *coef, const int64_t *roots,       \
      const int64_t *rps, const int64_t *rpd, const int64_t *roo, const T *proj
#define YE3T_REF_FA_SEG_VIEW(T)                                                                                   \
  ye3t::runtime::FactorizedAngularSegmentedPlanView<T> v;                                                        \
  v.segment_source_offsets = seg_src_off;                                                                        \
  v.segment_input_offsets = seg_in_off;                                                                          \
  v.segment_input_dimensions = seg_in_dim;                                                                       \
  v.segment_workspace_offsets = nullptr;                                                                         \
  v.segment_workspace_dimensions = nullptr;                                                                      \
  v.segment_node_offsets = seg_node_off;                                                                         \
  v.segment_root_offsets = seg_root_off;                                                                         \
  v.segment_projection_offsets = seg_proj_off;                                                                   \
  v.segment_projection_dimensions = seg_proj_dim;                                                                \
  v.segment_output_offsets = seg_out_off;                                                                        \
  v.node_offsets = noff;                                                                                         \
  v.node_dimensions = ndim;                                                                                      \
  v.node_leaf_offsets = nleaf;                                                                                   \
  v.node_left = nl;                                                                                              \
  v.node_right = nr;                                                                                             \
  v.node_coefficient_offsets = ncoef;                                                                            \
  v.coefficient_rows = rows;                                                                                     \
  v.coefficient_columns = cols;                                                                                  \
  v.coefficient_values = coef;                                                                                   \
  v.root_nodes = roots;                                                                                          \
  v.root_projection_starts = rps;                                                                                \
  v.root_projection_dimensions = rpd;                                                                            \
  v.root_output_offsets = roo;                                                                                   \
  v.projection_values = proj;                                                                                    \
  v.segment_count = seg_count;                                                                                   \
  v.packed_input_dimension = packed_dim;                                                                         \
  v.workspace_dimension = 0;                                                                                     \
  v.output_dimension = out_dim;
#define YE3T_REF_FA_SEG(SUFFIX, T)                                                                                \
  void ref_factorized_angular_segmented_##SUFFIX(const T *packed, YE3T_REF_FA_SEG_ARGS(T), T *out) {             \
    YE3T_REF_FA_SEG_VIEW(T)                                                                                      \
    ye3t::runtime::factorized_angular_segmented_forward<T>(packed, batch, v, out);                               \
  }                                                                                                              \
  void ref_factorized_angular_segmented_adjoint_##SUFFIX(const T *gout, const T *packed, YE3T_REF_FA_SEG_ARGS(T), \
                                                         T *gpacked) {                                           \
    YE3T_REF_FA_SEG_VIEW(T)                                                                                      \
    ye3t::runtime::factorized_angular_segmented_adjoint<T>(gout, packed, batch, v, gpacked);                     \
  }
YE3T_REF_FA_SEG(f64, double)
YE3T_REF_FA_SEG(c128, std::complex<double>)
#undef YE3T_REF_FA_SEG
#undef YE3T_REF_FA_SEG_VIEW
#undef YE3T_REF_FA_SEG_ARGS
}
