// Test-only C shim over the reference's own CPU core (ye3t_runtime_core.cpp),
// compiled from the reference sources in place by oracle/Makefile into
// oracle/_ref/.  Used to validate the C restatement and as a CPU baseline in
// this container.  Never part of the product.
#include <cstdint>
#include "ye3t_runtime_core.h"

extern "C" {
void ref_radial_table(const double* r, const double* c, const double* l, int64_t e, int64_t n,
                      double* v, double* d) {
  ye3t::runtime::cheb_exp_cos_radial_table_with_derivative<double>(r, c, l, e, n, v, d);
}
void ref_real_sph_table(const double* vec, int64_t e, int64_t lmax, double eps, double* v, double* d) {
  ye3t::runtime::real_spherical_harmonics_table_with_derivative<double>(vec, e, lmax, eps, v, d);
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
}
