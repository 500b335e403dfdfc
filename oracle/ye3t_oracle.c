/*
 * CPU ORACLE -- test infrastructure only.
 *
 * A plain-C restatement of the reference's CPU native algorithms for the ACE
 * hot path.  It is the checker for the HIP kernels and the timed CPU baseline;
 * nothing in the product library links, loads or calls it.
 *
 * Each function cites the reference routine it restates:
 *   ye3t/runtime/csrc/ye3t_runtime_core.cpp   (radial, real SH, scheduled edge channels, density, monomials)
 *   ye3t/core/csrc/factorized_runtime.cpp     (componentwise schedule evaluation)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ChebExpCos radial basis, one column per radial index.
 * Restates cheb_exp_cos_radial_with_derivative / ..._table_with_derivative
 * (ye3t_runtime_core.cpp:321-423): zero beyond the cutoff, n=0 -> 1,
 * n=1 -> (1+cos(pi r/rc))/2, n>=2 -> (1-T_n(x))(1+cos(pi r/rc))/4 with
 * x = 1 - 2 expm1(-lambda (r/rc - 1)) / expm1(lambda). */
void oracle_radial_table(const double* radii, const double* cutoffs, const double* lambdas,
                         int64_t edge_count, int64_t n_max, double* values, double* derivs) {
  const double pi = acos(-1.0);
  const double eps = 2.220446049250313e-16;
  const int64_t width = n_max + 1;
  for (int64_t e = 0; e < edge_count; ++e) {
    const double r = radii[e];
    const double rc = cutoffs[e] > eps ? cutoffs[e] : eps;
    const double lam = lambdas[e];
    const double s = r / rc;
    for (int64_t n = 0; n <= n_max; ++n) {
      double v, d;
      if (s > 1.0) {
        v = 0.0; d = 0.0;
      } else if (n == 0) {
        v = 1.0; d = 0.0;
      } else if (n == 1) {
        v = 0.5 * (1.0 + cos(pi * s));
        d = -0.5 * pi * sin(pi * s) / rc;
      } else {
        const double ex = exp(-lam * (s - 1.0));
        const double den = expm1(lam);
        const double x = 1.0 - 2.0 * expm1(-lam * (s - 1.0)) / den;
        double t0 = 1.0, t1 = x, u0 = 1.0, u1 = 2.0 * x;
        for (int64_t k = 2; k <= n; ++k) {
          const double t2 = 2.0 * x * t1 - t0;
          t0 = t1; t1 = t2;
          if (k < n) {
            const double u2 = 2.0 * x * u1 - u0;
            u0 = u1; u1 = u2;
          }
        }
        const double dcheb = (double)n * u1;
        const double dx = 2.0 * lam * ex / (den * rc);
        const double env = 1.0 + cos(pi * s);
        const double denv = -pi * sin(pi * s) / rc;
        v = 0.25 * (1.0 - t1) * env;
        d = 0.25 * (-dcheb * dx * env + (1.0 - t1) * denv);
      }
      values[e * width + n] = v;
      if (derivs) derivs[e * width + n] = d;
    }
  }
}

/* Ascending Legendre coefficients by Bonnet's recurrence (ye3t_runtime_core.cpp:34-56). */
static void legendre_coeffs(int64_t l, double* out /* l+1 */) {
  double prev[32], cur[32], next[32];
  memset(prev, 0, sizeof prev); memset(cur, 0, sizeof cur);
  if (l == 0) { out[0] = 1.0; return; }
  prev[0] = 1.0; cur[0] = 0.0; cur[1] = 1.0;
  for (int64_t n = 1; n < l; ++n) {
    memset(next, 0, sizeof next);
    const double fw = (double)(2 * n + 1) / (double)(n + 1);
    const double bw = (double)n / (double)(n + 1);
    for (int64_t p = 0; p <= n; ++p) next[p + 1] += fw * cur[p];
    for (int64_t p = 0; p <= n - 1; ++p) next[p] -= bw * prev[p];
    memcpy(prev, cur, sizeof cur); memcpy(cur, next, sizeof next);
  }
  for (int64_t p = 0; p <= l; ++p) out[p] = cur[p];
}

/* d^order/dz^order of an ascending polynomial (ye3t_runtime_core.cpp:57-72). */
static int64_t deriv_coeffs(const double* c, int64_t count, int64_t order, double* out) {
  double tmp[32];
  memcpy(tmp, c, (size_t)count * sizeof(double));
  for (int64_t k = 0; k < order; ++k) {
    if (count <= 1) { out[0] = 0.0; return 1; }
    for (int64_t p = 1; p < count; ++p) tmp[p - 1] = (double)p * tmp[p];
    count -= 1;
  }
  memcpy(out, tmp, (size_t)count * sizeof(double));
  return count;
}

static double horner(const double* c, int64_t count, double x) {
  double v = 0.0;
  for (int64_t p = count; p > 0; --p) v = v * x + c[p - 1];
  return v;
}

/* N_lm = sqrt((2l+1)/(4 pi) (l-m)!/(l+m)!) via logs (ye3t_runtime_core.cpp:213-222). */
static double sph_norm(int64_t l, int64_t m) {
  const double ln = 0.5 * (log((double)(2 * l + 1)) - log(4.0 * acos(-1.0)) +
                           lgamma((double)(l - m + 1)) - lgamma((double)(l + m + 1)));
  return exp(ln);
}

/* Real SH table (+ Cartesian gradient) for l = 0..l_max, degree l at columns
 * [l^2, (l+1)^2), m ascending.  Restates real_spherical_unit_value_and_gradient
 * and real_spherical_harmonics_(table_)with_derivative
 * (ye3t_runtime_core.cpp:224-286, 787-889). */
void oracle_real_sph_table(const double* vectors, int64_t edge_count, int64_t l_max, double epsilon,
                           double* values, double* grads) {
  const int64_t width = (l_max + 1) * (l_max + 1);
  for (int64_t e = 0; e < edge_count; ++e) {
    const double x = vectors[3 * e], y = vectors[3 * e + 1], z0 = vectors[3 * e + 2];
    const double r = sqrt(x * x + y * y + z0 * z0);
    const double sr = r > epsilon ? r : epsilon;
    const double u[3] = {x / sr, y / sr, z0 / sr};
    for (int64_t l = 0; l <= l_max; ++l) {
      double val[64], ug[64 * 3];
      const int64_t w = 2 * l + 1;
      memset(val, 0, sizeof val); memset(ug, 0, sizeof ug);
      double leg[32], dleg[32], dm[32], dm1[32];
      legendre_coeffs(l, leg);
      const int64_t nd = deriv_coeffs(leg, l + 1, 1, dleg);
      const double n0 = sph_norm(l, 0);
      val[l] = n0 * horner(leg, l + 1, u[2]);
      ug[l * 3 + 2] = n0 * horner(dleg, nd, u[2]);
      const double s2 = sqrt(2.0);
      double pr = 1.0, pi_ = 0.0, ppr = 1.0, ppi = 0.0;
      for (int64_t m = 1; m <= l; ++m) {
        ppr = pr; ppi = pi_;
        const double nr = pr * u[0] - pi_ * u[1];
        const double ni = pr * u[1] + pi_ * u[0];
        pr = nr; pi_ = ni;
        const int64_t c1 = deriv_coeffs(leg, l + 1, m, dm);
        const int64_t c2 = deriv_coeffs(leg, l + 1, m + 1, dm1);
        const double poly = horner(dm, c1, u[2]);
        const double polyz = horner(dm1, c2, u[2]);
        const double sc = s2 * sph_norm(l, m);
        const int64_t pos = l + m, neg = l - m;
        val[pos] = sc * poly * pr;
        ug[pos * 3 + 0] = sc * poly * ((double)m * ppr);
        ug[pos * 3 + 1] = sc * poly * (-(double)m * ppi);
        ug[pos * 3 + 2] = sc * polyz * pr;
        val[neg] = -sc * poly * pi_;
        ug[neg * 3 + 0] = -sc * poly * ((double)m * ppi);
        ug[neg * 3 + 1] = -sc * poly * ((double)m * ppr);
        ug[neg * 3 + 2] = -sc * polyz * pi_;
      }
      for (int64_t c = 0; c < w; ++c) {
        const int64_t o = e * width + l * l + c;
        values[o] = val[c];
        if (grads) {
          for (int a = 0; a < 3; ++a) {
            double g = 0.0;
            for (int b = 0; b < 3; ++b) {
              double jac = 0.0;
              if (r > epsilon) jac = ((a == b ? 1.0 : 0.0) - u[a] * u[b]) / sr;
              else if (a == b) jac = 1.0 / sr;
              g += ug[c * 3 + b] * jac;
            }
            grads[o * 3 + a] = g;
          }
        }
      }
    }
  }
}

/* Serial scatter of edge rows into their center rows (ye3t_runtime_core.cpp:1684-1702). */
void oracle_density_accumulate(const double* edge_values, const int64_t* centers, int64_t edge_count,
                               int64_t channel_count, int64_t atom_count, double* out) {
  memset(out, 0, (size_t)(atom_count * channel_count) * sizeof(double));
  for (int64_t e = 0; e < edge_count; ++e) {
    const double* src = edge_values + e * channel_count;
    double* dst = out + centers[e] * channel_count;
    for (int64_t c = 0; c < channel_count; ++c) dst[c] += src[c];
  }
}

/* Gather of centre-row adjoints to edge rows, edge_adjoint[e, :] =
 * atomic_adjoint[centers[e], :] (ye3t_runtime_core.cpp:1704-1715). */
void oracle_density_accumulate_adjoint(const double* atomic_adjoint, const int64_t* centers, int64_t edge_count,
                                       int64_t channel_count, double* edge_adjoint) {
  for (int64_t e = 0; e < edge_count; ++e) {
    const double* src = atomic_adjoint + centers[e] * channel_count;
    double* dst = edge_adjoint + e * channel_count;
    for (int64_t c = 0; c < channel_count; ++c) dst[c] = src[c];
  }
}

/* Scheduled radial-angular edge channels and their Cartesian derivatives
 * (ye3t_runtime_core.cpp:1550-1604): channel k of edge e is
 * scale_k R[e, ri_k] Y[e, ai_k] (products left to right) when channel_types[k]
 * is negative or equals edge_types[e], zero otherwise; the derivative is
 * scale_k (dR dir Y + R dY) per axis, in that order. */
void oracle_scheduled_channels(const double* rv, const double* rd, const double* av, const double* ad,
                               const double* dir, const int64_t* edge_types, const int64_t* cri,
                               const int64_t* cai, const int64_t* ctype, const double* cscale, int64_t edge_count,
                               int64_t radial_width, int64_t angular_width, int64_t channel_count,
                               double* values, double* derivs) {
  for (int64_t e = 0; e < edge_count; ++e) {
    for (int64_t k = 0; k < channel_count; ++k) {
      const int64_t o = e * channel_count + k;
      if (ctype[k] >= 0 && edge_types[e] != ctype[k]) {
        values[o] = 0.0;
        derivs[3 * o] = derivs[3 * o + 1] = derivs[3 * o + 2] = 0.0;
        continue;
      }
      const int64_t r_at = e * radial_width + cri[k], a_at = e * angular_width + cai[k];
      const double r = rv[r_at], a = av[a_at], sc = cscale[k];
      values[o] = sc * r * a;
      for (int x = 0; x < 3; ++x) derivs[3 * o + x] = sc * (rd[r_at] * dir[3 * e + x] * a + r * ad[3 * a_at + x]);
    }
  }
}

/* Stage 1 composed the reference way: radial table, real SH table, edge
 * product edge[e, (c, n, lm)] = w_c(e) * R_n(e) * Y_lm(e) (the semantics of
 * scheduled_radial_angular_channels, ye3t_runtime_core.cpp:1550-1604), then
 * density_accumulate over centers.  Channel weights w_c(e):
 *   species != NULL      : one-hot, w_c = [species[neighbor[e]] == c]
 *   node_features != NULL: w_c = node_features[neighbor[e], c]
 *   otherwise            : w_0 = 1 (channel_count must be 1).
 * With radial_mix != NULL ([C, n_max+1]) the radial of channel c is
 * sum_n radial_mix[c, n] R_n and the row has one radial per channel.
 * Output A[N, C, R, (l_max+1)^2] with R = n_max+1 (or 1 with radial_mix).
 * The edge loop is edge-parallel-free (serial), exactly like the reference. */
void oracle_ace_density(int64_t atom_count, int64_t edge_count, const int64_t* centers,
                        const int64_t* neighbors, const double* edge_vectors, const int32_t* species,
                        const double* node_features, const double* radial_mix, int64_t channel_count,
                        int64_t n_max, int64_t l_max, double cutoff, double lambda, double epsilon,
                        double* out) {
  const int64_t nr = n_max + 1;
  const int64_t lw = (l_max + 1) * (l_max + 1);
  const int64_t rows = radial_mix ? 1 : nr;
  const int64_t row = channel_count * rows * lw;
  double* radii = (double*)malloc((size_t)edge_count * sizeof(double));
  double* cuts = (double*)malloc((size_t)edge_count * sizeof(double));
  double* lams = (double*)malloc((size_t)edge_count * sizeof(double));
  double* R = (double*)malloc((size_t)(edge_count * nr) * sizeof(double));
  double* Y = (double*)malloc((size_t)(edge_count * lw) * sizeof(double));
  for (int64_t e = 0; e < edge_count; ++e) {
    const double* v = edge_vectors + 3 * e;
    radii[e] = sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    cuts[e] = cutoff; lams[e] = lambda;
  }
  oracle_radial_table(radii, cuts, lams, edge_count, n_max, R, NULL);
  oracle_real_sph_table(edge_vectors, edge_count, l_max, epsilon, Y, NULL);
  memset(out, 0, (size_t)(atom_count * row) * sizeof(double));
  double* edge_row = (double*)malloc((size_t)row * sizeof(double));
  for (int64_t e = 0; e < edge_count; ++e) {
    const int64_t j = neighbors ? neighbors[e] : 0;
    for (int64_t c = 0; c < channel_count; ++c) {
      double w;
      if (species) w = (species[j] == c) ? 1.0 : 0.0;
      else if (node_features) w = node_features[j * channel_count + c];
      else w = 1.0;
      for (int64_t n = 0; n < rows; ++n) {
        double rad;
        if (radial_mix) {
          rad = 0.0;
          for (int64_t q = 0; q < nr; ++q) rad += radial_mix[c * nr + q] * R[e * nr + q];
        } else {
          rad = R[e * nr + n];
        }
        for (int64_t k = 0; k < lw; ++k)
          edge_row[(c * rows + n) * lw + k] = w * rad * Y[e * lw + k];
      }
    }
    double* dst = out + centers[e] * row;
    for (int64_t k = 0; k < row; ++k) dst[k] += edge_row[k];
  }
  free(edge_row); free(radii); free(cuts); free(lams); free(R); free(Y);
}

/* Edge-vector gradient of stage 1 composed the reference way: per edge e
 * (centre i, neighbour j) and channel (c, r, k) the reference's scheduled
 * channel derivative (ye3t_runtime_core.cpp:1550-1604)
 *   d value / d v_e = w_c(j) (rad'_{c,r}(|v|) dir_e Y_k + rad_{c,r} dY_k / dv)
 * with radial and harmonic tables from oracle_radial_table /
 * oracle_real_sph_table (derivatives included), dir_e = v_e / max(|v_e|, eps)
 * (the unit vector of the harmonics) and rad = R_r, or sum_q mix[c, q] R_q when
 * radial_mix is set; contracted with the density adjoint gathered to the edge
 * (density_accumulate_adjoint, ye3t_runtime_core.cpp:1704-1715):
 *   grad[e, a] = sum_{c, r, k} adjoint[i, c, r, k] d value_{c,r,k} / d v_e[a]. */
void oracle_ace_density_edge_gradient(int64_t atom_count, int64_t edge_count, const int64_t* centers,
                                      const int64_t* neighbors, const double* edge_vectors, const int32_t* species,
                                      const double* node_features, const double* radial_mix, int64_t channel_count,
                                      int64_t n_max, int64_t l_max, double cutoff, double lambda, double epsilon,
                                      const double* density_adjoint, double* grad) {
  const int64_t nr = n_max + 1;
  const int64_t lw = (l_max + 1) * (l_max + 1);
  const int64_t rows = radial_mix ? 1 : nr;
  const int64_t row = channel_count * rows * lw;
  double* radii = (double*)malloc((size_t)edge_count * sizeof(double));
  double* cuts = (double*)malloc((size_t)edge_count * sizeof(double));
  double* lams = (double*)malloc((size_t)edge_count * sizeof(double));
  double* R = (double*)malloc((size_t)(edge_count * nr) * sizeof(double));
  double* dR = (double*)malloc((size_t)(edge_count * nr) * sizeof(double));
  double* Y = (double*)malloc((size_t)(edge_count * lw) * sizeof(double));
  double* dY = (double*)malloc((size_t)(edge_count * lw * 3) * sizeof(double));
  for (int64_t e = 0; e < edge_count; ++e) {
    const double* v = edge_vectors + 3 * e;
    radii[e] = sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    cuts[e] = cutoff; lams[e] = lambda;
  }
  (void)atom_count;
  oracle_radial_table(radii, cuts, lams, edge_count, n_max, R, dR);
  oracle_real_sph_table(edge_vectors, edge_count, l_max, epsilon, Y, dY);
  for (int64_t e = 0; e < edge_count; ++e) {
    const int64_t j = neighbors ? neighbors[e] : 0;
    const double* adj = density_adjoint + centers[e] * row;
    const double sr = radii[e] > epsilon ? radii[e] : epsilon;
    double dir[3];
    for (int a = 0; a < 3; ++a) dir[a] = edge_vectors[3 * e + a] / sr;
    double g[3] = {0.0, 0.0, 0.0};
    for (int64_t c = 0; c < channel_count; ++c) {
      double w;
      if (species) w = (species[j] == c) ? 1.0 : 0.0;
      else if (node_features) w = node_features[j * channel_count + c];
      else w = 1.0;
      for (int64_t n = 0; n < rows; ++n) {
        double rad, drad;
        if (radial_mix) {
          rad = 0.0; drad = 0.0;
          for (int64_t q = 0; q < nr; ++q) {
            rad += radial_mix[c * nr + q] * R[e * nr + q];
            drad += radial_mix[c * nr + q] * dR[e * nr + q];
          }
        } else {
          rad = R[e * nr + n];
          drad = dR[e * nr + n];
        }
        for (int64_t k = 0; k < lw; ++k) {
          const double ad = adj[(c * rows + n) * lw + k];
          for (int a = 0; a < 3; ++a)
            g[a] += ad * (w * (drad * dir[a] * Y[e * lw + k] + rad * dY[(e * lw + k) * 3 + a]));
        }
      }
    }
    for (int a = 0; a < 3; ++a) grad[3 * e + a] = g[a];
  }
  free(radii); free(cuts); free(lams); free(R); free(dR); free(Y); free(dY);
}

static double ipow(double b, int64_t e) {
  double v = 1.0;
  while (e > 0) { if (e & 1) v *= b; e >>= 1; if (e > 0) b *= b; }
  return v;
}

/* Symmetric-power monomial contraction (ye3t_runtime_core.cpp:5279-5315),
 * batch-parallel like execution_plan_torch.cpp:5488. */
void oracle_symmetric_power_monomial(const double* input, int64_t batch, int64_t in_dim,
                                     const int64_t* monomial_counts, const int64_t* output_offsets,
                                     const double* monomial_values, int64_t out_dim, double* output) {
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < batch; ++b) {
    const double* row = input + b * in_dim;
    for (int64_t o = 0; o < out_dim; ++o) {
      double v = 0.0;
      for (int64_t t = output_offsets[o]; t < output_offsets[o + 1]; ++t) {
        double mono = monomial_values[t];
        for (int64_t c = 0; c < in_dim; ++c) mono *= ipow(row[c], monomial_counts[t * in_dim + c]);
        v += mono;
      }
      output[b * out_dim + o] = v;
    }
  }
}

/* Componentwise schedule evaluation (factorized_runtime.cpp:251-285):
 * parallel over batch x component, each component walks its CSR term range. */
void oracle_evaluate_componentwise(const double* block_values, const int64_t* component_offsets,
                                   const int64_t* component_label_index, const int64_t* block_m_indices,
                                   const double* coeffs, double* out, int64_t batch, int64_t basis_count,
                                   int64_t magnetic_dim, int64_t component_count, int64_t block_count) {
  const int64_t total = batch * component_count;
#pragma omp parallel for schedule(static)
  for (int64_t lin = 0; lin < total; ++lin) {
    const int64_t b = lin / component_count;
    const int64_t k = lin - b * component_count;
    const int64_t label = component_label_index[k];
    double acc = 0.0;
    for (int64_t t = component_offsets[k]; t < component_offsets[k + 1]; ++t) {
      double v = coeffs[t];
      const int64_t* tm = block_m_indices + t * block_count;
      for (int64_t blk = 0; blk < block_count; ++blk)
        v *= block_values[((b * basis_count + label) * block_count + blk) * magnetic_dim + tm[blk]];
      acc += v;
    }
    out[b * component_count + k] = acc;
  }
}

/* ACE product, flat form: block values (leaf copies and symmetric-block
 * monomials, as symmetric_power_monomial_forward) then per column the
 * componentwise term loop (as evaluate_componentwise), over a [samples, a_width]
 * density.  value_factors / term_refs hold up to 4 indices, -1 = unused. */
void oracle_ace_product_flat(const double* A, int64_t samples, int64_t a_width,
                             int64_t value_count, const int64_t* value_offsets, const double* value_coeffs,
                             const int32_t* value_factors, int64_t column_count, const int64_t* column_offsets,
                             const double* term_coeffs, const int32_t* term_refs, double* B) {
#pragma omp parallel
  {
    double* vals = (double*)malloc((size_t)(value_count > 0 ? value_count : 1) * sizeof(double));
#pragma omp for schedule(static)
    for (int64_t s = 0; s < samples; ++s) {
      const double* row = A + s * a_width;
      for (int64_t v = 0; v < value_count; ++v) {
        double acc = 0.0;
        for (int64_t t = value_offsets[v]; t < value_offsets[v + 1]; ++t) {
          double m = value_coeffs[t];
          for (int q = 0; q < 4; ++q) {
            const int32_t f = value_factors[t * 4 + q];
            if (f >= 0) m *= row[f];
          }
          acc += m;
        }
        vals[v] = acc;
      }
      double* out = B + s * column_count;
      for (int64_t c = 0; c < column_count; ++c) {
        double acc = 0.0;
        for (int64_t t = column_offsets[c]; t < column_offsets[c + 1]; ++t) {
          double m = term_coeffs[t];
          for (int q = 0; q < 4; ++q) {
            const int32_t r = term_refs[t * 4 + q];
            if (r >= 0) m *= vals[r];
          }
          acc += m;
        }
        out[c] = acc;
      }
    }
    free(vals);
  }
}

/* Reverse mode of oracle_ace_product_flat: gA[s] = J(A[s])^T gB[s], where
 * B = f(A) is the flat form above (a polynomial of total degree <= 4 in A).
 * Each term's product rule is expanded factor by factor (the counterpart of
 * factorized_angular_adjoint, ye3t_runtime_core.h:1431-1456). */
void oracle_ace_product_flat_adjoint(const double* A, const double* gB, int64_t samples, int64_t a_width,
                                     int64_t value_count, const int64_t* value_offsets, const double* value_coeffs,
                                     const int32_t* value_factors, int64_t column_count,
                                     const int64_t* column_offsets, const double* term_coeffs,
                                     const int32_t* term_refs, double* gA) {
#pragma omp parallel
  {
    const size_t nv = (size_t)(value_count > 0 ? value_count : 1);
    double* vals = (double*)malloc(nv * sizeof(double));
    double* gv = (double*)malloc(nv * sizeof(double));
#pragma omp for schedule(static)
    for (int64_t s = 0; s < samples; ++s) {
      const double* row = A + s * a_width;
      const double* g = gB + s * column_count;
      double* out = gA + s * a_width;
      for (int64_t v = 0; v < value_count; ++v) {
        double acc = 0.0;
        for (int64_t t = value_offsets[v]; t < value_offsets[v + 1]; ++t) {
          double m = value_coeffs[t];
          for (int q = 0; q < 4; ++q) {
            const int32_t f = value_factors[t * 4 + q];
            if (f >= 0) m *= row[f];
          }
          acc += m;
        }
        vals[v] = acc;
        gv[v] = 0.0;
      }
      for (int64_t c = 0; c < column_count; ++c) {
        for (int64_t t = column_offsets[c]; t < column_offsets[c + 1]; ++t) {
          for (int q = 0; q < 4; ++q) {
            const int32_t r = term_refs[t * 4 + q];
            if (r < 0) continue;
            double m = term_coeffs[t] * g[c];
            for (int q2 = 0; q2 < 4; ++q2) {
              const int32_t r2 = term_refs[t * 4 + q2];
              if (q2 != q && r2 >= 0) m *= vals[r2];
            }
            gv[r] += m;
          }
        }
      }
      for (int64_t k = 0; k < a_width; ++k) out[k] = 0.0;
      for (int64_t v = 0; v < value_count; ++v) {
        for (int64_t t = value_offsets[v]; t < value_offsets[v + 1]; ++t) {
          for (int q = 0; q < 4; ++q) {
            const int32_t f = value_factors[t * 4 + q];
            if (f < 0) continue;
            double m = value_coeffs[t] * gv[v];
            for (int q2 = 0; q2 < 4; ++q2) {
              const int32_t f2 = value_factors[t * 4 + q2];
              if (q2 != q && f2 >= 0) m *= row[f2];
            }
            out[f] += m;
          }
        }
      }
    }
    free(vals);
    free(gv);
  }
}

/* Brute-force neighbour list (the reference has no builder).  Row i holds the
 * j != i, ascending, with |r_j - r_i|^2 < cutoff^2, each fp64 operation
 * rounded on its own: ((dx*dx + dy*dy) + dz*dz) with d = r_j - r_i.  That is
 * the CSR the density inputs take (centers, execution_plan.py:7913-7984) in the
 * order prepare_carrier_scatter_segments gives edges keyed target*N + source
 * (execution_plan.py:9316-9434).  positions are float (is_f32) or double; edge
 * vectors r_j - r_i are computed in that type and returned widened to double.
 * Pass 1 (centers == NULL) writes row_offsets[N + 1]; pass 2 fills the edges. */
static double pos_at(const void* pos, int is_f32, int64_t k) {
  return is_f32 ? (double)((const float*)pos)[k] : ((const double*)pos)[k];
}

void oracle_neighbor_list(const void* pos, int is_f32, int64_t n, double cutoff, int64_t* row_offsets,
                          int64_t* centers, int64_t* neighbors, double* vectors) {
  const double rc2 = cutoff * cutoff;
  const int fill = centers != NULL;
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t i = 0; i < n; ++i) {
    const double xi = pos_at(pos, is_f32, 3 * i), yi = pos_at(pos, is_f32, 3 * i + 1),
                 zi = pos_at(pos, is_f32, 3 * i + 2);
    int64_t e = fill ? row_offsets[i] : 0;
    for (int64_t j = 0; j < n; ++j) {
      if (j == i) continue;
      const double xj = pos_at(pos, is_f32, 3 * j), yj = pos_at(pos, is_f32, 3 * j + 1),
                   zj = pos_at(pos, is_f32, 3 * j + 2);
      const double dx = xj - xi, dy = yj - yi, dz = zj - zi;  /* built with -ffp-contract=off */
      const double d2 = (dx * dx + dy * dy) + dz * dz;
      if (!(d2 < rc2)) continue;
      if (fill) {
        centers[e] = i;
        neighbors[e] = j;
        if (is_f32) {
          const float* p = (const float*)pos;
          vectors[3 * e] = (double)(float)(p[3 * j] - p[3 * i]);
          vectors[3 * e + 1] = (double)(float)(p[3 * j + 1] - p[3 * i + 1]);
          vectors[3 * e + 2] = (double)(float)(p[3 * j + 2] - p[3 * i + 2]);
        } else {
          vectors[3 * e] = xj - xi;
          vectors[3 * e + 1] = yj - yi;
          vectors[3 * e + 2] = zj - zi;
        }
      }
      ++e;
    }
    if (!fill) row_offsets[i + 1] = e;
  }
  if (!fill) {
    row_offsets[0] = 0;
    for (int64_t i = 0; i < n; ++i) row_offsets[i + 1] += row_offsets[i];
  }
}
