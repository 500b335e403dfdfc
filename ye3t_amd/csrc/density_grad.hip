// Edge-vector gradient of the fused stage-1 density on gfx950 (forces).
//
// For a density adjoint gA[i, c, r, k] (same shape as A), the gradient of
// <gA, A(v)> with respect to every edge vector v_e, e in row i, neighbour j:
//
//   g_e = sum_{c, r, k} gA[i, c, r, k] w_c(j) (rad'_{c,r}(|v|) u Y_k(u) + rad_{c,r}(|v|) dY_k/dv)
//
// with u = v / max(|v|, eps), rad_{c,r} = R_r or sum_q mix[c, q] R_q.  This is
// the reference chain cheb_exp_cos_radial_table_with_derivative ->
// spherical_harmonics_table_with_derivative ->
// scheduled_radial_angular_channels_with_derivative (ye3t_runtime_core.cpp:
// 1550-1604) -> density_accumulate_adjoint (:1704-1715) contracted on the
// device in one pass, without materialising the [E, channels, 3] derivative
// table.  Per edge (one lane):
//   a   = sum_{c,r} w rad'_{c,r} (sum_k gA[c,r,k] Y_k)
//   t_k = sum_{c,r} w rad_{c,r} gA[c,r,k]
//   g   = a u + J^T sum_k t_k grad_u Y_k,   J = (I - u u^T) / |v|
// (the harmonics are polynomials in u; J is du/dv).  Arithmetic in fp64; Y, t
// and the radial values live in registers (the kernel is instantiated per
// l_max; radial loops run to a fixed maximum under a predicate).
#include "common.h"

namespace ye3t {
namespace {

constexpr int kGradMaxRadial = 16;  // n_max + 1 <= 16

template <typename In, typename G>
struct GradParams {
  const In* vec;             // [E, 3]
  const int64_t* row_offsets;  // [N + 1]
  const int64_t* neighbors;  // [E] or NULL
  const int32_t* species;    // [N] or NULL
  const In* feats;           // [N, C] or NULL
  const In* mix;             // [C, nr] or NULL
  const G* gA;               // [N, C, rows, lw]
  In* out;                   // [E, 3]
  int64_t N, E;
  int C, nr, rows;
  double cutoff, lambda, eps;
  NormTable nt;
};

// Y_k(u) for k < (LMAX + 1)^2 (the reference's real SH, same recurrence as
// real_sph_row) with compile-time bounds, so Y stays in registers.
template <int LMAX>
__device__ inline void sph_values(double x, double y, double z, const NormTable& nt, double* Y) {
  const double sqrt2 = 1.4142135623730950488016887242096981;
  double cr = 1.0, ci = 0.0, qmm = 1.0;
#pragma unroll
  for (int m = 0; m <= LMAX; ++m) {
    if (m > 0) {
      qmm *= double(2 * m - 1);
      const double nr = cr * x - ci * y;
      const double ni = cr * y + ci * x;
      cr = nr;
      ci = ni;
    }
    double q2 = 0.0, q1 = 0.0;
#pragma unroll
    for (int l = m; l <= LMAX; ++l) {
      double q;
      if (l == m) {
        q = qmm;
      } else if (l == m + 1) {
        q = double(2 * m + 1) * z * qmm;
      } else {
        q = (double(2 * l - 1) * z * q1 - double(l + m - 1) * q2) * nt.inv[l - m];
      }
      q2 = q1;
      q1 = q;
      const double n = nt.v[l * (kMaxL + 1) + m];
      const int base = l * l + l;
      if (m == 0) {
        Y[base] = n * q;
      } else {
        const double s = sqrt2 * n * q;
        Y[base + m] = s * cr;
        Y[base - m] = -s * ci;
      }
    }
  }
}

// G = sum_k t_k grad_u Y_k(u), the harmonics taken as polynomials in u:
// Y_{l,0} = N Q_l^0(z), Y_{l,+-m} = sqrt2 N Q_l^m(z) (Re, -Im) (x + i y)^m with
// Q_l^m = d^m P_l / dz^m, so d/dz brings Q_l^{m+1} and d/dx, d/dy bring
// m (x + i y)^{m-1}.
template <int LMAX>
__device__ inline void sph_gradient_dot(double x, double y, double z, const NormTable& nt, const double* t,
                                        double& gx, double& gy, double& gz) {
  const double sqrt2 = 1.4142135623730950488016887242096981;
  double Q[LMAX + 2][LMAX + 1];  // Q[m][l] = Q_l^m for l <= LMAX, m <= LMAX + 1
  double qmm = 1.0;
#pragma unroll
  for (int m = 0; m <= LMAX + 1; ++m) {
    if (m > 0) qmm *= double(2 * m - 1);
    double q2 = 0.0, q1 = 0.0;
#pragma unroll
    for (int l = 0; l <= LMAX; ++l) {
      double q = 0.0;
      if (l == m) {
        q = qmm;
      } else if (l == m + 1) {
        q = double(2 * m + 1) * z * qmm;
      } else if (l > m + 1) {
        q = (double(2 * l - 1) * z * q1 - double(l + m - 1) * q2) * nt.inv[l - m];
      }
      if (l >= m) {
        q2 = q1;
        q1 = q;
      }
      Q[m][l] = q;
    }
  }
  gx = gy = gz = 0.0;
  double cr = 1.0, ci = 0.0, pr = 1.0, pi = 0.0;  // (x + i y)^m and ^(m-1)
#pragma unroll
  for (int m = 0; m <= LMAX; ++m) {
    if (m > 0) {
      pr = cr;
      pi = ci;
      const double nr = cr * x - ci * y;
      const double ni = cr * y + ci * x;
      cr = nr;
      ci = ni;
    }
#pragma unroll
    for (int l = m; l <= LMAX; ++l) {
      const double n = nt.v[l * (kMaxL + 1) + m];
      const int base = l * l + l;
      if (m == 0) {
        gz += t[base] * (n * Q[1][l]);
      } else {
        const double s = sqrt2 * n;
        const double q = Q[m][l], qz = Q[m + 1][l];
        const double tp = t[base + m], tm = t[base - m];
        // grad Y_{l,+m} = s (m q pr, -m q pi, qz cr); grad Y_{l,-m} = -s (m q pi, m q pr, qz ci)
        gx += s * double(m) * q * (tp * pr - tm * pi);
        gy += -s * double(m) * q * (tp * pi + tm * pr);
        gz += s * qz * (tp * cr - tm * ci);
      }
    }
  }
}

// One channel c of edge e with weight w: a += w sum_r rad'_{c,r} z_{c,r},
// t_k += w sum_r rad_{c,r} gA[c, r, k], z_{c,r} = sum_k gA[c, r, k] Y_k.  The
// radial values R, dR are register arrays of kGradMaxRadial entries (computed
// to the fixed length; entries from nr on are not read).
template <int LW, int NRMAX, typename In, typename G>
__device__ inline void channel_terms(const GradParams<In, G>& p, const G* grow, int c, double w, const double* R,
                                     const double* dR, const double* Y, double& a, double* t) {
  if (p.mix) {
    double rad = 0.0, drad = 0.0;
#pragma unroll
    for (int q = 0; q < NRMAX; ++q) {
      if (q < p.nr) {
        const double mq = double(p.mix[c * p.nr + q]);
        rad += mq * R[q];
        drad += mq * dR[q];
      }
    }
    const G* gr = grow + int64_t(c) * LW;
    double z = 0.0;
#pragma unroll
    for (int k = 0; k < LW; ++k) z += double(gr[k]) * Y[k];
    a += w * drad * z;
    const double coef = w * rad;
#pragma unroll
    for (int k = 0; k < LW; ++k) t[k] += coef * double(gr[k]);
  } else {
#pragma unroll
    for (int n = 0; n < NRMAX; ++n) {
      if (n < p.nr) {
        const G* gr = grow + (int64_t(c) * p.nr + n) * LW;
        double z = 0.0;
#pragma unroll
        for (int k = 0; k < LW; ++k) z += double(gr[k]) * Y[k];
        a += w * dR[n] * z;
        const double coef = w * R[n];
#pragma unroll
        for (int k = 0; k < LW; ++k) t[k] += coef * double(gr[k]);
      }
    }
  }
}

// NRMAX: length of the radial register arrays (>= p.nr).  MIX16: node
// features with a mix over exactly 16 channels and l_max <= 3 (config 4's
// shape): the channel loop is unrolled, the neighbour's feature row is read
// once as a 64-byte row rather than as 16 four-byte gathers, and each
// channel's adjoint row is requested one channel ahead.
template <int LMAX, int NRMAX, bool MIX16, typename In, typename G>
__global__ __launch_bounds__(64) void density_edge_gradient_kernel(GradParams<In, G> p) {
  constexpr int LW = (LMAX + 1) * (LMAX + 1);
  const int lane = threadIdx.x;
  // centre of each edge: the largest i with row_offsets[i] <= e (then
  // e < row_offsets[i + 1]; rows of empty atoms own nothing).  `centre`
  // bisects [lo, hi) given row_offsets[lo] <= target and hi == N or
  // row_offsets[hi] > target.  The block's first edge is bracketed by
  // galloping from the atom a uniform degree would give it, its last edge by
  // galloping from the first's centre (wave-uniform, scalar loads: a few
  // dependent loads instead of log2 N), then each lane bisects the few rows
  // between them; every access stays inside [0, N).
  auto centre = [&](int64_t target, int64_t lo, int64_t hi) {
    while (hi - lo > 1) {
      const int64_t mid = (lo + hi) >> 1;
      if (p.row_offsets[mid] <= target) lo = mid;
      else hi = mid;
    }
    return lo;
  };
  auto gallop = [&](int64_t target, int64_t lo_bound, int64_t guess) {
    int64_t lo, hi;
    guess = guess < lo_bound ? lo_bound : (guess > p.N - 1 ? p.N - 1 : guess);
    if (p.row_offsets[guess] <= target) {  // bracket upwards
      lo = guess;
      int64_t step = 1;
      hi = lo + step;
      while (hi < p.N && p.row_offsets[hi] <= target) {
        lo = hi;
        step *= 2;
        hi = lo + step;
      }
      hi = hi < p.N ? hi : p.N;
    } else {  // bracket downwards: row_offsets[lo_bound] <= target holds
      hi = guess;
      int64_t step = 1;
      lo = hi - step;
      while (lo > lo_bound && p.row_offsets[lo] > target) {
        hi = lo;
        step *= 2;
        lo = hi - step;
      }
      lo = lo > lo_bound ? lo : lo_bound;
    }
    return centre(target, lo, hi);
  };
  const int64_t e_first = int64_t(blockIdx.x) * 64;
  const int64_t e_last = e_first + 63 < p.E ? e_first + 63 : p.E - 1;
  const int64_t i_first = gallop(e_first, 0, int64_t(double(e_first) * double(p.N) / double(p.E)));
  const int64_t i_last = gallop(e_last, i_first, i_first);
  const int64_t e = e_first + lane;
  if (e >= p.E) return;
  // a lane's centre: with few rows in the block, i_first plus the number of
  // rows k in (i_first, i_last] with row_offsets[k] <= e (the offsets rise, so
  // those rows are a prefix), the offsets read through the scalar cache
  // independently of one another; otherwise a per-lane bisection
  int64_t i;
  if (i_last - i_first <= 16) {
    i = i_first;
    for (int64_t k = i_first + 1; k <= i_last; ++k) i += p.row_offsets[k] <= e ? 1 : 0;
  } else {
    i = centre(e, i_first, i_last + 1);
  }
  int64_t j = p.neighbors ? p.neighbors[e] : 0;
  j = j < 0 ? 0 : (j >= p.N ? p.N - 1 : j);  // out-of-range input is clamped, never dereferenced
  const double vx = double(p.vec[3 * e]), vy = double(p.vec[3 * e + 1]), vz = double(p.vec[3 * e + 2]);
  const double r = d_sqrt(vx * vx + vy * vy + vz * vz);
  const double sr = r > p.eps ? r : p.eps;
  const double ux = vx / sr, uy = vy / sr, uz = vz / sr;
  double Y[LW];
  sph_values<LMAX>(ux, uy, uz, p.nt, Y);
  double R[NRMAX], dR[NRMAX];
  cheb_exp_cos_row<double, true, double>(r, p.cutoff, p.lambda, NRMAX - 1, R, dR);
  double a = 0.0;
  double t[LW];
#pragma unroll
  for (int k = 0; k < LW; ++k) t[k] = 0.0;
  const G* grow = p.gA + i * int64_t(p.C) * p.rows * LW;
  if (p.species) {  // one-hot: the neighbour's channel only
    int s = p.species[j];
    s = s < 0 ? 0 : (s >= p.C ? p.C - 1 : s);
    channel_terms<LW, NRMAX>(p, grow, s, 1.0, R, dR, Y, a, t);
  } else if constexpr (MIX16) {
    // the neighbour's 16 features as one 64-byte row (the channel index is
    // wave-uniform, so h[c] is a register-relative move), each channel's
    // adjoint row requested one channel ahead; the loop stays rolled so the
    // loads stay where they are written
    constexpr int C = 16;
    In h[C];
#pragma unroll
    for (int c = 0; c < C; ++c) h[c] = p.feats[j * C + c];
    G gn[LW];
#pragma unroll
    for (int k = 0; k < LW; ++k) gn[k] = grow[k];
#pragma unroll 1
    for (int c = 0; c < C; ++c) {
      G g[LW];
#pragma unroll
      for (int k = 0; k < LW; ++k) g[k] = gn[k];
      if (c + 1 < C) {
        const G* gr = grow + (c + 1) * LW;
#pragma unroll
        for (int k = 0; k < LW; ++k) gn[k] = gr[k];
      }
      const double w = double(h[c]);
      double rad = 0.0, drad = 0.0;
#pragma unroll
      for (int q = 0; q < NRMAX; ++q) {
        if (q < p.nr) {
          const double mq = double(p.mix[c * p.nr + q]);
          rad += mq * R[q];
          drad += mq * dR[q];
        }
      }
      double z = 0.0;
#pragma unroll
      for (int k = 0; k < LW; ++k) z += double(g[k]) * Y[k];
      a += w * drad * z;
      const double coef = w * rad;
#pragma unroll
      for (int k = 0; k < LW; ++k) t[k] += coef * double(g[k]);
    }
  } else if (p.mix) {
    // channel index uniform across the wave (the mix row is read through the
    // scalar cache).  For l_max <= 3 the next channel's adjoint row and
    // feature value are requested before this channel's arithmetic, so their
    // latency hides behind it (config 4: 198 -> 181 us); larger rows would not
    // fit twice in the registers, and each is loaded just before its use.
    constexpr bool kPrefetch = LW <= 16;
    G gn[kPrefetch ? LW : 1];
    In wn = In(1);
    if constexpr (kPrefetch) {
      wn = p.feats ? p.feats[j * p.C] : In(1);
#pragma unroll
      for (int k = 0; k < LW; ++k) gn[k] = grow[k];
    }
    for (int c = 0; c < p.C; ++c) {
      G g[LW];
      double w;
      if constexpr (kPrefetch) {
#pragma unroll
        for (int k = 0; k < LW; ++k) g[k] = gn[k];
        w = double(wn);
        if (c + 1 < p.C) {
          const G* gr = grow + int64_t(c + 1) * LW;
#pragma unroll
          for (int k = 0; k < LW; ++k) gn[k] = gr[k];
          wn = p.feats ? p.feats[j * p.C + c + 1] : In(1);
        }
      } else {
        w = p.feats ? double(p.feats[j * p.C + c]) : 1.0;
        const G* gr = grow + int64_t(c) * LW;
#pragma unroll
        for (int k = 0; k < LW; ++k) g[k] = gr[k];
      }
      double rad = 0.0, drad = 0.0;
#pragma unroll
      for (int q = 0; q < NRMAX; ++q) {
        if (q < p.nr) {
          const double mq = double(p.mix[c * p.nr + q]);
          rad += mq * R[q];
          drad += mq * dR[q];
        }
      }
      double z = 0.0;
#pragma unroll
      for (int k = 0; k < LW; ++k) z += double(g[k]) * Y[k];
      a += w * drad * z;
      const double coef = w * rad;
#pragma unroll
      for (int k = 0; k < LW; ++k) t[k] += coef * double(g[k]);
    }
  } else {  // channel index uniform across the wave
    for (int c = 0; c < p.C; ++c)
      channel_terms<LW, NRMAX>(p, grow, c, p.feats ? double(p.feats[j * p.C + c]) : 1.0, R, dR, Y, a, t);
  }
  double gx, gy, gz;
  sph_gradient_dot<LMAX>(ux, uy, uz, p.nt, t, gx, gy, gz);
  if (r > p.eps) {  // J^T G with J = (I - u u^T) / r
    const double ug = ux * gx + uy * gy + uz * gz;
    gx = (gx - ux * ug) / sr;
    gy = (gy - uy * ug) / sr;
    gz = (gz - uz * ug) / sr;
  } else {  // u = v / eps: J = I / eps
    gx /= sr;
    gy /= sr;
    gz /= sr;
  }
  p.out[3 * e] = In(a * ux + gx);
  p.out[3 * e + 1] = In(a * uy + gy);
  p.out[3 * e + 2] = In(a * uz + gz);
}

template <int LMAX, typename In, typename G>
int launch_lmax(const GradParams<In, G>& p, hipStream_t s) {
  const int64_t blocks = (p.E + 63) / 64;
  if constexpr (LMAX == 3) {
    if (!p.species && p.mix && p.feats && p.C == 16 && p.nr <= 9) {
      hipLaunchKernelGGL((density_edge_gradient_kernel<3, 9, true, In, G>), dim3(unsigned(blocks)), dim3(64), 0, s, p);
      return check_launch("density_edge_gradient_kernel");
    }
  }
  hipLaunchKernelGGL((density_edge_gradient_kernel<LMAX, kGradMaxRadial, false, In, G>), dim3(unsigned(blocks)),
                     dim3(64), 0, s, p);
  return check_launch("density_edge_gradient_kernel");
}

template <typename In, typename G>
int launch(const GradParams<In, G>& p, int lmax, hipStream_t s) {
  switch (lmax) {
    case 0: return launch_lmax<0>(p, s);
    case 1: return launch_lmax<1>(p, s);
    case 2: return launch_lmax<2>(p, s);
    case 3: return launch_lmax<3>(p, s);
    case 4: return launch_lmax<4>(p, s);
    case 5: return launch_lmax<5>(p, s);
    case 6: return launch_lmax<6>(p, s);
    case 7: return launch_lmax<7>(p, s);
    case 8: return launch_lmax<8>(p, s);
    default: return set_error(YE3T_EUNSUPPORTED, "l_max %d > 8", lmax);
  }
}

template <typename In, typename G>
int run(const ye3t_density_args* a, const void* gA, void* grad, hipStream_t s) {
  GradParams<In, G> p;
  p.vec = static_cast<const In*>(a->edge_vectors);
  p.row_offsets = a->row_offsets;
  p.neighbors = a->neighbors;
  p.species = a->species;
  p.feats = static_cast<const In*>(a->node_features);
  p.mix = static_cast<const In*>(a->radial_mix);
  p.gA = static_cast<const G*>(gA);
  p.out = static_cast<In*>(grad);
  p.N = a->atom_count;
  p.E = a->edge_count;
  p.C = int(a->channel_count);
  p.nr = int(a->max_radial_index + 1);
  p.rows = a->radial_mix ? 1 : p.nr;
  p.cutoff = a->cutoff;
  p.lambda = a->lambda;
  p.eps = a->epsilon;
  p.nt = norm_table();
  return launch<In, G>(p, int(a->max_angular), s);
}

}  // namespace
}  // namespace ye3t

using namespace ye3t;

extern "C" int ye3t_hip_ace_density_edge_gradient(const ye3t_density_args* a, int adjoint_dtype,
                                                  const void* density_adjoint, void* edge_gradient,
                                                  ye3t_stream_t stream) {
  clear_error();
  YE3T_REQUIRE(a != nullptr, "NULL arguments");
  YE3T_REQUIRE(a->atom_count >= 0 && a->edge_count >= 0, "negative size");
  if (a->edge_count == 0) return YE3T_OK;
  YE3T_REQUIRE(a->atom_count > 0, "edges without atoms");
  YE3T_REQUIRE(a->row_offsets && a->edge_vectors && density_adjoint && edge_gradient, "NULL input or output");
  YE3T_REQUIRE(a->channel_count >= 1, "channel_count must be positive");
  YE3T_REQUIRE(a->max_radial_index >= 0 && a->max_radial_index + 1 <= kGradMaxRadial, "n_max must be in [0, %d]",
               kGradMaxRadial - 1);
  YE3T_REQUIRE(a->max_angular >= 0 && a->max_angular <= 8, "l_max must be in [0, 8]");
  YE3T_REQUIRE(!(a->species && a->node_features), "species and node_features are exclusive");
  YE3T_REQUIRE((a->species || a->node_features) || a->channel_count == 1,
               "channel_count > 1 needs species or node_features");
  YE3T_REQUIRE(!(a->species || a->node_features) || a->neighbors, "species or node_features need neighbors");
  YE3T_REQUIRE((a->edge_count + 63) / 64 <= int64_t(0x7FFFFFFF), "too many edges for one launch");
  const hipStream_t s = as_stream(stream);
  if (a->dtype == YE3T_F64 && adjoint_dtype == YE3T_F64) return run<double, double>(a, density_adjoint,
                                                                                    edge_gradient, s);
  if (a->dtype == YE3T_F32 && adjoint_dtype == YE3T_F32) return run<float, float>(a, density_adjoint,
                                                                                  edge_gradient, s);
  if (a->dtype == YE3T_F32 && adjoint_dtype == YE3T_F64) return run<float, double>(a, density_adjoint,
                                                                                   edge_gradient, s);
  return set_error(YE3T_EDTYPE, "unsupported dtypes (edge vectors %d, adjoint %d)", a->dtype, adjoint_dtype);
}
