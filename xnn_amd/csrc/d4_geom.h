// Geometry and constants shared by the dispersion kernels (d4.hip, d4_tiles.hip): the
// structure's lattice with its inverse and interplanar spacings, the per-pair image window,
// the Casimir-Polder quadrature weights and the parameter blocks of the CN and pair terms.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstdint>

namespace xnn {

constexpr int kNW = 23;  // Casimir-Polder frequencies
constexpr double kBohr = 0.5291772109044924;
constexpr double kInvBohr = 1.0 / kBohr;
constexpr double kSqrtPi = 1.7724538509055160273;
constexpr double kInvSqrtPi = 1.0 / kSqrtPi;

// The Casimir-Polder frequency grid (hartree, d4.py:130-141) and its trapezoid weights
// times 3 / pi, folded by the compiler: (3 / pi) * (w[k+1] - w[k-1]) / 2, one-sided at the ends.
constexpr double kCpFreq[kNW] = {0.000001, 0.05, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9,
                                 1.0,      1.2,  1.4, 1.6, 1.8, 2.0, 2.5, 3.0, 4.0, 5.0, 7.5,
                                 10.0};
constexpr double cp3_weight(int k) {
  return (3.0 / M_PI) * 0.5 *
         ((k > 0 ? kCpFreq[k] - kCpFreq[k - 1] : 0.0) +
          (k < kNW - 1 ? kCpFreq[k + 1] - kCpFreq[k] : 0.0));
}

// coordination-number terms: cutoffs in bohr, the erf steepness kcn and the EN factor
// k4 exp(-(|dEN| + k5)^2 / k6) (d4.py:552-591)
struct CnParams {
  double cut_cn, cut_eeq, kcn, k4, k5, k6;
};

// two-body terms: s6, s8, BJ a1, a2; cutoff and switch width in bohr (d4.py:1044-1071)
struct PairParams {
  double s6, s8, a1, a2, cutoff, width;
};

// Structure geometry: cell rows (Angstrom), image counts per axis, and the columns of the
// inverse cell scaled to interplanar spacings (for image pruning).
struct Lattice {
  double a[9];
  double ab[9];    // cell rows in bohr
  double inv[9];   // inverse cell, f = d @ inv
  double sp[3];    // interplanar spacing per axis, 1 / |inv[:, axis]|
  int n0, n1, n2;
};

__device__ inline void lattice_inverse(Lattice& L) {
  const double* a = L.a;
  const double c00 = a[4] * a[8] - a[5] * a[7], c01 = a[2] * a[7] - a[1] * a[8],
               c02 = a[1] * a[5] - a[2] * a[4];
  const double det = a[0] * c00 + a[3] * c01 + a[6] * c02;
  if (fabs(det) < 1e-300) {
#pragma unroll
    for (int k = 0; k < 9; ++k) L.inv[k] = 0.0;
    L.sp[0] = L.sp[1] = L.sp[2] = 1e300;
    return;
  }
  const double id = 1.0 / det;
  L.inv[0] = c00 * id;
  L.inv[1] = c01 * id;
  L.inv[2] = c02 * id;
  L.inv[3] = (a[5] * a[6] - a[3] * a[8]) * id;
  L.inv[4] = (a[0] * a[8] - a[2] * a[6]) * id;
  L.inv[5] = (a[2] * a[3] - a[0] * a[5]) * id;
  L.inv[6] = (a[3] * a[7] - a[4] * a[6]) * id;
  L.inv[7] = (a[1] * a[6] - a[0] * a[7]) * id;
  L.inv[8] = (a[0] * a[4] - a[1] * a[3]) * id;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const double n2 = L.inv[c] * L.inv[c] + L.inv[3 + c] * L.inv[3 + c] + L.inv[6 + c] * L.inv[6 + c];
    L.sp[c] = n2 > 0.0 ? 1.0 / sqrt(n2) : 1e300;
  }
}

__device__ inline void load_lattice(const double* __restrict__ cell,
                                    const int32_t* __restrict__ images, int64_t b, Lattice& L) {
  if (cell == nullptr) {
#pragma unroll
    for (int k = 0; k < 9; ++k) L.a[k] = L.ab[k] = L.inv[k] = 0.0;
    L.sp[0] = L.sp[1] = L.sp[2] = 1e300;
    L.n0 = L.n1 = L.n2 = 0;
    return;
  }
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    L.a[k] = cell[9 * b + k];
    L.ab[k] = L.a[k] * kInvBohr;
  }
  L.n0 = images[3 * b + 0];
  L.n1 = images[3 * b + 1];
  L.n2 = images[3 * b + 2];
  lattice_inverse(L);
}

// Images n_c in [lo_c, hi_c] per axis that can lie within rc (Angstrom) of d: the
// fractional component f_c + n_c of d + n @ cell bounds its length from below by
// |f_c + n_c| sp_c, so other images are farther than rc (a small slack keeps the
// bound conservative under rounding). Returned as six scalars (an indexed array here
// lands in scratch memory, one store and one load per pair).
struct ImageRange {
  int lo0, hi0, lo1, hi1, lo2, hi2;
};

__device__ inline void axis_range(int nmax, double f, double w, int& lo, int& hi) {
  if (nmax == 0) {
    lo = hi = 0;
    return;
  }
  const double m = (double)nmax;
  lo = (int)fmax(ceil(-w - f), -m);  // clamped as doubles, then converted
  hi = (int)fmin(floor(w - f), m);
}

__device__ inline ImageRange image_window(const Lattice& L, double dx, double dy, double dz,
                                          double rc) {
  ImageRange r;
  axis_range(L.n0, dx * L.inv[0] + dy * L.inv[3] + dz * L.inv[6], rc / L.sp[0] + 1e-9, r.lo0,
             r.hi0);
  axis_range(L.n1, dx * L.inv[1] + dy * L.inv[4] + dz * L.inv[7], rc / L.sp[1] + 1e-9, r.lo1,
             r.hi1);
  axis_range(L.n2, dx * L.inv[2] + dy * L.inv[5] + dz * L.inv[8], rc / L.sp[2] + 1e-9, r.lo2,
             r.hi2);
  return r;
}

// bytes of workspace the D4 tile kernels need (d4_tiles.hip)
size_t d4_tiles_workspace_bytes(int64_t n_nodes, int64_t n_graphs, int64_t max_atoms);

}  // namespace xnn
