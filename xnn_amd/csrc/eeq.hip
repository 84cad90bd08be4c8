// The real-space part of the large-system EEQ operator (gfx950, float64).
//
// The large regime of the EEQ charges (common/models/eeq.py:170-397, the operator of
// eeq_charges_large, eeq.py:664) splits the Coulomb interaction of the charge
// distributions with an Ewald parameter alpha: the screened kernel
//   K_ij(r) = [erf(gamma_ij r) - erf(alpha r)] / r,  gamma_ij = (a_i^2 + a_j^2)^(-1/2),
// summed over every lattice image within the real-space cutoff (an atom's own images
// included, r > 0), and a reciprocal sum that the host forms from structure factors.
// A molecule takes alpha = 0 and the single image: K = erf(gamma r) / r.
//
// xnn_eeq_real_matrix forms R_ij = sum_n K_ij(|pos_j + n cell - pos_i|) as a dense (N, N)
// float64 matrix (symmetric): one thread per (i, j), the images of the pair in a window
// taken from its fractional coordinates and the cell's interplanar spacings (every image
// within the cutoff lies in it). With 288 GB of HBM the dense matrix is the MI355X form up
// to ~10^5 atoms: it is formed once per evaluation and factorized on the device.
//
// xnn_eeq_real_grad forms the derivatives of S = sum_ij u_i R_ij(pos, cell) w_j: with
// d = pos_j + n cell - pos_i and K' = dK/dr,
//   dS/dpos_k = -sum_{j,n} (u_k w_j + u_j w_k) K'(r) d / r,
//   dS/dcell = sum_k sum_{j,n} u_k w_j K'(r) n (x) d / r   (per-atom rows, summed by the caller),
// one wave per atom k, lanes over j, a fixed butterfly: bitwise reproducible.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "common.h"
#include "device.h"
#include "fp64.h"

namespace xnn {

struct EeqCell {
  double a[9];    // rows, bohr
  double inv[9];  // inverse, f = d @ inv
  double reach[3];  // cutoff / interplanar spacing per axis (0: not periodic)
  int periodic;
};

// the window of image offsets n_a for fractional difference f_a: |f_a + n_a| <= reach_a
__device__ inline void image_range(double f, double reach, int& lo, int& hi) {
  lo = (int)ceil(-reach - f);
  hi = (int)floor(reach - f);
}

// erf(gam r) - erf(alpha r) is evaluated as erfc(alpha r) - erfc(gam r), without the
// cancellation of two values near one; erfc(gam r) < 4e-20 for gam r >= 6.5, where it is
// dropped (most pairs of a long real-space range: one error function instead of two).
__device__ inline double screened(double r, double gam, double alpha) {
  if (alpha > 0.0) {
    const double x = gam * r;
    return (erfc(alpha * r) - (x < 6.5 ? erfc(x) : 0.0)) / r;
  }
  return erf(gam * r) / r;
}

// the same from r^2 and 1 / r
__device__ inline double screened_inv(double r2, double ir, double gam, double alpha) {
  const double r = r2 * ir;
  if (alpha > 0.0) {
    const double x = gam * r;
    return (erfc(alpha * r) - (x < 6.5 ? erfc(x) : 0.0)) * ir;
  }
  return erf(gam * r) * ir;
}

// dK/dr of the screened kernel
__device__ inline double screened_slope(double r, double gam, double alpha, double K) {
  constexpr double two_over_sqrt_pi = 1.1283791670955126;
  double g = gam * exp(-gam * gam * r * r);
  if (alpha > 0.0) g -= alpha * exp(-alpha * alpha * r * r);
  return (two_over_sqrt_pi * g - K) / r;
}

// calls fn(dx, dy, dz, n0, n1, n2) for every image n of a pair within distance^2 cut2,
// given the fractional difference f of its two atoms and the per-axis window reach (the
// image offsets with |f_a + n_a| <= reach_a hold every image within the range): f is
// wrapped to [-1/2, 1/2] first and the wrap folded into n. The zero vector (an atom and
// itself) is skipped.
template <typename Fn>
__device__ inline void for_images_frac(const EeqCell& C, const double* reach, double f0,
                                       double f1, double f2, double cut2, Fn&& fn) {
  double f[3] = {f0, f1, f2};
  int w[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    w[c] = (int)rint(f[c]);
    f[c] -= w[c];
  }
  int lo[3], hi[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) image_range(f[c], reach[c], lo[c], hi[c]);
  for (int n0 = lo[0]; n0 <= hi[0]; ++n0)
    for (int n1 = lo[1]; n1 <= hi[1]; ++n1)
      for (int n2 = lo[2]; n2 <= hi[2]; ++n2) {
        const double g0 = f[0] + n0, g1 = f[1] + n1, g2 = f[2] + n2;
        const double dx = g0 * C.a[0] + g1 * C.a[3] + g2 * C.a[6];
        const double dy = g0 * C.a[1] + g1 * C.a[4] + g2 * C.a[7];
        const double dz = g0 * C.a[2] + g1 * C.a[5] + g2 * C.a[8];
        const double r2 = dx * dx + dy * dy + dz * dz;
        if (r2 <= cut2 && r2 > 1e-20) fn(dx, dy, dz, n0 - w[0], n1 - w[1], n2 - w[2]);
      }
}

__device__ inline void to_frac(const EeqCell& C, double dx, double dy, double dz, double* f) {
#pragma unroll
  for (int c = 0; c < 3; ++c) f[c] = dx * C.inv[c] + dy * C.inv[3 + c] + dz * C.inv[6 + c];
}

// calls fn(dx, dy, dz, n0, n1, n2) for every image of the pair (i -> j) within the cutoff
template <typename Fn>
__device__ inline void for_images(const EeqCell& C, double dx0, double dy0, double dz0,
                                  double cut2, bool same, Fn&& fn) {
  if (!C.periodic) {
    const double r2 = dx0 * dx0 + dy0 * dy0 + dz0 * dz0;
    if (!same && r2 <= cut2) fn(dx0, dy0, dz0, 0, 0, 0);
    return;
  }
  double f[3];
  to_frac(C, dx0, dy0, dz0, f);
  for_images_frac(C, C.reach, f[0], f[1], f[2], cut2, fn);
}

// 16 x 16 tiles of the lower block triangle (the upper tiles return at once): each entry
// summed over its images, a tile below the diagonal also stored transposed through LDS, so
// the matrix is symmetric to the bit and half of its entries are summed.
__global__ __launch_bounds__(256) void eeq_real_matrix_kernel(
    const double* __restrict__ pos, int64_t n, EeqCell C, const double* __restrict__ rad,
    double alpha, double cut2, double* __restrict__ R) {
  __shared__ double tile[16][17];
  if (blockIdx.x > blockIdx.y) return;            // uniform: mirrored from below
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int64_t j = (int64_t)blockIdx.x * 16 + tx;
  const int64_t i = (int64_t)blockIdx.y * 16 + ty;
  double sum = 0.0;
  if (i < n && j < n) {
    const double ai = rad[i], aj = rad[j];
    const double gam = 1.0 / sqrt(ai * ai + aj * aj);
    for_images(C, pos[3 * j] - pos[3 * i], pos[3 * j + 1] - pos[3 * i + 1],
               pos[3 * j + 2] - pos[3 * i + 2], cut2, i == j,
               [&](double dx, double dy, double dz, int, int, int) {
                 sum += screened(sqrt(dx * dx + dy * dy + dz * dz), gam, alpha);
               });
    R[i * n + j] = sum;
  }
  if (blockIdx.x == blockIdx.y) return;           // uniform: a diagonal tile is whole
  tile[ty][tx] = sum;
  __syncthreads();
  const int64_t it = (int64_t)blockIdx.x * 16 + ty, jt = (int64_t)blockIdx.y * 16 + tx;
  if (it < n && jt < n) R[it * n + jt] = tile[tx][ty];
}

__global__ __launch_bounds__(256) void eeq_real_grad_kernel(
    const double* __restrict__ pos, int64_t n, EeqCell C, const double* __restrict__ rad,
    double alpha, double cut2, const double* __restrict__ u, const double* __restrict__ w,
    double* __restrict__ grad_pos, double* __restrict__ cell_partial) {
  const int lane = threadIdx.x % kWave;
  const int64_t k = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (k >= n) return;
  const double pk0 = pos[3 * k], pk1 = pos[3 * k + 1], pk2 = pos[3 * k + 2];
  const double ak = rad[k], uk = u[k], wk = w[k];
  double g[3] = {0.0, 0.0, 0.0};
  double c[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
  const bool want_cell = cell_partial != nullptr;
  for (int64_t j = lane; j < n; j += kWave) {
    const double aj = rad[j];
    const double gam = 1.0 / sqrt(ak * ak + aj * aj);
    const double sym = uk * w[j] + u[j] * wk, own = uk * w[j];
    for_images(C, pos[3 * j] - pk0, pos[3 * j + 1] - pk1, pos[3 * j + 2] - pk2, cut2, j == k,
               [&](double dx, double dy, double dz, int n0, int n1, int n2) {
                 const double r = sqrt(dx * dx + dy * dy + dz * dz);
                 const double K = screened(r, gam, alpha);
                 const double s = screened_slope(r, gam, alpha, K) / r;
                 g[0] -= sym * s * dx;
                 g[1] -= sym * s * dy;
                 g[2] -= sym * s * dz;
                 if (want_cell) {
                   const double t = own * s;
                   c[0] += t * n0 * dx; c[1] += t * n0 * dy; c[2] += t * n0 * dz;
                   c[3] += t * n1 * dx; c[4] += t * n1 * dy; c[5] += t * n1 * dz;
                   c[6] += t * n2 * dx; c[7] += t * n2 * dy; c[8] += t * n2 * dz;
                 }
               });
  }
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) {
#pragma unroll
    for (int q = 0; q < 3; ++q) g[q] += __shfl_xor(g[q], m, kWave);
    if (want_cell) {
#pragma unroll
      for (int q = 0; q < 9; ++q) c[q] += __shfl_xor(c[q], m, kWave);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < 3; ++q) grad_pos[3 * k + q] = g[q];
    if (want_cell) {
#pragma unroll
      for (int q = 0; q < 9; ++q) cell_partial[9 * k + q] = c[q];
    }
  }
}

// ------------------------------------------------------------------ matrix-free product
// out = R v for one or two right-hand sides (the conjugate-gradient regime): R is never
// stored. Atoms come in tiles of kApplyTile consecutive indices; block (i tile, split)
// takes the i tile, one atom per thread, against the j tiles of its split, staged in LDS
// (fractional coordinates, width, v), and writes its partial sums; the splits are added
// in a fixed order afterwards (bitwise reproducible). With tile bounds (center, radius of
// a sphere holding the tile's atoms, in the coordinates of pos), a j tile is skipped when
// no lattice image of it comes within the cutoff of the i tile: ordered along space (the
// cell list of the caller), most tiles of a large cell are skipped.
constexpr int kApplyTile = 256;
constexpr int kApplyBlocks = 2048;   // target blocks per launch (8 per CU)

__device__ inline bool eeq_tiles_meet(const EeqCell& C, const double* __restrict__ tiles,
                                      int64_t ti, int64_t tj, double cutoff) {
  const double* a = tiles + 4 * ti;
  const double* b = tiles + 4 * tj;
  const double R = cutoff + a[3] + b[3];
  const double dx = b[0] - a[0], dy = b[1] - a[1], dz = b[2] - a[2];
  if (!C.periodic) return dx * dx + dy * dy + dz * dz <= R * R;
  double f[3], reach[3];
  to_frac(C, dx, dy, dz, f);
#pragma unroll
  for (int c = 0; c < 3; ++c) reach[c] = C.reach[c] * (R / cutoff) + 1e-12;
  bool hit = dx * dx + dy * dy + dz * dz <= R * R;   // the zero image, which the walk skips
  for_images_frac(C, reach, f[0], f[1], f[2], R * R,
                  [&](double, double, double, int, int, int) { hit = true; });
  return hit;
}

template <int NRHS>
__global__ __launch_bounds__(kApplyTile) void eeq_real_apply_kernel(
    const double* __restrict__ pos, int64_t n, EeqCell C, const double* __restrict__ rad,
    double alpha, double cutoff, const double* __restrict__ tiles,
    const double* __restrict__ v, int64_t tiles_per_split, double* __restrict__ part) {
  __shared__ double sp[3][kApplyTile], sa[kApplyTile], sv[NRHS][kApplyTile];
  const int64_t ti = blockIdx.x, split = blockIdx.y;
  const int64_t n_tiles = (n + kApplyTile - 1) / kApplyTile;
  const int64_t i = ti * kApplyTile + threadIdx.x;
  const bool vi = i < n;
  const int64_t ic = vi ? i : 0;
  double pi[3];
  if (C.periodic) {
    to_frac(C, pos[3 * ic], pos[3 * ic + 1], pos[3 * ic + 2], pi);
  } else {
#pragma unroll
    for (int c = 0; c < 3; ++c) pi[c] = pos[3 * ic + c];
  }
  const double ai2 = rad[ic] * rad[ic];
  const double cut2 = cutoff * cutoff;
  double acc[NRHS];
#pragma unroll
  for (int r = 0; r < NRHS; ++r) acc[r] = 0.0;
  const int64_t t0 = split * tiles_per_split;
  const int64_t t1 = t0 + tiles_per_split < n_tiles ? t0 + tiles_per_split : n_tiles;
  for (int64_t tj = t0; tj < t1; ++tj) {
    if (tiles != nullptr && !eeq_tiles_meet(C, tiles, ti, tj, cutoff)) continue;  // uniform
    const int64_t j0 = tj * kApplyTile;
    const int cnt = (int)(n - j0 < kApplyTile ? n - j0 : kApplyTile);
    __syncthreads();
    if ((int)threadIdx.x < cnt) {
      const int64_t j = j0 + threadIdx.x;
      double pj[3];
      if (C.periodic) {
        to_frac(C, pos[3 * j], pos[3 * j + 1], pos[3 * j + 2], pj);
      } else {
#pragma unroll
        for (int c = 0; c < 3; ++c) pj[c] = pos[3 * j + c];
      }
#pragma unroll
      for (int c = 0; c < 3; ++c) sp[c][threadIdx.x] = pj[c];
      sa[threadIdx.x] = rad[j] * rad[j];
#pragma unroll
      for (int r = 0; r < NRHS; ++r) sv[r][threadIdx.x] = v[j * NRHS + r];
    }
    __syncthreads();
    if (!vi) continue;
    for (int q = 0; q < cnt; ++q) {
      // refined hardware reciprocal square roots (about an ulp) instead of the IEEE square
      // roots and divisions: the kernel value only needs float64 accuracy, not rounding
      const double gam = rsq_nr(ai2 + sa[q]);
      double k = 0.0;
      const auto add = [&](double dx, double dy, double dz, int, int, int) {
        const double r2 = dx * dx + dy * dy + dz * dz;
        k += screened_inv(r2, rsq_nr(r2), gam, alpha);
      };
      if (C.periodic) {
        for_images_frac(C, C.reach, sp[0][q] - pi[0], sp[1][q] - pi[1], sp[2][q] - pi[2], cut2,
                        add);
      } else if (j0 + q != i) {
        const double dx = sp[0][q] - pi[0], dy = sp[1][q] - pi[1], dz = sp[2][q] - pi[2];
        if (dx * dx + dy * dy + dz * dz <= cut2) add(dx, dy, dz, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < NRHS; ++r) acc[r] = fma(k, sv[r][q], acc[r]);
    }
  }
  if (vi) {
#pragma unroll
    for (int r = 0; r < NRHS; ++r) part[(split * n + i) * NRHS + r] = acc[r];
  }
}

// out[k] = sum over the splits of part[s][k], in split order
__global__ __launch_bounds__(256) void eeq_sum_splits_kernel(const double* __restrict__ part,
                                                             int64_t splits, int64_t m,
                                                             double* __restrict__ out) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= m) return;
  double s = 0.0;
  for (int64_t q = 0; q < splits; ++q) s += part[q * m + k];
  out[k] = s;
}

static int64_t eeq_apply_splits(int64_t n) {
  const int64_t tiles = (n + kApplyTile - 1) / kApplyTile;
  if (tiles == 0) return 1;
  const int64_t want = (kApplyBlocks + tiles - 1) / tiles;
  return std::max<int64_t>(1, std::min<int64_t>(want, tiles));
}

// host: the cell's inverse and per-axis reach; false for a singular cell
static bool eeq_cell(const double* cell, double cutoff, EeqCell& C) {
  C.periodic = cell != nullptr;
  for (int q = 0; q < 9; ++q) {
    C.a[q] = cell ? cell[q] : 0.0;
    C.inv[q] = 0.0;
  }
  C.reach[0] = C.reach[1] = C.reach[2] = 0.0;
  if (!C.periodic) return true;
  const double* a = C.a;
  const double c00 = a[4] * a[8] - a[5] * a[7], c01 = a[2] * a[7] - a[1] * a[8],
               c02 = a[1] * a[5] - a[2] * a[4];
  const double det = a[0] * c00 + a[3] * c01 + a[6] * c02;
  if (!(std::fabs(det) > 1e-12)) return false;
  const double id = 1.0 / det;
  C.inv[0] = c00 * id;
  C.inv[1] = c01 * id;
  C.inv[2] = c02 * id;
  C.inv[3] = (a[5] * a[6] - a[3] * a[8]) * id;
  C.inv[4] = (a[0] * a[8] - a[2] * a[6]) * id;
  C.inv[5] = (a[2] * a[3] - a[0] * a[5]) * id;
  C.inv[6] = (a[3] * a[7] - a[4] * a[6]) * id;
  C.inv[7] = (a[1] * a[6] - a[0] * a[7]) * id;
  C.inv[8] = (a[0] * a[4] - a[1] * a[3]) * id;
  // interplanar spacing of axis c: 1 / |column c of the inverse|; a little slack so that
  // rounding never drops an image at the cutoff (the r test decides)
  for (int col = 0; col < 3; ++col) {
    const double x = C.inv[col], y = C.inv[3 + col], z = C.inv[6 + col];
    C.reach[col] = cutoff * std::sqrt(x * x + y * y + z * z) * (1.0 + 1e-12) + 1e-12;
  }
  return true;
}

// the image windows stay bounded: at most kMaxReach cell lengths along any axis
constexpr double kMaxReach = 32.0;
static bool eeq_reach_ok(const EeqCell& C, double cutoff) {
  if (!C.periodic) return true;
  if (!std::isfinite(cutoff)) return false;
  return C.reach[0] <= kMaxReach && C.reach[1] <= kMaxReach && C.reach[2] <= kMaxReach;
}


// One diagonal block of the blocked Cholesky factorization of the (symmetric positive
// definite) operator, in place: rows and columns k0 .. k0+b of the row-major matrix a
// (leading dimension lda), whose trailing updates the host has applied. One workgroup of
// 512 threads; thread (ty, tx) holds the 32 elements (ty + 16 p, tx + 32 q) in registers,
// of the block and of E, which starts as the identity.
//
// Elimination with unscaled columns: column j's pivot d_j = a_jj, a_ic -= a_ij a_cj / d_j
// for j < c <= i, and the same row operations on E, row i -= (a_ij / d_j) row j for i > j.
// Afterwards L_ij = a_ij / sqrt(d_j) and E is the inverse of the unit lower factor, so
// L^-1 = diag(d)^(-1/2) E. A step eliminates two columns: it reads columns j and j + 1 of
// the block and rows j and j + 1 of E as their owners published them to LDS at the end of
// the step before (two buffers, one barrier per step), column j + 1 and row j + 1 not yet
// reduced by column j; every thread applies that reduction itself, g = a_{j+1,j} / d_j:
// y1_i = a_{i,j+1} - a_ij g, d_{j+1} = a_{j+1,j+1} - a_{j+1,j} g, E row j+1 -= g E row j.
// Written: L (lower; the block's upper triangle zeroed) and inv = L^-1 (b, b) row-major,
// which the host multiplies into the panel below the block. A pivot that is not positive
// and finite stores k0 + j + 1 into *info if it still holds 0 and leaves the block
// unwritten. Entries of the block outside rows and columns < b stay zero throughout.
constexpr int kCholBlock = 128;
constexpr int kCholThreads = 512;
constexpr int kCholP = kCholBlock / (kCholThreads / 32);  // row groups of 16
constexpr int kCholQ = kCholBlock / 32;                   // column groups of 32
static_assert(kCholP == 8 && kCholQ == 4, "the pivot publish switches list 8 and 4 groups");

// 1 / d for a positive normal d: the hardware estimate refined by two Newton steps
// r <- r + r (1 - d r) (each squares the relative error), on the barrier-bound path of the
// column steps where the full division sequence costs a large part of a step.
__device__ inline double refined_rcp(double d) {
  double r = __builtin_amdgcn_rcp(d);
  r = fma(r, fma(-d, r, 1.0), r);
  return fma(r, fma(-d, r, 1.0), r);
}

__global__ __launch_bounds__(kCholThreads) void eeq_cholesky_block_kernel(
    double* __restrict__ a, int64_t lda, int64_t k0, int b, double* __restrict__ inv,
    int* __restrict__ info) {
  __shared__ double col_buf[2][2][kCholBlock];  // columns j, j + 1 of the block
  __shared__ double row_buf[2][2][kCholBlock];  // rows j, j + 1 of E
  __shared__ double piv[kCholBlock];
  const int t = threadIdx.x, tx = t & 31, ty = t >> 5;
  double* blk = a + k0 * lda + k0;
  double v[kCholP][kCholQ], e[kCholP][kCholQ];
#pragma unroll
  for (int p = 0; p < kCholP; ++p)
#pragma unroll
    for (int q = 0; q < kCholQ; ++q) {
      const int i = ty + 16 * p, c = tx + 32 * q;
      v[p][q] = (i < b && c <= i) ? blk[i * lda + c] : 0.0;
      e[p][q] = i == c ? 1.0 : 0.0;
    }
  for (int k = t; k < 4 * kCholBlock; k += kCholThreads) {
    (&col_buf[0][0][0])[k] = 0.0;
    (&row_buf[0][0][0])[k] = 0.0;
  }
  __syncthreads();
  if (tx < 2)
#pragma unroll
    for (int p = 0; p < kCholP; ++p) col_buf[0][tx][ty + 16 * p] = v[p][0];
  if (ty < 2)
#pragma unroll
    for (int q = 0; q < kCholQ; ++q) row_buf[0][ty][tx + 32 * q] = e[0][q];
  for (int j = 0, step = 0; j < b; j += 2, ++step) {
    __syncthreads();
    const double* c0 = col_buf[step & 1][0];
    const double* c1 = col_buf[step & 1][1];
    const double* r0w = row_buf[step & 1][0];
    const double* r1w = row_buf[step & 1][1];
    const double d0 = c0[j], x = c0[j + 1], e1 = c1[j + 1];
    double l0[kCholP], l1[kCholP], m0[kCholQ], m1[kCholQ], w0[kCholQ], w1[kCholQ];
#pragma unroll
    for (int p = 0; p < kCholP; ++p) {
      l0[p] = c0[ty + 16 * p];
      l1[p] = c1[ty + 16 * p];
    }
#pragma unroll
    for (int q = 0; q < kCholQ; ++q) {
      m0[q] = c0[tx + 32 * q];
      m1[q] = c1[tx + 32 * q];
      w0[q] = r0w[tx + 32 * q];
      w1[q] = r1w[tx + 32 * q];
    }
    const bool pair = j + 1 < b;
    const double r0 = refined_rcp(d0);
    const double g = x * r0;
    const double d1 = e1 - x * g;
    const double r1 = pair ? refined_rcp(d1) : 0.0;
    // Columns c <= j (c <= j + 1 for the second) take zero factors and rows i <= j
    // (i <= j + 1) zero multipliers: exact no-ops. Rows and columns past the block's
    // diagonal hold values that are never read again, and E's rows vanish right of their
    // index, so the updates run unmasked over the row groups that reach below j (uniform
    // branches) and the column groups left of the diagonal.
#pragma unroll
    for (int q = 0; q < kCholQ; ++q) {
      const int c = tx + 32 * q;
      const double y1 = m1[q] - m0[q] * g;
      m0[q] = c > j ? m0[q] * r0 : 0.0;
      m1[q] = c > j + 1 ? y1 * r1 : 0.0;
      w1[q] -= g * w0[q];
    }
#pragma unroll
    for (int p = 0; p < kCholP; ++p) {
      if (16 * p + 15 <= j) continue;
      const int i = ty + 16 * p;
      const double y0 = l0[p], y1 = l1[p] - l0[p] * g;
      const double f0 = i > j ? y0 * r0 : 0.0;
      const double f1 = i > j + 1 ? y1 * r1 : 0.0;
#pragma unroll
      for (int q = 0; q <= (p >> 1); ++q) {
        v[p][q] -= y0 * m0[q] + y1 * m1[q];
        e[p][q] -= f0 * w0[q] + f1 * w1[q];
      }
    }
    // uniform: every thread read the same pivots
    const bool bad0 = !(d0 > 0.0 && d0 < INFINITY), bad1 = pair && !(d1 > 0.0 && d1 < INFINITY);
    if (bad0 || bad1) {
      if (t == 0 && *info == 0) *info = (int)(k0 + j + (bad0 ? 1 : 2));
      return;
    }
    if (t == 0) {
      piv[j] = d0;
      if (pair) piv[j + 1] = d1;
    }
    const int jn = j + 2;
    if (jn < b) {
      const int nb = (step + 1) & 1;
      // jn is even, so columns jn and jn + 1 lie in one register column group and E rows jn
      // and jn + 1 in one row group: a uniform switch picks the registers, two lanes of each
      // 32 write the columns and two thread rows the E rows. The columns' rows above jn go
      // out too: every later update takes them with zero column factors.
      const int qs = __builtin_amdgcn_readfirstlane(jn >> 5);
      const int ps = __builtin_amdgcn_readfirstlane(jn >> 4);
      double vc[kCholP], er[kCholQ];
      switch (qs) {
#define XNN_CHOL_COL(Q)                                          \
  case Q:                                                        \
    _Pragma("unroll") for (int p = 0; p < kCholP; ++p) vc[p] = v[p][Q]; \
    break;
        XNN_CHOL_COL(0)
        XNN_CHOL_COL(1)
        XNN_CHOL_COL(2)
        default:
#pragma unroll
          for (int p = 0; p < kCholP; ++p) vc[p] = v[p][kCholQ - 1];
      }
#undef XNN_CHOL_COL
      switch (ps) {
#define XNN_CHOL_ROW(P)                                          \
  case P:                                                        \
    _Pragma("unroll") for (int q = 0; q < kCholQ; ++q) er[q] = e[P][q]; \
    break;
        XNN_CHOL_ROW(0)
        XNN_CHOL_ROW(1)
        XNN_CHOL_ROW(2)
        XNN_CHOL_ROW(3)
        XNN_CHOL_ROW(4)
        XNN_CHOL_ROW(5)
        XNN_CHOL_ROW(6)
        default:
#pragma unroll
          for (int q = 0; q < kCholQ; ++q) er[q] = e[kCholP - 1][q];
      }
#undef XNN_CHOL_ROW
      const int hc = tx - (jn & 31), hr = ty - (jn & 15);
      if (hc == 0 || hc == 1) {
#pragma unroll
        for (int p = 0; p < kCholP; ++p) col_buf[nb][hc][ty + 16 * p] = vc[p];
      }
      if (hr == 0 || hr == 1) {
#pragma unroll
        for (int q = 0; q < kCholQ; ++q) row_buf[nb][hr][tx + 32 * q] = er[q];
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < kCholP; ++p) {
    const int i = ty + 16 * p;
    if (i >= b) continue;
    const double rroot = 1.0 / sqrt(piv[i]);
#pragma unroll
    for (int q = 0; q < kCholQ; ++q) {
      const int c = tx + 32 * q;
      if (c >= b) continue;
      double l = 0.0, y = 0.0;
      if (c <= i) {
        const double root = sqrt(piv[c]);
        l = c == i ? root : v[p][q] / root;
        y = e[p][q] * rroot;
      }
      blk[i * lda + c] = l;
      inv[i * b + c] = y;
    }
  }
}

// ---------------------------------------------------------------- solves with the factor
// (L L^T) X = B with L from eeq_cholesky_block_kernel and the inverses of its diagonal
// blocks (block j: rows [128 j, 128 j + b_j), inverse at inv + 128 * 128 j, row stride
// b_j), X (n, NRHS) row-major. Forward L Y = B walks the blocks down, backward L^T X = Y
// up, one launch per block. Launch k: every workgroup solves block k from its residual
// rows with the block's inverse (forward y = inv r, backward x = inv^T r; a 128 x 128
// product, repeated per workgroup rather than waiting for one), workgroup 0 stores it,
// and every row still to come takes away the block's contribution (forward: r_i -= L[i,
// k0:k0 + b_k] y_k, a wave per row over its contiguous entries, 8 rows' loads in flight at
// once; backward: r_i -= L[k0:k0 + b_k, i]^T x_k for i < k0, a thread per row, the block
// row read across threads). The solution goes to another array than the residual rows
// the launch reads (forward: residual in X, solution in the work array; backward the
// reverse), so no workgroup reads a row another one rewrites. Sums in a fixed order.
constexpr int kTrsvBlock = kCholBlock;
constexpr int kTrsvFwdRows = 32;      // rows per workgroup (forward)
constexpr int kTrsvBwdRows = 256;     // rows per workgroup (backward)

__device__ __forceinline__ double wave_sum_xor(double v) {
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// out = inv rb (TRANS: inv^T rb) over one block of size b <= 128 with its lower-triangular
// inverse (row stride b), rb and out in LDS: two threads per entry, each over half of the
// columns (the loads independent of the sums, so they are in flight together), the halves
// added by one exchange.
template <int NRHS, bool TRANS>
__device__ __forceinline__ void trsv_block_inverse(const double* __restrict__ ib, int b,
                                                   const double (*rb)[NRHS],
                                                   double (*out)[NRHS]) {
  const int t = threadIdx.x, i = t >> 1, h = t & 1;
  const int ii = i < b ? i : 0;
  double s[NRHS];
#pragma unroll
  for (int r = 0; r < NRHS; ++r) s[r] = 0.0;
#pragma unroll 16
  for (int q = 0; q < kTrsvBlock / 2; ++q) {
    const int c = h * (kTrsvBlock / 2) + q;
    // forward: inv[i][c], c <= i; backward: inv[c][i], c >= i
    const bool use = c < b && (TRANS ? c >= ii : c <= ii);
    const double l = use ? (TRANS ? ib[(int64_t)c * b + ii] : ib[(int64_t)ii * b + c]) : 0.0;
#pragma unroll
    for (int r = 0; r < NRHS; ++r) s[r] = fma(l, rb[use ? c : 0][r], s[r]);
  }
#pragma unroll
  for (int r = 0; r < NRHS; ++r) s[r] += __shfl_xor(s[r], 1, kWave);
  if (h == 0 && i < b) {
#pragma unroll
    for (int r = 0; r < NRHS; ++r) out[i][r] = s[r];
  }
}

template <int NRHS, bool TRANS>
__global__ __launch_bounds__(256) void eeq_trsv_step_kernel(const double* __restrict__ L,
                                                            int64_t n,
                                                            const double* __restrict__ inv,
                                                            int k, double* __restrict__ res,
                                                            double* __restrict__ sol) {
  __shared__ double rs[kTrsvBlock][NRHS];     // block k's residual
  __shared__ double xs[kTrsvBlock][NRHS];     // its solution
  const int t = threadIdx.x, lane = t & (kWave - 1), wv = t >> 6;
  const int64_t k0 = (int64_t)k * kTrsvBlock;
  const int bk = (int)(n - k0 < kTrsvBlock ? n - k0 : kTrsvBlock);
  for (int i = t; i < bk * NRHS; i += blockDim.x) (&rs[0][0])[i] = res[k0 * NRHS + i];
  __syncthreads();
  trsv_block_inverse<NRHS, TRANS>(inv + (int64_t)k * kTrsvBlock * kTrsvBlock, bk, rs, xs);
  __syncthreads();
  if (blockIdx.x == 0)
    for (int i = t; i < bk * NRHS; i += blockDim.x) sol[k0 * NRHS + i] = (&xs[0][0])[i];
  if (!TRANS) {
    // rows after the block, kTrsvFwdRows per workgroup; a wave takes 8 rows at a time
    constexpr int kBatch = 8;
    const int64_t r0 = k0 + bk + (int64_t)blockIdx.x * kTrsvFwdRows;
    const int64_t r1 = r0 + kTrsvFwdRows < n ? r0 + kTrsvFwdRows : n;
    const int ca = lane < bk ? lane : 0, cb = lane + kWave < bk ? lane + kWave : 0;
    for (int64_t base = r0 + (int64_t)wv * kBatch; base < r1;
         base += (int64_t)(blockDim.x / kWave) * kBatch) {
      double v0[kBatch], v1[kBatch], old[kBatch][NRHS];
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int64_t i = base + q;
        const bool ok = i < r1;
        const double* row = L + (ok ? i : k0) * n + k0;
        v0[q] = ok && lane < bk ? row[lane] : 0.0;
        v1[q] = ok && lane + kWave < bk ? row[lane + kWave] : 0.0;
#pragma unroll
        for (int r = 0; r < NRHS; ++r) old[q][r] = ok ? res[i * NRHS + r] : 0.0;
      }
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int64_t i = base + q;
        if (i >= r1) break;                       // uniform in the wave
#pragma unroll
        for (int r = 0; r < NRHS; ++r) {
          const double sr = wave_sum_xor(fma(v0[q], xs[ca][r], v1[q] * xs[cb][r]));
          if (lane == 0) res[i * NRHS + r] = old[q][r] - sr;
        }
      }
    }
  } else {
    // rows before the block, kTrsvBwdRows per workgroup, a thread per row
    const int64_t r0 = (int64_t)blockIdx.x * kTrsvBwdRows;
    const int64_t r1 = r0 + kTrsvBwdRows < k0 ? r0 + kTrsvBwdRows : k0;
    for (int64_t i = r0 + t; i < r1; i += blockDim.x) {
      double s[NRHS], old[NRHS];
#pragma unroll
      for (int r = 0; r < NRHS; ++r) {
        s[r] = 0.0;
        old[r] = res[i * NRHS + r];
      }
#pragma unroll 16
      for (int c = 0; c < kTrsvBlock; ++c) {
        const bool use = c < bk;
        const double l = use ? L[(k0 + c) * n + i] : 0.0;
#pragma unroll
        for (int r = 0; r < NRHS; ++r) s[r] = fma(l, xs[use ? c : 0][r], s[r]);
      }
#pragma unroll
      for (int r = 0; r < NRHS; ++r) res[i * NRHS + r] = old[r] - s[r];
    }
  }
}

}  // namespace xnn

using namespace xnn;

extern "C" {

int xnn_eeq_real_matrix(const double* pos, int64_t n_nodes, const double* cell,
                        const double* rad, double alpha, double cutoff, double* matrix,
                        xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0, "negative size");
  if (n_nodes == 0) return XNN_OK;
  XNN_REQUIRE(pos && rad && matrix, "NULL input or output");
  XNN_REQUIRE(n_nodes <= (int64_t(1) << 20), "at most 2^20 atoms");
  XNN_REQUIRE(cutoff > 0.0 && alpha >= 0.0, "cutoff must be positive, alpha non-negative");
  XNN_REQUIRE(cell != nullptr || alpha == 0.0, "a molecule takes alpha = 0");
  EeqCell C;
  XNN_REQUIRE(eeq_cell(cell, cutoff, C), "singular cell");
  XNN_REQUIRE(eeq_reach_ok(C, cutoff), "the real-space range spans more than %g cells",
              kMaxReach);
  const dim3 grid((unsigned)((n_nodes + 15) / 16), (unsigned)((n_nodes + 15) / 16));
  hipLaunchKernelGGL(eeq_real_matrix_kernel, grid, dim3(256), 0, as_hip(stream), pos, n_nodes, C,
                     rad, alpha, cutoff * cutoff, matrix);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_eeq_real_grad(const double* pos, int64_t n_nodes, const double* cell, const double* rad,
                      double alpha, double cutoff, const double* u, const double* w,
                      double* grad_pos, double* cell_partial, xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0, "negative size");
  if (n_nodes == 0) return XNN_OK;
  XNN_REQUIRE(pos && rad && u && w && grad_pos, "NULL input or output");
  XNN_REQUIRE(cutoff > 0.0 && alpha >= 0.0, "cutoff must be positive, alpha non-negative");
  XNN_REQUIRE(cell != nullptr || (alpha == 0.0 && cell_partial == nullptr),
              "a molecule takes alpha = 0 and has no cell gradient");
  EeqCell C;
  XNN_REQUIRE(eeq_cell(cell, cutoff, C), "singular cell");
  XNN_REQUIRE(eeq_reach_ok(C, cutoff), "the real-space range spans more than %g cells",
              kMaxReach);
  hipLaunchKernelGGL(eeq_real_grad_kernel, dim3((unsigned)grid_1d(n_nodes, 4)), dim3(256), 0,
                     as_hip(stream), pos, n_nodes, C, rad, alpha, cutoff * cutoff, u, w, grad_pos,
                     cell_partial);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_eeq_real_apply_work_size(int64_t n_nodes, int32_t nrhs, size_t* bytes) {
  XNN_REQUIRE(n_nodes >= 0 && bytes != nullptr, "negative size or NULL output");
  XNN_REQUIRE(nrhs == 1 || nrhs == 2, "one or two right-hand sides (got %d)", (int)nrhs);
  *bytes = sizeof(double) * (size_t)std::max<int64_t>(eeq_apply_splits(n_nodes) * n_nodes * nrhs, 1);
  return XNN_OK;
}

int xnn_eeq_real_apply(const double* pos, int64_t n_nodes, const double* cell, const double* rad,
                       double alpha, double cutoff, const double* tiles, const double* v,
                       int32_t nrhs, double* out, void* work, size_t work_bytes,
                       xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0, "negative size");
  XNN_REQUIRE(nrhs == 1 || nrhs == 2, "one or two right-hand sides (got %d)", (int)nrhs);
  if (n_nodes == 0) return XNN_OK;
  XNN_REQUIRE(pos && rad && v && out && work, "NULL input, output or workspace");
  XNN_REQUIRE(n_nodes <= (int64_t(1) << 26), "at most 2^26 atoms");
  XNN_REQUIRE(cutoff > 0.0 && alpha >= 0.0, "cutoff must be positive, alpha non-negative");
  XNN_REQUIRE(cell != nullptr || alpha == 0.0, "a molecule takes alpha = 0");
  const int64_t splits = eeq_apply_splits(n_nodes);
  XNN_REQUIRE(work_bytes >= sizeof(double) * (size_t)(splits * n_nodes * nrhs),
              "workspace too small");
  EeqCell C;
  XNN_REQUIRE(eeq_cell(cell, cutoff, C), "singular cell");
  XNN_REQUIRE(eeq_reach_ok(C, cutoff), "the real-space range spans more than %g cells",
              kMaxReach);
  const int64_t n_tiles = (n_nodes + kApplyTile - 1) / kApplyTile;
  const int64_t per = (n_tiles + splits - 1) / splits;
  const dim3 grid((unsigned)n_tiles, (unsigned)splits);
  hipStream_t s = as_hip(stream);
  double* part = static_cast<double*>(work);
  if (nrhs == 1)
    hipLaunchKernelGGL(eeq_real_apply_kernel<1>, grid, dim3(kApplyTile), 0, s, pos, n_nodes, C,
                       rad, alpha, cutoff, tiles, v, per, part);
  else
    hipLaunchKernelGGL(eeq_real_apply_kernel<2>, grid, dim3(kApplyTile), 0, s, pos, n_nodes, C,
                       rad, alpha, cutoff, tiles, v, per, part);
  XNN_LAUNCH_CHECK();
  const int64_t m = n_nodes * nrhs;
  hipLaunchKernelGGL(eeq_sum_splits_kernel, dim3((unsigned)grid_1d(m, 256)), dim3(256), 0, s, part,
                     splits, m, out);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_eeq_cholesky_solve(const double* factor, int64_t n, const double* inv_blocks, double* x,
                           int32_t nrhs, double* work, xnn_stream_t stream) {
  XNN_REQUIRE(n >= 0, "negative size");
  XNN_REQUIRE(nrhs == 1 || nrhs == 2, "one or two right-hand sides (got %d)", (int)nrhs);
  if (n == 0) return XNN_OK;
  XNN_REQUIRE(factor && inv_blocks && x && work, "NULL factor, inverses, right-hand side or work");
  XNN_REQUIRE(n <= (int64_t(1) << 20), "at most 2^20 rows");
  const int nb = (int)((n + kTrsvBlock - 1) / kTrsvBlock);
  hipStream_t s = as_hip(stream);
  for (int k = 0; k < nb; ++k) {          // forward: residual in x, solution into work
    const int64_t after = n - std::min<int64_t>(n, (int64_t)(k + 1) * kTrsvBlock);
    const unsigned grid = (unsigned)std::max<int64_t>(1, (after + kTrsvFwdRows - 1) / kTrsvFwdRows);
    if (nrhs == 1)
      hipLaunchKernelGGL((eeq_trsv_step_kernel<1, false>), dim3(grid), dim3(256), 0, s, factor, n,
                         inv_blocks, k, x, work);
    else
      hipLaunchKernelGGL((eeq_trsv_step_kernel<2, false>), dim3(grid), dim3(256), 0, s, factor, n,
                         inv_blocks, k, x, work);
  }
  for (int k = nb - 1; k >= 0; --k) {     // backward: residual in work, solution into x
    const int64_t before = (int64_t)k * kTrsvBlock;
    const unsigned grid = (unsigned)std::max<int64_t>(1, (before + kTrsvBwdRows - 1) / kTrsvBwdRows);
    if (nrhs == 1)
      hipLaunchKernelGGL((eeq_trsv_step_kernel<1, true>), dim3(grid), dim3(256), 0, s, factor, n,
                         inv_blocks, k, work, x);
    else
      hipLaunchKernelGGL((eeq_trsv_step_kernel<2, true>), dim3(grid), dim3(256), 0, s, factor, n,
                         inv_blocks, k, work, x);
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_eeq_cholesky_block(double* matrix, int64_t n, int64_t k0, int64_t b, double* inv,
                           int* info, xnn_stream_t stream) {
  XNN_REQUIRE(matrix && inv && info, "NULL matrix, inverse or info");
  XNN_REQUIRE(n > 0 && k0 >= 0 && b >= 1 && b <= kCholBlock && k0 + b <= n,
              "block [%lld, %lld) outside the matrix or wider than %d", (long long)k0,
              (long long)(k0 + b), kCholBlock);
  hipLaunchKernelGGL(eeq_cholesky_block_kernel, dim3(1), dim3(kCholThreads), 0, as_hip(stream), matrix,
                     n, k0, (int)b, inv, info);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

}  // extern "C"
