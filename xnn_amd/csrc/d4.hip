// D4 and D3 dispersion pair terms on lattice images (gfx950, wave64, float64).
//
// xnn_d4_coordination(_backward)  DFTD4.coordination_numbers (d4.py:552-591): the
//                                 EN-weighted erf-count CN and the plain erf count
//                                 of the charge model, summed to the receiver
// xnn_d4_two_body(_backward)      DFTD4.two_body_energy / pair_damping / pair_c6
//                                 (d4.py:1044-1071, 910-934) with the quintic
//                                 switch (dispersion.py:42-67): -1/2 C6 f(r) to the
//                                 receiver of every directed pair image; the backward
//                                 gives grad_pos, the cell gradient and dE/d alpha, the
//                                 quantities of the reference's native kernel run_d4
//                                 (dispersion_fast/cpu.py:834-935)
// xnn_d3_coordination(_backward)  DFTD3.coordination_numbers (d3.py:632-642), the
//                                 exponential count
// xnn_d3_two_body(_backward)      DFTD3.pair_c6 / two_body_energy (d3.py:651-722): C6
//                                 from per-atom reference weights and the species-pair
//                                 reference block, bj / zero / mzero / op damping
//
// No edge list: the long pair cutoff (60 bohr by default) makes the image list dense,
// so the kernels walk all (receiver, source, image) triples of each structure. Work
// item = one wave: a tile of 64 consecutive receivers (one per lane) against one chunk
// of source atoms, staged through LDS 64 at a time; images are looped in registers.
// Every directed pair is evaluated by its receiver's lane, both directions of a pair
// use their own weights, so forces need no scatter. Each item writes per-receiver
// partials for its chunk; xnn_d4 reductions sum the chunks in a fixed order
// (deterministic, no atomics). Positions and cells in Angstrom, lengths in the kernel
// in bohr, all float64.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "common.h"
#include "device.h"
#include "fp64.h"

namespace xnn {

constexpr int kD4Tile = 64;     // receivers per item (lanes of one wave)
constexpr int kD4Sub = 64;      // sources per LDS stage
constexpr int kD4MaxChunks = 128;
constexpr int kNW = 23;         // Casimir-Polder frequencies
constexpr double kBohr = 0.5291772109044924;
constexpr double kInvBohr = 1.0 / kBohr;
constexpr double kSqrtPi = 1.7724538509055160273;
constexpr double kInvSqrtPi = 1.0 / kSqrtPi;

struct D4Work {
  int64_t chunk;   // source atoms per chunk (multiple of kD4Sub)
  int64_t n_cy;    // chunk slots per tile
  int64_t n_tiles;
};

// chunk size and slots: at most kD4MaxChunks chunks of the largest structure, and the
// slots cover the source span of any 64-receiver tile (one structure: N atoms; a batch:
// the tile's structures, at most 64 + 2 (max_atoms - 1) atoms)
static D4Work d4_work(int64_t n_nodes, int64_t n_graphs, int64_t max_atoms) {
  D4Work w;
  const int64_t span = n_graphs <= 1 ? n_nodes : std::min<int64_t>(n_nodes, kD4Tile + 2 * max_atoms);
  int64_t subs = (std::max<int64_t>(max_atoms, 1) + (int64_t)kD4Sub * kD4MaxChunks - 1) /
                 ((int64_t)kD4Sub * kD4MaxChunks);
  w.chunk = kD4Sub * std::max<int64_t>(subs, 1);
  w.n_cy = (span + w.chunk - 1) / w.chunk + 1;
  w.n_tiles = (n_nodes + kD4Tile - 1) / kD4Tile;
  return w;
}

// Structure geometry of one lane: cell rows (Angstrom), image counts per axis, and the
// columns of the inverse cell scaled to interplanar spacings (for image pruning).
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

__device__ inline void load_lattice(const double* __restrict__ cell,
                                    const int32_t* __restrict__ images, int b, Lattice& L) {
  if (cell == nullptr) {
#pragma unroll
    for (int k = 0; k < 9; ++k) L.a[k] = L.ab[k] = L.inv[k] = 0.0;
    L.sp[0] = L.sp[1] = L.sp[2] = 1e300;
    L.n0 = L.n1 = L.n2 = 0;
    return;
  }
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    L.a[k] = cell[9 * (int64_t)b + k];
    L.ab[k] = L.a[k] * kInvBohr;
  }
  L.n0 = images[3 * b + 0];
  L.n1 = images[3 * b + 1];
  L.n2 = images[3 * b + 2];
  lattice_inverse(L);
}


// source data staged in LDS (one stage of kD4Sub atoms)
struct D4Stage {
  double x[kD4Sub], y[kD4Sub], z[kD4Sub];
  double w[kD4Sub];       // backward weight of the source (its upstream gradient)
  double w2[kD4Sub];      // second weight (CN: EEQ-count gradient)
  double p[kD4Sub], q[kD4Sub];  // per-source table values (CN: rcov, EN; pair: r4r2 and
                                // its square root), read once per stage, not per pair
  int sp[kD4Sub];         // species
  int b[kD4Sub];          // structure
};

// ---------------------------------------------------------------- coordination numbers
struct CnParams {
  double cut_cn, cut_eeq, kcn, k4, k5, k6;
};

// BACKWARD = false: partial[cy][0/1][i] = (cn_d4, cn_raw) sums of this chunk.
// BACKWARD = true:  partial[cy][0..11][i] = grad_pos (3), cell gradient n (x) g (9).
template <bool BACKWARD, bool D3 = false>
__global__ __launch_bounds__(64, 3) void d4_cn_kernel(
    const double* __restrict__ pos, int64_t n_nodes, const int32_t* __restrict__ species,
    const int32_t* __restrict__ batch, const int64_t* __restrict__ node_ptr,
    const double* __restrict__ cell, const int32_t* __restrict__ images,
    const double* __restrict__ rcov, const double* __restrict__ en, CnParams prm,
    const double* __restrict__ g_cn, const double* __restrict__ g_raw, int64_t chunk,
    int64_t n_cy, double* __restrict__ partial) {
  __shared__ D4Stage st;
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x, cy = blockIdx.y;
  const int64_t i = t * kD4Tile + lane;
  const bool live = i < n_nodes;
  // source range of the tile's structures, in chunks
  const int64_t i_first = t * kD4Tile, i_last = std::min<int64_t>(i_first + kD4Tile, n_nodes) - 1;
  const int64_t s_lo = node_ptr[batch[i_first]], s_hi = node_ptr[batch[i_last] + 1];
  const int64_t c = s_lo / chunk + cy;
  const int64_t j0 = std::max<int64_t>(c * chunk, s_lo), j1 = std::min<int64_t>((c + 1) * chunk, s_hi);
  constexpr int NP = BACKWARD ? 12 : 2;
  double acc[NP];
#pragma unroll
  for (int k = 0; k < NP; ++k) acc[k] = 0.0;
  double xi = 0, yi = 0, zi = 0, rci = 0, eni = 0, gi = 0, g2i = 0;
  int bi = -1;
  Lattice L;
  if (live) {
    xi = pos[3 * i];
    yi = pos[3 * i + 1];
    zi = pos[3 * i + 2];
    const int s = species[i];
    rci = rcov[s];
    eni = en[s];
    bi = batch[i];
    if (BACKWARD) {
      gi = g_cn ? g_cn[i] : 0.0;
      g2i = g_raw ? g_raw[i] : 0.0;
    }
    load_lattice(cell, images, bi, L);
  } else {
    load_lattice(nullptr, nullptr, 0, L);
  }
  const double cmax = prm.cut_cn > prm.cut_eeq ? prm.cut_cn : prm.cut_eeq;
  const double inv_k6 = 1.0 / prm.k6;
  for (int64_t base = j0; base < j1; base += kD4Sub) {
    const int cnt = (int)std::min<int64_t>(kD4Sub, j1 - base);
    __syncthreads();
    if (lane < cnt) {
      const int64_t j = base + lane;
      st.x[lane] = pos[3 * j];
      st.y[lane] = pos[3 * j + 1];
      st.z[lane] = pos[3 * j + 2];
      const int sj = species[j];
      st.sp[lane] = sj;
      st.b[lane] = batch[j];
      st.p[lane] = rcov[sj];
      if (!D3) st.q[lane] = en[sj];
      if (BACKWARD) {
        st.w[lane] = g_cn ? g_cn[j] : 0.0;
        st.w2[lane] = g_raw ? g_raw[j] : 0.0;
      }
    }
    __syncthreads();
    if (!live) continue;
    for (int jj = 0; jj < cnt; ++jj) {
      if (st.b[jj] != bi) continue;
      const double rc = rci + st.p[jj];
      double enf = 1.0;
      if (!D3) {
        const double den = fabs(eni - st.q[jj]) + prm.k5;
        enf = prm.k4 * exp(-den * den * inv_k6);
      }
      // per pair: k0 / rc and the erf count's slope factor -k0 / (rc sqrt(pi))
      const double k_rc = prm.kcn / rc;
      const double dk = -k_rc * kInvSqrtPi;
      const double dx = xi - st.x[jj], dy = yi - st.y[jj], dz = zi - st.z[jj];
      const double bx = dx * kInvBohr, by = dy * kInvBohr, bz = dz * kInvBohr;
      const double wsum = BACKWARD ? gi + st.w[jj] : 0.0;
      const double w2sum = BACKWARD ? g2i + st.w2[jj] : 0.0;
      const ImageRange win = image_window(L, dx, dy, dz, cmax * kBohr);
      for (int n0 = win.lo0; n0 <= win.hi0; ++n0)
        for (int n1 = win.lo1; n1 <= win.hi1; ++n1) {
          // the image's vector in bohr, d + n @ cell
          const double px = bx + n0 * L.ab[0] + n1 * L.ab[3];
          const double py = by + n0 * L.ab[1] + n1 * L.ab[4];
          const double pz = bz + n0 * L.ab[2] + n1 * L.ab[5];
          for (int n2 = win.lo2; n2 <= win.hi2; ++n2) {
            const double vx = px + n2 * L.ab[6], vy = py + n2 * L.ab[7], vz = pz + n2 * L.ab[8];
            const double r2 = vx * vx + vy * vy + vz * vz;
            if (r2 <= 0.0 || r2 > cmax * cmax) continue;
            const double rinv = rsq_nr(r2);
            const double r = r2 * rinv;
            const bool in_cn = r <= prm.cut_cn, in_eeq = !D3 && r <= prm.cut_eeq;
            double count, dcount;
            if (D3) {
              // 1 / (1 + exp(-k1 (rc / r - 1))) (d3.py:632-642); d/dr = -s (1 - s) k1 rc / r^2
              const double sg = rcp_nr(1.0 + exp(-prm.kcn * (rc * rinv - 1.0)));
              count = sg;
              dcount = -sg * (1.0 - sg) * prm.kcn * rc * rinv * rinv;
            } else {
              // (1 + erf(-k0 (r - rc) / rc)) / 2; d/dr = -k0 exp(-x^2) / (rc sqrt(pi))
              const double x = k_rc * (rc - r);
              count = 0.5 * (1.0 + erf(x));
              dcount = BACKWARD ? dk * exp(-x * x) : 0.0;
            }
            if (!BACKWARD) {
              if (in_cn) acc[0] += enf * count;
              if (in_eeq) acc[1] += count;
            } else {
              const double both = (in_cn ? wsum * enf : 0.0) + (in_eeq ? w2sum : 0.0);
              const double own = (in_cn ? gi * enf : 0.0) + (in_eeq ? g2i : 0.0);
              // per Angstrom of the edge vector: d r_bohr / d v = v_bohr / (r bohr)
              const double s = dcount * rinv * kInvBohr;
              acc[0] += both * s * vx;
              acc[1] += both * s * vy;
              acc[2] += both * s * vz;
              const double ox = own * s * vx, oy = own * s * vy, oz = own * s * vz;
              acc[3] += n0 * ox; acc[4] += n0 * oy; acc[5] += n0 * oz;
              acc[6] += n1 * ox; acc[7] += n1 * oy; acc[8] += n1 * oz;
              acc[9] += n2 * ox; acc[10] += n2 * oy; acc[11] += n2 * oz;
            }
          }
        }
    }
  }
  if (live) {
#pragma unroll
    for (int k = 0; k < NP; ++k) partial[((int64_t)cy * NP + k) * n_nodes + i] = acc[k];
  }
}

// ---------------------------------------------------------------- two-body term
struct PairParams {
  double s6, s8, a1, a2, cutoff, width;  // cutoff, width in bohr
};

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
__constant__ double c_cp3[kNW] = {
    cp3_weight(0),  cp3_weight(1),  cp3_weight(2),  cp3_weight(3),  cp3_weight(4),
    cp3_weight(5),  cp3_weight(6),  cp3_weight(7),  cp3_weight(8),  cp3_weight(9),
    cp3_weight(10), cp3_weight(11), cp3_weight(12), cp3_weight(13), cp3_weight(14),
    cp3_weight(15), cp3_weight(16), cp3_weight(17), cp3_weight(18), cp3_weight(19),
    cp3_weight(20), cp3_weight(21), cp3_weight(22)};
static_assert(sizeof(c_cp3) / sizeof(c_cp3[0]) == kNW, "one weight per frequency");

// BACKWARD = false: partial[cy][0][i] = sum of -1/2 C6 f(r) over this chunk.
// BACKWARD = true:  partial[cy][0..11][i] = grad_pos (3), cell gradient (9), and
//                   partial_alpha[cy][w][i] = dE/d alpha_i(w) (23).
// (64, 2): at most 256 registers, two waves per SIMD. The backward would take 284 and run
// one wave per SIMD; with the cap it spills a few values to scratch and the step runs 12 %
// faster (2.72 -> 2.40 ms on the 5,000-atom box). A cap of 3 waves spills far more and
// is slower.
template <bool BACKWARD>
__global__ __launch_bounds__(64, 2) void d4_pair_kernel(
    const double* __restrict__ pos, int64_t n_nodes, const int32_t* __restrict__ species,
    const int32_t* __restrict__ batch, const int64_t* __restrict__ node_ptr,
    const double* __restrict__ cell, const int32_t* __restrict__ images,
    const double* __restrict__ r4r2, const double* __restrict__ alpha, PairParams prm,
    const double* __restrict__ g_e2, int64_t chunk, int64_t n_cy, double* __restrict__ partial,
    double* __restrict__ partial_alpha) {
  __shared__ D4Stage st;
  __shared__ double sa[kNW][kD4Sub];  // the sources' alpha(i w) times the grid weights c_cp3
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x, cy = blockIdx.y;
  const int64_t i = t * kD4Tile + lane;
  const bool live = i < n_nodes;
  const int64_t i_first = t * kD4Tile, i_last = std::min<int64_t>(i_first + kD4Tile, n_nodes) - 1;
  const int64_t s_lo = node_ptr[batch[i_first]], s_hi = node_ptr[batch[i_last] + 1];
  const int64_t c = s_lo / chunk + cy;
  const int64_t j0 = std::max<int64_t>(c * chunk, s_lo), j1 = std::min<int64_t>((c + 1) * chunk, s_hi);
  constexpr int NP = BACKWARD ? 12 : 1;
  double acc[NP];
#pragma unroll
  for (int k = 0; k < NP; ++k) acc[k] = 0.0;
  double ai[kNW], da[kNW];
#pragma unroll
  for (int w = 0; w < kNW; ++w) {
    ai[w] = 0.0;
    da[w] = 0.0;
  }
  double xi = 0, yi = 0, zi = 0, qi = 0, sq3qi = 0, gi = 0;
  int bi = -1;
  Lattice L;
  if (live) {
    xi = pos[3 * i];
    yi = pos[3 * i + 1];
    zi = pos[3 * i + 2];
    qi = r4r2[species[i]];
    sq3qi = sqrt(3.0 * qi);
    bi = batch[i];
    if (BACKWARD) gi = g_e2[i];
#pragma unroll
    for (int w = 0; w < kNW; ++w) ai[w] = alpha[(int64_t)kNW * i + w];
    load_lattice(cell, images, bi, L);
  } else {
    load_lattice(nullptr, nullptr, 0, L);
  }
  const double rc2 = prm.cutoff * prm.cutoff;
  // below r = cutoff - width the switch is 1 with zero slope: r itself is not needed
  const double wzone = prm.width > 0.0 ? fmax(prm.cutoff - fmin(prm.width, prm.cutoff), 0.0)
                                       : prm.cutoff;
  const double wz2 = wzone * wzone;
  for (int64_t base = j0; base < j1; base += kD4Sub) {
    const int cnt = (int)std::min<int64_t>(kD4Sub, j1 - base);
    __syncthreads();
    if (lane < cnt) {
      const int64_t j = base + lane;
      st.x[lane] = pos[3 * j];
      st.y[lane] = pos[3 * j + 1];
      st.z[lane] = pos[3 * j + 2];
      const double qj = r4r2[species[j]];
      st.p[lane] = qj;
      st.q[lane] = sqrt(qj);
      st.b[lane] = batch[j];
      if (BACKWARD) st.w[lane] = g_e2[j];
#pragma unroll
      for (int w = 0; w < kNW; ++w) sa[w][lane] = alpha[(int64_t)kNW * j + w] * c_cp3[w];
    }
    __syncthreads();
    if (!live) continue;
    for (int jj = 0; jj < cnt; ++jj) {
      if (st.b[jj] != bi) continue;
      double c6 = 0.0;
#pragma unroll
      for (int w = 0; w < kNW; ++w) c6 += ai[w] * sa[w][jj];
      // rr = 3 r4r2_i r4r2_j and R0 = a1 sqrt(rr) + a2, sqrt(rr) = sqrt(3 r4r2_i) sqrt(r4r2_j)
      const double rr = 3.0 * qi * st.p[jj];
      const double s8rr = prm.s8 * rr;
      const double r0 = prm.a1 * (sq3qi * st.q[jj]) + prm.a2;
      const double r02 = r0 * r0;
      const double r06 = r02 * r02 * r02, r08 = r06 * r02;
      const double dx = xi - st.x[jj], dy = yi - st.y[jj], dz = zi - st.z[jj];
      const double bx = dx * kInvBohr, by = dy * kInvBohr, bz = dz * kInvBohr;
      const double wsum = BACKWARD ? gi + st.w[jj] : 0.0;
      double fsum = 0.0;  // sum over images of f(r): d E / d C6 of the pair
      const ImageRange win = image_window(L, dx, dy, dz, prm.cutoff * kBohr);
      for (int n0 = win.lo0; n0 <= win.hi0; ++n0)
        for (int n1 = win.lo1; n1 <= win.hi1; ++n1) {
          // the image's vector in bohr, d + n @ cell
          const double px = bx + n0 * L.ab[0] + n1 * L.ab[3];
          const double py = by + n0 * L.ab[1] + n1 * L.ab[4];
          const double pz = bz + n0 * L.ab[2] + n1 * L.ab[5];
          for (int n2 = win.lo2; n2 <= win.hi2; ++n2) {
            const double vx = px + n2 * L.ab[6], vy = py + n2 * L.ab[7], vz = pz + n2 * L.ab[8];
            const double r2 = vx * vx + vy * vy + vz * vz;
            if (r2 <= 0.0 || r2 > rc2) continue;
            // t6 = 1 / (r^6 + r0^6), t8 = 1 / (r^8 + r0^8) from one reciprocal
            const double r4 = r2 * r2, r6 = r4 * r2, r8 = r6 * r2;
            const double p6 = r6 + r06, p8 = r8 + r08;
            const double inv = rcp_nr(p6 * p8);
            const double t6 = p8 * inv, t8 = p6 * inv;
            const double g = prm.s6 * t6 + s8rr * t8;
            double sw = 1.0, dsw_r = 0.0;  // the switch and its slope over r
            if (r2 > wz2) {
              const double rinv = rsq_nr(r2);
              double dsw;
              switch_d(r2 * rinv, prm.cutoff, prm.width, sw, dsw);
              dsw_r = dsw * rinv;
            }
            const double f = sw * g;
            if (!BACKWARD) {
              acc[0] += -0.5 * c6 * f;
            } else {
              fsum += f;
              // (d f / d r) / r, and d r_bohr / d v_Angstrom = v_bohr / (r_bohr bohr)
              const double dg_r = -6.0 * prm.s6 * r4 * t6 * t6 - 8.0 * s8rr * r6 * t8 * t8;
              const double df_r = dsw_r * g + sw * dg_r;
              const double s = -0.5 * kInvBohr * c6 * df_r;
              acc[0] += wsum * s * vx;
              acc[1] += wsum * s * vy;
              acc[2] += wsum * s * vz;
              const double ox = gi * s * vx, oy = gi * s * vy, oz = gi * s * vz;
              acc[3] += n0 * ox; acc[4] += n0 * oy; acc[5] += n0 * oz;
              acc[6] += n1 * ox; acc[7] += n1 * oy; acc[8] += n1 * oz;
              acc[9] += n2 * ox; acc[10] += n2 * oy; acc[11] += n2 * oz;
            }
          }
        }
      if (BACKWARD && fsum != 0.0) {
        const double k = -0.5 * wsum * fsum;
#pragma unroll
        for (int w = 0; w < kNW; ++w) da[w] += k * sa[w][jj];
      }
    }
  }
  if (live) {
#pragma unroll
    for (int k = 0; k < NP; ++k) partial[((int64_t)cy * NP + k) * n_nodes + i] = acc[k];
    if (BACKWARD) {
#pragma unroll
      for (int w = 0; w < kNW; ++w) partial_alpha[((int64_t)cy * kNW + w) * n_nodes + i] = da[w];
    }
  }
}

// ---------------------------------------------------------------- D3 two-body term
constexpr int kNR = 7;  // D3 reference systems per element

struct D3PairParams {
  double s6, s8, a1, a2, rs6, rs8, alp, bet, cutoff, width;
  int damping;  // 0 bj, 1 zero, 2 mzero, 3 op
};

// t6, t8 of the damping variants (d3.py:698-720) and their r-derivatives
__device__ inline void d3_damp(const D3PairParams& p, double r, double r0, double& t6, double& t8,
                               double& d6, double& d8) {
  const double r2 = r * r, r6 = r2 * r2 * r2, r8 = r6 * r2;
  if (p.damping == 0) {                       // rational (Becke-Johnson)
    const double q2 = r0 * r0, q6 = q2 * q2 * q2, q8 = q6 * q2;
    t6 = 1.0 / (r6 + q6);
    t8 = 1.0 / (r8 + q8);
    d6 = -6.0 * r * r2 * r2 * t6 * t6;
    d8 = -8.0 * r * r6 * t8 * t8;
  } else if (p.damping == 1 || p.damping == 2) {  // zero / modified zero
    double a6, a8, da6, da8;
    if (p.damping == 1) {
      a6 = pow(p.rs6 * r0 / r, p.alp);
      a8 = pow(p.rs8 * r0 / r, p.alp + 2.0);
      da6 = -p.alp * a6 / r;
      da8 = -(p.alp + 2.0) * a8 / r;
    } else {
      const double x6 = r / (p.rs6 * r0) + p.bet * r0, x8 = r / (p.rs8 * r0) + p.bet * r0;
      a6 = pow(x6, -p.alp);
      a8 = pow(x8, -(p.alp + 2.0));
      da6 = -p.alp * a6 / x6 / (p.rs6 * r0);
      da8 = -(p.alp + 2.0) * a8 / x8 / (p.rs8 * r0);
    }
    t6 = 1.0 / ((1.0 + 6.0 * a6) * r6);
    t8 = 1.0 / ((1.0 + 6.0 * a8) * r8);
    d6 = -t6 * (6.0 * da6 / (1.0 + 6.0 * a6) + 6.0 / r);
    d8 = -t8 * (6.0 * da8 / (1.0 + 6.0 * a8) + 8.0 / r);
  } else {                                    // optimized power
    const double rb = pow(r, p.bet), ab = pow(r0, p.bet);
    const double q2 = r0 * r0, q6 = q2 * q2 * q2, q8 = q6 * q2;
    const double den6 = rb * r6 + ab * q6, den8 = rb * r8 + ab * q8;
    t6 = rb / den6;
    t8 = rb / den8;
    // t = 1 / (r^n + c r^-bet), c = ab q^n: dt/dr = -t^2 (n r^(n-1) - bet c r^(-bet-1))
    const double c6 = ab * q6 / rb, c8 = ab * q8 / rb;
    d6 = -t6 * t6 * (6.0 * r * r2 * r2 - p.bet * c6 / r);
    d8 = -t8 * t8 * (8.0 * r * r6 - p.bet * c8 / r);
  }
}

// BACKWARD = false: partial[cy][0][i] = sum of -1/2 C6 f(r) over this chunk.
// BACKWARD = true:  partial[cy][0..11][i] = grad_pos (3), cell gradient (9), and
//                   partial_w[cy][a][i] = dE / dW_i[a] (7).
// C6_ij = sum_ab W_i[a] W_j[b] C6ref[s_i][s_j][a][b] (d3.py:651-674).
// D3 reference-C6 vectors staged per receiver species (see d3_pair_kernel): species rows
// padded by two doubles so that lanes of different species read different banks
constexpr int kD3SvStride = kNR * kD4Sub + 2;
constexpr int kD3MaxStaged = 16;  // 16 x 3.5 KB of LDS at most

// BJ: the rational damping compiled alone (the default; the general loop with all four
// dampings holds more registers)
template <bool BACKWARD, bool STAGED, bool BJ>
__global__ __launch_bounds__(64, 2) void d3_pair_kernel(
    const double* __restrict__ pos, int64_t n_nodes, const int32_t* __restrict__ species,
    const int32_t* __restrict__ batch, const int64_t* __restrict__ node_ptr,
    const double* __restrict__ cell, const int32_t* __restrict__ images,
    const double* __restrict__ r4r2, const double* __restrict__ rvdw,
    const double* __restrict__ c6ref, int n_species, const double* __restrict__ wref,
    D3PairParams prm, const double* __restrict__ g_e2, int64_t chunk, int64_t n_cy,
    double* __restrict__ partial, double* __restrict__ partial_w) {
  __shared__ D4Stage st;
  // STAGED: for every receiver species s, v_s[a] = sum_b C6ref[s][s_j][a][b] W_j[b] of each
  // staged source j (dynamic LDS, kD3SvStride doubles per species), so that a pair reads
  // its seven values instead of the 7 x 7 reference block; otherwise the sources' weights
  __shared__ double sw_[STAGED ? 1 : kNR][kD4Sub];
  extern __shared__ double d3_sv[];
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x, cy = blockIdx.y;
  const int64_t i = t * kD4Tile + lane;
  const bool live = i < n_nodes;
  const int64_t i_first = t * kD4Tile, i_last = std::min<int64_t>(i_first + kD4Tile, n_nodes) - 1;
  const int64_t s_lo = node_ptr[batch[i_first]], s_hi = node_ptr[batch[i_last] + 1];
  const int64_t c = s_lo / chunk + cy;
  const int64_t j0 = std::max<int64_t>(c * chunk, s_lo), j1 = std::min<int64_t>((c + 1) * chunk, s_hi);
  constexpr int NP = BACKWARD ? 12 : 1;
  double acc[NP];
#pragma unroll
  for (int k = 0; k < NP; ++k) acc[k] = 0.0;
  double wi[kNR], dw[kNR];
#pragma unroll
  for (int a = 0; a < kNR; ++a) {
    wi[a] = 0.0;
    dw[a] = 0.0;
  }
  double xi = 0, yi = 0, zi = 0, qi = 0, sq3qi = 0, gi = 0;
  int bi = -1, si = 0;
  Lattice L;
  if (live) {
    xi = pos[3 * i];
    yi = pos[3 * i + 1];
    zi = pos[3 * i + 2];
    si = species[i];
    qi = r4r2[si];
    sq3qi = sqrt(3.0 * qi);
    bi = batch[i];
    if (BACKWARD) gi = g_e2[i];
#pragma unroll
    for (int a = 0; a < kNR; ++a) wi[a] = wref[(int64_t)kNR * i + a];
    load_lattice(cell, images, bi, L);
  } else {
    load_lattice(nullptr, nullptr, 0, L);
  }
  const double rc2 = prm.cutoff * prm.cutoff;
  // below r = cutoff - width the switch is 1 with zero slope
  const double wzone = prm.width > 0.0 ? fmax(prm.cutoff - fmin(prm.width, prm.cutoff), 0.0)
                                       : prm.cutoff;
  const double wz2 = wzone * wzone;
  for (int64_t base = j0; base < j1; base += kD4Sub) {
    const int cnt = (int)std::min<int64_t>(kD4Sub, j1 - base);
    __syncthreads();
    if (lane < cnt) {
      const int64_t j = base + lane;
      st.x[lane] = pos[3 * j];
      st.y[lane] = pos[3 * j + 1];
      st.z[lane] = pos[3 * j + 2];
      const int sj = species[j];
      st.sp[lane] = sj;
      st.b[lane] = batch[j];
      st.p[lane] = r4r2[sj];
      st.q[lane] = sqrt(st.p[lane]);
      if (BACKWARD) st.w[lane] = g_e2[j];
      if (STAGED) {
        double wj[kNR];
#pragma unroll
        for (int b = 0; b < kNR; ++b) wj[b] = wref[(int64_t)kNR * j + b];
        for (int s2 = 0; s2 < n_species; ++s2) {
          const double* blk = c6ref + ((int64_t)s2 * n_species + sj) * (kNR * kNR);
#pragma unroll
          for (int a = 0; a < kNR; ++a) {
            double sa = 0.0;
#pragma unroll
            for (int b = 0; b < kNR; ++b) sa += blk[a * kNR + b] * wj[b];
            d3_sv[s2 * kD3SvStride + a * kD4Sub + lane] = sa;
          }
        }
      } else {
#pragma unroll
        for (int a = 0; a < kNR; ++a) sw_[a][lane] = wref[(int64_t)kNR * j + a];
      }
    }
    __syncthreads();
    if (!live) continue;
    for (int jj = 0; jj < cnt; ++jj) {
      if (st.b[jj] != bi) continue;
      const int sj = st.sp[jj];
      double v[kNR];  // v[a] = sum_b C6ref[a][b] W_j[b]
      if (STAGED) {
#pragma unroll
        for (int a = 0; a < kNR; ++a) v[a] = d3_sv[si * kD3SvStride + a * kD4Sub + jj];
      } else {
        const double* blk = c6ref + ((int64_t)si * n_species + sj) * (kNR * kNR);
#pragma unroll
        for (int a = 0; a < kNR; ++a) {
          double sa = 0.0;
#pragma unroll
          for (int b = 0; b < kNR; ++b) sa += blk[a * kNR + b] * sw_[b][jj];
          v[a] = sa;
        }
      }
      double c6 = 0.0;
#pragma unroll
      for (int a = 0; a < kNR; ++a) c6 += wi[a] * v[a];
      // rr = 3 r4r2_i r4r2_j; BJ and op: R0 = a1 sqrt(rr) + a2 with sqrt(rr) =
      // sqrt(3 r4r2_i) sqrt(r4r2_j), zero and mzero: R0 from the vdW radii table
      const double rr = 3.0 * qi * st.p[jj];
      const double r0 = (prm.damping == 0 || prm.damping == 3) ? prm.a1 * (sq3qi * st.q[jj]) + prm.a2
                                                               : rvdw[si * n_species + sj];
      const double s8rr = prm.s8 * rr;
      const double r02 = r0 * r0, r06 = r02 * r02 * r02, r08 = r06 * r02;
      const double dx = xi - st.x[jj], dy = yi - st.y[jj], dz = zi - st.z[jj];
      const double wsum = BACKWARD ? gi + st.w[jj] : 0.0;
      double fsum = 0.0;
      const ImageRange win = image_window(L, dx, dy, dz, prm.cutoff * kBohr);
      const double bx = dx * kInvBohr, by = dy * kInvBohr, bz = dz * kInvBohr;
      for (int n0 = win.lo0; n0 <= win.hi0; ++n0)
        for (int n1 = win.lo1; n1 <= win.hi1; ++n1) {
          // the image's vector in bohr, d + n @ cell
          const double px = bx + n0 * L.ab[0] + n1 * L.ab[3];
          const double py = by + n0 * L.ab[1] + n1 * L.ab[4];
          const double pz = bz + n0 * L.ab[2] + n1 * L.ab[5];
          for (int n2 = win.lo2; n2 <= win.hi2; ++n2) {
            const double vx = px + n2 * L.ab[6], vy = py + n2 * L.ab[7], vz = pz + n2 * L.ab[8];
            const double r2 = vx * vx + vy * vy + vz * vz;
            if (r2 <= 0.0 || r2 > rc2) continue;
            double f, df_r;  // f(r) and (d f / d r) / r
            if (BJ) {
              // BJ, as the D4 pair kernel: t6 = 1 / (r^6 + R0^6), t8 = 1 / (r^8 + R0^8) from
              // one reciprocal, r itself only inside the switching zone
              const double r4 = r2 * r2, r6 = r4 * r2, r8 = r6 * r2;
              const double p6 = r6 + r06, p8 = r8 + r08;
              const double inv = rcp_nr(p6 * p8);
              const double t6 = p8 * inv, t8 = p6 * inv;
              const double g = prm.s6 * t6 + s8rr * t8;
              double sw = 1.0, dsw_r = 0.0;
              if (r2 > wz2) {
                const double rinv = rsq_nr(r2);
                double dsw;
                switch_d(r2 * rinv, prm.cutoff, prm.width, sw, dsw);
                dsw_r = dsw * rinv;
              }
              f = sw * g;
              df_r = BACKWARD ? dsw_r * g + sw * (-6.0 * prm.s6 * r4 * t6 * t6 -
                                                  8.0 * s8rr * r6 * t8 * t8)
                              : 0.0;
            } else {
              // every damping (BJ included: prm.damping selects), r explicit
              const double rinv = rsq_nr(r2);
              const double r = r2 * rinv;
              double sw, dsw, t6, t8, d6, d8;
              switch_d(r, prm.cutoff, prm.width, sw, dsw);
              d3_damp(prm, r, r0, t6, t8, d6, d8);
              const double g = prm.s6 * t6 + s8rr * t8;
              f = sw * g;
              df_r = BACKWARD ? (dsw * g + sw * (prm.s6 * d6 + s8rr * d8)) * rinv : 0.0;
            }
            if (!BACKWARD) {
              acc[0] += -0.5 * c6 * f;
            } else {
              fsum += f;
              // d r_bohr / d v_Angstrom = v_bohr / (r_bohr bohr)
              const double s = -0.5 * kInvBohr * c6 * df_r;
              acc[0] += wsum * s * vx;
              acc[1] += wsum * s * vy;
              acc[2] += wsum * s * vz;
              const double ox = gi * s * vx, oy = gi * s * vy, oz = gi * s * vz;
              acc[3] += n0 * ox; acc[4] += n0 * oy; acc[5] += n0 * oz;
              acc[6] += n1 * ox; acc[7] += n1 * oy; acc[8] += n1 * oz;
              acc[9] += n2 * ox; acc[10] += n2 * oy; acc[11] += n2 * oz;
            }
          }
        }
      if (BACKWARD && fsum != 0.0) {
        const double k = -0.5 * wsum * fsum;
#pragma unroll
        for (int a = 0; a < kNR; ++a) dw[a] += k * v[a];
      }
    }
  }
  if (live) {
#pragma unroll
    for (int k = 0; k < NP; ++k) partial[((int64_t)cy * NP + k) * n_nodes + i] = acc[k];
    if (BACKWARD) {
#pragma unroll
      for (int a = 0; a < kNR; ++a) partial_w[((int64_t)cy * kNR + a) * n_nodes + i] = dw[a];
    }
  }
}

// out[i * nk + (k - k0)] = sum over chunk slots cy of partial[cy][k][i], for the
// components k0 <= k < k0 + nk of a partial array of np components. The kReduceWaves
// waves of a block share 64 outputs: wave w sums the slots cy = w, w + kReduceWaves, ...
// in order, and wave 0 adds the waves' sums in wave order (a fixed order, so repeated
// calls agree bit for bit; the slot loop of one output is ~n_cy / kReduceWaves loads long
// instead of n_cy dependent ones). The 64 outputs of a block are 64 consecutive atoms of
// one component, so that every load of a wave reads one contiguous run of the partials.
constexpr int kReduceWaves = 8;

__global__ __launch_bounds__(64 * kReduceWaves) void d4_reduce_kernel(
    const double* __restrict__ partial, int64_t n_nodes, int np, int k0, int nk, int64_t n_cy,
    double* __restrict__ out) {
  __shared__ double red[kReduceWaves][64];
  const int lane = threadIdx.x & 63;
  const int wv = wave_in_block();
  const int64_t i = (int64_t)blockIdx.x * 64 + lane;
  const int k = k0 + (int)blockIdx.y;
  const bool live = i < n_nodes;
  double s = 0.0;
  if (live) {
    const double* src = partial + (int64_t)k * n_nodes + i;
    const int64_t stride = (int64_t)np * n_nodes;
    for (int64_t cy = wv; cy < n_cy; cy += kReduceWaves) s += src[cy * stride];
  }
  red[wv][lane] = s;
  __syncthreads();
  if (wv == 0 && live) {
    double t = red[0][lane];
#pragma unroll
    for (int w = 1; w < kReduceWaves; ++w) t += red[w][lane];
    out[i * nk + (k - k0)] = t;
  }
}

static void reduce_into(const double* partial, int64_t n_nodes, int np, int k0, int nk,
                        int64_t n_cy, double* out, hipStream_t s) {
  const int64_t n = n_nodes * nk;
  if (n == 0 || out == nullptr) return;
  hipLaunchKernelGGL(d4_reduce_kernel, dim3(grid_1d(n_nodes, 64), nk), dim3(64 * kReduceWaves),
                     0, s, partial, n_nodes, np, k0, nk, n_cy, out);
}

// ---------------------------------------------------------------- polarizabilities
constexpr int kD4Ref = 7;                                  // reference systems per element
constexpr double kD4NormEps = 1.4916681462400413e-154;     // smallest usable weight norm

struct AlphaTables {
  int n_el;
  const int32_t* nref;     // (n_el,)
  const int32_t* ngw;      // (n_el, 7)
  const double* refcn;     // (n_el, 7)
  const double* refq;      // (n_el, 7)
  const double* zeff;      // (n_el,)
  const double* gi;        // (n_el,) hardness x gc
  const double* refalpha;  // (n_el, 7, 23)
  double ga, wf;
};

// One thread per atom. Reference r of element z weighs
// g_r = sum_{j=1..ngw} exp(-wf j (cn - cnref_r)^2), normalised over the element's
// references (d4.py:984-1023; a norm below kD4NormEps puts weight 1 on the references of
// the largest cnref), times the charge scaling zeta_r(q) = exp(ga (1 - exp(gi (1 - qref_r /
// (q + zeff))))) with qref_r = refq_r + zeff, or exp(ga) when q + zeff < 0
// (dispersion.py:70-121); alpha_k = sum_r w_r zeta_r refalpha[z][r][k] (d4.py:1036-1042).
// BACKWARD contracts g_alpha with d alpha / d cn (through w) into g_cn and with
// d alpha / d q (through zeta) into g_q, as the reference's native d4_alpha
// (dispersion_fast/cpu.py:774-829). An atomic number outside the tables gives NaN.
template <bool BACKWARD>
__global__ __launch_bounds__(256) void d4_alpha_kernel(
    int64_t n, const int64_t* __restrict__ z, const double* __restrict__ cn,
    const double* __restrict__ q, AlphaTables T, const double* __restrict__ g_alpha,
    double* __restrict__ alpha, double* __restrict__ g_cn, double* __restrict__ g_q) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t zz = z[i];
  const int nr = (zz >= 0 && zz < T.n_el) ? T.nref[zz] : -1;
  if (nr < 0 || nr > kD4Ref) {
    const double bad = __builtin_nan("");
    if (!BACKWARD) {
      for (int k = 0; k < kNW; ++k) alpha[i * kNW + k] = bad;
    } else {
      if (g_cn) g_cn[i] = bad;
      if (g_q) g_q[i] = bad;
    }
    return;
  }
  const double c = cn[i];
  double w[kD4Ref], dw[kD4Ref];
  double norm = 0.0, dnorm = 0.0;
#pragma unroll
  for (int r = 0; r < kD4Ref; ++r) {
    double g = 0.0, dg = 0.0;
    if (r < nr) {
      const double d = c - T.refcn[zz * kD4Ref + r];
      const double d2 = d * d;
      const int ng = T.ngw[zz * kD4Ref + r];
      for (int j = 1; j <= ng; ++j) {
        const double e = exp(-T.wf * j * d2);
        g += e;
        dg += e * (-2.0 * T.wf * j * d);
      }
    }
    w[r] = g;
    dw[r] = dg;
    norm += g;
    dnorm += dg;
  }
  if (norm > kD4NormEps) {
#pragma unroll
    for (int r = 0; r < kD4Ref; ++r) {
      const double wr = w[r] / norm;
      dw[r] = (dw[r] - wr * dnorm) / norm;
      w[r] = wr;
    }
  } else {
    double top = -__builtin_inf();
    for (int r = 0; r < nr; ++r) top = fmax(top, T.refcn[zz * kD4Ref + r]);
#pragma unroll
    for (int r = 0; r < kD4Ref; ++r) {
      w[r] = (r < nr && fabs(T.refcn[zz * kD4Ref + r] - top) < 1e-12) ? 1.0 : 0.0;
      dw[r] = 0.0;
    }
  }
  const double zi = T.zeff[zz], gi = T.gi[zz];
  const double qmod = q[i] + zi;
  double zeta[kD4Ref], dzeta[kD4Ref];
#pragma unroll
  for (int r = 0; r < kD4Ref; ++r) {
    zeta[r] = 0.0;
    dzeta[r] = 0.0;
    if (r < nr) {
      if (qmod < 0.0) {
        zeta[r] = exp(T.ga);
      } else {
        const double qref = T.refq[zz * kD4Ref + r] + zi;
        const double eu = exp(gi * (1.0 - qref / qmod));
        zeta[r] = exp(T.ga * (1.0 - eu));
        dzeta[r] = zeta[r] * (-T.ga * eu) * gi * qref / (qmod * qmod);
      }
    }
  }
  const double* ra = T.refalpha + zz * (kD4Ref * kNW);
  if (!BACKWARD) {
    double a[kNW];
#pragma unroll
    for (int k = 0; k < kNW; ++k) a[k] = 0.0;
    for (int r = 0; r < nr; ++r) {
      const double wz = w[r] * zeta[r];
#pragma unroll
      for (int k = 0; k < kNW; ++k) a[k] += wz * ra[r * kNW + k];
    }
#pragma unroll
    for (int k = 0; k < kNW; ++k) alpha[i * kNW + k] = a[k];
  } else {
    double ga[kNW];
#pragma unroll
    for (int k = 0; k < kNW; ++k) ga[k] = g_alpha[i * kNW + k];
    double gc = 0.0, gq = 0.0;
    for (int r = 0; r < nr; ++r) {
      double t = 0.0;  // sum_k g_alpha_k refalpha[r][k]
#pragma unroll
      for (int k = 0; k < kNW; ++k) t += ga[k] * ra[r * kNW + k];
      gc += dw[r] * zeta[r] * t;
      gq += w[r] * dzeta[r] * t;
    }
    if (g_cn) g_cn[i] = gc;
    if (g_q) g_q[i] = gq;
  }
}

// One thread per atom: the D3 reference weights w_r = g_r / sum_r' g_r' with
// g_r = exp(-wf (cn - cnref_r)^2) over the species' nref references (d3.py:644-649,
// dispersion.py:70-121; a zero norm puts weight 1 on the references of the largest cnref).
// BACKWARD: g_cn = sum_r g_w[r] d w_r / d cn. A species outside the tables gives NaN.
template <bool BACKWARD>
__global__ __launch_bounds__(256) void d3_weights_kernel(
    int64_t n, const int32_t* __restrict__ species, const double* __restrict__ cn,
    int n_species, const int32_t* __restrict__ nref, const double* __restrict__ refcn,
    double wf, const double* __restrict__ g_w, double* __restrict__ w_out,
    double* __restrict__ g_cn) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int sp = species[i];
  const int nr = (sp >= 0 && sp < n_species) ? nref[sp] : -1;
  if (nr < 0 || nr > kNR) {
    const double bad = __builtin_nan("");
    if (!BACKWARD) {
      for (int r = 0; r < kNR; ++r) w_out[i * kNR + r] = bad;
    } else {
      g_cn[i] = bad;
    }
    return;
  }
  const double c = cn[i];
  double w[kNR], dw[kNR];
  double norm = 0.0, dnorm = 0.0;
#pragma unroll
  for (int r = 0; r < kNR; ++r) {
    double g = 0.0, dg = 0.0;
    if (r < nr) {
      const double d = c - refcn[sp * kNR + r];
      g = exp(-wf * (d * d));
      dg = g * (-2.0 * wf * d);
    }
    w[r] = g;
    dw[r] = dg;
    norm += g;
    dnorm += dg;
  }
  if (norm > 0.0) {
#pragma unroll
    for (int r = 0; r < kNR; ++r) {
      const double wr = w[r] / norm;
      dw[r] = (dw[r] - wr * dnorm) / norm;
      w[r] = wr;
    }
  } else {
    double top = -__builtin_inf();
    for (int r = 0; r < nr; ++r) top = fmax(top, refcn[sp * kNR + r]);
#pragma unroll
    for (int r = 0; r < kNR; ++r) {
      w[r] = (r < nr && fabs(refcn[sp * kNR + r] - top) < 1e-12) ? 1.0 : 0.0;
      dw[r] = 0.0;
    }
  }
  if (!BACKWARD) {
#pragma unroll
    for (int r = 0; r < kNR; ++r) w_out[i * kNR + r] = w[r];
  } else {
    double gc = 0.0;
#pragma unroll
    for (int r = 0; r < kNR; ++r) gc += g_w[i * kNR + r] * dw[r];
    g_cn[i] = gc;
  }
}

static int d4_check(const double* pos, int64_t n_nodes, const int32_t* species,
                    const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                    const double* cell, const int32_t* images, int64_t max_atoms) {
  XNN_REQUIRE(n_nodes >= 0 && n_graphs >= 1, "negative size or no structure");
  XNN_REQUIRE(n_nodes == 0 || (pos && species && batch && node_ptr), "NULL atom input");
  XNN_REQUIRE(cell == nullptr || images != nullptr, "a cell needs the image counts");
  XNN_REQUIRE(max_atoms >= 1 || n_nodes == 0, "max_atoms must be >= 1");
  return XNN_OK;
}

}  // namespace xnn

using namespace xnn;

extern "C" {

size_t xnn_d4_workspace_bytes(int64_t n_nodes, int64_t n_graphs, int64_t max_atoms) {
  if (n_nodes <= 0) return 0;
  const D4Work w = d4_work(n_nodes, n_graphs, max_atoms);
  // the largest user: the pair backward, 12 + 23 values per receiver and chunk slot
  return (size_t)(w.n_cy * (12 + kNW) * n_nodes) * sizeof(double);
}

int xnn_d4_coordination(const double* pos, int64_t n_nodes, const int32_t* species,
                        const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                        int64_t max_atoms, const double* cell, const int32_t* images,
                        const double* rcov, const double* en, const xnn_d4_cn_params* prm,
                        double* cn_d4, double* cn_raw, void* workspace, size_t workspace_bytes,
                        xnn_stream_t stream) {
  const int st = d4_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images, max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(prm && rcov && en, "NULL tables or params");
  XNN_REQUIRE(n_nodes == 0 || (cn_d4 && cn_raw), "NULL output");
  if (n_nodes == 0) return XNN_OK;
  const D4Work w = d4_work(n_nodes, n_graphs, max_atoms);
  const size_t need = (size_t)(w.n_cy * 2 * n_nodes) * sizeof(double);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small (%zu < %zu)",
              workspace_bytes, need);
  const CnParams p{prm->cutoff_cn, prm->cutoff_eeq_cn, prm->kcn, prm->k4, prm->k5, prm->k6};
  hipStream_t s = as_hip(stream);
  double* part = static_cast<double*>(workspace);
  hipLaunchKernelGGL(d4_cn_kernel<false>, dim3((unsigned)w.n_tiles, (unsigned)w.n_cy),
                     dim3(kD4Tile), 0, s, pos, n_nodes, species, batch, node_ptr, cell, images,
                     rcov, en, p, nullptr, nullptr, w.chunk, w.n_cy, part);
  XNN_LAUNCH_CHECK();
  reduce_into(part, n_nodes, 2, 0, 1, w.n_cy, cn_d4, s);
  reduce_into(part, n_nodes, 2, 1, 1, w.n_cy, cn_raw, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d4_coordination_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                                 const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                                 int64_t max_atoms, const double* cell, const int32_t* images,
                                 const double* rcov, const double* en,
                                 const xnn_d4_cn_params* prm, const double* g_cn_d4,
                                 const double* g_cn_raw, double* grad_pos, double* cell_partial,
                                 void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  const int st = d4_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images, max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(prm && rcov && en, "NULL tables or params");
  XNN_REQUIRE(n_nodes == 0 || grad_pos, "NULL grad_pos");
  if (n_nodes == 0) return XNN_OK;
  const D4Work w = d4_work(n_nodes, n_graphs, max_atoms);
  const size_t need = (size_t)(w.n_cy * 12 * n_nodes) * sizeof(double);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small (%zu < %zu)",
              workspace_bytes, need);
  const CnParams p{prm->cutoff_cn, prm->cutoff_eeq_cn, prm->kcn, prm->k4, prm->k5, prm->k6};
  hipStream_t s = as_hip(stream);
  double* part = static_cast<double*>(workspace);
  hipLaunchKernelGGL(d4_cn_kernel<true>, dim3((unsigned)w.n_tiles, (unsigned)w.n_cy),
                     dim3(kD4Tile), 0, s, pos, n_nodes, species, batch, node_ptr, cell, images,
                     rcov, en, p, g_cn_d4, g_cn_raw, w.chunk, w.n_cy, part);
  XNN_LAUNCH_CHECK();
  reduce_into(part, n_nodes, 12, 0, 3, w.n_cy, grad_pos, s);
  reduce_into(part, n_nodes, 12, 3, 9, w.n_cy, cell_partial, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d4_two_body(const double* pos, int64_t n_nodes, const int32_t* species,
                    const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                    int64_t max_atoms, const double* cell, const int32_t* images,
                    const double* r4r2, const double* alpha, const xnn_d4_pair_params* prm,
                    double* e2, void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  const int st = d4_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images, max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(prm && r4r2, "NULL tables or params");
  XNN_REQUIRE(n_nodes == 0 || (alpha && e2), "NULL alpha or output");
  XNN_REQUIRE(prm->cutoff > 0.0, "pair cutoff must be positive");
  if (n_nodes == 0) return XNN_OK;
  const D4Work w = d4_work(n_nodes, n_graphs, max_atoms);
  const size_t need = (size_t)(w.n_cy * n_nodes) * sizeof(double);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small (%zu < %zu)",
              workspace_bytes, need);
  hipStream_t s = as_hip(stream);
  const PairParams p{prm->s6, prm->s8, prm->a1, prm->a2, prm->cutoff, prm->width};
  double* part = static_cast<double*>(workspace);
  hipLaunchKernelGGL(d4_pair_kernel<false>, dim3((unsigned)w.n_tiles, (unsigned)w.n_cy),
                     dim3(kD4Tile), 0, s, pos, n_nodes, species, batch, node_ptr, cell, images,
                     r4r2, alpha, p, nullptr, w.chunk, w.n_cy, part, nullptr);
  XNN_LAUNCH_CHECK();
  reduce_into(part, n_nodes, 1, 0, 1, w.n_cy, e2, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d4_two_body_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                             const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                             int64_t max_atoms, const double* cell, const int32_t* images,
                             const double* r4r2, const double* alpha,
                             const xnn_d4_pair_params* prm, const double* g_e2, double* grad_pos,
                             double* cell_partial, double* grad_alpha, void* workspace,
                             size_t workspace_bytes, xnn_stream_t stream) {
  const int st = d4_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images, max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(prm && r4r2, "NULL tables or params");
  XNN_REQUIRE(n_nodes == 0 || (alpha && g_e2 && grad_pos), "NULL alpha, g_e2 or grad_pos");
  XNN_REQUIRE(prm->cutoff > 0.0, "pair cutoff must be positive");
  if (n_nodes == 0) return XNN_OK;
  const D4Work w = d4_work(n_nodes, n_graphs, max_atoms);
  const size_t need = (size_t)(w.n_cy * (12 + kNW) * n_nodes) * sizeof(double);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small (%zu < %zu)",
              workspace_bytes, need);
  hipStream_t s = as_hip(stream);
  const PairParams p{prm->s6, prm->s8, prm->a1, prm->a2, prm->cutoff, prm->width};
  double* part = static_cast<double*>(workspace);
  double* part_a = part + w.n_cy * 12 * n_nodes;
  hipLaunchKernelGGL(d4_pair_kernel<true>, dim3((unsigned)w.n_tiles, (unsigned)w.n_cy),
                     dim3(kD4Tile), 0, s, pos, n_nodes, species, batch, node_ptr, cell, images,
                     r4r2, alpha, p, g_e2, w.chunk, w.n_cy, part, part_a);
  XNN_LAUNCH_CHECK();
  reduce_into(part, n_nodes, 12, 0, 3, w.n_cy, grad_pos, s);
  reduce_into(part, n_nodes, 12, 3, 9, w.n_cy, cell_partial, s);
  reduce_into(part_a, n_nodes, kNW, 0, kNW, w.n_cy, grad_alpha, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d3_coordination(const double* pos, int64_t n_nodes, const int32_t* species,
                        const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                        int64_t max_atoms, const double* cell, const int32_t* images,
                        const double* rcov, double cutoff_cn, double kcn, double* cn,
                        void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  const int st = d4_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images, max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(rcov != nullptr, "NULL rcov");
  XNN_REQUIRE(n_nodes == 0 || cn, "NULL output");
  if (n_nodes == 0) return XNN_OK;
  const D4Work w = d4_work(n_nodes, n_graphs, max_atoms);
  const size_t need = (size_t)(w.n_cy * 2 * n_nodes) * sizeof(double);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small (%zu < %zu)",
              workspace_bytes, need);
  const CnParams p{cutoff_cn, 0.0, kcn, 0.0, 0.0, 1.0};
  hipStream_t s = as_hip(stream);
  double* part = static_cast<double*>(workspace);
  hipLaunchKernelGGL((d4_cn_kernel<false, true>), dim3((unsigned)w.n_tiles, (unsigned)w.n_cy),
                     dim3(kD4Tile), 0, s, pos, n_nodes, species, batch, node_ptr, cell, images,
                     rcov, rcov, p, nullptr, nullptr, w.chunk, w.n_cy, part);
  XNN_LAUNCH_CHECK();
  reduce_into(part, n_nodes, 2, 0, 1, w.n_cy, cn, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d3_coordination_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                                 const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                                 int64_t max_atoms, const double* cell, const int32_t* images,
                                 const double* rcov, double cutoff_cn, double kcn,
                                 const double* g_cn, double* grad_pos, double* cell_partial,
                                 void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  const int st = d4_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images, max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(rcov != nullptr, "NULL rcov");
  XNN_REQUIRE(n_nodes == 0 || (grad_pos && g_cn), "NULL g_cn or grad_pos");
  if (n_nodes == 0) return XNN_OK;
  const D4Work w = d4_work(n_nodes, n_graphs, max_atoms);
  const size_t need = (size_t)(w.n_cy * 12 * n_nodes) * sizeof(double);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small (%zu < %zu)",
              workspace_bytes, need);
  const CnParams p{cutoff_cn, 0.0, kcn, 0.0, 0.0, 1.0};
  hipStream_t s = as_hip(stream);
  double* part = static_cast<double*>(workspace);
  hipLaunchKernelGGL((d4_cn_kernel<true, true>), dim3((unsigned)w.n_tiles, (unsigned)w.n_cy),
                     dim3(kD4Tile), 0, s, pos, n_nodes, species, batch, node_ptr, cell, images,
                     rcov, rcov, p, g_cn, nullptr, w.chunk, w.n_cy, part);
  XNN_LAUNCH_CHECK();
  reduce_into(part, n_nodes, 12, 0, 3, w.n_cy, grad_pos, s);
  reduce_into(part, n_nodes, 12, 3, 9, w.n_cy, cell_partial, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

static int d3_pair_check(const xnn_d3_pair_params* prm, const double* r4r2, const double* rvdw,
                         const double* c6ref, int n_species) {
  XNN_REQUIRE(prm && r4r2 && rvdw && c6ref, "NULL tables or params");
  XNN_REQUIRE(n_species >= 1, "n_species must be >= 1");
  XNN_REQUIRE(prm->damping >= 0 && prm->damping <= 3, "damping must be 0..3 (bj, zero, mzero, op)");
  XNN_REQUIRE(prm->cutoff > 0.0, "pair cutoff must be positive");
  return XNN_OK;
}

static D3PairParams d3_params(const xnn_d3_pair_params* p) {
  return D3PairParams{p->s6, p->s8, p->a1, p->a2, p->rs6, p->rs8, p->alp, p->bet, p->cutoff,
                      p->width, p->damping};
}

int xnn_d3_two_body(const double* pos, int64_t n_nodes, const int32_t* species,
                    const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                    int64_t max_atoms, const double* cell, const int32_t* images,
                    const double* r4r2, const double* rvdw, const double* c6ref,
                    int32_t n_species, const double* weights, const xnn_d3_pair_params* prm,
                    double* e2, void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  const int st = d4_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images, max_atoms);
  if (st != XNN_OK) return st;
  const int st2 = d3_pair_check(prm, r4r2, rvdw, c6ref, n_species);
  if (st2 != XNN_OK) return st2;
  XNN_REQUIRE(n_nodes == 0 || (weights && e2), "NULL weights or output");
  if (n_nodes == 0) return XNN_OK;
  const D4Work w = d4_work(n_nodes, n_graphs, max_atoms);
  const size_t need = (size_t)(w.n_cy * n_nodes) * sizeof(double);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small (%zu < %zu)",
              workspace_bytes, need);
  hipStream_t s = as_hip(stream);
  double* part = static_cast<double*>(workspace);
  {
    const size_t sv_bytes = (size_t)n_species * kD3SvStride * sizeof(double);
    const bool staged = n_species <= kD3MaxStaged, bj = prm->damping == 0;
    auto k = staged ? (bj ? d3_pair_kernel<false, true, true> : d3_pair_kernel<false, true, false>)
                    : (bj ? d3_pair_kernel<false, false, true> : d3_pair_kernel<false, false, false>);
    hipLaunchKernelGGL(k, dim3((unsigned)w.n_tiles, (unsigned)w.n_cy), dim3(kD4Tile),
                       staged ? sv_bytes : 0, s, pos, n_nodes, species, batch, node_ptr, cell,
                       images, r4r2, rvdw, c6ref, n_species, weights, d3_params(prm), nullptr, w.chunk, w.n_cy, part,
                       nullptr);
  }
  XNN_LAUNCH_CHECK();
  reduce_into(part, n_nodes, 1, 0, 1, w.n_cy, e2, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d3_two_body_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                             const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                             int64_t max_atoms, const double* cell, const int32_t* images,
                             const double* r4r2, const double* rvdw, const double* c6ref,
                             int32_t n_species, const double* weights,
                             const xnn_d3_pair_params* prm, const double* g_e2, double* grad_pos,
                             double* cell_partial, double* grad_weights, void* workspace,
                             size_t workspace_bytes, xnn_stream_t stream) {
  const int st = d4_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images, max_atoms);
  if (st != XNN_OK) return st;
  const int st2 = d3_pair_check(prm, r4r2, rvdw, c6ref, n_species);
  if (st2 != XNN_OK) return st2;
  XNN_REQUIRE(n_nodes == 0 || (weights && g_e2 && grad_pos), "NULL weights, g_e2 or grad_pos");
  if (n_nodes == 0) return XNN_OK;
  const D4Work w = d4_work(n_nodes, n_graphs, max_atoms);
  const size_t need = (size_t)(w.n_cy * (12 + kNR) * n_nodes) * sizeof(double);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small (%zu < %zu)",
              workspace_bytes, need);
  hipStream_t s = as_hip(stream);
  double* part = static_cast<double*>(workspace);
  double* part_w = part + w.n_cy * 12 * n_nodes;
  {
    const size_t sv_bytes = (size_t)n_species * kD3SvStride * sizeof(double);
    const bool staged = n_species <= kD3MaxStaged, bj = prm->damping == 0;
    auto k = staged ? (bj ? d3_pair_kernel<true, true, true> : d3_pair_kernel<true, true, false>)
                    : (bj ? d3_pair_kernel<true, false, true> : d3_pair_kernel<true, false, false>);
    hipLaunchKernelGGL(k, dim3((unsigned)w.n_tiles, (unsigned)w.n_cy), dim3(kD4Tile),
                       staged ? sv_bytes : 0, s, pos, n_nodes, species, batch, node_ptr, cell,
                       images, r4r2, rvdw, c6ref, n_species, weights, d3_params(prm), g_e2, w.chunk, w.n_cy, part,
                       part_w);
  }
  XNN_LAUNCH_CHECK();
  reduce_into(part, n_nodes, 12, 0, 3, w.n_cy, grad_pos, s);
  reduce_into(part, n_nodes, 12, 3, 9, w.n_cy, cell_partial, s);
  reduce_into(part_w, n_nodes, kNR, 0, kNR, w.n_cy, grad_weights, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

static int alpha_tables(const xnn_d4_alpha_tables* t, AlphaTables& T) {
  XNN_REQUIRE(t != nullptr, "NULL tables");
  XNN_REQUIRE(t->n_elements >= 1, "empty tables");
  XNN_REQUIRE(t->nref && t->ngw && t->refcn && t->refq && t->zeff && t->gi && t->refalpha,
              "NULL table");
  T = AlphaTables{t->n_elements, t->nref, t->ngw, t->refcn, t->refq, t->zeff, t->gi,
                  t->refalpha, t->ga, t->wf};
  return XNN_OK;
}

int xnn_d4_polarizabilities(int64_t n_nodes, const int64_t* atomic_numbers, const double* cn,
                            const double* q, const xnn_d4_alpha_tables* tables, double* alpha,
                            xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0, "negative size");
  AlphaTables T;
  const int st = alpha_tables(tables, T);
  if (st != XNN_OK) return st;
  if (n_nodes == 0) return XNN_OK;
  XNN_REQUIRE(atomic_numbers && cn && q && alpha, "NULL input or output");
  hipLaunchKernelGGL(d4_alpha_kernel<false>, dim3(grid_1d(n_nodes, 256)), dim3(256), 0,
                     as_hip(stream), n_nodes, atomic_numbers, cn, q, T, nullptr, alpha, nullptr,
                     nullptr);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d4_polarizabilities_backward(int64_t n_nodes, const int64_t* atomic_numbers,
                                     const double* cn, const double* q,
                                     const xnn_d4_alpha_tables* tables, const double* g_alpha,
                                     double* g_cn, double* g_q, xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0, "negative size");
  AlphaTables T;
  const int st = alpha_tables(tables, T);
  if (st != XNN_OK) return st;
  if (n_nodes == 0 || (g_cn == nullptr && g_q == nullptr)) return XNN_OK;
  XNN_REQUIRE(atomic_numbers && cn && q && g_alpha, "NULL input");
  hipLaunchKernelGGL(d4_alpha_kernel<true>, dim3(grid_1d(n_nodes, 256)), dim3(256), 0,
                     as_hip(stream), n_nodes, atomic_numbers, cn, q, T, g_alpha, nullptr, g_cn,
                     g_q);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d3_weights(int64_t n_nodes, const int32_t* species, const double* cn,
                   int32_t n_species, const int32_t* nref, const double* refcn, double wf,
                   double* weights, xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_species >= 1, "negative size or no species");
  XNN_REQUIRE(nref && refcn, "NULL tables");
  if (n_nodes == 0) return XNN_OK;
  XNN_REQUIRE(species && cn && weights, "NULL input or output");
  hipLaunchKernelGGL(d3_weights_kernel<false>, dim3(grid_1d(n_nodes, 256)), dim3(256), 0,
                     as_hip(stream), n_nodes, species, cn, (int)n_species, nref, refcn, wf,
                     nullptr, weights, nullptr);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d3_weights_backward(int64_t n_nodes, const int32_t* species, const double* cn,
                            int32_t n_species, const int32_t* nref, const double* refcn,
                            double wf, const double* g_weights, double* g_cn,
                            xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_species >= 1, "negative size or no species");
  XNN_REQUIRE(nref && refcn, "NULL tables");
  if (n_nodes == 0) return XNN_OK;
  XNN_REQUIRE(species && cn && g_weights && g_cn, "NULL input or output");
  hipLaunchKernelGGL(d3_weights_kernel<true>, dim3(grid_1d(n_nodes, 256)), dim3(256), 0,
                     as_hip(stream), n_nodes, species, cn, (int)n_species, nref, refcn, wf,
                     g_weights, nullptr, g_cn);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

}  // extern "C"
