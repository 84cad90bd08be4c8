// D3 dispersion pair terms on lattice images and the D4 polarizabilities (gfx950, wave64,
// float64). The D4 coordination numbers and two-body term walk spatially ordered tiles
// (d4_tiles.hip).
//
// xnn_d3_coordination(_backward)  DFTD3.coordination_numbers (d3.py:632-642), the
//                                 exponential count
// xnn_d3_two_body(_backward)      DFTD3.pair_c6 / two_body_energy (d3.py:651-722): C6
//                                 from per-atom reference weights and the species-pair
//                                 reference block, bj / zero / mzero / op damping
// xnn_d4_polarizabilities(_backward)  DFTD4.weights / polarizabilities (d4.py:984-1042)
//
// No edge list: the long pair cutoff (60 bohr by default) makes the image list dense,
// so the D3 kernels walk all (receiver, source, image) triples of each structure. Work
// item = one wave: a tile of 64 consecutive receivers (one per lane) against one chunk
// of source atoms, staged through LDS 64 at a time; images are looped in registers.
// Every directed pair is evaluated by its receiver's lane, both directions of a pair
// use their own weights, so forces need no scatter. Each item writes per-receiver
// partials for its chunk; the reductions sum the chunks in a fixed order
// (deterministic, no atomics). Positions and cells in Angstrom, lengths in the kernel
// in bohr, all float64.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "common.h"
#include "device.h"
#include "d4_geom.h"
#include "fp64.h"

namespace xnn {

constexpr int kD4Tile = 64;     // receivers per item (lanes of one wave)
constexpr int kD4Sub = 64;      // sources per LDS stage
constexpr int kD4MaxChunks = 128;

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

// source data staged in LDS (one stage of kD4Sub atoms)
struct D4Stage {
  double x[kD4Sub], y[kD4Sub], z[kD4Sub];
  double w[kD4Sub];       // backward weight of the source (its upstream gradient)
  double p[kD4Sub], q[kD4Sub];  // per-source table values (CN: rcov; pair: r4r2 and its
                                // square root), read once per stage, not per pair
  int sp[kD4Sub];         // species
  int b[kD4Sub];          // structure
};

// ---------------------------------------------------------------- D3 coordination numbers
// The exponential count 1 / (1 + exp(-k1 (rc / r - 1))) within cut_cn (d3.py:632-642).
// BACKWARD = false: partial[cy][0][i] = the count of this chunk (np = 2, component 1 unused).
// BACKWARD = true:  partial[cy][0..11][i] = grad_pos (3), cell gradient n (x) g (9).
template <bool BACKWARD>
__global__ __launch_bounds__(64, 3) void d3_cn_kernel(
    const double* __restrict__ pos, int64_t n_nodes, const int32_t* __restrict__ species,
    const int32_t* __restrict__ batch, const int64_t* __restrict__ node_ptr,
    const double* __restrict__ cell, const int32_t* __restrict__ images,
    const double* __restrict__ rcov, CnParams prm, const double* __restrict__ g_cn,
    int64_t chunk, int64_t n_cy, double* __restrict__ partial) {
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
  double xi = 0, yi = 0, zi = 0, rci = 0, gi = 0;
  int bi = -1;
  Lattice L;
  if (live) {
    xi = pos[3 * i];
    yi = pos[3 * i + 1];
    zi = pos[3 * i + 2];
    rci = rcov[species[i]];
    bi = batch[i];
    if (BACKWARD) gi = g_cn[i];
    load_lattice(cell, images, bi, L);
  } else {
    load_lattice(nullptr, nullptr, 0, L);
  }
  const double cmax = prm.cut_cn;
  for (int64_t base = j0; base < j1; base += kD4Sub) {
    const int cnt = (int)std::min<int64_t>(kD4Sub, j1 - base);
    __syncthreads();
    if (lane < cnt) {
      const int64_t j = base + lane;
      st.x[lane] = pos[3 * j];
      st.y[lane] = pos[3 * j + 1];
      st.z[lane] = pos[3 * j + 2];
      st.b[lane] = batch[j];
      st.p[lane] = rcov[species[j]];
      if (BACKWARD) st.w[lane] = g_cn[j];
    }
    __syncthreads();
    if (!live) continue;
    for (int jj = 0; jj < cnt; ++jj) {
      if (st.b[jj] != bi) continue;
      const double rc = rci + st.p[jj];
      const double dx = xi - st.x[jj], dy = yi - st.y[jj], dz = zi - st.z[jj];
      const double bx = dx * kInvBohr, by = dy * kInvBohr, bz = dz * kInvBohr;
      const double wsum = BACKWARD ? gi + st.w[jj] : 0.0;
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
            // d/dr of the count = -s (1 - s) k1 rc / r^2
            const double sg = rcp_nr(1.0 + exp(-prm.kcn * (rc * rinv - 1.0)));
            if (!BACKWARD) {
              acc[0] += sg;
            } else {
              const double dcount = -sg * (1.0 - sg) * prm.kcn * rc * rinv * rinv;
              // per Angstrom of the edge vector: d r_bohr / d v = v_bohr / (r bohr)
              const double s = dcount * rinv * kInvBohr;
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
    }
  }
  if (live) {
#pragma unroll
    for (int k = 0; k < NP; ++k) partial[((int64_t)cy * NP + k) * n_nodes + i] = acc[k];
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
  // the D3 kernels' largest user, the pair backward: 12 + 7 values per receiver and chunk
  // slot; the D4 tile kernels: their own layout
  const size_t d3 = (size_t)(w.n_cy * (12 + kNR) * n_nodes) * sizeof(double);
  return std::max(d3, d4_tiles_workspace_bytes(n_nodes, n_graphs, max_atoms));
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
  hipLaunchKernelGGL(d3_cn_kernel<false>, dim3((unsigned)w.n_tiles, (unsigned)w.n_cy),
                     dim3(kD4Tile), 0, s, pos, n_nodes, species, batch, node_ptr, cell, images,
                     rcov, p, nullptr, w.chunk, w.n_cy, part);
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
  hipLaunchKernelGGL(d3_cn_kernel<true>, dim3((unsigned)w.n_tiles, (unsigned)w.n_cy),
                     dim3(kD4Tile), 0, s, pos, n_nodes, species, batch, node_ptr, cell, images,
                     rcov, p, g_cn, w.chunk, w.n_cy, part);
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
