// The Axilrod-Teller-Muto three-body dispersion term of D4 and D3 over an edge list
// (gfx950, wave64, float64).
//
// xnn_atm_plan_size, xnn_atm_plan  the triplet plan of an edge list
//                                  (dispersion_fast/atm.py:318-352): the edges sorted by
//                                  (center, neighbor), per-center edge ranges and the
//                                  centers that have repeated-atom triangles
// xnn_atm_work_size, xnn_atm_energy
//                                  per-atom energies (atm.py:84-162, 380-399, the formula
//                                  of dispersion.py:183-222)
// xnn_atm_energy_backward          their gradients in the edge vectors and in both C6
//                                  factor matrices (atm.py:165-294, 402-443)
// xnn_atm_tangent_work_size, xnn_atm_energy_backward_tangent
//                                  second derivatives: the tangents of the energies and
//                                  of those gradients along a direction (atm.py:475-509,
//                                  atm_tangents.py)
//
// Bookkeeping (dispersion.py:253-270, 343-398): a triangle of three distinct atoms is
// evaluated once, from its smallest-index corner c (the pairs among c's edges to
// larger-index neighbors), and a third of its energy goes to each corner; a triangle with
// a repeated atom (an atom and its own periodic image, or two images of one neighbor) is
// evaluated at every visit, its third going to the visiting center. The per-atom
// energies are those of visiting every corner.
//
// Distinct triangles: work item = one wave = a center c and a tile of 64 of its edges to
// larger-index neighbors, a = (j -> c) one per lane; the wave walks the later edges
// b = (k -> c) of c in lockstep. b is wave-uniform, so its 64-byte record and the C6
// factor row of k load through the scalar unit, the per-lane sums (edge a, atom j) stay
// in registers until the item ends, and the per-b sums (edge b, atom k) are reduced
// across the wave once per b (in the backward a transposing butterfly that leaves each
// lane pair holding one of up to 32 sums) and added atomically as reproducible sums: a
// head and a tail of fixed quanta whose float64 sums are exact in any order (atm_acc), so
// the results do not depend on the order of the atomics. Items run heaviest tile first.
// Repeated-atom triangles: one wave per flagged center, lanes over its edges, each lane
// walking the few later edges that share an atom with its own.
//
// Pair C6 = <fa[x], fb[y]> over K <= 32 components (held per lane for j); the damping
// radius is the product of three species-pair factors. Energies in hartree, lengths in
// bohr.
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cstdint>

#include "common.h"
#include "device.h"
#include "fp64.h"

namespace xnn {

constexpr int kAtmTile = 64;          // upper edges per item, one per lane
constexpr int kAtmWaves = 4;          // waves (centers) per block
constexpr int kAtmMaxK = 32;          // C6 factor components
constexpr int kAtmMaxSpecies = 32;    // side of the damping-radius factor table
constexpr double kAtmEps = 2.220446049250313e-16;   // lower bound on r_jk^2 (dispersion.py:200)

// one edge (j -> c) as the triplet kernels read it (one 64-byte scalar load)
struct __align__(16) AtmEdge {
  double vx, vy, vz;   // edge vector, bohr
  double c6;           // <fa[c], fb[j]>
  double p;            // damping-radius factor of the species pair (c, j)
  double sw;           // switch at r = |v|
  double dsw;          // its slope in r^2: sw'(r) / (2 r)
  uint32_t nbs;        // the neighbor j (low 26 bits) and its species (high 6)
  int32_t pos;         // the edge's position in the (center, neighbor) order
};
static_assert(sizeof(AtmEdge) == 64, "AtmEdge is one 64-byte record");
constexpr int kAtmNbBits = 26;         // atoms < 2^26

__device__ __forceinline__ int32_t atm_nb(const AtmEdge& e) {
  return (int32_t)(e.nbs & ((1u << kAtmNbBits) - 1u));
}
__device__ __forceinline__ int atm_snb(const AtmEdge& e) { return (int)(e.nbs >> kAtmNbBits); }

// 30-bit Morton code of an edge vector inside the cutoff sphere (10 bits per axis)
__device__ __forceinline__ uint32_t atm_spread10(uint32_t v) {
  v &= 0x3ffu;
  v = (v | (v << 16)) & 0x030000ffu;
  v = (v | (v << 8)) & 0x0300f00fu;
  v = (v | (v << 4)) & 0x030c30c3u;
  v = (v | (v << 2)) & 0x09249249u;
  return v;
}
__device__ __forceinline__ uint32_t atm_morton(double x, double y, double z, double inv_2rc) {
  const auto q = [&](double t) {
    const double u = (t * inv_2rc + 0.5) * 1024.0;
    return (uint32_t)(u < 0.0 ? 0.0 : (u > 1023.0 ? 1023.0 : u));
  };
  return (atm_spread10(q(x)) << 2) | (atm_spread10(q(y)) << 1) | atm_spread10(q(z));
}

struct AtmConst {
  double s9_3;         // s9 / 3: a third of every triangle per corner
  double alp3;
  double cut2;
  double cutoff;
  double width;        // <= 0: sharp cutoff
};

static size_t atm_align(size_t x) { return (x + 255) & ~(size_t)255; }

struct AtmPlanLayout {
  size_t keys, perm, nbr, ctr, lo, lo1, flag, stats, by_src, lo_src, keys_in, vals_in, keys2,
      cub, cub_bytes, total;
};

static int atm_end_bit(int64_t n) {
  const uint64_t top = (uint64_t)n * (uint64_t)n;   // the out-of-range sentinel key
  int b = 1;
  while (b < 64 && (top >> b) != 0) ++b;
  return b;
}

static AtmPlanLayout atm_plan_layout(int64_t E, int64_t N) {
  AtmPlanLayout L;
  size_t at = 0;
  L.keys = at; at += atm_align(sizeof(uint64_t) * std::max<int64_t>(E, 1));
  L.perm = at; at += atm_align(sizeof(int32_t) * std::max<int64_t>(E, 1));
  L.nbr = at; at += atm_align(sizeof(int32_t) * std::max<int64_t>(E, 1));
  L.ctr = at; at += atm_align(sizeof(int32_t) * std::max<int64_t>(E, 1));
  L.lo = at; at += atm_align(sizeof(int32_t) * (N + 1));
  L.lo1 = at; at += atm_align(sizeof(int32_t) * std::max<int64_t>(N, 1));
  L.flag = at; at += atm_align(sizeof(int32_t) * std::max<int64_t>(N, 1));
  L.stats = at; at += atm_align(sizeof(int32_t) * 4);
  L.by_src = at; at += atm_align(sizeof(int32_t) * std::max<int64_t>(E, 1));
  L.lo_src = at; at += atm_align(sizeof(int32_t) * (N + 1));
  L.keys_in = at; at += atm_align(sizeof(uint64_t) * std::max<int64_t>(E, 1));
  L.vals_in = at; at += atm_align(sizeof(int32_t) * std::max<int64_t>(E, 1));
  L.keys2 = at; at += atm_align(sizeof(uint64_t) * std::max<int64_t>(E, 1));
  size_t cub_bytes = 0;
  (void)hipcub::DeviceRadixSort::SortPairs(nullptr, cub_bytes, (uint64_t*)nullptr,
                                           (uint64_t*)nullptr, (int32_t*)nullptr,
                                           (int32_t*)nullptr, (int)std::max<int64_t>(E, 1), 0,
                                           atm_end_bit(N));
  L.cub = at;
  L.cub_bytes = atm_align(cub_bytes + 256);
  at += L.cub_bytes;
  L.total = at;
  return L;
}

struct AtmWorkLayout {
  size_t rec, rec_up, fa, fb, gs, skey, sval, skey_out, sperm, cub, cub_bytes, tail,
      tail_count, total;
};

static int atm_bitlen(int64_t n) {
  int b = 1;
  while (b < 62 && (n >> b) != 0) ++b;
  return b;
}

static AtmWorkLayout atm_work_layout(int64_t E, int64_t N, int kp, bool backward) {
  AtmWorkLayout L;
  size_t at = 0;
  const int64_t e1 = std::max<int64_t>(E, 1);
  L.rec = at; at += atm_align(sizeof(AtmEdge) * e1);
  L.rec_up = at; at += atm_align(sizeof(AtmEdge) * e1);
  L.skey = at; at += atm_align(sizeof(uint64_t) * e1);
  L.sval = at; at += atm_align(sizeof(int32_t) * e1);
  L.skey_out = at; at += atm_align(sizeof(uint64_t) * e1);
  L.sperm = at; at += atm_align(sizeof(int32_t) * e1);
  size_t cub_bytes = 0;
  (void)hipcub::DeviceRadixSort::SortPairs(nullptr, cub_bytes, (uint64_t*)nullptr,
                                           (uint64_t*)nullptr, (int32_t*)nullptr,
                                           (int32_t*)nullptr, (int)e1, 0,
                                           33 + atm_bitlen(std::max<int64_t>(N, 1)));
  L.cub = at;
  L.cub_bytes = atm_align(cub_bytes + 256);
  at += L.cub_bytes;
  L.fa = at; at += atm_align(sizeof(double) * kp * std::max<int64_t>(N, 1));
  L.fb = at; at += atm_align(sizeof(double) * kp * std::max<int64_t>(N, 1));
  L.gs = at;
  if (backward) at += atm_align(sizeof(double) * 4 * std::max<int64_t>(E, 1));
  // the tails of the reproducible sums: energies (forward); or gs, gfa and gfb (backward)
  L.tail = at;
  L.tail_count = backward ? 4 * E + 2 * N * (int64_t)kp : N;
  at += atm_align(sizeof(double) * std::max<int64_t>((int64_t)L.tail_count, 1));
  L.total = at;
  return L;
}

template <typename T>
static T* at_off(void* base, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}
template <typename T>
static const T* at_off(const void* base, size_t off) {
  return reinterpret_cast<const T*>(static_cast<const char*>(base) + off);
}

// ------------------------------------------------------------------------------ plan
__global__ __launch_bounds__(256) void atm_fill_i32_kernel(int32_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

__global__ __launch_bounds__(256) void atm_fill_f64_kernel(double* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0;
}

// head[i] += tail[i]: the one rounding of a reproducible sum
__global__ __launch_bounds__(256) void atm_add_tail_kernel(double* __restrict__ head,
                                                           const double* __restrict__ tail,
                                                           int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) head[i] += tail[i];
}

// key = center * N + neighbor; an index out of range gets the sentinel N^2 (sorted last)
// and raises the plan's error flag
__global__ __launch_bounds__(256) void atm_keys_kernel(const int64_t* __restrict__ ei, int64_t E, int64_t N,
                                uint64_t* __restrict__ keys, int32_t* __restrict__ vals,
                                int32_t* __restrict__ stats) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int64_t s = ei[e], d = ei[E + e];
  uint64_t key = (uint64_t)N * (uint64_t)N;
  if (s >= 0 && s < N && d >= 0 && d < N)
    key = (uint64_t)d * (uint64_t)N + (uint64_t)s;
  else
    stats[2] = 1;
  keys[e] = key;
  vals[e] = (int32_t)e;
}

__device__ inline int64_t atm_lower_bound(const uint64_t* __restrict__ keys, int64_t n,
                                          uint64_t v) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < v)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// neighbor of every sorted edge; a center with two edges to images of one neighbor has
// repeated-atom triangles
__global__ __launch_bounds__(256) void atm_neighbors_kernel(const uint64_t* __restrict__ keys, int64_t E, int64_t N,
                                     int32_t* __restrict__ nbr, int32_t* __restrict__ ctr,
                                     uint64_t* __restrict__ keys2, int32_t* __restrict__ vals2,
                                     int32_t* __restrict__ flag, int32_t* __restrict__ stats) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= E) return;
  const uint64_t k = keys[p];
  const uint64_t top = (uint64_t)N * (uint64_t)N;
  const uint64_t cj = k < top ? k / (uint64_t)N : 0, jj = k < top ? k % (uint64_t)N : 0;
  nbr[p] = (int32_t)jj;
  ctr[p] = (int32_t)cj;
  // (neighbor, center) keys: the by-source order of the backward's center sides
  keys2[p] = k < top ? jj * (uint64_t)N + cj : top;
  vals2[p] = (int32_t)p;
  if (k < top && p + 1 < E && keys[p + 1] == k) {
    flag[k / (uint64_t)N] = 1;
    stats[1] = 1;
  }
}

// per-center ranges: [lo[c], lo1[c]) neighbors <= c, [lo1[c], lo[c+1]) neighbors > c; an
// edge to the center's own image flags it; stats[0] = most tiles of upper edges
__global__ __launch_bounds__(256) void atm_rows_kernel(const uint64_t* __restrict__ keys, int64_t E, int64_t N,
                                int32_t* __restrict__ lo, int32_t* __restrict__ lo1,
                                int32_t* __restrict__ flag, int32_t* __restrict__ stats) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c > N) return;
  const uint64_t base = (uint64_t)c * (uint64_t)N;
  const int64_t l = atm_lower_bound(keys, E, base);
  lo[c] = (int32_t)l;
  if (c == N) return;
  const int64_t u = atm_lower_bound(keys, E, base + (uint64_t)c + 1);
  const int64_t h = atm_lower_bound(keys, E, base + (uint64_t)N);
  lo1[c] = (int32_t)u;
  if (u > l && keys[u - 1] == base + (uint64_t)c) {
    flag[c] = 1;
    stats[1] = 1;
  }
  const int64_t n_up = h - u;
  if (n_up >= 2) atomicMax(&stats[0], (int32_t)((n_up + kAtmTile - 1) / kAtmTile));
}

// lo_src[j]: first by-source position of neighbor j
__global__ __launch_bounds__(256) void atm_src_rows_kernel(const uint64_t* __restrict__ keys2, int64_t E, int64_t N,
                                    int32_t* __restrict__ lo_src) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j > N) return;
  lo_src[j] = (int32_t)atm_lower_bound(keys2, E, (uint64_t)j * (uint64_t)N);
}

// ------------------------------------------------------------------------------ records
template <int KP>
__global__ __launch_bounds__(256) void atm_pad_kernel(const double* __restrict__ f, int64_t N, int K,
                               double* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * KP) return;
  const int64_t n = i / KP;
  const int w = (int)(i - n * KP);
  out[i] = w < K ? f[n * K + w] : 0.0;
}

template <int KP>
__global__ __launch_bounds__(256) void atm_edges_kernel(const uint64_t* __restrict__ keys,
                                 const int32_t* __restrict__ perm,
                                 const int32_t* __restrict__ nbr, int64_t E, int64_t N,
                                 const double* __restrict__ vec, const double* __restrict__ fa,
                                 const double* __restrict__ fb,
                                 const int32_t* __restrict__ species,
                                 const double* __restrict__ table, int S, AtmConst kc,
                                 AtmEdge* __restrict__ rec, uint64_t* __restrict__ skey,
                                 int32_t* __restrict__ sval) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= E) return;
  const int64_t e = perm[p];
  const int64_t c = (int64_t)(keys[p] / (uint64_t)N);
  const int32_t j = nbr[p];
  AtmEdge r;
  r.vx = vec[3 * e + 0];
  r.vy = vec[3 * e + 1];
  r.vz = vec[3 * e + 2];
  double c6 = 0.0;
#pragma unroll
  for (int w = 0; w < KP; ++w) c6 = fma(fa[c * KP + w], fb[(int64_t)j * KP + w], c6);
  r.c6 = c6;
  // a species outside the table gives a NaN factor (and stays a valid table index)
  const int sc = species[c], sj = species[j];
  const bool ok = sc >= 0 && sc < S && sj >= 0 && sj < S;
  r.p = ok ? table[sc * S + sj] : __builtin_nan("");
  r.sw = 1.0;
  r.dsw = 0.0;
  if (kc.width > 0.0) {
    const double r2 = r.vx * r.vx + r.vy * r.vy + r.vz * r.vz;
    const double len = sqrt(r2);
    double sw, dsw;
    switch_d(len, kc.cutoff, kc.width, sw, dsw);
    r.sw = sw;
    r.dsw = len > 0.0 ? 0.5 * dsw / len : 0.0;
  }
  r.nbs = (uint32_t)j | ((uint32_t)(sj >= 0 && sj < S ? sj : 0) << kAtmNbBits);
  r.pos = (int32_t)p;
  rec[p] = r;
  // the walk order of the distinct-triangle kernel: a center's edges to smaller-index
  // neighbors first, in the plan's order (equal keys, stable sort), then its edges to
  // larger-index neighbors along a Morton curve of the edge vector, so that a tile of 64
  // of them is compact in space and the walked edges far from it fail for all lanes
  const bool up = (int64_t)j > c;
  skey[p] = ((uint64_t)c << 33) |
            (up ? ((1ull << 32) | atm_morton(r.vx, r.vy, r.vz, 0.5 / kc.cutoff)) : 0ull);
  sval[p] = (int32_t)p;
}

// the walk-ordered copy of the records
__global__ __launch_bounds__(256) void atm_walk_order_kernel(const AtmEdge* __restrict__ rec,
                                      const int32_t* __restrict__ sperm, int64_t E,
                                      AtmEdge* __restrict__ rec_up) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q < E) rec_up[q] = rec[sperm[q]];
}

// ------------------------------------------------------------------------------ triangle
// q^(16/3), the damping power at the upstream exponent alp / 3 = 16 / 3 (D4: alp = 16; D3:
// (alp + 2) / 3 with alp = 14): q^6 z^2 with z = q^(-1/3) from the single-precision estimate
// 2^(-log2(q) / 3) refined by two Newton steps z <- z (4 - q z^3) / 3 (quadratic: about
// 2e-7, then 1e-13, then rounding); outside [1e-30, 1e30], beyond the estimate's range,
// the general power.
__device__ __forceinline__ double atm_pow_16_3(double q) {
  if (!(q > 1e-30 && q < 1e30)) return exp((16.0 / 3.0) * log(q));
  double z = (double)__builtin_amdgcn_exp2f(-0.333333343f * __builtin_amdgcn_logf((float)q));
  z = z * fma(-q * z, z * z, 4.0) * (1.0 / 3.0);
  z = z * fma(-q * z, z * z, 4.0) * (1.0 / 3.0);
  const double q2 = q * q;
  return q2 * q2 * q2 * (z * z);
}

// The energy of one triangle visit (weight * s9/3 * C9 * angular * damping * switches)
// and, in the backward, its derivatives in the squared sides x = r_cj^2, y = r_ck^2,
// w = r_jk^2 (dispersion.py:183-222; closed form of dispersion.py:413-510). P16: the
// exponent is 16/3.
template <bool SWITCH, bool BWD, bool P16>
__device__ __forceinline__ void atm_triangle(const AtmConst& kc, double x, double y, double w,
                                             double ix, double iy, double c6abs, double r0,
                                             double swa, double swb, double dswa, double dswb,
                                             double weight, double& e, double& gx, double& gy,
                                             double& gw) {
  const double s = rsq_nr(x * y * w);            // 1 / (r_cj r_ck r_jk)
  const double s2 = s * s;
  const double s3 = s2 * s;
  const double s5 = s3 * s2;
  // (R0 / (r_cj r_ck r_jk))^alp3
  const double t = P16 ? atm_pow_16_3(r0 * s) : exp(kc.alp3 * log(r0 * s));
  const double damp = rcp_nr(fma(6.0, t, 1.0));
  const double f1 = x + w - y, f2 = x - w + y, f3 = w + y - x;
  const double nn = f1 * f2 * f3;
  const double ang = fma(0.375 * nn, s5, s3);
  double swjk = 1.0, dswjk = 0.0;
  if (SWITCH) {
    const double r = w * rsq_nr(w);
    double sw, dsw;
    switch_d(r, kc.cutoff, kc.width, sw, dsw);
    swjk = sw;
    dswjk = 0.5 * dsw / r;
  }
  const double sw = swa * swb * swjk;
  const double base = weight * kc.s9_3 * sqrt(c6abs);
  e = base * ang * damp * sw;
  if (BWD) {
    const double iw = rcp_nr(w);
    const double a23 = f2 * f3, a13 = f1 * f3, a12 = f1 * f2;
    const double q = 0.375 * s5;
    const double ang_x = fma(q, fma(-2.5 * nn, ix, a23 + a13 - a12), -1.5 * s3 * ix);
    const double ang_y = fma(q, fma(-2.5 * nn, iy, a13 + a12 - a23), -1.5 * s3 * iy);
    const double ang_w = fma(q, fma(-2.5 * nn, iw, a23 + a12 - a13), -1.5 * s3 * iw);
    const double dc = 3.0 * kc.alp3 * t * damp * damp;   // x d(damp)/dx
    const double bd = base * damp * sw;
    const double ba = base * ang;
    const double dcs = dc * sw;
    gx = fma(bd, ang_x, ba * fma(dcs, ix, damp * dswa * swb * swjk));
    gy = fma(bd, ang_y, ba * fma(dcs, iy, damp * swa * dswb * swjk));
    gw = fma(bd, ang_w, ba * fma(dcs, iw, damp * swa * swb * dswjk));
  }
}

// ------------------------------------------------------------------------------ exchanges
// Cross-lane exchanges of doubles without LDS address arithmetic: gfx950's row-swap permutes
// for the two halves of the wave (lane ^ 32) and the two 16-lane rows of each half (lane ^
// 16), a DPP row rotation by 8 (lane ^ 8 within a row), an xor swizzle for lane ^ 4 and DPP
// quad permutations for lane ^ 2 and lane ^ 1. Every lane of the wave must be active.
struct AtmLanes {
  int unused;
};

__device__ __forceinline__ AtmLanes atm_lanes(int) { return {0}; }

// v_permlane32_swap exchanges lanes 32-63 of its first operand with lanes 0-31 of its second,
// so the sum of its two results is A_l + A_{l+32} on lanes l < 32 and B_{l-32} + B_l on the
// others (a reduce-scatter step that needs no select); v_permlane16_swap does the same for
// the odd and even 16-lane rows (A on rows 0 and 2, B on rows 1 and 3).
__device__ __forceinline__ double atm_swap32_sum(double A, double B) {
  const auto lo = __builtin_amdgcn_permlane32_swap((unsigned)__double2loint(A),
                                                   (unsigned)__double2loint(B), false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap((unsigned)__double2hiint(A),
                                                   (unsigned)__double2hiint(B), false, false);
  return __hiloint2double((int)hi[0], (int)lo[0]) + __hiloint2double((int)hi[1], (int)lo[1]);
}

__device__ __forceinline__ double atm_swap16_sum(double A, double B) {
  const auto lo = __builtin_amdgcn_permlane16_swap((unsigned)__double2loint(A),
                                                   (unsigned)__double2loint(B), false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap((unsigned)__double2hiint(A),
                                                   (unsigned)__double2hiint(B), false, false);
  return __hiloint2double((int)hi[0], (int)lo[0]) + __hiloint2double((int)hi[1], (int)lo[1]);
}

constexpr int kDppXor1 = 0xB1;   // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;   // quad_perm [2, 3, 0, 1]
constexpr int kDppRor8 = 0x128;  // row_ror:8, lane ^ 8 within a 16-lane row

template <int CTRL>
__device__ __forceinline__ double atm_dpp(double v) {
  const int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, 0xF, 0xF, false);
  return __hiloint2double(hi, lo);
}

// lane ^ 4: ds_swizzle in bit mode (and 0x1F, or 0, xor 4)
__device__ __forceinline__ double atm_xor4(double v) {
  const int lo = __builtin_amdgcn_ds_swizzle(__double2loint(v), 0x1F | (4 << 10));
  const int hi = __builtin_amdgcn_ds_swizzle(__double2hiint(v), 0x1F | (4 << 10));
  return __hiloint2double(hi, lo);
}

// the wave-wide sum in every lane (a fixed butterfly: every lane gets the same bits)
__device__ __forceinline__ double atm_wave_sum(double v, const AtmLanes&) {
  v = atm_swap32_sum(v, v);
  v = atm_swap16_sum(v, v);
  v += atm_dpp<kDppRor8>(v);
  v += atm_xor4(v);
  v += atm_dpp<kDppXor2>(v);
  v += atm_dpp<kDppXor1>(v);
  return v;
}

// The wave-wide sums of the 32 products g * f[s] (f zero beyond its length): lanes 2s and
// 2s + 1 return the total of slot s. The first two halvings are row-swap sums (lanes below
// 32 keep slots 0-15, then rows 0 and 2 keep the lower 8 of their 16), the last four
// exchange with lane ^ 8, 4, 2, 1; for those each lane holds its row permuted, fp[i] =
// f[i ^ ((lane >> 1) & 7)], so that at every halving the lane keeps its first half and
// receives its partner's second half, which holds the same slots: no selects.
// fp[i][lane] lives in LDS (a column per lane: conflict-free, and 64 registers fewer).
// atm_fold16 is every halving after the first, atm_fold32 the whole fold.
__device__ __forceinline__ double atm_fold16(double (&p)[16]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = atm_swap16_sum(p[i], p[i + 8]);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] += atm_dpp<kDppRor8>(p[i + 4]);
#pragma unroll
  for (int i = 0; i < 2; ++i) p[i] += atm_xor4(p[i + 2]);
  p[0] += atm_dpp<kDppXor2>(p[1]);
  return p[0] + atm_dpp<kDppXor1>(p[0]);
}

__device__ __forceinline__ double atm_fold32(const double (*fp)[kWave], int lane, double g,
                                             const AtmLanes&) {
  double p[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) p[i] = atm_swap32_sum(g * fp[i][lane], g * fp[i + 16][lane]);
  return atm_fold16(p);
}

// The same sums of g * f[s] + h * u[s] (two permuted tables, one fold).
__device__ __forceinline__ double atm_fold32x2(const double (*fp)[kWave],
                                               const double (*up)[kWave], int lane, double g,
                                               double h) {
  double p[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    p[i] = atm_swap32_sum(fma(h, up[i][lane], g * fp[i][lane]),
                          fma(h, up[i + 16][lane], g * fp[i + 16][lane]));
  return atm_fold16(p);
}

// The wave-wide sums of four per-lane values: lanes 16 s .. 16 s + 15 return slot s.
__device__ __forceinline__ double atm_fold4(double s0, double s1, double s2, double s3,
                                            int, const AtmLanes&) {
  // lanes below 32 keep slots 0 and 1, the others 2 and 3; then rows 0 and 2 keep the first
  const double k0 = atm_swap32_sum(s0, s2);
  const double k1 = atm_swap32_sum(s1, s3);
  double v = atm_swap16_sum(k0, k1);
  v += atm_dpp<kDppRor8>(v);
  v += atm_xor4(v);
  v += atm_dpp<kDppXor2>(v);
  return v + atm_dpp<kDppXor1>(v);
}

// Reproducible sums. Every addend v is split into a head, v rounded to a multiple of
// 2^-40, and a tail, the rest rounded to a multiple of 2^-70 (both splits exact: v - head
// is exact since |v - head| <= 2^-41 and both are multiples of the ulp of v), and the two
// are added atomically to two arrays. Sums of multiples of 2^-40 below 2^13 in magnitude
// and of multiples of 2^-70 below 2^-17 (fewer than 2^24 tails per target) are exact in
// float64, so every order of the atomics gives the same bits: the totals head + tail are
// reproducible run to run, within 2^-71 per addend of the exact sum. Non-finite addends
// give NaN.
struct AtmTail {
  double* energy;   // (N)
  double* gs;       // (E, 4)
  double* gfa;      // (N, K)
  double* gfb;      // (N, K)
};

__device__ __forceinline__ void atm_acc(double* __restrict__ head, double* __restrict__ tail,
                                        int64_t i, double v) {
  const double h = __builtin_rint(v * 0x1p40) * 0x1p-40;
  const double t = __builtin_rint((v - h) * 0x1p70) * 0x1p-70;
  unsafeAtomicAdd(head + i, h);
  unsafeAtomicAdd(tail + i, t);
}

// Per-wave ring of the energies of the last kAtmRing walked edges b (one row per b, one
// column per lane) and their atoms k: the wave sums them 16 rows at a time, a quarter row
// per lane, instead of one butterfly per b.
constexpr int kAtmRing = 16;

__device__ __forceinline__ void atm_ring_flush(double (*ring)[kWave + 1], const int32_t* ring_k,
                                               int n, int lane, const AtmLanes& L,
                                               double* __restrict__ energy,
                                               double* __restrict__ energy_tail) {
  wave_sync();
  const int r = lane & (kAtmRing - 1), q = lane >> 4;
  double v = 0.0;
#pragma unroll
  for (int i = 0; i < kWave / 4; ++i) v += ring[r][q * (kWave / 4) + i];
  v = atm_swap16_sum(v, v);
  v = atm_swap32_sum(v, v);
  if (q == 0 && r < n) atm_acc(energy, energy_tail, ring_k[r], v);
  wave_sync();
}

__device__ __forceinline__ void atm_stage_table(const double* __restrict__ table, int S,
                                                double* sTab) {
  for (int i = threadIdx.x; i < S * S; i += blockDim.x) sTab[i] = table[i];
  __syncthreads();
}

// ------------------------------------------------------------------------------ kernels
// Distinct triangles from their smallest corner. Forward: energy[c], energy[j],
// energy[k] += e. Backward (weights go_c + go_j + go_k): gs[edge] += (dE/dv, dE/dC6) for
// both edges, gfa[j] += dE/dC6_jk fb[k], gfb[k] += dE/dC6_jk fa[j].
template <int KP, bool SWITCH, bool BWD, bool P16>
__global__ __launch_bounds__(kAtmWaves * kWave) void atm_upper_kernel(
    const AtmEdge* __restrict__ rec, const int32_t* __restrict__ lo,
    const int32_t* __restrict__ lo1, int64_t N, int64_t n_groups,
    const double* __restrict__ fa, const double* __restrict__ fb,
    const double* __restrict__ table, int S, AtmConst kc, double* __restrict__ energy,
    const double* __restrict__ go, double* __restrict__ gs, double* __restrict__ gfa,
    double* __restrict__ gfb, int K, AtmTail tail) {
  __shared__ double sTab[kAtmMaxSpecies * kAtmMaxSpecies];
  // the forward's energy ring (one per wave; a placeholder in the backward)
  __shared__ double sRing[BWD ? 1 : kAtmWaves][BWD ? 1 : kAtmRing][kWave + 1];
  __shared__ int32_t sRingK[BWD ? 1 : kAtmWaves][kAtmRing];
  // the backward's permuted factor rows, fp[i][lane] = fa[j][i ^ ((lane >> 1) & 7)]
  __shared__ double sFp[BWD ? kAtmWaves : 1][BWD ? 32 : 1][kWave];
  atm_stage_table(table, S, sTab);
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = wave_in_block();
  const int64_t t = blockIdx.x / n_groups;
  const int64_t c = (blockIdx.x - t * n_groups) * kAtmWaves + wv;
  if (c >= N) return;
  const int32_t hi = lo[c + 1];
  const int32_t a0 = lo1[c] + (int32_t)t * kAtmTile;
  if (a0 + 1 >= hi) return;                       // fewer than two edges left: no pair
  const AtmLanes L = atm_lanes(lane);
  const int32_t a = a0 + lane;
  const bool va = a < hi;
  const AtmEdge ea = rec[va ? a : a0];
  const double ax = ea.vx, ay = ea.vy, az = ea.vz;
  const double x = ax * ax + ay * ay + az * az;
  const double ix = BWD ? rcp_nr(x) : 0.0;
  const double hc6a = BWD ? 0.5 / (ea.c6 != 0.0 ? ea.c6 : 1.0) : 0.0;   // dC9/C9 per dC6_cj
  const int32_t j = atm_nb(ea);
  const int sj = atm_snb(ea);
  double fj[KP];
#pragma unroll
  for (int w = 0; w < KP; ++w) fj[w] = fa[(int64_t)j * KP + w];
  if (BWD) {
    const int m = (lane >> 1) & 7;
#pragma unroll
    for (int i = 0; i < 32; ++i)
      sFp[wv][i][lane] = (i ^ m) < KP ? fa[(int64_t)j * KP + (i ^ m)] : 0.0;
    wave_sync();
  }
  const double go_c = BWD ? go[c] : 0.0;
  const double go_j = BWD ? go[j] : 0.0;
  double e_row = 0.0;
  double gax = 0.0, gay = 0.0, gaz = 0.0, gc6a = 0.0;
  double gfj[BWD ? KP : 1];
#pragma unroll
  for (int w = 0; w < (BWD ? KP : 1); ++w) gfj[w] = 0.0;
  int n_ring = 0;

  // the forward loads the walked edge's record one step ahead (its latency under the
  // current step; measured 3 % faster there, 3 % slower in the register-bound backward)
  AtmEdge eb_next = rec[a0 + 1];
  for (int32_t b = a0 + 1; b < hi; ++b) {
    const AtmEdge eb = BWD ? rec[b] : eb_next;      // wave-uniform
    if (!BWD && b + 1 < hi) eb_next = rec[b + 1];
    const int32_t k = atm_nb(eb);
    const double dx = ax - eb.vx, dy = ay - eb.vy, dz = az - eb.vz;
    const double w2 = dx * dx + dy * dy + dz * dz;
    const bool keep = va && a < b && j != k && w2 <= kc.cut2 && w2 > kAtmEps;
    if (__ballot(keep) == 0) continue;
    const double y = eb.vx * eb.vx + eb.vy * eb.vy + eb.vz * eb.vz;
    const double iy = BWD ? rcp_nr(y) : 0.0;
    const double* __restrict__ fk = fb + (int64_t)k * KP;
    double e = 0.0, gx = 0.0, gy = 0.0, gw = 0.0, c6jk = 1.0;
    if (keep) {
      c6jk = 0.0;
#pragma unroll
      for (int w = 0; w < KP; ++w) c6jk = fma(fj[w], fk[w], c6jk);
      const double r0 = ea.p * eb.p * sTab[sj * S + atm_snb(eb)];
      const double weight = BWD ? go_c + go_j + go[k] : 1.0;
      atm_triangle<SWITCH, BWD, P16>(kc, x, y, w2, ix, iy, fabs(ea.c6 * eb.c6 * c6jk), r0,
                                     ea.sw, eb.sw, ea.dsw, eb.dsw, weight, e, gx, gy, gw);
    }
    if (!BWD) {
      e_row += e;
      sRing[wv][n_ring][lane] = e;
      if (lane == 0) sRingK[wv][n_ring] = k;
      if (++n_ring == kAtmRing) {
        atm_ring_flush(sRing[wv], sRingK[wv], n_ring, lane, L, energy, tail.energy);
        n_ring = 0;
      }
    } else {
      // dE/dC6 = E / (2 C6) for each of the three pair coefficients (C9 = sqrt(C6 C6 C6))
      const double g3 = keep ? 0.5 * e * rcp_nr(c6jk != 0.0 ? c6jk : 1.0) : 0.0;
      gax = fma(2.0, fma(gx, ax, gw * dx), gax);
      gay = fma(2.0, fma(gx, ay, gw * dy), gay);
      gaz = fma(2.0, fma(gx, az, gw * dz), gaz);
      gc6a = fma(e, hc6a, gc6a);
#pragma unroll
      for (int w = 0; w < KP; ++w) gfj[w] = fma(g3, fk[w], gfj[w]);
      // edge b and atom k: the wave's sums of g3 fa[j] (per component) and of the four
      // scalars (vector gradient of edge b, dE/dC6_ck)
      const double vf = atm_fold32(sFp[BWD ? wv : 0], lane, g3, L);
      const double vs = atm_fold4(2.0 * fma(gy, eb.vx, -gw * dx), 2.0 * fma(gy, eb.vy, -gw * dy),
                                  2.0 * fma(gy, eb.vz, -gw * dz),
                                  0.5 * e / (eb.c6 != 0.0 ? eb.c6 : 1.0), lane, L);
      const int slot = lane >> 1;
      if ((lane & 1) == 0 && slot < K) atm_acc(gfb, tail.gfb, (int64_t)k * K + slot, vf);
      if ((lane & 15) == 0) atm_acc(gs, tail.gs, (int64_t)eb.pos * 4 + (lane >> 4), vs);
    }
  }
  if (!BWD) {
    if (n_ring > 0) atm_ring_flush(sRing[wv], sRingK[wv], n_ring, lane, L, energy, tail.energy);
    if (va) atm_acc(energy, tail.energy, j, e_row);
    const double ec = atm_wave_sum(e_row, L);
    if (lane == 0) atm_acc(energy, tail.energy, c, ec);
  } else if (va) {
    atm_acc(gs, tail.gs, (int64_t)ea.pos * 4 + 0, gax);
    atm_acc(gs, tail.gs, (int64_t)ea.pos * 4 + 1, gay);
    atm_acc(gs, tail.gs, (int64_t)ea.pos * 4 + 2, gaz);
    atm_acc(gs, tail.gs, (int64_t)ea.pos * 4 + 3, gc6a);
#pragma unroll
    for (int w = 0; w < KP; ++w)
      if (w < K) atm_acc(gfa, tail.gfa, (int64_t)j * K + w, gfj[w]);
  }
}

// Triangles with a repeated atom, at every visit of a flagged center c, a third to c:
// the pairs of c's edges where one edge goes to an image of c itself (any partner) or
// both go to images of one neighbor. Edges of c are sorted by neighbor, so the partners
// of an edge are its run of equal neighbors and the run of self-image edges, which ends
// the lower range [lo[c], lo1[c]).
template <int KP, bool SWITCH, bool BWD>
__global__ __launch_bounds__(kAtmWaves * kWave) void atm_repeat_kernel(
    const AtmEdge* __restrict__ rec, const int32_t* __restrict__ lo,
    const int32_t* __restrict__ lo1, const int32_t* __restrict__ flag, int64_t N,
    const double* __restrict__ fa, const double* __restrict__ fb,
    const double* __restrict__ table, int S, AtmConst kc, double* __restrict__ energy,
    const double* __restrict__ go, double* __restrict__ gs, double* __restrict__ gfa,
    double* __restrict__ gfb, int K, AtmTail tail) {
  __shared__ double sTab[kAtmMaxSpecies * kAtmMaxSpecies];
  atm_stage_table(table, S, sTab);
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t c = (int64_t)blockIdx.x * kAtmWaves + wave_in_block();
  if (c >= N || flag[c] == 0) return;
  const int32_t l0 = lo[c], u0 = lo1[c], hi = lo[c + 1];
  int32_t s0 = u0;                                  // self-image edges: [s0, u0)
  while (s0 > l0 && atm_nb(rec[s0 - 1]) == (int32_t)c) --s0;
  const double go_c = BWD ? go[c] : 0.0;
  double e_acc = 0.0;
  for (int32_t a0 = l0; a0 < hi; a0 += kAtmTile) {
    const int32_t a = a0 + lane;
    if (a >= hi) break;
    const AtmEdge ea = rec[a];
    const double ax = ea.vx, ay = ea.vy, az = ea.vz;
    const double x = ax * ax + ay * ay + az * az;
    const double ix = BWD ? rcp_nr(x) : 0.0;
    const int32_t j = atm_nb(ea);
    double fj[KP];
#pragma unroll
    for (int w = 0; w < KP; ++w) fj[w] = fa[(int64_t)j * KP + w];
    double gax = 0.0, gay = 0.0, gaz = 0.0, gc6a = 0.0;
    double gfj[BWD ? KP : 1];
#pragma unroll
    for (int w = 0; w < (BWD ? KP : 1); ++w) gfj[w] = 0.0;
    // partner ranges: a self edge pairs with every later edge; another edge with its
    // run of equal neighbors and with the later self edges
    const bool self = j == (int32_t)c;
    int32_t run_end = a + 1;
    if (!self)
      while (run_end < hi && atm_nb(rec[run_end]) == j) ++run_end;
    const int32_t r1_end = self ? hi : run_end;
    bool any = false;                               // a triangle was kept for this edge
    const int32_t r2_beg = self ? hi : (s0 > a + 1 ? s0 : a + 1);
    const int32_t r2_end = self ? hi : u0;
    for (int pass = 0; pass < 2; ++pass) {
      const int32_t b_beg = pass == 0 ? a + 1 : r2_beg;
      const int32_t b_end = pass == 0 ? r1_end : r2_end;
      for (int32_t b = b_beg; b < b_end; ++b) {
        const AtmEdge eb = rec[b];
        const double dx = ax - eb.vx, dy = ay - eb.vy, dz = az - eb.vz;
        const double w2 = dx * dx + dy * dy + dz * dz;
        if (!(w2 <= kc.cut2 && w2 > kAtmEps)) continue;
        any = true;
        const int32_t k = atm_nb(eb);
        const double y = eb.vx * eb.vx + eb.vy * eb.vy + eb.vz * eb.vz;
        const double* __restrict__ fk = fb + (int64_t)k * KP;
        double c6jk = 0.0;
#pragma unroll
        for (int w = 0; w < KP; ++w) c6jk = fma(fj[w], fk[w], c6jk);
        const double r0 = ea.p * eb.p * sTab[atm_snb(ea) * S + atm_snb(eb)];
        double e, gx = 0.0, gy = 0.0, gw = 0.0;
        atm_triangle<SWITCH, BWD, false>(kc, x, y, w2, ix, BWD ? rcp_nr(y) : 0.0,
                                  fabs(ea.c6 * eb.c6 * c6jk), r0, ea.sw, eb.sw, ea.dsw, eb.dsw,
                                  BWD ? go_c : 1.0, e, gx, gy, gw);
        if (!BWD) {
          e_acc += e;
        } else {
          const double g3 = 0.5 * e / (c6jk != 0.0 ? c6jk : 1.0);
          gax = fma(2.0, fma(gx, ax, gw * dx), gax);
          gay = fma(2.0, fma(gx, ay, gw * dy), gay);
          gaz = fma(2.0, fma(gx, az, gw * dz), gaz);
          gc6a += 0.5 * e / (ea.c6 != 0.0 ? ea.c6 : 1.0);
#pragma unroll
          for (int w = 0; w < KP; ++w) gfj[w] = fma(g3, fk[w], gfj[w]);
          atm_acc(gs, tail.gs, (int64_t)b * 4 + 0, 2.0 * fma(gy, eb.vx, -gw * dx));
          atm_acc(gs, tail.gs, (int64_t)b * 4 + 1, 2.0 * fma(gy, eb.vy, -gw * dy));
          atm_acc(gs, tail.gs, (int64_t)b * 4 + 2, 2.0 * fma(gy, eb.vz, -gw * dz));
          atm_acc(gs, tail.gs, (int64_t)b * 4 + 3, 0.5 * e / (eb.c6 != 0.0 ? eb.c6 : 1.0));
#pragma unroll
          for (int w = 0; w < KP; ++w)
            if (w < K) atm_acc(gfb, tail.gfb, (int64_t)k * K + w, g3 * fj[w]);
        }
      }
    }
    if (BWD && any) {
      atm_acc(gs, tail.gs, (int64_t)a * 4 + 0, gax);
      atm_acc(gs, tail.gs, (int64_t)a * 4 + 1, gay);
      atm_acc(gs, tail.gs, (int64_t)a * 4 + 2, gaz);
      atm_acc(gs, tail.gs, (int64_t)a * 4 + 3, gc6a);
#pragma unroll
      for (int w = 0; w < KP; ++w)
        if (w < K) atm_acc(gfa, tail.gfa, (int64_t)j * K + w, gfj[w]);
    }
  }
  if (!BWD) {
    const double ec = atm_wave_sum(e_acc, atm_lanes(lane));
    if (lane == 0) atm_acc(energy, tail.energy, c, ec);
  }
}

// grad_vec[original edge] = the sorted edge's vector gradient
__global__ __launch_bounds__(256) void atm_vec_grad_kernel(const int32_t* __restrict__ perm,
                                    const double* __restrict__ gs, int64_t E,
                                    double* __restrict__ gvec) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= E) return;
  const int64_t e = perm[p];
  gvec[3 * e + 0] = gs[4 * p + 0];
  gvec[3 * e + 1] = gs[4 * p + 1];
  gvec[3 * e + 2] = gs[4 * p + 2];
}

// The center sides C6_cj = <fa[c], fb[j]> of every edge, one wave per atom x, no atomics:
// gfa[x] += sum over x's row (x the center) of dE/dC6 fb[j], gfb[x] += sum over the edges
// whose neighbor is x (the plan's by-source order) of dE/dC6 fa[c].
template <int KP>
__global__ __launch_bounds__(kAtmWaves * kWave) void atm_center_side_kernel(
    const int32_t* __restrict__ lo, const int32_t* __restrict__ nbr,
    const int32_t* __restrict__ lo_src, const int32_t* __restrict__ by_src,
    const int32_t* __restrict__ ctr, const double* __restrict__ gs,
    const double* __restrict__ fa, const double* __restrict__ fb, int64_t N, int K,
    double* __restrict__ gfa, double* __restrict__ gfb) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t x = (int64_t)blockIdx.x * kAtmWaves + wave_in_block();
  if (x >= N) return;
  const AtmLanes L = atm_lanes(lane);
  for (int side = 0; side < 2; ++side) {
    const int32_t p0 = side == 0 ? lo[x] : lo_src[x];
    const int32_t p1 = side == 0 ? lo[x + 1] : lo_src[x + 1];
    if (p0 == p1) continue;                         // uniform
    double acc[KP];
#pragma unroll
    for (int w = 0; w < KP; ++w) acc[w] = 0.0;
    for (int32_t q = p0 + lane; q < p1; q += kWave) {
      const int64_t p = side == 0 ? q : by_src[q];
      const double g = gs[4 * p + 3];
      const double* __restrict__ f = side == 0 ? fb + (int64_t)nbr[p] * KP : fa + (int64_t)ctr[p] * KP;
#pragma unroll
      for (int w = 0; w < KP; ++w) acc[w] = fma(g, f[w], acc[w]);
    }
    double* __restrict__ out = side == 0 ? gfa : gfb;
#pragma unroll
    for (int w = 0; w < KP; ++w) {
      const double v = atm_wave_sum(acc[w], L);
      if (lane == 0 && w < K) out[x * K + w] += v;
    }
  }
}

// Diagnostics for the roofline: counts[0] += edge pairs tested by the upper kernel,
// counts[1] += distinct triangles it keeps, counts[2] += repeated-atom triangle visits.
// Same walk as the triangle kernels, reading the vectors through the plan's permutation.
__global__ __launch_bounds__(kAtmWaves * kWave) void atm_count_kernel(
    const int32_t* __restrict__ perm, const int32_t* __restrict__ nbr,
    const int32_t* __restrict__ lo, const int32_t* __restrict__ lo1,
    const int32_t* __restrict__ flag, int64_t N, int64_t n_groups, int64_t max_tiles,
    const double* __restrict__ vec, double cut2, unsigned long long* __restrict__ counts) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t t = blockIdx.x / n_groups;
  const int64_t c = (blockIdx.x - t * n_groups) * kAtmWaves + wave_in_block();
  if (c >= N) return;
  const int32_t l0 = lo[c], u0 = lo1[c], hi = lo[c + 1];
  unsigned long long tested = 0, kept = 0, rep = 0;
  const int32_t a0 = u0 + (int32_t)t * kAtmTile;
  if (t < max_tiles && a0 + 1 < hi) {
    const int32_t a = a0 + lane;
    const bool va = a < hi;
    const int64_t ea = perm[va ? a : a0];
    const double ax = vec[3 * ea], ay = vec[3 * ea + 1], az = vec[3 * ea + 2];
    const int32_t j = nbr[va ? a : a0];
    for (int32_t b = a0 + 1; b < hi; ++b) {
      const int64_t eb = perm[b];
      const double dx = ax - vec[3 * eb], dy = ay - vec[3 * eb + 1], dz = az - vec[3 * eb + 2];
      const double w2 = dx * dx + dy * dy + dz * dz;
      const bool live = va && a < b;
      tested += live;
      kept += live && j != nbr[b] && w2 <= cut2 && w2 > kAtmEps;
    }
  }
  if (t == 0 && flag[c] != 0) {
    int32_t s0 = u0;
    while (s0 > l0 && nbr[s0 - 1] == (int32_t)c) --s0;
    for (int32_t a = l0 + lane; a < hi; a += kWave) {
      const int64_t ea = perm[a];
      const double ax = vec[3 * ea], ay = vec[3 * ea + 1], az = vec[3 * ea + 2];
      const int32_t j = nbr[a];
      const bool self = j == (int32_t)c;
      int32_t run_end = a + 1;
      if (!self)
        while (run_end < hi && nbr[run_end] == j) ++run_end;
      for (int pass = 0; pass < 2; ++pass) {
        const int32_t b_beg = pass == 0 ? a + 1 : (self ? hi : (s0 > a + 1 ? s0 : a + 1));
        const int32_t b_end = pass == 0 ? (self ? hi : run_end) : (self ? hi : u0);
        for (int32_t b = b_beg; b < b_end; ++b) {
          const int64_t eb = perm[b];
          const double dx = ax - vec[3 * eb], dy = ay - vec[3 * eb + 1],
                       dz = az - vec[3 * eb + 2];
          const double w2 = dx * dx + dy * dy + dz * dz;
          rep += w2 <= cut2 && w2 > kAtmEps;
        }
      }
    }
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    tested += __shfl_xor(tested, o);
    kept += __shfl_xor(kept, o);
    rep += __shfl_xor(rep, o);
  }
  if (lane == 0) {
    if (tested) atomicAdd(&counts[0], tested);
    if (kept) atomicAdd(&counts[1], kept);
    if (rep) atomicAdd(&counts[2], rep);
  }
}

// ------------------------------------------------------------------------------ tangents
// Second derivatives (dispersion_fast/atm.py:475-509, atm_tangents.py): along a direction
// (edge vectors, both factor matrices), the derivative of the per-atom energies and of the
// gradient of sum_i go_i E_i at fixed go, i.e. the Hessian of that sum times the direction.
// Every quantity of a triangle's energy and of its closed-form gradient (atm_triangle)
// carries its derivative along the direction as a forward-mode number, so those formulas
// are differentiated exactly as written. Sums are the reproducible head/tail sums.

struct AtmDual {
  double v, t;   // value, derivative along the direction
};
using Dl = AtmDual;
__device__ __forceinline__ Dl operator+(Dl a, Dl b) { return {a.v + b.v, a.t + b.t}; }
__device__ __forceinline__ Dl operator-(Dl a, Dl b) { return {a.v - b.v, a.t - b.t}; }
__device__ __forceinline__ Dl operator-(Dl a) { return {-a.v, -a.t}; }
__device__ __forceinline__ Dl operator*(Dl a, Dl b) { return {a.v * b.v, fma(a.v, b.t, a.t * b.v)}; }
__device__ __forceinline__ Dl operator*(double s, Dl a) { return {s * a.v, s * a.t}; }
__device__ __forceinline__ Dl operator+(Dl a, double s) { return {a.v + s, a.t}; }
__device__ __forceinline__ Dl operator/(Dl a, Dl b) {
  const double r = 1.0 / b.v, q = a.v * r;
  return {q, (a.t - q * b.t) * r};
}
__device__ __forceinline__ Dl dl_rcp(Dl a) {
  const double r = 1.0 / a.v;
  return {r, -a.t * r * r};
}
__device__ __forceinline__ Dl dl_sqrt(Dl a) {
  const double s = sqrt(a.v);
  return {s, a.v > 0.0 ? 0.5 * a.t / s : 0.0};
}
__device__ __forceinline__ Dl dl_rsqrt(Dl a) {
  const double r = 1.0 / sqrt(a.v);
  return {r, -0.5 * a.t * r / a.v};
}
// a^p, a > 0
__device__ __forceinline__ Dl dl_pow(Dl a, double p) {
  const double v = exp(p * log(a.v));
  return {v, p * v * a.t / a.v};
}
// a / b with the kernels' guard: b = 0 divides by one
__device__ __forceinline__ Dl dl_over(Dl a, Dl b) {
  return b.v != 0.0 ? a / b : a;
}

// the switch of one side and its slope in r^2 (switch_d, width > 0), from r^2
__device__ __forceinline__ void atm_switch_t(Dl r2, const AtmConst& kc, Dl& sw, Dl& dsw2) {
  const Dl r = dl_sqrt(r2);
  const Dl u = (1.0 / kc.width) * (Dl{kc.cutoff, 0.0} - r);
  if (u.v >= 1.0 || u.v <= 0.0) {
    sw = {u.v >= 1.0 ? 1.0 : 0.0, 0.0};
    dsw2 = {0.0, 0.0};
    return;
  }
  sw = u * u * u * ((6.0 * u + (-15.0)) * u + 10.0);
  const Dl om = Dl{1.0, 0.0} - u;
  const Dl dsw = (-30.0 / kc.width) * (u * u * om * om);
  dsw2 = 0.5 * (r.v > 0.0 ? dsw / r : Dl{0.0, 0.0});
}

// atm_triangle's energy and derivatives in x, y, w at unit weight, as forward-mode numbers;
// c9sq = |C6_cj C6_ck C6_jk|, the three switches and their slopes in the squared sides
// given for the two walked sides (the third from w).
template <bool SWITCH>
__device__ __forceinline__ void atm_triangle_t(const AtmConst& kc, Dl x, Dl y, Dl w, Dl c9sq,
                                               double r0, Dl swa, Dl swb, Dl dswa, Dl dswb,
                                               Dl& e, Dl& gx, Dl& gy, Dl& gw) {
  const Dl s = dl_rsqrt(x * y * w);
  const Dl s2 = s * s;
  const Dl s3 = s2 * s;
  const Dl s5 = s3 * s2;
  const Dl t = dl_pow(r0 * s, kc.alp3);
  const Dl damp = dl_rcp(6.0 * t + 1.0);
  const Dl f1 = x + w - y, f2 = x - w + y, f3 = w + y - x;
  const Dl nn = f1 * f2 * f3;
  const Dl ang = 0.375 * nn * s5 + s3;
  Dl swjk{1.0, 0.0}, dswjk{0.0, 0.0};
  if (SWITCH) atm_switch_t(w, kc, swjk, dswjk);
  const Dl sw = swa * swb * swjk;
  const Dl base = kc.s9_3 * dl_sqrt(c9sq);
  e = base * ang * damp * sw;
  const Dl ix = dl_rcp(x), iy = dl_rcp(y), iw = dl_rcp(w);
  const Dl a23 = f2 * f3, a13 = f1 * f3, a12 = f1 * f2;
  const Dl q = 0.375 * s5;
  const Dl ang_x = q * (-2.5 * nn * ix + a23 + a13 - a12) - 1.5 * s3 * ix;
  const Dl ang_y = q * (-2.5 * nn * iy + a13 + a12 - a23) - 1.5 * s3 * iy;
  const Dl ang_w = q * (-2.5 * nn * iw + a23 + a12 - a13) - 1.5 * s3 * iw;
  const Dl dc = 3.0 * kc.alp3 * t * damp * damp;
  const Dl bd = base * damp * sw;
  const Dl ba = base * ang;
  const Dl dcs = dc * sw;
  gx = bd * ang_x + ba * (dcs * ix + damp * dswa * swb * swjk);
  gy = bd * ang_y + ba * (dcs * iy + damp * swa * dswb * swjk);
  gw = bd * ang_w + ba * (dcs * iw + damp * swa * swb * dswjk);
}

// one edge's tangents: the vector's and that of C6_cj = <fa[c], fb[j]>
struct __align__(32) AtmEdgeT {
  double vx, vy, vz, c6;
};

// the tangent kernels' sums (heads, or their tails)
struct AtmTanSums {
  double* energy_t;   // (N)   tangents of the per-atom energies
  double* gs;         // (E,4) column 3: dE/dC6_cj (the value, for the center sides)
  double* gs_t;       // (E,4) tangents of the edge gradients (vector, C6_cj)
  double* gfa_t;      // (N,K)
  double* gfb_t;      // (N,K)
};

// one wave (center) per block: the two permuted factor tables take 32 KB of LDS per wave
constexpr int kAtmTanWaves = 1;

template <int KP>
__global__ __launch_bounds__(256) void atm_edges_tangent_kernel(
    const uint64_t* __restrict__ keys, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ nbr, int64_t E, int64_t N, const double* __restrict__ vec_t,
    const double* __restrict__ fa, const double* __restrict__ fb,
    const double* __restrict__ fa_t, const double* __restrict__ fb_t,
    AtmEdgeT* __restrict__ rec_t) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= E) return;
  const int64_t e = perm[p];
  const int64_t c = (int64_t)(keys[p] / (uint64_t)N);
  const int64_t j = nbr[p];
  double c6 = 0.0;
#pragma unroll
  for (int w = 0; w < KP; ++w)
    c6 = fma(fa_t[c * KP + w], fb[j * KP + w], fma(fa[c * KP + w], fb_t[j * KP + w], c6));
  rec_t[p] = AtmEdgeT{vec_t[3 * e + 0], vec_t[3 * e + 1], vec_t[3 * e + 2], c6};
}

// The distinct-triangle walk of atm_upper_kernel (same items, same order of b) with
// forward-mode numbers: per triangle the energy tangent to c, j and k, and the tangents of
// both edges' gradients and of the jk side's factor gradients at weight go_c + go_j + go_k,
// with the value of dE/dC6 of both edges for the center sides. The walked edge's sums go
// through the fold (fa[j] and its tangent permuted in LDS) and atm_fold4.
template <int KP, bool SWITCH>
__global__ __launch_bounds__(kAtmTanWaves * kWave) void atm_upper_tangent_kernel(
    const AtmEdge* __restrict__ rec, const AtmEdgeT* __restrict__ rec_t,
    const int32_t* __restrict__ lo, const int32_t* __restrict__ lo1, int64_t N,
    int64_t n_groups, const double* __restrict__ fa, const double* __restrict__ fb,
    const double* __restrict__ fa_t, const double* __restrict__ fb_t,
    const double* __restrict__ table, int S, AtmConst kc, const double* __restrict__ go, int K,
    AtmTanSums out, AtmTanSums tail) {
  __shared__ double sTab[kAtmMaxSpecies * kAtmMaxSpecies];
  __shared__ double sFp[kAtmTanWaves][32][kWave];   // fa[j][i ^ ((lane >> 1) & 7)]
  __shared__ double sFq[kAtmTanWaves][32][kWave];   // fa_t[j], same permutation
  atm_stage_table(table, S, sTab);
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = wave_in_block();
  const int64_t t = blockIdx.x / n_groups;
  const int64_t c = (blockIdx.x - t * n_groups) * kAtmTanWaves + wv;
  if (c >= N) return;
  const int32_t hi = lo[c + 1];
  const int32_t a0 = lo1[c] + (int32_t)t * kAtmTile;
  if (a0 + 1 >= hi) return;
  const AtmLanes L = atm_lanes(lane);
  const int32_t a = a0 + lane;
  const bool va = a < hi;
  const AtmEdge ea = rec[va ? a : a0];
  const AtmEdgeT eat = rec_t[ea.pos];
  const Dl avx{ea.vx, eat.vx}, avy{ea.vy, eat.vy}, avz{ea.vz, eat.vz};
  const Dl x = avx * avx + avy * avy + avz * avz;
  Dl swa{ea.sw, 0.0}, dswa{ea.dsw, 0.0};
  if (SWITCH) atm_switch_t(x, kc, swa, dswa);
  const Dl c6a{ea.c6, eat.c6};
  const int32_t j = atm_nb(ea);
  const int sj = atm_snb(ea);
  const int m = (lane >> 1) & 7;
  double fj[KP];
#pragma unroll
  for (int w = 0; w < KP; ++w) fj[w] = fa[(int64_t)j * KP + w];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    sFp[wv][i][lane] = (i ^ m) < KP ? fa[(int64_t)j * KP + (i ^ m)] : 0.0;
    sFq[wv][i][lane] = (i ^ m) < KP ? fa_t[(int64_t)j * KP + (i ^ m)] : 0.0;
  }
  wave_sync();
  const double go_cj = go[c] + go[j];
  double e_row_t = 0.0, gax_t = 0.0, gay_t = 0.0, gaz_t = 0.0, gc6a = 0.0, gc6a_t = 0.0;
  double gfj_t[KP];
#pragma unroll
  for (int w = 0; w < KP; ++w) gfj_t[w] = 0.0;

  for (int32_t b = a0 + 1; b < hi; ++b) {
    const AtmEdge eb = rec[b];                      // wave-uniform
    const int32_t k = atm_nb(eb);
    const double dx = ea.vx - eb.vx, dy = ea.vy - eb.vy, dz = ea.vz - eb.vz;
    const double w2 = dx * dx + dy * dy + dz * dz;
    const bool keep = va && a < b && j != k && w2 <= kc.cut2 && w2 > kAtmEps;
    if (__ballot(keep) == 0) continue;
    const AtmEdgeT ebt = rec_t[eb.pos];
    const double* __restrict__ fk = fb + (int64_t)k * KP;
    const double* __restrict__ fkt = fb_t + (int64_t)k * KP;
    double bx_t = 0.0, by_t = 0.0, bz_t = 0.0, bc6 = 0.0, bc6_t = 0.0, ek_t = 0.0;
    double g3 = 0.0, g3_t = 0.0;
    if (keep) {
      const Dl bvx{eb.vx, ebt.vx}, bvy{eb.vy, ebt.vy}, bvz{eb.vz, ebt.vz};
      const Dl y = bvx * bvx + bvy * bvy + bvz * bvz;
      Dl swb{eb.sw, 0.0}, dswb{eb.dsw, 0.0};
      if (SWITCH) atm_switch_t(y, kc, swb, dswb);
      const Dl ddx = avx - bvx, ddy = avy - bvy, ddz = avz - bvz;
      const Dl w = ddx * ddx + ddy * ddy + ddz * ddz;
      double c6jk = 0.0, c6jk_t = 0.0;
#pragma unroll
      for (int q = 0; q < KP; ++q) {
        c6jk = fma(fj[q], fk[q], c6jk);
        c6jk_t = fma(fj[q], fkt[q], fma(sFq[wv][q ^ m][lane], fk[q], c6jk_t));
      }
      const Dl cjk{c6jk, c6jk_t}, c6b{eb.c6, ebt.c6};
      const Dl pr = c6a * c6b * cjk;
      const double r0 = ea.p * eb.p * sTab[sj * S + atm_snb(eb)];
      Dl e, gx, gy, gw;
      atm_triangle_t<SWITCH>(kc, x, y, w, pr.v < 0.0 ? -pr : pr, r0, swa, swb, dswa, dswb, e,
                             gx, gy, gw);
      const double W = go_cj + go[k];
      e_row_t += e.t;
      ek_t = e.t;
      const Dl eW = W * e, gxW = W * gx, gyW = W * gy, gwW = W * gw;
      // edge a's vector gradient 2 (gx v_a + gw d), edge b's 2 (gy v_b - gw d)
      gax_t = fma(2.0, (gxW * avx + gwW * ddx).t, gax_t);
      gay_t = fma(2.0, (gxW * avy + gwW * ddy).t, gay_t);
      gaz_t = fma(2.0, (gxW * avz + gwW * ddz).t, gaz_t);
      bx_t = 2.0 * (gyW * bvx - gwW * ddx).t;
      by_t = 2.0 * (gyW * bvy - gwW * ddy).t;
      bz_t = 2.0 * (gyW * bvz - gwW * ddz).t;
      // dE/dC6 = E / (2 C6) for each of the three pair coefficients
      const Dl ha = 0.5 * dl_over(eW, c6a), hb = 0.5 * dl_over(eW, c6b);
      const Dl h3 = 0.5 * dl_over(eW, cjk);
      gc6a += ha.v;
      gc6a_t += ha.t;
      bc6 = hb.v;
      bc6_t = hb.t;
      g3 = h3.v;
      g3_t = h3.t;
#pragma unroll
      for (int q = 0; q < KP; ++q) gfj_t[q] = fma(g3_t, fk[q], fma(g3, fkt[q], gfj_t[q]));
    }
    // edge b and atom k: the wave's sums
    const double vf = atm_fold32x2(sFp[wv], sFq[wv], lane, g3_t, g3);
    const double vs = atm_fold4(bx_t, by_t, bz_t, bc6_t, lane, L);
    const double vp = atm_fold4(bc6, ek_t, 0.0, 0.0, lane, L);
    const int slot = lane >> 1;
    if ((lane & 1) == 0 && slot < K) atm_acc(out.gfb_t, tail.gfb_t, (int64_t)k * K + slot, vf);
    if ((lane & 15) == 0) atm_acc(out.gs_t, tail.gs_t, (int64_t)eb.pos * 4 + (lane >> 4), vs);
    if (lane == 0) atm_acc(out.gs, tail.gs, (int64_t)eb.pos * 4 + 3, vp);
    if (lane == 16) atm_acc(out.energy_t, tail.energy_t, k, vp);
  }
  if (va) {
    atm_acc(out.gs_t, tail.gs_t, (int64_t)ea.pos * 4 + 0, gax_t);
    atm_acc(out.gs_t, tail.gs_t, (int64_t)ea.pos * 4 + 1, gay_t);
    atm_acc(out.gs_t, tail.gs_t, (int64_t)ea.pos * 4 + 2, gaz_t);
    atm_acc(out.gs_t, tail.gs_t, (int64_t)ea.pos * 4 + 3, gc6a_t);
    atm_acc(out.gs, tail.gs, (int64_t)ea.pos * 4 + 3, gc6a);
    atm_acc(out.energy_t, tail.energy_t, j, e_row_t);
#pragma unroll
    for (int w = 0; w < KP; ++w)
      if (w < K) atm_acc(out.gfa_t, tail.gfa_t, (int64_t)j * K + w, gfj_t[w]);
  }
  const double ec = atm_wave_sum(e_row_t, L);
  if (lane == 0) atm_acc(out.energy_t, tail.energy_t, c, ec);
}

// atm_repeat_kernel's walk with forward-mode numbers (weight go_c, energy tangent to c).
template <int KP, bool SWITCH>
__global__ __launch_bounds__(kAtmWaves * kWave) void atm_repeat_tangent_kernel(
    const AtmEdge* __restrict__ rec, const AtmEdgeT* __restrict__ rec_t,
    const int32_t* __restrict__ lo, const int32_t* __restrict__ lo1,
    const int32_t* __restrict__ flag, int64_t N, const double* __restrict__ fa,
    const double* __restrict__ fb, const double* __restrict__ fa_t,
    const double* __restrict__ fb_t, const double* __restrict__ table, int S, AtmConst kc,
    const double* __restrict__ go, int K, AtmTanSums out, AtmTanSums tail) {
  __shared__ double sTab[kAtmMaxSpecies * kAtmMaxSpecies];
  atm_stage_table(table, S, sTab);
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t c = (int64_t)blockIdx.x * kAtmWaves + wave_in_block();
  if (c >= N || flag[c] == 0) return;
  const int32_t l0 = lo[c], u0 = lo1[c], hi = lo[c + 1];
  int32_t s0 = u0;                                  // self-image edges: [s0, u0)
  while (s0 > l0 && atm_nb(rec[s0 - 1]) == (int32_t)c) --s0;
  const double go_c = go[c];
  double e_acc_t = 0.0;
  for (int32_t a0 = l0; a0 < hi; a0 += kAtmTile) {
    const int32_t a = a0 + lane;
    if (a >= hi) break;
    const AtmEdge ea = rec[a];
    const AtmEdgeT eat = rec_t[a];
    const Dl avx{ea.vx, eat.vx}, avy{ea.vy, eat.vy}, avz{ea.vz, eat.vz};
    const Dl x = avx * avx + avy * avy + avz * avz;
    Dl swa{ea.sw, 0.0}, dswa{ea.dsw, 0.0};
    if (SWITCH) atm_switch_t(x, kc, swa, dswa);
    const Dl c6a{ea.c6, eat.c6};
    const int32_t j = atm_nb(ea);
    double fj[KP], fjt[KP], gfj_t[KP];
#pragma unroll
    for (int w = 0; w < KP; ++w) {
      fj[w] = fa[(int64_t)j * KP + w];
      fjt[w] = fa_t[(int64_t)j * KP + w];
      gfj_t[w] = 0.0;
    }
    double gax_t = 0.0, gay_t = 0.0, gaz_t = 0.0, gc6a = 0.0, gc6a_t = 0.0;
    const bool self = j == (int32_t)c;
    int32_t run_end = a + 1;
    if (!self)
      while (run_end < hi && atm_nb(rec[run_end]) == j) ++run_end;
    const int32_t r1_end = self ? hi : run_end;
    bool any = false;
    const int32_t r2_beg = self ? hi : (s0 > a + 1 ? s0 : a + 1);
    const int32_t r2_end = self ? hi : u0;
    for (int pass = 0; pass < 2; ++pass) {
      const int32_t b_beg = pass == 0 ? a + 1 : r2_beg;
      const int32_t b_end = pass == 0 ? r1_end : r2_end;
      for (int32_t b = b_beg; b < b_end; ++b) {
        const AtmEdge eb = rec[b];
        const double dx = ea.vx - eb.vx, dy = ea.vy - eb.vy, dz = ea.vz - eb.vz;
        const double w2 = dx * dx + dy * dy + dz * dz;
        if (!(w2 <= kc.cut2 && w2 > kAtmEps)) continue;
        any = true;
        const AtmEdgeT ebt = rec_t[b];
        const int32_t k = atm_nb(eb);
        const Dl bvx{eb.vx, ebt.vx}, bvy{eb.vy, ebt.vy}, bvz{eb.vz, ebt.vz};
        const Dl y = bvx * bvx + bvy * bvy + bvz * bvz;
        Dl swb{eb.sw, 0.0}, dswb{eb.dsw, 0.0};
        if (SWITCH) atm_switch_t(y, kc, swb, dswb);
        const Dl ddx = avx - bvx, ddy = avy - bvy, ddz = avz - bvz;
        const Dl w = ddx * ddx + ddy * ddy + ddz * ddz;
        const double* __restrict__ fk = fb + (int64_t)k * KP;
        const double* __restrict__ fkt = fb_t + (int64_t)k * KP;
        double c6jk = 0.0, c6jk_t = 0.0;
#pragma unroll
        for (int q = 0; q < KP; ++q) {
          c6jk = fma(fj[q], fk[q], c6jk);
          c6jk_t = fma(fj[q], fkt[q], fma(fjt[q], fk[q], c6jk_t));
        }
        const Dl cjk{c6jk, c6jk_t}, c6b{eb.c6, ebt.c6};
        const Dl pr = c6a * c6b * cjk;
        const double r0 = ea.p * eb.p * sTab[atm_snb(ea) * S + atm_snb(eb)];
        Dl e, gx, gy, gw;
        atm_triangle_t<SWITCH>(kc, x, y, w, pr.v < 0.0 ? -pr : pr, r0, swa, swb, dswa, dswb,
                               e, gx, gy, gw);
        e_acc_t += e.t;
        const Dl eW = go_c * e, gxW = go_c * gx, gyW = go_c * gy, gwW = go_c * gw;
        gax_t = fma(2.0, (gxW * avx + gwW * ddx).t, gax_t);
        gay_t = fma(2.0, (gxW * avy + gwW * ddy).t, gay_t);
        gaz_t = fma(2.0, (gxW * avz + gwW * ddz).t, gaz_t);
        const Dl ha = 0.5 * dl_over(eW, c6a), hb = 0.5 * dl_over(eW, c6b);
        const Dl h3 = 0.5 * dl_over(eW, cjk);
        gc6a += ha.v;
        gc6a_t += ha.t;
#pragma unroll
        for (int q = 0; q < KP; ++q) gfj_t[q] = fma(h3.t, fk[q], fma(h3.v, fkt[q], gfj_t[q]));
        atm_acc(out.gs_t, tail.gs_t, (int64_t)b * 4 + 0, 2.0 * (gyW * bvx - gwW * ddx).t);
        atm_acc(out.gs_t, tail.gs_t, (int64_t)b * 4 + 1, 2.0 * (gyW * bvy - gwW * ddy).t);
        atm_acc(out.gs_t, tail.gs_t, (int64_t)b * 4 + 2, 2.0 * (gyW * bvz - gwW * ddz).t);
        atm_acc(out.gs_t, tail.gs_t, (int64_t)b * 4 + 3, hb.t);
        atm_acc(out.gs, tail.gs, (int64_t)b * 4 + 3, hb.v);
#pragma unroll
        for (int q = 0; q < KP; ++q)
          if (q < K)
            atm_acc(out.gfb_t, tail.gfb_t, (int64_t)k * K + q, fma(h3.t, fj[q], h3.v * fjt[q]));
      }
    }
    if (any) {
      atm_acc(out.gs_t, tail.gs_t, (int64_t)a * 4 + 0, gax_t);
      atm_acc(out.gs_t, tail.gs_t, (int64_t)a * 4 + 1, gay_t);
      atm_acc(out.gs_t, tail.gs_t, (int64_t)a * 4 + 2, gaz_t);
      atm_acc(out.gs_t, tail.gs_t, (int64_t)a * 4 + 3, gc6a_t);
      atm_acc(out.gs, tail.gs, (int64_t)a * 4 + 3, gc6a);
#pragma unroll
      for (int w = 0; w < KP; ++w)
        if (w < K) atm_acc(out.gfa_t, tail.gfa_t, (int64_t)j * K + w, gfj_t[w]);
    }
  }
  const double ec = atm_wave_sum(e_acc_t, atm_lanes(lane));
  if (lane == 0) atm_acc(out.energy_t, tail.energy_t, c, ec);
}

// ------------------------------------------------------------------------------ host
static AtmConst atm_const(const xnn_atm_params* prm) {
  AtmConst k;
  k.s9_3 = prm->s9 / 3.0;
  k.alp3 = prm->alp3;
  k.cut2 = prm->cutoff * prm->cutoff;
  k.cutoff = prm->cutoff;
  k.width = prm->width > 0.0 ? std::min(prm->width, prm->cutoff) : 0.0;
  return k;
}

static int atm_kp(int K) { return K <= 24 ? 24 : (K <= 28 ? 28 : 32); }

static void atm_zero(double* p, int64_t n, hipStream_t s) {
  if (n > 0) hipLaunchKernelGGL(atm_fill_f64_kernel, dim3(grid_1d(n, 256)), dim3(256), 0, s, p, n);
}

static void atm_add_tail(double* head, const double* tail, int64_t n, hipStream_t s) {
  if (n > 0)
    hipLaunchKernelGGL(atm_add_tail_kernel, dim3(grid_1d(n, 256)), dim3(256), 0, s, head, tail, n);
}

struct AtmArgs {
  const void* plan;
  int64_t E, N, max_tiles, has_repeats;
  const double* vec;
  const double* fa;
  const double* fb;
  int K;
  const int32_t* species;
  const double* table;
  int S;
  AtmConst kc;
  double* energy;
  const double* go;
  double* gvec;
  double* gfa;
  double* gfb;
  void* work;
  hipStream_t s;
};

template <int KP, bool SWITCH, bool BWD, bool P16>
static int atm_run(const AtmArgs& A) {
  const AtmPlanLayout P = atm_plan_layout(A.E, A.N);
  const AtmWorkLayout W = atm_work_layout(A.E, A.N, KP, BWD);
  const uint64_t* keys = at_off<uint64_t>(A.plan, P.keys);
  const int32_t* perm = at_off<int32_t>(A.plan, P.perm);
  const int32_t* nbr = at_off<int32_t>(A.plan, P.nbr);
  const int32_t* lo = at_off<int32_t>(A.plan, P.lo);
  const int32_t* lo1 = at_off<int32_t>(A.plan, P.lo1);
  const int32_t* flag = at_off<int32_t>(A.plan, P.flag);
  AtmEdge* rec = at_off<AtmEdge>(A.work, W.rec);
  AtmEdge* rec_up = at_off<AtmEdge>(A.work, W.rec_up);
  uint64_t* skey = at_off<uint64_t>(A.work, W.skey);
  int32_t* sval = at_off<int32_t>(A.work, W.sval);
  int32_t* sperm = at_off<int32_t>(A.work, W.sperm);
  double* faP = at_off<double>(A.work, W.fa);
  double* fbP = at_off<double>(A.work, W.fb);
  double* gs = BWD ? at_off<double>(A.work, W.gs) : nullptr;
  const int64_t nk = A.N * (int64_t)A.K;
  double* tails = at_off<double>(A.work, W.tail);
  AtmTail tail{nullptr, nullptr, nullptr, nullptr};
  if (!BWD) {
    tail.energy = tails;
    atm_zero(A.energy, A.N, A.s);
    atm_zero(tail.energy, A.N, A.s);
  } else {
    tail.gs = tails;
    tail.gfa = tail.gs + 4 * A.E;
    tail.gfb = tail.gfa + nk;
    atm_zero(gs, 4 * A.E, A.s);
    atm_zero(A.gfa, nk, A.s);
    atm_zero(A.gfb, nk, A.s);
    atm_zero(tails, 4 * A.E + 2 * nk, A.s);
  }
  XNN_LAUNCH_CHECK();
  if (A.E == 0 || A.N == 0) return XNN_OK;
  hipLaunchKernelGGL((atm_pad_kernel<KP>), dim3(grid_1d(A.N * KP, 256)), dim3(256), 0, A.s, A.fa,
                     A.N, A.K, faP);
  hipLaunchKernelGGL((atm_pad_kernel<KP>), dim3(grid_1d(A.N * KP, 256)), dim3(256), 0, A.s, A.fb,
                     A.N, A.K, fbP);
  hipLaunchKernelGGL((atm_edges_kernel<KP>), dim3(grid_1d(A.E, 256)), dim3(256), 0, A.s, keys,
                     perm, nbr, A.E, A.N, A.vec, faP, fbP, A.species, A.table, A.S, A.kc, rec,
                     skey, sval);
  XNN_LAUNCH_CHECK();
  size_t cub_bytes = W.cub_bytes;
  XNN_HIP_CHECK(hipcub::DeviceRadixSort::SortPairs(
      at_off<void>(A.work, W.cub), cub_bytes, skey, at_off<uint64_t>(A.work, W.skey_out), sval,
      sperm, (int)A.E, 0, 33 + atm_bitlen(A.N), A.s));
  hipLaunchKernelGGL(atm_walk_order_kernel, dim3(grid_1d(A.E, 256)), dim3(256), 0, A.s, rec,
                     sperm, A.E, rec_up);
  XNN_LAUNCH_CHECK();
  const int64_t n_groups = (A.N + kAtmWaves - 1) / kAtmWaves;
  if (A.max_tiles > 0) {
    const int64_t blocks = A.max_tiles * n_groups;
    XNN_REQUIRE(blocks <= 0x7fffffff, "ATM: too many triplet work items");
    hipLaunchKernelGGL((atm_upper_kernel<KP, SWITCH, BWD, P16>), dim3((unsigned)blocks),
                       dim3(kAtmWaves * kWave), 0, A.s, rec_up, lo, lo1, A.N, n_groups, faP, fbP,
                       A.table, A.S, A.kc, A.energy, A.go, gs, A.gfa, A.gfb, A.K, tail);
    XNN_LAUNCH_CHECK();
  }
  if (A.has_repeats) {
    hipLaunchKernelGGL((atm_repeat_kernel<KP, SWITCH, BWD>), dim3((unsigned)n_groups),
                       dim3(kAtmWaves * kWave), 0, A.s, rec, lo, lo1, flag, A.N, faP, fbP,
                       A.table, A.S, A.kc, A.energy, A.go, gs, A.gfa, A.gfb, A.K, tail);
    XNN_LAUNCH_CHECK();
  }
  if (!BWD) {
    atm_add_tail(A.energy, tail.energy, A.N, A.s);
  } else {
    atm_add_tail(gs, tail.gs, 4 * A.E, A.s);
    atm_add_tail(A.gfa, tail.gfa, nk, A.s);
    atm_add_tail(A.gfb, tail.gfb, nk, A.s);
  }
  if (BWD) {
    hipLaunchKernelGGL(atm_vec_grad_kernel, dim3(grid_1d(A.E, 256)), dim3(256), 0, A.s, perm, gs,
                       A.E, A.gvec);
    hipLaunchKernelGGL((atm_center_side_kernel<KP>), dim3((unsigned)n_groups),
                       dim3(kAtmWaves * kWave), 0, A.s, lo, nbr,
                       at_off<int32_t>(A.plan, P.lo_src), at_off<int32_t>(A.plan, P.by_src),
                       at_off<int32_t>(A.plan, P.ctr), gs, faP, fbP, A.N, A.K, A.gfa, A.gfb);
    XNN_LAUNCH_CHECK();
  }
  return XNN_OK;
}

template <int KP, bool BWD, bool P16>
static int atm_dispatch_sw(const AtmArgs& A) {
  return A.kc.width > 0.0 ? atm_run<KP, true, BWD, P16>(A) : atm_run<KP, false, BWD, P16>(A);
}

template <bool BWD>
static int atm_dispatch(const AtmArgs& A) {
  // the upstream exponent 16/3 takes the power without exp and log
  const bool p16 = fabs(A.kc.alp3 - 16.0 / 3.0) < 1e-12;
  if (atm_kp(A.K) == 24)
    return p16 ? atm_dispatch_sw<24, BWD, true>(A) : atm_dispatch_sw<24, BWD, false>(A);
  if (atm_kp(A.K) == 28)
    return p16 ? atm_dispatch_sw<28, BWD, true>(A) : atm_dispatch_sw<28, BWD, false>(A);
  return p16 ? atm_dispatch_sw<32, BWD, true>(A) : atm_dispatch_sw<32, BWD, false>(A);
}

// The tangent workspace: the backward's layout, then the padded directions of both factor
// matrices, the edges' tangent records, the tangents of the edge gradients and the tails of
// the energy and edge-gradient tangents.
struct AtmTanLayout {
  AtmWorkLayout base;
  size_t fa_t, fb_t, rec_t, gs_t, tail2, total;
};

static AtmTanLayout atm_tangent_layout(int64_t E, int64_t N, int kp) {
  AtmTanLayout T;
  T.base = atm_work_layout(E, N, kp, true);
  size_t at = T.base.total;
  const int64_t e1 = std::max<int64_t>(E, 1), n1 = std::max<int64_t>(N, 1);
  T.fa_t = at; at += atm_align(sizeof(double) * kp * n1);
  T.fb_t = at; at += atm_align(sizeof(double) * kp * n1);
  T.rec_t = at; at += atm_align(sizeof(AtmEdgeT) * e1);
  T.gs_t = at; at += atm_align(sizeof(double) * 4 * e1);
  T.tail2 = at; at += atm_align(sizeof(double) * (n1 + 4 * e1));
  T.total = at;
  return T;
}

struct AtmTanArgs {
  const double* vec_t;
  const double* fa_t;
  const double* fb_t;
  double* energy_t;
  double* gvec_t;
  double* gfa_t;
  double* gfb_t;
};

template <int KP, bool SWITCH>
static int atm_tangent_run(const AtmArgs& A, const AtmTanArgs& D) {
  const AtmPlanLayout P = atm_plan_layout(A.E, A.N);
  const AtmTanLayout T = atm_tangent_layout(A.E, A.N, KP);
  const AtmWorkLayout& W = T.base;
  const uint64_t* keys = at_off<uint64_t>(A.plan, P.keys);
  const int32_t* perm = at_off<int32_t>(A.plan, P.perm);
  const int32_t* nbr = at_off<int32_t>(A.plan, P.nbr);
  const int32_t* lo = at_off<int32_t>(A.plan, P.lo);
  const int32_t* lo1 = at_off<int32_t>(A.plan, P.lo1);
  const int32_t* flag = at_off<int32_t>(A.plan, P.flag);
  AtmEdge* rec = at_off<AtmEdge>(A.work, W.rec);
  AtmEdge* rec_up = at_off<AtmEdge>(A.work, W.rec_up);
  AtmEdgeT* rec_t = at_off<AtmEdgeT>(A.work, T.rec_t);
  uint64_t* skey = at_off<uint64_t>(A.work, W.skey);
  int32_t* sval = at_off<int32_t>(A.work, W.sval);
  int32_t* sperm = at_off<int32_t>(A.work, W.sperm);
  double* faP = at_off<double>(A.work, W.fa);
  double* fbP = at_off<double>(A.work, W.fb);
  double* fatP = at_off<double>(A.work, T.fa_t);
  double* fbtP = at_off<double>(A.work, T.fb_t);
  const int64_t nk = A.N * (int64_t)A.K;
  AtmTanSums out{D.energy_t, at_off<double>(A.work, W.gs), at_off<double>(A.work, T.gs_t),
                 D.gfa_t, D.gfb_t};
  double* tails = at_off<double>(A.work, W.tail);     // gs, gfa_t, gfb_t
  double* tails2 = at_off<double>(A.work, T.tail2);   // energy_t, gs_t
  AtmTanSums tail{tails2, tails, tails2 + A.N, tails + 4 * A.E, tails + 4 * A.E + nk};
  atm_zero(out.energy_t, A.N, A.s);
  atm_zero(out.gs, 4 * A.E, A.s);
  atm_zero(out.gs_t, 4 * A.E, A.s);
  atm_zero(out.gfa_t, nk, A.s);
  atm_zero(out.gfb_t, nk, A.s);
  atm_zero(tails, 4 * A.E + 2 * nk, A.s);
  atm_zero(tails2, A.N + 4 * A.E, A.s);
  if (A.E > 0) atm_zero(D.gvec_t, 3 * A.E, A.s);
  XNN_LAUNCH_CHECK();
  if (A.E == 0 || A.N == 0) return XNN_OK;
  const double* f4[4] = {A.fa, A.fb, D.fa_t, D.fb_t};
  double* p4[4] = {faP, fbP, fatP, fbtP};
  for (int i = 0; i < 4; ++i)
    hipLaunchKernelGGL((atm_pad_kernel<KP>), dim3(grid_1d(A.N * KP, 256)), dim3(256), 0, A.s,
                       f4[i], A.N, A.K, p4[i]);
  hipLaunchKernelGGL((atm_edges_kernel<KP>), dim3(grid_1d(A.E, 256)), dim3(256), 0, A.s, keys,
                     perm, nbr, A.E, A.N, A.vec, faP, fbP, A.species, A.table, A.S, A.kc, rec,
                     skey, sval);
  hipLaunchKernelGGL((atm_edges_tangent_kernel<KP>), dim3(grid_1d(A.E, 256)), dim3(256), 0, A.s,
                     keys, perm, nbr, A.E, A.N, D.vec_t, faP, fbP, fatP, fbtP, rec_t);
  XNN_LAUNCH_CHECK();
  size_t cub_bytes = W.cub_bytes;
  XNN_HIP_CHECK(hipcub::DeviceRadixSort::SortPairs(
      at_off<void>(A.work, W.cub), cub_bytes, skey, at_off<uint64_t>(A.work, W.skey_out), sval,
      sperm, (int)A.E, 0, 33 + atm_bitlen(A.N), A.s));
  hipLaunchKernelGGL(atm_walk_order_kernel, dim3(grid_1d(A.E, 256)), dim3(256), 0, A.s, rec,
                     sperm, A.E, rec_up);
  XNN_LAUNCH_CHECK();
  if (A.max_tiles > 0) {
    const int64_t n_groups = (A.N + kAtmTanWaves - 1) / kAtmTanWaves;
    const int64_t blocks = A.max_tiles * n_groups;
    XNN_REQUIRE(blocks <= 0x7fffffff, "ATM: too many triplet work items");
    hipLaunchKernelGGL((atm_upper_tangent_kernel<KP, SWITCH>), dim3((unsigned)blocks),
                       dim3(kAtmTanWaves * kWave), 0, A.s, rec_up, rec_t, lo, lo1, A.N, n_groups,
                       faP, fbP, fatP, fbtP, A.table, A.S, A.kc, A.go, A.K, out, tail);
    XNN_LAUNCH_CHECK();
  }
  if (A.has_repeats) {
    const int64_t n_groups = (A.N + kAtmWaves - 1) / kAtmWaves;
    hipLaunchKernelGGL((atm_repeat_tangent_kernel<KP, SWITCH>), dim3((unsigned)n_groups),
                       dim3(kAtmWaves * kWave), 0, A.s, rec, rec_t, lo, lo1, flag, A.N, faP, fbP,
                       fatP, fbtP, A.table, A.S, A.kc, A.go, A.K, out, tail);
    XNN_LAUNCH_CHECK();
  }
  atm_add_tail(out.energy_t, tail.energy_t, A.N, A.s);
  atm_add_tail(out.gs, tail.gs, 4 * A.E, A.s);
  atm_add_tail(out.gs_t, tail.gs_t, 4 * A.E, A.s);
  atm_add_tail(out.gfa_t, tail.gfa_t, nk, A.s);
  atm_add_tail(out.gfb_t, tail.gfb_t, nk, A.s);
  hipLaunchKernelGGL(atm_vec_grad_kernel, dim3(grid_1d(A.E, 256)), dim3(256), 0, A.s, perm,
                     out.gs_t, A.E, D.gvec_t);
  // the center sides C6_cj = <fa[c], fb[j]>: tangents of their gradients with the values of
  // the factors, then their gradients with the factors' directions
  const int64_t n_groups = (A.N + kAtmWaves - 1) / kAtmWaves;
  for (int pass = 0; pass < 2; ++pass)
    hipLaunchKernelGGL((atm_center_side_kernel<KP>), dim3((unsigned)n_groups),
                       dim3(kAtmWaves * kWave), 0, A.s, lo, nbr,
                       at_off<int32_t>(A.plan, P.lo_src), at_off<int32_t>(A.plan, P.by_src),
                       at_off<int32_t>(A.plan, P.ctr), pass == 0 ? out.gs_t : out.gs,
                       pass == 0 ? faP : fatP, pass == 0 ? fbP : fbtP, A.N, A.K, D.gfa_t,
                       D.gfb_t);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

static int atm_tangent_dispatch(const AtmArgs& A, const AtmTanArgs& D) {
  const bool sw = A.kc.width > 0.0;
  switch (atm_kp(A.K)) {
    case 24: return sw ? atm_tangent_run<24, true>(A, D) : atm_tangent_run<24, false>(A, D);
    case 28: return sw ? atm_tangent_run<28, true>(A, D) : atm_tangent_run<28, false>(A, D);
    default: return sw ? atm_tangent_run<32, true>(A, D) : atm_tangent_run<32, false>(A, D);
  }
}

static int atm_check(int64_t E, int64_t N, int64_t max_tiles, const double* vec, const double* fa,
                     const double* fb, int32_t K, const int32_t* species, const double* table,
                     int32_t S, const xnn_atm_params* prm, const void* plan, void* work,
                     size_t work_bytes, bool bwd) {
  XNN_REQUIRE(E >= 0 && N >= 0 && max_tiles >= 0, "negative size");
  XNN_REQUIRE(E <= 0x7fffffff && N < (1 << kAtmNbBits),
              "ATM: at most 2^31 - 1 edges and 2^26 - 1 atoms");
  XNN_REQUIRE(K >= 1 && K <= kAtmMaxK, "ATM: the C6 factors need 1 to %d components (got %d)",
              kAtmMaxK, (int)K);
  XNN_REQUIRE(S >= 1 && S <= kAtmMaxSpecies, "ATM: 1 to %d species (got %d)", kAtmMaxSpecies,
              (int)S);
  XNN_REQUIRE(prm != nullptr && prm->cutoff > 0.0, "ATM: a positive cutoff is required");
  XNN_REQUIRE(plan != nullptr && work != nullptr, "NULL plan or workspace");
  XNN_REQUIRE(work_bytes >= atm_work_layout(E, N, atm_kp(K), bwd).total, "workspace too small");
  XNN_REQUIRE(N == 0 || (fa && fb && species && table), "NULL input");
  XNN_REQUIRE(E == 0 || vec, "NULL edge vectors");
  return XNN_OK;
}

}  // namespace xnn

using namespace xnn;

extern "C" {

int xnn_atm_plan_size(int64_t n_edges, int64_t n_atoms, size_t* bytes) {
  XNN_REQUIRE(n_edges >= 0 && n_atoms >= 0 && bytes, "negative size or NULL output");
  XNN_REQUIRE(n_edges <= 0x7fffffff && n_atoms < 0x7fffffff,
              "ATM: at most 2^31 - 1 edges and atoms");
  *bytes = atm_plan_layout(n_edges, n_atoms).total;
  return XNN_OK;
}

int xnn_atm_plan(const int64_t* edge_index, int64_t n_edges, int64_t n_atoms, void* plan,
                 size_t plan_bytes, int64_t* info, xnn_stream_t stream) {
  XNN_REQUIRE(n_edges >= 0 && n_atoms >= 0, "negative size");
  XNN_REQUIRE(n_edges <= 0x7fffffff && n_atoms < (1 << kAtmNbBits),
              "ATM: at most 2^31 - 1 edges and 2^26 - 1 atoms");
  XNN_REQUIRE(plan != nullptr && info != nullptr, "NULL plan or info");
  XNN_REQUIRE(n_edges == 0 || edge_index != nullptr, "NULL edge_index");
  const AtmPlanLayout L = atm_plan_layout(n_edges, n_atoms);
  XNN_REQUIRE(plan_bytes >= L.total, "plan buffer too small (%zu < %zu bytes)", plan_bytes,
              L.total);
  hipStream_t s = as_hip(stream);
  const int64_t E = n_edges, N = n_atoms;
  int32_t* flag = at_off<int32_t>(plan, L.flag);
  int32_t* stats = at_off<int32_t>(plan, L.stats);
  hipLaunchKernelGGL(atm_fill_i32_kernel, dim3(grid_1d(std::max<int64_t>(N, 1), 256)), dim3(256),
                     0, s, flag, std::max<int64_t>(N, 1));
  hipLaunchKernelGGL(atm_fill_i32_kernel, dim3(1), dim3(64), 0, s, stats, 4);
  XNN_LAUNCH_CHECK();
  if (E > 0) {
    uint64_t* keys_in = at_off<uint64_t>(plan, L.keys_in);
    int32_t* vals_in = at_off<int32_t>(plan, L.vals_in);
    uint64_t* keys = at_off<uint64_t>(plan, L.keys);
    int32_t* perm = at_off<int32_t>(plan, L.perm);
    hipLaunchKernelGGL(atm_keys_kernel, dim3(grid_1d(E, 256)), dim3(256), 0, s, edge_index, E, N,
                       keys_in, vals_in, stats);
    XNN_LAUNCH_CHECK();
    size_t cub_bytes = L.cub_bytes;
    XNN_HIP_CHECK(hipcub::DeviceRadixSort::SortPairs(at_off<void>(plan, L.cub), cub_bytes, keys_in,
                                                     keys, vals_in, perm, (int)E, 0,
                                                     atm_end_bit(N), s));
    hipLaunchKernelGGL(atm_neighbors_kernel, dim3(grid_1d(E, 256)), dim3(256), 0, s, keys, E, N,
                       at_off<int32_t>(plan, L.nbr), at_off<int32_t>(plan, L.ctr),
                       at_off<uint64_t>(plan, L.keys2), vals_in, flag, stats);
    XNN_LAUNCH_CHECK();
    // the by-source order (sorted keys into the free keys_in buffer)
    cub_bytes = L.cub_bytes;
    XNN_HIP_CHECK(hipcub::DeviceRadixSort::SortPairs(
        at_off<void>(plan, L.cub), cub_bytes, at_off<uint64_t>(plan, L.keys2), keys_in, vals_in,
        at_off<int32_t>(plan, L.by_src), (int)E, 0, atm_end_bit(N), s));
  }
  hipLaunchKernelGGL(atm_src_rows_kernel, dim3(grid_1d(N + 1, 256)), dim3(256), 0, s,
                     at_off<uint64_t>(plan, L.keys_in), E, N, at_off<int32_t>(plan, L.lo_src));
  XNN_LAUNCH_CHECK();
  hipLaunchKernelGGL(atm_rows_kernel, dim3(grid_1d(N + 1, 256)), dim3(256), 0, s,
                     at_off<uint64_t>(plan, L.keys), E, N, at_off<int32_t>(plan, L.lo),
                     at_off<int32_t>(plan, L.lo1), flag, stats);
  XNN_LAUNCH_CHECK();
  int32_t h[4];
  XNN_HIP_CHECK(hipMemcpyAsync(h, stats, sizeof(h), hipMemcpyDeviceToHost, s));
  XNN_HIP_CHECK(hipStreamSynchronize(s));
  XNN_REQUIRE(h[2] == 0, "ATM: edge_index holds an atom index outside [0, %lld)",
              (long long)N);
  info[0] = h[0];
  info[1] = h[1];
  return XNN_OK;
}

int xnn_atm_work_size(int64_t n_edges, int64_t n_atoms, int32_t k, int32_t backward,
                      size_t* bytes) {
  XNN_REQUIRE(n_edges >= 0 && n_atoms >= 0 && bytes, "negative size or NULL output");
  XNN_REQUIRE(k >= 1 && k <= kAtmMaxK, "ATM: the C6 factors need 1 to %d components (got %d)",
              kAtmMaxK, (int)k);
  *bytes = atm_work_layout(n_edges, n_atoms, atm_kp(k), backward != 0).total;
  return XNN_OK;
}

int xnn_atm_energy(const void* plan, int64_t n_edges, int64_t n_atoms, int64_t max_tiles,
                   int64_t has_repeats, const double* edge_vec, const double* feat_a,
                   const double* feat_b, int32_t k, const int32_t* species, const double* table,
                   int32_t n_species, const xnn_atm_params* prm, double* energy, void* work,
                   size_t work_bytes, xnn_stream_t stream) {
  const int rc = atm_check(n_edges, n_atoms, max_tiles, edge_vec, feat_a, feat_b, k, species,
                           table, n_species, prm, plan, work, work_bytes, false);
  if (rc != XNN_OK) return rc;
  XNN_REQUIRE(n_atoms == 0 || energy != nullptr, "NULL output");
  AtmArgs A{plan, n_edges, n_atoms, max_tiles, has_repeats, edge_vec, feat_a, feat_b, k,
            species, table, n_species, atm_const(prm), energy, nullptr, nullptr, nullptr,
            nullptr, work, as_hip(stream)};
  return atm_dispatch<false>(A);
}

int xnn_atm_energy_backward(const void* plan, int64_t n_edges, int64_t n_atoms,
                            int64_t max_tiles, int64_t has_repeats, const double* edge_vec,
                            const double* feat_a, const double* feat_b, int32_t k,
                            const int32_t* species, const double* table, int32_t n_species,
                            const xnn_atm_params* prm, const double* grad_energy,
                            double* grad_vec, double* grad_fa, double* grad_fb, void* work,
                            size_t work_bytes, xnn_stream_t stream) {
  const int rc = atm_check(n_edges, n_atoms, max_tiles, edge_vec, feat_a, feat_b, k, species,
                           table, n_species, prm, plan, work, work_bytes, true);
  if (rc != XNN_OK) return rc;
  XNN_REQUIRE(n_atoms == 0 || (grad_energy && grad_fa && grad_fb), "NULL input or output");
  XNN_REQUIRE(n_edges == 0 || grad_vec, "NULL output");
  AtmArgs A{plan, n_edges, n_atoms, max_tiles, has_repeats, edge_vec, feat_a, feat_b, k,
            species, table, n_species, atm_const(prm), nullptr, grad_energy, grad_vec, grad_fa,
            grad_fb, work, as_hip(stream)};
  return atm_dispatch<true>(A);
}

int xnn_atm_tangent_work_size(int64_t n_edges, int64_t n_atoms, int32_t k, size_t* bytes) {
  XNN_REQUIRE(n_edges >= 0 && n_atoms >= 0 && bytes, "negative size or NULL output");
  XNN_REQUIRE(k >= 1 && k <= kAtmMaxK, "ATM: the C6 factors need 1 to %d components (got %d)",
              kAtmMaxK, (int)k);
  *bytes = atm_tangent_layout(n_edges, n_atoms, atm_kp(k)).total;
  return XNN_OK;
}

int xnn_atm_energy_backward_tangent(
    const void* plan, int64_t n_edges, int64_t n_atoms, int64_t max_tiles, int64_t has_repeats,
    const double* edge_vec, const double* feat_a, const double* feat_b, int32_t k,
    const int32_t* species, const double* table, int32_t n_species, const xnn_atm_params* prm,
    const double* grad_energy, const double* edge_vec_t, const double* feat_a_t,
    const double* feat_b_t, double* energy_t, double* grad_vec_t, double* grad_fa_t,
    double* grad_fb_t, void* work, size_t work_bytes, xnn_stream_t stream) {
  const int rc = atm_check(n_edges, n_atoms, max_tiles, edge_vec, feat_a, feat_b, k, species,
                           table, n_species, prm, plan, work, work_bytes, true);
  if (rc != XNN_OK) return rc;
  XNN_REQUIRE(work_bytes >= atm_tangent_layout(n_edges, n_atoms, atm_kp(k)).total,
              "workspace too small");
  XNN_REQUIRE(n_atoms == 0 || (grad_energy && feat_a_t && feat_b_t && energy_t && grad_fa_t &&
                               grad_fb_t),
              "NULL input or output");
  XNN_REQUIRE(n_edges == 0 || (edge_vec_t && grad_vec_t), "NULL edge tangents or output");
  AtmArgs A{plan, n_edges, n_atoms, max_tiles, has_repeats, edge_vec, feat_a, feat_b, k,
            species, table, n_species, atm_const(prm), nullptr, grad_energy, nullptr, nullptr,
            nullptr, work, as_hip(stream)};
  AtmTanArgs D{edge_vec_t, feat_a_t, feat_b_t, energy_t, grad_vec_t, grad_fa_t, grad_fb_t};
  return atm_tangent_dispatch(A, D);
}

int xnn_atm_count(const void* plan, int64_t n_edges, int64_t n_atoms, int64_t max_tiles,
                  const double* edge_vec, double cutoff, int64_t* counts, xnn_stream_t stream) {
  XNN_REQUIRE(n_edges >= 0 && n_atoms >= 0 && max_tiles >= 0, "negative size");
  XNN_REQUIRE(n_edges <= 0x7fffffff && n_atoms < 0x7fffffff,
              "ATM: at most 2^31 - 1 edges and atoms");
  XNN_REQUIRE(plan != nullptr && counts != nullptr, "NULL plan or output");
  XNN_REQUIRE(n_edges == 0 || edge_vec != nullptr, "NULL edge vectors");
  counts[0] = counts[1] = counts[2] = 0;
  if (n_edges == 0 || n_atoms == 0) return XNN_OK;
  const AtmPlanLayout L = atm_plan_layout(n_edges, n_atoms);
  hipStream_t s = as_hip(stream);
  unsigned long long* dev = nullptr;
  XNN_HIP_CHECK(hipMallocAsync((void**)&dev, 3 * sizeof(unsigned long long), s));
  XNN_HIP_CHECK(hipMemsetAsync(dev, 0, 3 * sizeof(unsigned long long), s));
  const int64_t n_groups = (n_atoms + kAtmWaves - 1) / kAtmWaves;
  const int64_t blocks = std::max<int64_t>(max_tiles, 1) * n_groups;
  XNN_REQUIRE(blocks <= 0x7fffffff, "ATM: too many triplet work items");
  hipLaunchKernelGGL(atm_count_kernel, dim3((unsigned)blocks), dim3(kAtmWaves * kWave), 0, s,
                     at_off<int32_t>(plan, L.perm), at_off<int32_t>(plan, L.nbr),
                     at_off<int32_t>(plan, L.lo), at_off<int32_t>(plan, L.lo1),
                     at_off<int32_t>(plan, L.flag), n_atoms, n_groups, max_tiles, edge_vec,
                     cutoff * cutoff, dev);
  XNN_LAUNCH_CHECK();
  unsigned long long h[3];
  XNN_HIP_CHECK(hipMemcpyAsync(h, dev, sizeof(h), hipMemcpyDeviceToHost, s));
  XNN_HIP_CHECK(hipFreeAsync(dev, s));
  XNN_HIP_CHECK(hipStreamSynchronize(s));
  counts[0] = (int64_t)h[0];
  counts[1] = (int64_t)h[1];
  counts[2] = (int64_t)h[2];
  return XNN_OK;
}

}  // extern "C"
