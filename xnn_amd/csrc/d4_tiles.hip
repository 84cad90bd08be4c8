// D4 coordination numbers and two-body dispersion over spatially ordered atom tiles
// (gfx950, wave64, float64).
//
// xnn_d4_coordination(_backward)  DFTD4.coordination_numbers (d4.py:552-591): the
//                                 EN-weighted erf-count CN and the plain erf count of the
//                                 charge model
// xnn_d4_two_body(_backward)      DFTD4.two_body_energy / pair_damping / pair_c6
//                                 (d4.py:1044-1071, 910-934) with the quintic switch
//                                 (dispersion.py:42-67): -1/2 C6 f(r) to each atom of every
//                                 pair image; the backward gives grad_pos, the cell gradient
//                                 and dE/d alpha, the quantities of the reference's native
//                                 kernel run_d4 (dispersion_fast/cpu.py:834-935)
//
// Layout. A call first orders the atoms of every structure along a Morton curve of a bin
// grid over their coordinates (fractional ones for a periodic structure), so that 64
// consecutive atoms -- a tile -- fill a compact box. The tiles of a structure are numbered
// 0..nt-1; a work item is one wave, receiver tile t (one atom per lane) against source
// tile t + d, d >= 0, staged in LDS:
//  * d > 0: every unordered pair (i in t, j in t + d) once, over all its lattice images.
//    The images of source j are one wave-uniform window: those whose fractional box around
//    the receiver tile's bounds can reach the cutoff; an image that none of the 64
//    receivers reaches is skipped by the whole wave. Both atoms of a pair get their share:
//    the receiver's in its lane's registers, the source's summed over the 64 lanes by a
//    reduce-scatter tree in registers over groups of 8 lanes and the 8 group sums added
//    through LDS every 8 sources. The backward keeps each pair's sum over images of f(r)
//    in its workspace block and ends with dE/d alpha of both atoms from them (small
//    products staged through LDS).
//  * d = 0: the directed pairs inside one tile, self images included, receiver side only.
// Per-atom partial sums go to slot (the other tile) of a (slots x components x atoms)
// array in tile order; every slot of an atom is written exactly once, and a reduce sums
// them in slot order, so a call repeats bit for bit (no atomics). Positions and cells in
// Angstrom, lengths inside the kernels in bohr, all float64.
#include <algorithm>
#include <initializer_list>
#include <cmath>
#include <cstdint>

#include "common.h"
#include "d4_geom.h"
#include "device.h"
#include "fp64.h"

namespace xnn {
namespace {

constexpr int kT = 64;                 // atoms per tile (lanes of a wave)
constexpr int kOrderThreads = 1024;    // one workgroup orders one structure
constexpr int kOrderBits = 4;          // at most 16 bins per axis
constexpr int kOrderBins = 1 << (3 * kOrderBits);
constexpr int kRedWaves = 8;           // waves of a slot-reduction block

__constant__ double c_cp3[kNW] = {
    cp3_weight(0),  cp3_weight(1),  cp3_weight(2),  cp3_weight(3),  cp3_weight(4),
    cp3_weight(5),  cp3_weight(6),  cp3_weight(7),  cp3_weight(8),  cp3_weight(9),
    cp3_weight(10), cp3_weight(11), cp3_weight(12), cp3_weight(13), cp3_weight(14),
    cp3_weight(15), cp3_weight(16), cp3_weight(17), cp3_weight(18), cp3_weight(19),
    cp3_weight(20), cp3_weight(21), cp3_weight(22)};

// ---------------------------------------------------------------- spatial order

// a structure's atoms [a0, a1), clamped to the n_nodes atoms that exist
__device__ inline void atom_range(const int64_t* __restrict__ node_ptr, int64_t b, int64_t n_nodes,
                                  int64_t& a0, int64_t& a1) {
  a0 = std::min<int64_t>(std::max<int64_t>(node_ptr[b], 0), n_nodes);
  a1 = std::min<int64_t>(std::max<int64_t>(node_ptr[b + 1], a0), n_nodes);
}


__device__ inline uint32_t morton3(uint32_t x, uint32_t y, uint32_t z) {
  uint32_t m = 0;
#pragma unroll
  for (int b = 0; b < kOrderBits; ++b)
    m |= (((x >> b) & 1u) << (3 * b)) | (((y >> b) & 1u) << (3 * b + 1)) |
         (((z >> b) & 1u) << (3 * b + 2));
  return m;
}

// exclusive prefix sum of one int per thread over the 1024-thread block
__device__ int block_exclusive_scan(int v, int* wave_sums, int& total) {
  const int lane = threadIdx.x & (kT - 1), wv = threadIdx.x / kT;
  int incl = v;
#pragma unroll
  for (int o = 1; o < kT; o <<= 1) {
    const int u = __shfl_up(incl, o, kT);
    if (lane >= o) incl += u;
  }
  if (lane == kT - 1) wave_sums[wv] = incl;
  __syncthreads();
  int base = 0, tot = 0;
  for (int w = 0; w < kOrderThreads / kT; ++w) {
    const int s = wave_sums[w];
    base += w < wv ? s : 0;
    tot += s;
  }
  __syncthreads();
  total = tot;
  return base + incl - v;
}

__device__ inline double block_reduce(double v, bool is_max, double* red) {
#pragma unroll
  for (int o = 1; o < kT; o <<= 1) {
    const double u = __shfl_xor(v, o, kT);
    v = is_max ? fmax(v, u) : fmin(v, u);
  }
  const int lane = threadIdx.x & (kT - 1), wv = threadIdx.x / kT;
  if (lane == 0) red[wv] = v;
  __syncthreads();
  double r = red[0];
  for (int w = 1; w < kOrderThreads / kT; ++w) r = is_max ? fmax(r, red[w]) : fmin(r, red[w]);
  __syncthreads();
  return r;
}

// the sort coordinates of atom p: fractional for a periodic structure, else Cartesian
__device__ inline void order_coords(const double* __restrict__ pos, int64_t p, bool periodic,
                                    const double* inv, double* c) {
  const double x = pos[3 * p], y = pos[3 * p + 1], z = pos[3 * p + 2];
  if (periodic) {
#pragma unroll
    for (int k = 0; k < 3; ++k) c[k] = x * inv[k] + y * inv[3 + k] + z * inv[6 + k];
  } else {
    c[0] = x;
    c[1] = y;
    c[2] = z;
  }
}

__device__ inline uint32_t order_code(const double* c, const double* lo, const double* scale,
                                      int side) {
  uint32_t b[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    // fmax / fmin return the number when the other operand is NaN: every bin is in range
    const double u = fmin(fmax((c[k] - lo[k]) * scale[k], 0.0), (double)(side - 1));
    b[k] = (uint32_t)u;
  }
  return morton3(b[0], b[1], b[2]);
}

// Workgroup b < n_graphs: order[node_ptr[b] + k] = the atom of structure b at place k of
// the Morton order of its bins (ties in atom order). Workgroup n_graphs: tile_ptr[b] =
// tiles of the structures before b.
__global__ __launch_bounds__(kOrderThreads) void d4_order_kernel(
    const double* __restrict__ pos, int64_t n_nodes, const int64_t* __restrict__ node_ptr,
    int64_t n_graphs, const double* __restrict__ cell, const int32_t* __restrict__ images,
    int32_t* __restrict__ order, int32_t* __restrict__ tile_ptr) {
  __shared__ int32_t cnt[kOrderBins], cur[kOrderBins];
  __shared__ int32_t wsum[kOrderThreads / kT];
  __shared__ double red[kOrderThreads / kT];
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  if (b == n_graphs) {
    int carry = 0;
    for (int64_t g0 = 0; g0 < n_graphs; g0 += kOrderThreads) {
      const int64_t g = g0 + tid;
      int v = 0;
      if (g < n_graphs) {
        int64_t a0, a1;
        atom_range(node_ptr, g, n_nodes, a0, a1);
        v = (int)((a1 - a0 + kT - 1) / kT);
      }
      int total;
      const int ex = block_exclusive_scan(v, wsum, total);
      if (g < n_graphs) tile_ptr[g] = carry + ex;
      carry += total;
    }
    if (tid == 0) tile_ptr[n_graphs] = carry;
    return;
  }
  int64_t a0, a1;
  atom_range(node_ptr, b, n_nodes, a0, a1);
  const int64_t n = a1 - a0;
  if (n <= kT) {
    for (int64_t p = tid; p < n; p += kOrderThreads) order[a0 + p] = (int32_t)(a0 + p);
    return;
  }
  Lattice L;
  load_lattice(cell, images, b, L);
  const bool periodic = (L.n0 | L.n1 | L.n2) != 0;
  double lo[3], hi[3], scale[3];
  {
    double mn[3] = {1e300, 1e300, 1e300}, mx[3] = {-1e300, -1e300, -1e300};
    for (int64_t p = tid; p < n; p += kOrderThreads) {
      double c[3];
      order_coords(pos, a0 + p, periodic, L.inv, c);
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        mn[k] = fmin(mn[k], c[k]);
        mx[k] = fmax(mx[k], c[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      lo[k] = block_reduce(mn[k], false, red);
      hi[k] = block_reduce(mx[k], true, red);
    }
  }
  // bins per axis: the smallest power of two whose cube holds ~2 atoms per bin
  int bits = 1;
  while (bits < kOrderBits && (int64_t(1) << (3 * bits)) * 2 < n) ++bits;
  const int side = 1 << bits, nb = 1 << (3 * bits);
#pragma unroll
  for (int k = 0; k < 3; ++k) scale[k] = hi[k] > lo[k] ? side / (hi[k] - lo[k]) : 0.0;
  for (int e = tid; e < nb; e += kOrderThreads) cnt[e] = 0;
  __syncthreads();
  for (int64_t p = tid; p < n; p += kOrderThreads) {
    double c[3];
    order_coords(pos, a0 + p, periodic, L.inv, c);
    atomicAdd(&cnt[order_code(c, lo, scale, side)], 1);
  }
  __syncthreads();
  // bin starts: thread t scans bins [4t, 4t + 4)
  {
    int v[4], s = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = 4 * tid + q;
      v[q] = e < nb ? cnt[e] : 0;
      s += v[q];
    }
    int total;
    int run = block_exclusive_scan(s, wsum, total);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = 4 * tid + q;
      if (e < nb) cur[e] = run;
      run += v[q];
    }
  }
  __syncthreads();
  // place each atom in its bin (arrival order), then sort every bin by atom index
  for (int64_t p = tid; p < n; p += kOrderThreads) {
    double c[3];
    order_coords(pos, a0 + p, periodic, L.inv, c);
    const int slot = atomicAdd(&cur[order_code(c, lo, scale, side)], 1);
    order[a0 + slot] = (int32_t)(a0 + p);
  }
  __syncthreads();
  for (int e = tid; e < nb; e += kOrderThreads) {
    const int end = cur[e], beg = end - cnt[e];
    for (int u = beg + 1; u < end; ++u) {
      const int32_t key = order[a0 + u];
      int q = u - 1;
      while (q >= beg && order[a0 + q] > key) {
        order[a0 + q + 1] = order[a0 + q];
        --q;
      }
      order[a0 + q + 1] = key;
    }
  }
}

// ---------------------------------------------------------------- work items

// one wave's pair of tiles: structure b, receiver tile lt (first sorted position r0,
// rcnt atoms), source tile ls (s0, scnt)
struct TileItem {
  int64_t b, r0, s0;
  int lt, ls, rcnt, scnt;
};

// false for an idle block: past the last tile, past the structure's last tile, or in a
// structure with more tiles than the max_nt slots (its atoms reduce to NaN)
__device__ inline bool tile_item(const int32_t* __restrict__ tile_ptr,
                                 const int64_t* __restrict__ node_ptr, int64_t n_graphs,
                                 int64_t n_nodes, int max_nt, TileItem& it) {
  const int64_t t = blockIdx.x, d = blockIdx.y;
  if (t >= tile_ptr[n_graphs]) return false;
  int64_t lo = 0, hi = n_graphs;  // the last structure whose first tile is <= t
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (tile_ptr[mid] <= t) lo = mid;
    else hi = mid;
  }
  const int nt = tile_ptr[lo + 1] - tile_ptr[lo];
  if (nt > max_nt) return false;
  it.b = lo;
  it.lt = (int)(t - tile_ptr[lo]);
  it.ls = it.lt + (int)d;
  if (it.ls >= nt) return false;
  int64_t a0, a1;
  atom_range(node_ptr, lo, n_nodes, a0, a1);
  it.r0 = a0 + (int64_t)it.lt * kT;
  it.s0 = a0 + (int64_t)it.ls * kT;
  it.rcnt = (int)std::min<int64_t>(kT, a1 - it.r0);
  it.scnt = (int)std::min<int64_t>(kT, a1 - it.s0);
  return true;
}

// the structure's cell (wave-uniform): bohr rows, inverse, per-axis window half-widths in
// fractional units for cutoff rc (Angstrom), image counts
struct TileGeo {
  double ab[9], inv[9], wf[3];
  double isp[3];  // 1 / interplanar spacing per axis (Angstrom^-1)
  int nmax[3];
  bool periodic;
};

// a float64 the whole wave holds, moved to scalar registers (the lattice is derived on the
// vector ALU, which has no way to tell that its result is the same in every lane)
__device__ inline double wave_uniform(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ inline void tile_geo(const double* __restrict__ cell,
                                const int32_t* __restrict__ images, int64_t b, double rc,
                                TileGeo& G) {
  Lattice L;
  load_lattice(cell, images, b, L);
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    G.ab[k] = wave_uniform(L.ab[k]);
    G.inv[k] = wave_uniform(L.inv[k]);
  }
  G.nmax[0] = L.n0;
  G.nmax[1] = L.n1;
  G.nmax[2] = L.n2;
  G.periodic = (L.n0 | L.n1 | L.n2) != 0;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    G.wf[c] = wave_uniform(rc / L.sp[c] + 1e-9);
    G.isp[c] = wave_uniform(1.0 / L.sp[c]);
  }
}

__device__ inline double wave_min(double v) { return wave_extreme<false>(v); }
__device__ inline double wave_max(double v) { return wave_extreme<true>(v); }

// receiver tile bounds in fractional coordinates (over the live lanes)
__device__ inline void tile_bounds(const TileGeo& G, double x, double y, double z, bool live,
                                   double* flo, double* fhi) {
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    flo[c] = 0.0;
    fhi[c] = 0.0;
  }
  if (!G.periodic) return;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const double f = x * G.inv[c] + y * G.inv[3 + c] + z * G.inv[6 + c];
    flo[c] = wave_min(live ? f : 1e300);
    fhi[c] = wave_max(live ? f : -1e300);
  }
}

__device__ inline int pack_window(int lo, int hi) { return (lo & 0xffff) | (hi << 16); }
__device__ inline int window_lo(int w) { return (int)(int16_t)(w & 0xffff); }
__device__ inline int window_hi(int w) { return w >> 16; }

// Images n_c of source j (fractional coordinate fj on axis c) that can lie within the
// cutoff of some receiver of the tile: the vector d + n @ cell of receiver i has
// fractional component f_i - fj + n_c, and |f_i - fj + n_c| sp_c bounds its length from
// below, so n_c in [ceil(-w - (fhi - fj)), floor(w - (flo - fj))], clamped to the image
// counts. Packed as two int16.
__device__ inline int tile_window(int nmax, double fj, double flo, double fhi, double w) {
  if (nmax == 0) return pack_window(0, 0);
  const double m = fmin((double)nmax, 32767.0);
  const int lo = (int)fmax(ceil(-w - (fhi - fj)), -m);
  const int hi = (int)fmin(floor(w - (flo - fj)), m);
  return pack_window(lo, hi);
}

// rc_aa > 0: a cutoff of this source's own (Angstrom) in place of the structure's
__device__ inline void source_windows(const TileGeo& G, double x, double y, double z,
                                      const double* flo, const double* fhi, int* w,
                                      double rc_aa = 0.0) {
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const double f = G.periodic ? x * G.inv[c] + y * G.inv[3 + c] + z * G.inv[6 + c] : 0.0;
    const double half = rc_aa > 0.0 ? rc_aa * G.isp[c] + 1e-9 : G.wf[c];
    w[c] = tile_window(G.nmax[c], f, flo[c], fhi[c], half);
  }
}

// Sums over the 64 lanes of one value per step, one step per source, in two stages. First a
// reduce-scatter tree in registers over groups of 8 lanes: step values enter at level 0;
// two items of level v (steps s and s + 2^v) combine into one of level v + 1, in which the
// lane with bit v clear keeps the first item's sums and the lane with it set the second's,
// each adding its partner's (lane ^ 2^v) share. After a step s = 7 (mod 8), lane L holds
// the sum over its group (lanes 8 (L / 8) .. + 7) of step s - 7 + L % 8. Then the 8 group
// sums of each of those 8 steps meet in LDS (lane_finish8).
template <int NV>
struct LaneTree8 {
  double p[3][NV];
};

template <int LV, int NV>
__device__ __forceinline__ void lane_combine(const double (&a)[NV], double (&v)[NV], int lane) {
  const bool upper = (lane >> LV) & 1;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const double send = upper ? a[k] : v[k];
    const double keep = upper ? v[k] : a[k];
    v[k] = keep + xor_lanes<1 << LV>(send);
  }
}

template <int NV>
__device__ __forceinline__ void lane_keep(double (&dst)[NV], const double (&v)[NV]) {
#pragma unroll
  for (int k = 0; k < NV; ++k) dst[k] = v[k];
}

// push step s (wave-uniform); true after a step s = 7 (mod 8), with the group sums in v
template <int NV>
__device__ __forceinline__ bool lane_push8(LaneTree8<NV>& t, int s, double (&v)[NV], int lane) {
  if (!(s & 1)) { lane_keep(t.p[0], v); return false; }
  lane_combine<0>(t.p[0], v, lane);
  if (!(s & 2)) { lane_keep(t.p[1], v); return false; }
  lane_combine<1>(t.p[1], v, lane);
  if (!(s & 4)) { lane_keep(t.p[2], v); return false; }
  lane_combine<2>(t.p[2], v, lane);
  return true;
}

// The totals of the 8 steps s0 .. s0 + 7 from the group sums v of lane_push8, added in group
// order through buf (64 NV doubles of LDS): lane q < 8 NV gets component q / 8 of step
// s0 + q % 8 and returns true.
template <int NV>
__device__ __forceinline__ bool lane_finish8(double* __restrict__ buf, const double (&v)[NV],
                                             int lane, double& total) {
#pragma unroll
  for (int k = 0; k < NV; ++k) buf[((lane & 7) * 8 + (lane >> 3)) * NV + k] = v[k];
  __syncthreads();
  total = 0.0;
  const bool mine = lane < 8 * NV;
  if (mine) {
    const int step = lane & 7, k = lane >> 3;
#pragma unroll
    for (int g = 0; g < 8; ++g) total += buf[(step * 8 + g) * NV + k];
  }
  __syncthreads();
  return mine;
}

// ---------------------------------------------------------------- two-body term

// The backward deals a work item's 64 sources over the W waves of its block, kT / W
// consecutive sources to a wave (whole 8-source flushes), every wave holding all 64
// receivers: three waves per SIMD hold about as many waves as there are tile pairs, so one
// wave per item would leave the kernel as long as its slowest items; finer items keep the
// SIMDs filled to the end. The sources are staged once per block; the receiver-side sums
// of the waves meet in LDS in wave order (the same order on every run).
template <bool BACKWARD, int W>
struct PairStage {
  double w[kT];                        // the sources' upstream gradient g_e2
  double gr[BACKWARD ? kT : 1];        // the receivers' (the dE/d alpha products)
  int id[BACKWARD ? 2 : 1][kT];        // atom ids of the receivers, the sources
  double sa[BACKWARD ? 1 : kT][kNW + 1];  // the energy kernel: the sources' alpha(i w) times
                                          // the quadrature weight c_cp3(w)
  int win[3][kT];                      // packed image windows
  union {
    struct {
      double x[kT], y[kT], z[kT];      // bohr
      double p[kT], q[kT];             // r4r2, its square root
      double red[W][8 * 8 * 3];        // lane_finish8, one buffer per wave
    } s;
    double comb[W > 1 ? 12 * kT : 1];  // receiver-side sums on their way across waves
  } u;
};

// The receiver-side sums v of the block's W waves, added in wave order through comb (NC x 64
// doubles); true in the last wave, whose v then holds the totals. Every wave of the block
// calls it; comb is free again when it returns.
template <int W, int NC>
__device__ __forceinline__ bool waves_combine(double* __restrict__ comb, double (&v)[NC], int wv,
                                              int lane) {
  if constexpr (W == 1) {
    return true;
  } else {
    for (int k = 0; k < W; ++k) {
      if (wv == k) {
        if (k > 0) {
#pragma unroll
          for (int c = 0; c < NC; ++c) v[c] = comb[c * kT + lane] + v[c];
        }
        if (k < W - 1) {
#pragma unroll
          for (int c = 0; c < NC; ++c) comb[c * kT + lane] = v[c];
        }
      }
      __syncthreads();
    }
    return wv == W - 1;
  }
}

// dE/d alpha(i w) of both atoms of every pair of the work item, from the pairs' image sums
// of f(r) the block's waves left in its workspace block: dE/d C6_ij = -1/2 (g_i + g_j) fsum_ij =: K_ij and
// d C6_ij / d alpha_i(w) = cp3(w) alpha_j(w), so
//   receivers: D_r[r][w] = sum_s K[s][r] cp3(w) alpha_s(w)   (64 x 23, K = 64 sources)
//   sources:   D_s[s][w] = sum_r K[s][r] cp3(w) alpha_r(w)   (tile pairs d > 0 only)
// two 64 x 64 x 24 products on the float64 matrix cores (v_mfma_f64_16x16x4: lane l gives
// A[l % 16][l / 16] and B[l / 16][l % 16] and gets D[4 v + l / 16][l % 16] in register v --
// not the float32 form's row 4 (l / 16) + v; checked on gfx950 with one-hot operands). The
// A operand is read from the block (still in cache), the B operand from the alpha table.
typedef double doublex4 __attribute__((ext_vector_type(4)));

template <bool DIAG, int W>
__device__ __forceinline__ void pair_alpha_products(
    const PairStage<true, W>& st, const TileItem& it, const double* __restrict__ alpha,
    int64_t n_nodes, const double* __restrict__ fb, double* __restrict__ partial_alpha) {
  __syncthreads();  // the block's rows, written by every lane, read across lanes and waves
  const int lane = threadIdx.x % kT, lo = lane & 15, hi = lane >> 4, wv = wave_in_block();
#pragma unroll 1
  for (int side = 0; side < (DIAG ? 1 : 2); ++side) {
    // side 0: output rows the receivers, contracted over the sources (an A load reads 16
    // consecutive doubles of four rows of K); side 1: output rows the sources, contracted
    // over the receivers (an A load reads four consecutive doubles of 16 rows)
    const int out_cnt = side == 0 ? it.rcnt : it.scnt;
    const int b_cnt = side == 0 ? it.scnt : it.rcnt;
    const int* __restrict__ bid = st.id[1 - side];
    // every B element of the side, then the A elements of one 16-row tile at a time: the
    // loads of a batch are in flight together, the products wait once per batch
    double b[kT / 4][2];
#pragma unroll
    for (int ks = 0; ks < kT / 4; ++ks) {
      const int kk = 4 * ks + hi;  // the contracted atom of this lane's B elements
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int w = 16 * nt + lo;
        b[ks][nt] = (kk < b_cnt && w < kNW)
                        ? alpha[(int64_t)kNW * bid[kk] + w] * c_cp3[w < kNW ? w : 0]
                        : 0.0;
      }
    }
    const int slot = side == 0 ? it.ls : it.lt;
    const int64_t p0 = side == 0 ? it.r0 : it.s0;
    double* __restrict__ pa = partial_alpha + (int64_t)slot * kNW * n_nodes + p0;
#pragma unroll 1
    for (int mt = wv % 4; mt < 4; mt += W) {  // the wave's 16-row tiles
      const int m = 16 * mt + lo;  // output row of this lane's A elements
      double a[kT / 4];
#pragma unroll
      for (int ks = 0; ks < kT / 4; ++ks) {
        const int kk = 4 * ks + hi;
        const int s = side == 0 ? kk : m, r = side == 0 ? m : kk;
        a[ks] = (s < it.scnt && r < it.rcnt) ? -0.5 * (st.gr[r] + st.w[s]) * fb[s * kT + r]
                                             : 0.0;
      }
      doublex4 acc[2] = {doublex4{0.0, 0.0, 0.0, 0.0}, doublex4{0.0, 0.0, 0.0, 0.0}};
#pragma unroll
      for (int ks = 0; ks < kT / 4; ++ks)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          acc[nt] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[ks], b[ks][nt], acc[nt], 0, 0, 0);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int w = 16 * nt + lo;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int mo = 16 * mt + 4 * v + hi;
          if (w < kNW && mo < out_cnt) pa[(int64_t)w * n_nodes + mo] = acc[nt][v];
        }
      }
    }
  }
}

// BACKWARD = false: partial[slot][0][p] = the atom's sum of -1/2 C6 f(r).
// BACKWARD = true:  partial[slot][0..2][p] = grad_pos, [3..11] the cell gradient (CELL),
//                   partial_alpha[slot][w][p] = dE/d alpha(i w); fsum_out[jj][lane] (this
//                   wave's 64 x 64 block of workspace) holds the pairs' sums over images of
//                   f(r), from which pair_alpha_products forms dE/d alpha at the end. The
//                   block first holds the pairs' C6, which the lane writes
//                   before the source loop (its receiver's alpha then leaves the registers)
//                   and reads back one source at a time, just before that source's row takes
//                   the image sum: no alpha table in LDS and no 23 alpha registers in the
//                   loop, so three waves fit on a SIMD.
template <bool BACKWARD, bool CELL, bool DIAG, int W>
__device__ __forceinline__ void pair_tile(
    PairStage<BACKWARD, W>& st, const TileItem& it, const TileGeo& G, const PairParams& prm,
    const double* __restrict__ pos, const int32_t* __restrict__ species,
    const double* __restrict__ r4r2, const double* __restrict__ alpha,
    const double* __restrict__ g_e2, const int32_t* __restrict__ order, int64_t n_nodes,
    double* __restrict__ partial, double* __restrict__ fsum_out,
    double* __restrict__ partial_alpha) {
  constexpr int NV = BACKWARD ? 3 : 1;
  constexpr int NP = BACKWARD ? (CELL ? 12 : 3) : 1;
  constexpr int S = kT / W;  // sources of a wave
  static_assert(S % 8 == 0 && (BACKWARD || W == 1), "whole 8-source flushes per wave");
  const int lane = threadIdx.x % kT, wv = wave_in_block();
  const int j_lo = wv * S, j_end = std::min(j_lo + S, it.scnt);
  const bool live = lane < it.rcnt;
  const int64_t pi = it.r0 + (live ? lane : 0);
  const int i = order[pi];
  const double xa = pos[3 * (int64_t)i], ya = pos[3 * (int64_t)i + 1], za = pos[3 * (int64_t)i + 2];
  const double xb = xa * kInvBohr, yb = ya * kInvBohr, zb = za * kInvBohr;
  const double qi = r4r2[species[i]], sq3qi = sqrt(3.0 * qi);
  const double gi = BACKWARD ? g_e2[i] : 0.0;
  double ai[kNW];
#pragma unroll
  for (int w = 0; w < kNW; ++w) ai[w] = alpha[(int64_t)kNW * i + w];
  if constexpr (BACKWARD) {
    // C6 of this lane's pair with each of the wave's sources, into the block's rows; the
    // source's alpha is wave-uniform (scalar loads)
    for (int jj = j_lo; jj < j_end; ++jj) {
      const int j = __builtin_amdgcn_readfirstlane(order[it.s0 + jj]);
      const double* __restrict__ aj = alpha + (int64_t)kNW * j;
      double c6p[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int w = 0; w < kNW; ++w) c6p[w & 3] += ai[w] * (aj[w] * c_cp3[w]);
      fsum_out[jj * kT + lane] = (c6p[0] + c6p[1]) + (c6p[2] + c6p[3]);
    }
  }
  if (wv == 0) {  // the sources, staged by the first wave
    double flo[3], fhi[3];
    tile_bounds(G, xa, ya, za, live, flo, fhi);
    if (lane < it.scnt) {
    const int j = order[it.s0 + lane];
    const double xs = pos[3 * (int64_t)j], ys = pos[3 * (int64_t)j + 1], zs = pos[3 * (int64_t)j + 2];
    st.u.s.x[lane] = xs * kInvBohr;
    st.u.s.y[lane] = ys * kInvBohr;
    st.u.s.z[lane] = zs * kInvBohr;
    const double pj = r4r2[species[j]];
    st.u.s.p[lane] = pj;
    st.u.s.q[lane] = sqrt(pj);
    if constexpr (BACKWARD) {
      st.w[lane] = g_e2[j];
      st.id[1][lane] = j;
    } else {
#pragma unroll
      for (int w = 0; w < kNW; ++w) st.sa[lane][w] = alpha[(int64_t)kNW * j + w] * c_cp3[w];
    }
    int win[3];
    source_windows(G, xs, ys, zs, flo, fhi, win);
#pragma unroll
    for (int c = 0; c < 3; ++c) st.win[c][lane] = win[c];
  } else {
    st.win[0][lane] = pack_window(1, 0);  // empty
    st.win[1][lane] = pack_window(0, 0);
    st.win[2][lane] = pack_window(0, 0);
    if constexpr (BACKWARD) {
      st.w[lane] = 0.0;
      st.id[1][lane] = i;
    }
  }
    if constexpr (BACKWARD) {
      st.gr[lane] = live ? gi : 0.0;
      st.id[0][lane] = i;
    }
  }
  __syncthreads();

  const double rc2 = prm.cutoff * prm.cutoff;
  // below r = cutoff - width the switch is 1 with zero slope: r itself is not needed
  const double wzone = prm.width > 0.0 ? fmax(prm.cutoff - fmin(prm.width, prm.cutoff), 0.0)
                                       : prm.cutoff;
  const double wz2 = wzone * wzone;
  const bool switched = prm.width > 0.0;
  double e_acc = 0.0, g3[3] = {0.0, 0.0, 0.0}, cacc[9];
#pragma unroll
  for (int m = 0; m < 9; ++m) cacc[m] = 0.0;
  LaneTree8<NV> tree;
  for (int jj = j_lo; jj < j_lo + S; ++jj) {
    double vs[NV];  // this source's share from this lane's pair
#pragma unroll
    for (int k = 0; k < NV; ++k) vs[k] = 0.0;
    const int w0 = __builtin_amdgcn_readfirstlane(st.win[0][jj]);
    const int w1 = __builtin_amdgcn_readfirstlane(st.win[1][jj]);
    const int w2 = __builtin_amdgcn_readfirstlane(st.win[2][jj]);
    const int lo0 = window_lo(w0), hi0 = window_hi(w0), lo1 = window_lo(w1), hi1 = window_hi(w1),
              lo2 = window_lo(w2), hi2 = window_hi(w2);
    double fs = 0.0;  // the pair's sum over images of f(r)
    if (lo0 <= hi0 && lo1 <= hi1 && lo2 <= hi2) {
      double c6;
      if constexpr (BACKWARD) {
        c6 = fsum_out[jj * kT + lane];
      } else {
        // four partial sums: four short dependency chains instead of one of 23
        double c6p[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int w = 0; w < kNW; ++w) c6p[w & 3] += ai[w] * st.sa[jj][w];
        c6 = (c6p[0] + c6p[1]) + (c6p[2] + c6p[3]);
      }
      // rr = 3 r4r2_i r4r2_j and R0 = a1 sqrt(rr) + a2, sqrt(rr) = sqrt(3 r4r2_i) sqrt(r4r2_j)
      const double rr = 3.0 * qi * st.u.s.p[jj];
      const double s8rr = prm.s8 * rr;
      const double r0 = prm.a1 * (sq3qi * st.u.s.q[jj]) + prm.a2;
      const double r02 = r0 * r0;
      const double r06 = r02 * r02 * r02, r08 = r06 * r02;
      const double dx = xb - st.u.s.x[jj], dy = yb - st.u.s.y[jj], dz = zb - st.u.s.z[jj];
      // E = sum_i g_i e_i: the pair's energy enters with (g_i + g_j) (-1/2 C6 f); the
      // vector's gradient per Angstrom carries d r_bohr / d v = v_bohr / (r_bohr bohr)
      const double wsum = BACKWARD ? gi + st.w[jj] : 0.0;
      const double k2 = -0.5 * kInvBohr * c6;
      double fsum = 0.0;                       // sum over images of f(r)
      double sv[3] = {0.0, 0.0, 0.0};          // sum of (df/dr / r) v
      double wv[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};  // sum of v (x) (df/dr / r) v, symmetric
      for (int n0 = lo0; n0 <= hi0; ++n0)
        for (int n1 = lo1; n1 <= hi1; ++n1) {
          // the image's vector in bohr, d + n @ cell
          const double px = dx + n0 * G.ab[0] + n1 * G.ab[3];
          const double py = dy + n0 * G.ab[1] + n1 * G.ab[4];
          const double pz = dz + n0 * G.ab[2] + n1 * G.ab[5];
          for (int n2 = lo2; n2 <= hi2; ++n2) {
            const double vx = px + n2 * G.ab[6], vy = py + n2 * G.ab[7], vz = pz + n2 * G.ab[8];
            const double r2 = vx * vx + vy * vy + vz * vz;
            const bool in = live && r2 > 0.0 && r2 <= rc2;
            if (!__any(in)) continue;
            // every lane evaluates the term (a lane outside the cutoff takes as long either
            // way) and the ones outside discard it by a select: no divergent branch
            // t6 = 1 / (r^6 + r0^6), t8 = 1 / (r^8 + r0^8) from one reciprocal
            const double r4 = r2 * r2, r6 = r4 * r2, r8 = r6 * r2;
            const double p6 = r6 + r06, p8 = r8 + r08;
            const double inv = rcp_nr(p6 * p8);
            const double t6 = p8 * inv, t8 = p6 * inv;
            const double g = prm.s6 * t6 + s8rr * t8;
            double sw = 1.0, dsw_r = 0.0;  // the switch and its slope over r
            if (switched && r2 > wz2) {
              const double rinv = rsq_nr(r2);
              double dsw;
              switch_d(r2 * rinv, prm.cutoff, prm.width, sw, dsw);
              dsw_r = dsw * rinv;
            }
            fsum += in ? sw * g : 0.0;
            if (BACKWARD) {
              // (d f / d r) / r
              const double dg_r = -6.0 * prm.s6 * r4 * t6 * t6 - 8.0 * s8rr * r6 * t8 * t8;
              const double df_r = in ? dsw_r * g + sw * dg_r : 0.0;
              const double ox = df_r * vx, oy = df_r * vy, oz = df_r * vz;
              sv[0] += ox;
              sv[1] += oy;
              sv[2] += oz;
              if (CELL) {
                wv[0] += vx * ox;
                wv[1] += vx * oy;
                wv[2] += vx * oz;
                wv[3] += vy * oy;
                wv[4] += vy * oz;
                wv[5] += vz * oz;
              }
            }
          }
        }
      if (BACKWARD && CELL) {
        // sum over images of n (x) (df/dr / r) v through n @ cell = v - d: the cell-space
        // moments (v - d) (x) (df/dr / r) v, mapped back by the inverse cell at the end.
        // The weight: a directed pair of the own tile carries its receiver's g only (its
        // reverse, also in the tile, carries the source's).
        const double cs = (DIAG ? gi : wsum) * k2;
        const double w9[9] = {wv[0], wv[1], wv[2], wv[1], wv[3], wv[4], wv[2], wv[4], wv[5]};
        const double dd[3] = {dx, dy, dz};
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
          for (int k = 0; k < 3; ++k) cacc[3 * m + k] += cs * (w9[3 * m + k] - dd[m] * sv[k]);
      }
      fs = fsum;
      if (!BACKWARD) {
        const double e = -0.5 * c6 * fsum;
        e_acc += e;
        vs[0] = e;
      } else {
        const double gs = wsum * k2;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          g3[k] += gs * sv[k];
          vs[k] = -gs * sv[k];
        }
      }
    }
    if (BACKWARD) fsum_out[jj * kT + lane] = fs;
    if (!DIAG && lane_push8(tree, jj, vs, lane)) {
      // the source tile's side of the last 8 sources
      double total;
      const int js = jj - 7 + (lane & 7);
      double* po = partial + (int64_t)it.lt * NP * n_nodes + it.s0 + js;
      if (lane_finish8(st.u.s.red[wv], vs, lane, total) && js < it.scnt)
        po[(int64_t)(lane >> 3) * n_nodes] = total;
      if (BACKWARD && CELL && lane < 8 && js < it.scnt) {
#pragma unroll
        for (int m = 0; m < 9; ++m) po[(int64_t)(3 + m) * n_nodes] = 0.0;
      }
    }
  }
  // the receivers' side, summed over the waves (the staging area is reused for it)
  if constexpr (W > 1) __syncthreads();
  double v[NP];
  if constexpr (!BACKWARD) {
    v[0] = e_acc;
  } else {
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] = g3[k];
    if constexpr (CELL) {
#pragma unroll
      for (int m = 0; m < 9; ++m) v[3 + m] = cacc[m];
    }
  }
  if (waves_combine<W>(st.u.comb, v, wv, lane) && live) {
    double* po = partial + (int64_t)it.ls * NP * n_nodes + pi;
#pragma unroll
    for (int k = 0; k < (BACKWARD ? 3 : 1); ++k) po[(int64_t)k * n_nodes] = v[k];
    if constexpr (BACKWARD && CELL) {
      // n_c = sum_m (v - d)_m inverse(cell in bohr)_mc, the inverse in bohr being bohr
      // times that in Angstrom
#pragma unroll
      for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          const double t = G.inv[c] * v[3 + k] + G.inv[3 + c] * v[6 + k] + G.inv[6 + c] * v[9 + k];
          po[(int64_t)(3 + 3 * c + k) * n_nodes] = kBohr * t;
        }
    }
  }
  if constexpr (BACKWARD) pair_alpha_products<DIAG, W>(st, it, alpha, n_nodes, fsum_out,
                                                        partial_alpha);
}

// The energy kernel (64, 2): at most 256 registers, two waves per SIMD (18 KB of LDS). The
// backward (64 W, 3): at most 168 registers, three waves per SIMD.
template <bool BACKWARD, bool CELL, int W>
__global__ __launch_bounds__(kT * W, BACKWARD ? 3 : 2) void d4_pair_tiles_kernel(
    const double* __restrict__ pos, const int32_t* __restrict__ species,
    const int64_t* __restrict__ node_ptr, int64_t n_graphs, const double* __restrict__ cell,
    const int32_t* __restrict__ images, const double* __restrict__ r4r2,
    const double* __restrict__ alpha, PairParams prm, const double* __restrict__ g_e2,
    const int32_t* __restrict__ order, const int32_t* __restrict__ tile_ptr, int64_t n_nodes,
    int max_nt, double* __restrict__ partial, double* __restrict__ fsum,
    double* __restrict__ partial_alpha) {
  __shared__ PairStage<BACKWARD, W> st;
  TileItem it;
  if (!tile_item(tile_ptr, node_ptr, n_graphs, n_nodes, max_nt, it)) return;
  TileGeo G;
  tile_geo(cell, images, it.b, prm.cutoff * kBohr, G);
  double* fb = BACKWARD ? fsum + ((int64_t)blockIdx.x * max_nt + blockIdx.y) * (kT * kT) : nullptr;
  if (it.ls == it.lt)
    pair_tile<BACKWARD, CELL, true, W>(st, it, G, prm, pos, species, r4r2, alpha, g_e2, order,
                                       n_nodes, partial, fb, partial_alpha);
  else
    pair_tile<BACKWARD, CELL, false, W>(st, it, G, prm, pos, species, r4r2, alpha, g_e2, order,
                                        n_nodes, partial, fb, partial_alpha);
}

// ---------------------------------------------------------------- coordination numbers

// As the pair backward, a work item's sources dealt over the W waves of its block.
template <int W>
struct CnStage {
  int win[3][kT];
  union {
    struct {
      double x[kT], y[kT], z[kT];  // bohr
      double rc[kT], en[kT];       // covalent radius (bohr), electronegativity
      double w[kT], w2[kT];        // upstream gradients of cn_d4 and cn_raw
      double red[W][8 * 8 * 3];    // lane_finish8, one buffer per wave
    } s;
    double comb[W > 1 ? 12 * kT : 1];  // receiver-side sums on their way across waves
  } u;
};

// BACKWARD = false: partial[slot][0/1][p] = (cn_d4, cn_raw) sums.
// BACKWARD = true:  partial[slot][0..2][p] = grad_pos, [3..11] the cell gradient (CELL).
template <bool BACKWARD, bool CELL, bool DIAG, int W>
__device__ __forceinline__ void cn_tile(
    CnStage<W>& st, const TileItem& it, const TileGeo& G, const CnParams& prm,
    const double* __restrict__ pos, const int32_t* __restrict__ species,
    const double* __restrict__ rcov, const double* __restrict__ en,
    const double* __restrict__ g_cn, const double* __restrict__ g_raw,
    const int32_t* __restrict__ order, int64_t n_nodes, double* __restrict__ partial) {
  constexpr int NV = BACKWARD ? 3 : 2;
  constexpr int NP = BACKWARD ? (CELL ? 12 : 3) : 2;
  constexpr int S = kT / W;  // sources of a wave
  static_assert(S % 8 == 0, "whole 8-source flushes per wave");
  const int lane = threadIdx.x % kT, wv = wave_in_block();
  const int j_lo = wv * S;
  const bool live = lane < it.rcnt;
  const int64_t pi = it.r0 + (live ? lane : 0);
  const int i = order[pi];
  const double xa = pos[3 * (int64_t)i], ya = pos[3 * (int64_t)i + 1], za = pos[3 * (int64_t)i + 2];
  const double xb = xa * kInvBohr, yb = ya * kInvBohr, zb = za * kInvBohr;
  const int si = species[i];
  const double rci = rcov[si], eni = en[si];
  const double gi = BACKWARD && g_cn ? g_cn[i] : 0.0;
  const double g2i = BACKWARD && g_raw ? g_raw[i] : 0.0;
  const double cmax = prm.cut_cn > prm.cut_eeq ? prm.cut_cn : prm.cut_eeq;
  const double cmax2 = cmax * cmax;
  // Beyond r = rc (1 + 27.5 / kcn) the erf argument is below -27.5: the count rounds to exactly
  // zero and so does its slope, -kcn / (rc sqrt(pi)) exp(-x^2) (exp(-756) underflows). Such
  // pairs are skipped: each source's window reaches only as far as its largest rc with the
  // tile's receivers allows, and each pair as far as its own rc allows.
  const double zfac = 1.0 + 27.5 / prm.kcn;
  if (wv == 0) {  // the sources, staged by the first wave
    double flo[3], fhi[3];
    tile_bounds(G, xa, ya, za, live, flo, fhi);
    const double rc_tile = wave_max(live ? rci : 0.0);
    if (lane < it.scnt) {
      const int j = order[it.s0 + lane];
      const double xs = pos[3 * (int64_t)j], ys = pos[3 * (int64_t)j + 1],
                   zs = pos[3 * (int64_t)j + 2];
      st.u.s.x[lane] = xs * kInvBohr;
      st.u.s.y[lane] = ys * kInvBohr;
      st.u.s.z[lane] = zs * kInvBohr;
      const int sj = species[j];
      st.u.s.rc[lane] = rcov[sj];
      st.u.s.en[lane] = en[sj];
      if (BACKWARD) {
        st.u.s.w[lane] = g_cn ? g_cn[j] : 0.0;
        st.u.s.w2[lane] = g_raw ? g_raw[j] : 0.0;
      }
      const double r_src = fmin(cmax, (rc_tile + rcov[sj]) * zfac);
      int win[3];
      source_windows(G, xs, ys, zs, flo, fhi, win, r_src * kBohr);
#pragma unroll
      for (int c = 0; c < 3; ++c) st.win[c][lane] = win[c];
    } else {
      st.win[0][lane] = pack_window(1, 0);
      st.win[1][lane] = pack_window(0, 0);
      st.win[2][lane] = pack_window(0, 0);
    }
  }
  __syncthreads();
  // a tile pair none of whose sources reaches the receivers' box (most of them, the CN's
  // reach being a few Angstrom): its slots hold zeros, written without the source loop
  if (!DIAG) {
    bool reach = false;
    if (lane < it.scnt) {
      const int w0 = st.win[0][lane], w1 = st.win[1][lane], w2 = st.win[2][lane];
      reach = window_lo(w0) <= window_hi(w0) && window_lo(w1) <= window_hi(w1) &&
              window_lo(w2) <= window_hi(w2);
    }
    if (!__any(reach)) {  // the same answer in every wave of the block
      if (live && wv == 0) {
        double* po = partial + (int64_t)it.ls * NP * n_nodes + pi;
#pragma unroll
        for (int k = 0; k < NP; ++k) po[(int64_t)k * n_nodes] = 0.0;
      }
      if (lane < it.scnt && wv == 0) {
        double* po = partial + (int64_t)it.lt * NP * n_nodes + it.s0 + lane;
#pragma unroll
        for (int k = 0; k < NP; ++k) po[(int64_t)k * n_nodes] = 0.0;
      }
      return;
    }
  }

  const double inv_k6 = 1.0 / prm.k6;
  double acc[2] = {0.0, 0.0}, g3[3] = {0.0, 0.0, 0.0}, cacc[9];
#pragma unroll
  for (int m = 0; m < 9; ++m) cacc[m] = 0.0;
  LaneTree8<NV> tree;
  for (int jj = j_lo; jj < j_lo + S; ++jj) {
    double vs[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) vs[k] = 0.0;
    const int w0 = __builtin_amdgcn_readfirstlane(st.win[0][jj]);
    const int w1 = __builtin_amdgcn_readfirstlane(st.win[1][jj]);
    const int w2 = __builtin_amdgcn_readfirstlane(st.win[2][jj]);
    const int lo0 = window_lo(w0), hi0 = window_hi(w0), lo1 = window_lo(w1), hi1 = window_hi(w1),
              lo2 = window_lo(w2), hi2 = window_hi(w2);
    if (lo0 <= hi0 && lo1 <= hi1 && lo2 <= hi2) {
      const double rc = rci + st.u.s.rc[jj];
      const double den = fabs(eni - st.u.s.en[jj]) + prm.k5;
      const double enf = prm.k4 * exp(-den * den * inv_k6);
      // per pair: k0 / rc and the erf count's slope factor -k0 / (rc sqrt(pi))
      const double k_rc = prm.kcn / rc;
      const double dk = -k_rc * kInvSqrtPi;
      const double dx = xb - st.u.s.x[jj], dy = yb - st.u.s.y[jj], dz = zb - st.u.s.z[jj];
      const double wsum = BACKWARD ? gi + st.u.s.w[jj] : 0.0;
      const double w2sum = BACKWARD ? g2i + st.u.s.w2[jj] : 0.0;
      const double reach2 = fmin(cmax2, rc * zfac * (rc * zfac));
      double c_cn = 0.0, c_eeq = 0.0;          // counts within the two cutoffs
      double sv[3] = {0.0, 0.0, 0.0};          // sum of the weighted gradients
      double sc[3] = {0.0, 0.0, 0.0};          // the same with the cell's weights (own tile)
      double wv[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};  // v (x) cell-weighted gradient
      for (int n0 = lo0; n0 <= hi0; ++n0)
        for (int n1 = lo1; n1 <= hi1; ++n1) {
          const double px = dx + n0 * G.ab[0] + n1 * G.ab[3];
          const double py = dy + n0 * G.ab[1] + n1 * G.ab[4];
          const double pz = dz + n0 * G.ab[2] + n1 * G.ab[5];
          for (int n2 = lo2; n2 <= hi2; ++n2) {
            const double vx = px + n2 * G.ab[6], vy = py + n2 * G.ab[7], vz = pz + n2 * G.ab[8];
            const double r2 = vx * vx + vy * vy + vz * vz;
            const bool in = live && r2 > 0.0 && r2 <= reach2;
            if (!__any(in)) continue;
            // every lane evaluates the term and the ones outside the cutoffs discard it
            const double rinv = rsq_nr(fmax(r2, 1e-300));
            const double r = r2 * rinv;
            const bool in_cn = in && r <= prm.cut_cn, in_eeq = in && r <= prm.cut_eeq;
            // (1 + erf(-k0 (r - rc) / rc)) / 2; d/dr = -k0 exp(-x^2) / (rc sqrt(pi))
            const double x = k_rc * (rc - r);
            if (!BACKWARD) {
              const double count = 0.5 * (1.0 + erf(x));
              c_cn += in_cn ? count : 0.0;
              c_eeq += in_eeq ? count : 0.0;
            } else {
              const double dcount = dk * exp(-x * x);
              // per Angstrom of the vector: d r_bohr / d v = v_bohr / (r bohr)
              const double s = dcount * rinv * kInvBohr;
              const double bs = ((in_cn ? wsum * enf : 0.0) + (in_eeq ? w2sum : 0.0)) * s;
              sv[0] += bs * vx;
              sv[1] += bs * vy;
              sv[2] += bs * vz;
              if (CELL) {
                // a directed pair of the own tile carries its receiver's weights only
                const double os = DIAG ? ((in_cn ? gi * enf : 0.0) + (in_eeq ? g2i : 0.0)) * s
                                       : bs;
                const double ox = os * vx, oy = os * vy, oz = os * vz;
                if (DIAG) {
                  sc[0] += ox;
                  sc[1] += oy;
                  sc[2] += oz;
                }
                wv[0] += vx * ox;
                wv[1] += vx * oy;
                wv[2] += vx * oz;
                wv[3] += vy * oy;
                wv[4] += vy * oz;
                wv[5] += vz * oz;
              }
            }
          }
        }
      if (!BACKWARD) {
        acc[0] += enf * c_cn;
        acc[1] += c_eeq;
        vs[0] = enf * c_cn;
        vs[1] = c_eeq;
      } else {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          g3[k] += sv[k];
          vs[k] = -sv[k];
        }
        if (CELL) {
          // sum over images of n (x) gradient through n @ cell = v - d (mapped back by the
          // inverse cell at the end)
          const double w9[9] = {wv[0], wv[1], wv[2], wv[1], wv[3], wv[4], wv[2], wv[4], wv[5]};
          const double dd[3] = {dx, dy, dz};
#pragma unroll
          for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int k = 0; k < 3; ++k) cacc[3 * m + k] += w9[3 * m + k] - dd[m] * (DIAG ? sc[k] : sv[k]);
        }
      }
    }
    if (!DIAG && lane_push8(tree, jj, vs, lane)) {
      double total;
      const int js = jj - 7 + (lane & 7);
      double* po = partial + (int64_t)it.lt * NP * n_nodes + it.s0 + js;
      if (lane_finish8(st.u.s.red[wv], vs, lane, total) && js < it.scnt)
        po[(int64_t)(lane >> 3) * n_nodes] = total;
      if (BACKWARD && CELL && lane < 8 && js < it.scnt) {
#pragma unroll
        for (int m = 0; m < 9; ++m) po[(int64_t)(3 + m) * n_nodes] = 0.0;
      }
    }
  }
  // the receivers' side, summed over the waves (the staging area is reused for it)
  if constexpr (W > 1) __syncthreads();
  double v[NP];
  if constexpr (!BACKWARD) {
    v[0] = acc[0];
    v[1] = acc[1];
  } else {
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] = g3[k];
    if constexpr (CELL) {
#pragma unroll
      for (int m = 0; m < 9; ++m) v[3 + m] = cacc[m];
    }
  }
  if (waves_combine<W>(st.u.comb, v, wv, lane) && live) {
    double* po = partial + (int64_t)it.ls * NP * n_nodes + pi;
#pragma unroll
    for (int k = 0; k < (BACKWARD ? 3 : 2); ++k) po[(int64_t)k * n_nodes] = v[k];
    if constexpr (BACKWARD && CELL) {
#pragma unroll
      for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          const double t = G.inv[c] * v[3 + k] + G.inv[3 + c] * v[6 + k] + G.inv[6 + c] * v[9 + k];
          po[(int64_t)(3 + 3 * c + k) * n_nodes] = kBohr * t;
        }
    }
  }
}

template <bool BACKWARD, bool CELL, int W>
__global__ __launch_bounds__(kT * W, 3) void d4_cn_tiles_kernel(
    const double* __restrict__ pos, const int32_t* __restrict__ species,
    const int64_t* __restrict__ node_ptr, int64_t n_graphs, const double* __restrict__ cell,
    const int32_t* __restrict__ images, const double* __restrict__ rcov,
    const double* __restrict__ en, CnParams prm, const double* __restrict__ g_cn,
    const double* __restrict__ g_raw, const int32_t* __restrict__ order,
    const int32_t* __restrict__ tile_ptr, int64_t n_nodes, int max_nt,
    double* __restrict__ partial) {
  __shared__ CnStage<W> st;
  TileItem it;
  if (!tile_item(tile_ptr, node_ptr, n_graphs, n_nodes, max_nt, it)) return;
  TileGeo G;
  const double cmax = prm.cut_cn > prm.cut_eeq ? prm.cut_cn : prm.cut_eeq;
  tile_geo(cell, images, it.b, cmax * kBohr, G);
  if (it.ls == it.lt)
    cn_tile<BACKWARD, CELL, true, W>(st, it, G, prm, pos, species, rcov, en, g_cn, g_raw, order,
                                     n_nodes, partial);
  else
    cn_tile<BACKWARD, CELL, false, W>(st, it, G, prm, pos, species, rcov, en, g_cn, g_raw, order,
                                      n_nodes, partial);
}

// ---------------------------------------------------------------- image counts

// images[b][c] = ceil(cutoff / spacing_c) for periodic axes, the interplanar spacing of axis
// c being the cell volume over |a_(c+1) x a_(c+2)| (the image range of
// neighborlist.py:74-104); 0 on non-periodic axes (pbc[b][c] == 0; pbc NULL: all periodic)
// and for an all-zero or degenerate cell; at most 32767. One thread per structure.
__global__ void d4_image_counts_kernel(const double* __restrict__ cell,
                                       const uint8_t* __restrict__ pbc, int64_t n_graphs,
                                       double cutoff, int32_t* __restrict__ images) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_graphs) return;
  const double* a = cell + 9 * b;
  double x[3][3];  // x[c] = a_(c+1) x a_(c+2)
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const double* u = a + 3 * ((c + 1) % 3);
    const double* v = a + 3 * ((c + 2) % 3);
    x[c][0] = u[1] * v[2] - u[2] * v[1];
    x[c][1] = u[2] * v[0] - u[0] * v[2];
    x[c][2] = u[0] * v[1] - u[1] * v[0];
  }
  const double vol = fabs(a[0] * x[0][0] + a[1] * x[0][1] + a[2] * x[0][2]);
  double total = 0.0;
#pragma unroll
  for (int k = 0; k < 9; ++k) total += fabs(a[k]);
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const double norm = sqrt(x[c][0] * x[c][0] + x[c][1] * x[c][1] + x[c][2] * x[c][2]);
    const bool live = total > 1e-8 && vol > 0.0 && norm > 0.0 && (pbc == nullptr || pbc[3 * b + c]);
    const double n = live ? ceil(cutoff * norm / vol) : 0.0;
    images[3 * b + c] = (int32_t)fmin(fmax(n, 0.0), 32767.0);
  }
}

// ---------------------------------------------------------------- slot reduction

// out[order[p] * nk + (k - k0)] = sum over the slots s < nt of p's structure of
// partial[s][k][p], for the components k0 <= k < k0 + nk of a partial array of np
// components. The 8 waves of a block share 64 outputs (64 consecutive places of one
// component): wave w sums the slots w, w + 8, ... in order and wave 0 adds the waves' sums
// in wave order. A structure larger than max_atoms (more tiles than slots) gives NaN.
// The slot sums of up to three partial arrays in one launch: grid row y belongs to target q
// with y0[q] <= y < y0[q + 1], component k = k0 + (y - y0[q]) of its partial array (np
// components) into out[i * nk + (k - k0)]. Per atom the slots are added in slot order.
struct ReduceTarget {
  const double* partial;
  double* out;
  int np, k0, nk;
};
struct ReduceTargets {
  ReduceTarget t[3];
  int y0[4];
  int n;
};

__global__ __launch_bounds__(kT * kRedWaves) void d4_tiles_reduce_kernel(
    ReduceTargets R, int64_t n_nodes, const int32_t* __restrict__ order,
    const int32_t* __restrict__ batch, const int64_t* __restrict__ node_ptr, int max_nt) {
  __shared__ double red[kRedWaves][kT];
  const int lane = threadIdx.x % kT;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kT));
  const int y = (int)blockIdx.y;
  const int q = y < R.y0[1] ? 0 : (y < R.y0[2] ? 1 : 2);   // uniform
  const ReduceTarget T = R.t[q];
  const int64_t p = (int64_t)blockIdx.x * kT + lane;
  const int k = T.k0 + (y - R.y0[q]);
  const bool live = p < n_nodes;
  double s = 0.0;
  int nt = 0;
  int64_t i = 0;
  if (live) {
    i = std::min<int64_t>(std::max<int64_t>(order[p], 0), n_nodes - 1);
    const int b = batch[i];
    nt = (int)((node_ptr[b + 1] - node_ptr[b] + kT - 1) / kT);
    const double* src = T.partial + (int64_t)k * n_nodes + p;
    const int64_t stride = (int64_t)T.np * n_nodes;
    const int ns = std::min(nt, max_nt);
    for (int slot = wv; slot < ns; slot += kRedWaves) s += src[slot * stride];
  }
  red[wv][lane] = s;
  __syncthreads();
  if (wv == 0 && live) {
    double t = red[0][lane];
#pragma unroll
    for (int w = 1; w < kRedWaves; ++w) t += red[w][lane];
    T.out[i * T.nk + (k - T.k0)] = nt > max_nt ? __builtin_nan("") : t;
  }
}

// ---------------------------------------------------------------- host side

struct TilesWs {
  int32_t* order;     // sorted place -> atom (plan part 1)
  int32_t* tile_ptr;  // first tile of each structure (plan part 2)
  double* partial;
  double* partial_alpha;
  double* fsum;       // pair sums of the two-body backward, kT x kT per work item
  int max_nt;
  int64_t grid_tiles;
  size_t need;
};

size_t ws_align(size_t x) { return (x + 255) & ~size_t(255); }

// workspace layout for components np (+ 23 alpha components when alpha is set)
TilesWs tiles_layout(void* ws, int64_t n_nodes, int64_t n_graphs, int64_t max_atoms, int np,
                     bool alpha) {
  TilesWs w{};
  w.max_nt = (int)((std::max<int64_t>(max_atoms, 1) + kT - 1) / kT);
  // tiles of all structures: sum of ceil(n_b / 64) <= (n_nodes + 63 n_graphs) / 64
  w.grid_tiles = std::min<int64_t>(n_nodes, (n_nodes + (kT - 1) * n_graphs) / kT);
  char* base = static_cast<char*>(ws);
  size_t o = 0;
  const size_t o_order = o;
  o += ws_align(4 * (size_t)n_nodes);
  const size_t o_tiles = o;
  o += ws_align(4 * (size_t)(n_graphs + 1));
  const size_t o_part = o;
  o += ws_align((size_t)w.max_nt * np * n_nodes * sizeof(double));
  const size_t o_alpha = o;
  if (alpha) o += ws_align((size_t)w.max_nt * kNW * n_nodes * sizeof(double));
  const size_t o_fsum = o;
  if (alpha) o += ws_align((size_t)w.grid_tiles * w.max_nt * kT * kT * sizeof(double));
  w.need = o;
  if (base) {
    w.order = reinterpret_cast<int32_t*>(base + o_order);
    w.tile_ptr = reinterpret_cast<int32_t*>(base + o_tiles);
    w.partial = reinterpret_cast<double*>(base + o_part);
    w.partial_alpha = alpha ? reinterpret_cast<double*>(base + o_alpha) : nullptr;
    w.fsum = alpha ? reinterpret_cast<double*>(base + o_fsum) : nullptr;
  }
  return w;
}

int tiles_check(const double* pos, int64_t n_nodes, const int32_t* species, const int32_t* batch,
                const int64_t* node_ptr, int64_t n_graphs, const double* cell,
                const int32_t* images, int64_t max_atoms) {
  XNN_REQUIRE(n_nodes >= 0 && n_graphs >= 1, "negative size or no structure");
  XNN_REQUIRE(n_nodes == 0 || (pos && species && batch && node_ptr), "NULL atom input");
  XNN_REQUIRE(cell == nullptr || images != nullptr, "a cell needs the image counts");
  XNN_REQUIRE(max_atoms >= 1 || n_nodes == 0, "max_atoms must be >= 1");
  XNN_REQUIRE(n_nodes < (int64_t(1) << 31), "more than 2^31 atoms");
  XNN_REQUIRE((max_atoms + kT - 1) / kT <= 65535, "max_atoms above 64 x 65535");
  return XNN_OK;
}

// the plan: order (n_nodes int32) then tile_ptr (n_graphs + 1 int32)
size_t plan_bytes(int64_t n_nodes, int64_t n_graphs) {
  return ws_align(4 * (size_t)n_nodes) + 4 * (size_t)(n_graphs + 1);
}

void build_plan(const double* pos, int64_t n_nodes, const int64_t* node_ptr, int64_t n_graphs,
                const double* cell, const int32_t* images, int32_t* order, int32_t* tile_ptr,
                hipStream_t s) {
  hipLaunchKernelGGL(d4_order_kernel, dim3((unsigned)(n_graphs + 1)), dim3(kOrderThreads), 0, s,
                     pos, n_nodes, node_ptr, n_graphs, cell, images, order, tile_ptr);
}

// the caller's plan (from xnn_d4_plan on the same positions and cells), or one built now in
// the workspace
void launch_order(const double* pos, int64_t n_nodes, const int64_t* node_ptr, int64_t n_graphs,
                  const double* cell, const int32_t* images, const int32_t* plan, TilesWs& w,
                  hipStream_t s) {
  if (plan != nullptr) {
    w.order = const_cast<int32_t*>(plan);
    w.tile_ptr = const_cast<int32_t*>(plan) + ws_align(4 * (size_t)n_nodes) / 4;
    return;
  }
  build_plan(pos, n_nodes, node_ptr, n_graphs, cell, images, w.order, w.tile_ptr, s);
}

// the targets with an output, in one launch
void launch_reduce(std::initializer_list<ReduceTarget> targets, int64_t n_nodes, const TilesWs& w,
                   const int32_t* batch, const int64_t* node_ptr, hipStream_t s) {
  ReduceTargets R{};
  int rows = 0;
  for (const ReduceTarget& t : targets) {
    if (t.out == nullptr) continue;
    R.t[R.n] = t;
    R.y0[R.n] = rows;
    rows += t.nk;
    ++R.n;
  }
  for (int q = R.n; q < 4; ++q) R.y0[q] = rows;
  if (rows == 0) return;
  hipLaunchKernelGGL(d4_tiles_reduce_kernel, dim3((unsigned)((n_nodes + kT - 1) / kT), rows),
                     dim3(kT * kRedWaves), 0, s, R, n_nodes, w.order, batch, node_ptr, w.max_nt);
}

dim3 tiles_grid(const TilesWs& w) { return dim3((unsigned)w.grid_tiles, (unsigned)w.max_nt); }

// waves per block of the pair backward: two (measured on the C5 box against one and four:
// 396 us, 436 us, 399 us)
constexpr int kPairWaves = 2;
constexpr int kCnWaves = 2;   // the same for the coordination-number kernels

void launch_pair_backward(bool with_cell, dim3 grid, hipStream_t s, const double* pos,
                          const int32_t* species, const int64_t* node_ptr, int64_t n_graphs,
                          const double* cell, const int32_t* images, const double* r4r2,
                          const double* alpha, const PairParams& p, const double* g_e2,
                          const int32_t* order, const int32_t* tile_ptr, int64_t n_nodes,
                          int max_nt, double* partial, double* fsum, double* partial_alpha) {
  auto k = with_cell ? d4_pair_tiles_kernel<true, true, kPairWaves>
                     : d4_pair_tiles_kernel<true, false, kPairWaves>;
  hipLaunchKernelGGL(k, grid, dim3(kT * kPairWaves), 0, s, pos, species, node_ptr, n_graphs, cell,
                     images, r4r2, alpha, p, g_e2, order, tile_ptr, n_nodes, max_nt, partial, fsum,
                     partial_alpha);
}

}  // namespace

size_t d4_tiles_workspace_bytes(int64_t n_nodes, int64_t n_graphs, int64_t max_atoms) {
  if (n_nodes <= 0) return 0;
  // the largest user: the pair backward with the cell, 12 + 23 components
  return tiles_layout(nullptr, n_nodes, n_graphs, max_atoms, 12, true).need;
}

}  // namespace xnn

using namespace xnn;

extern "C" {

int xnn_d4_coordination(const double* pos, int64_t n_nodes, const int32_t* species,
                        const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                        int64_t max_atoms, const double* cell, const int32_t* images,
                        const int32_t* plan,
                        const double* rcov, const double* en, const xnn_d4_cn_params* prm,
                        double* cn_d4, double* cn_raw, void* workspace, size_t workspace_bytes,
                        xnn_stream_t stream) {
  const int st = tiles_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images,
                             max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(prm && rcov && en, "NULL tables or params");
  XNN_REQUIRE(n_nodes == 0 || (cn_d4 && cn_raw), "NULL output");
  if (n_nodes == 0) return XNN_OK;
  const TilesWs need = tiles_layout(nullptr, n_nodes, n_graphs, max_atoms, 2, false);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need.need,
              "workspace too small (%zu < %zu)", workspace_bytes, need.need);
  TilesWs w = tiles_layout(workspace, n_nodes, n_graphs, max_atoms, 2, false);
  const CnParams p{prm->cutoff_cn, prm->cutoff_eeq_cn, prm->kcn, prm->k4, prm->k5, prm->k6};
  hipStream_t s = as_hip(stream);
  launch_order(pos, n_nodes, node_ptr, n_graphs, cell, images, plan, w, s);
  hipLaunchKernelGGL((d4_cn_tiles_kernel<false, false, kCnWaves>), tiles_grid(w),
                     dim3(kT * kCnWaves), 0, s, pos,
                     species, node_ptr, n_graphs, cell, images, rcov, en, p, nullptr, nullptr,
                     w.order, w.tile_ptr, n_nodes, w.max_nt, w.partial);
  launch_reduce({{w.partial, cn_d4, 2, 0, 1}, {w.partial, cn_raw, 2, 1, 1}}, n_nodes, w, batch,
                node_ptr, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d4_coordination_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                                 const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                                 int64_t max_atoms, const double* cell, const int32_t* images,
                        const int32_t* plan,
                                 const double* rcov, const double* en,
                                 const xnn_d4_cn_params* prm, const double* g_cn_d4,
                                 const double* g_cn_raw, double* grad_pos, double* cell_partial,
                                 void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  const int st = tiles_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images,
                             max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(prm && rcov && en, "NULL tables or params");
  XNN_REQUIRE(n_nodes == 0 || grad_pos, "NULL grad_pos");
  if (n_nodes == 0) return XNN_OK;
  // without a cell every image is n = 0 and the cell gradient comes out zero
  const bool with_cell = cell_partial != nullptr;
  const int np = with_cell ? 12 : 3;
  const TilesWs need = tiles_layout(nullptr, n_nodes, n_graphs, max_atoms, np, false);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need.need,
              "workspace too small (%zu < %zu)", workspace_bytes, need.need);
  TilesWs w = tiles_layout(workspace, n_nodes, n_graphs, max_atoms, np, false);
  const CnParams p{prm->cutoff_cn, prm->cutoff_eeq_cn, prm->kcn, prm->k4, prm->k5, prm->k6};
  hipStream_t s = as_hip(stream);
  launch_order(pos, n_nodes, node_ptr, n_graphs, cell, images, plan, w, s);
  auto k = with_cell ? d4_cn_tiles_kernel<true, true, kCnWaves>
                     : d4_cn_tiles_kernel<true, false, kCnWaves>;
  hipLaunchKernelGGL(k, tiles_grid(w), dim3(kT * kCnWaves), 0, s, pos, species, node_ptr, n_graphs,
                     cell,
                     images, rcov, en, p, g_cn_d4, g_cn_raw, w.order, w.tile_ptr, n_nodes,
                     w.max_nt, w.partial);
  launch_reduce({{w.partial, grad_pos, np, 0, 3}, {w.partial, cell_partial, np, 3, 9}}, n_nodes, w,
                batch, node_ptr, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d4_two_body(const double* pos, int64_t n_nodes, const int32_t* species,
                    const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                    int64_t max_atoms, const double* cell, const int32_t* images,
                        const int32_t* plan,
                    const double* r4r2, const double* alpha, const xnn_d4_pair_params* prm,
                    double* e2, void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  const int st = tiles_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images,
                             max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(prm && r4r2, "NULL tables or params");
  XNN_REQUIRE(n_nodes == 0 || (alpha && e2), "NULL alpha or output");
  XNN_REQUIRE(prm->cutoff > 0.0, "pair cutoff must be positive");
  if (n_nodes == 0) return XNN_OK;
  const TilesWs need = tiles_layout(nullptr, n_nodes, n_graphs, max_atoms, 1, false);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need.need,
              "workspace too small (%zu < %zu)", workspace_bytes, need.need);
  TilesWs w = tiles_layout(workspace, n_nodes, n_graphs, max_atoms, 1, false);
  const PairParams p{prm->s6, prm->s8, prm->a1, prm->a2, prm->cutoff, prm->width};
  hipStream_t s = as_hip(stream);
  launch_order(pos, n_nodes, node_ptr, n_graphs, cell, images, plan, w, s);
  hipLaunchKernelGGL((d4_pair_tiles_kernel<false, false, 1>), tiles_grid(w), dim3(kT), 0, s, pos,
                     species, node_ptr, n_graphs, cell, images, r4r2, alpha, p, nullptr, w.order,
                     w.tile_ptr, n_nodes, w.max_nt, w.partial, nullptr, nullptr);
  launch_reduce({{w.partial, e2, 1, 0, 1}}, n_nodes, w, batch, node_ptr, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d4_two_body_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                             const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                             int64_t max_atoms, const double* cell, const int32_t* images,
                        const int32_t* plan,
                             const double* r4r2, const double* alpha,
                             const xnn_d4_pair_params* prm, const double* g_e2, double* grad_pos,
                             double* cell_partial, double* grad_alpha, void* workspace,
                             size_t workspace_bytes, xnn_stream_t stream) {
  const int st = tiles_check(pos, n_nodes, species, batch, node_ptr, n_graphs, cell, images,
                             max_atoms);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(prm && r4r2, "NULL tables or params");
  XNN_REQUIRE(n_nodes == 0 || (alpha && g_e2 && grad_pos), "NULL alpha, g_e2 or grad_pos");
  XNN_REQUIRE(prm->cutoff > 0.0, "pair cutoff must be positive");
  if (n_nodes == 0) return XNN_OK;
  // without a cell every image is n = 0 and the cell gradient comes out zero
  const bool with_cell = cell_partial != nullptr;
  const int np = with_cell ? 12 : 3;
  const TilesWs need = tiles_layout(nullptr, n_nodes, n_graphs, max_atoms, np, true);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need.need,
              "workspace too small (%zu < %zu)", workspace_bytes, need.need);
  TilesWs w = tiles_layout(workspace, n_nodes, n_graphs, max_atoms, np, true);
  const PairParams p{prm->s6, prm->s8, prm->a1, prm->a2, prm->cutoff, prm->width};
  hipStream_t s = as_hip(stream);
  launch_order(pos, n_nodes, node_ptr, n_graphs, cell, images, plan, w, s);
  launch_pair_backward(with_cell, tiles_grid(w), s, pos, species, node_ptr, n_graphs, cell, images,
                       r4r2, alpha, p, g_e2, w.order, w.tile_ptr, n_nodes, w.max_nt, w.partial,
                       w.fsum, w.partial_alpha);
  launch_reduce({{w.partial, grad_pos, np, 0, 3}, {w.partial, cell_partial, np, 3, 9},
                 {w.partial_alpha, grad_alpha, kNW, 0, kNW}},
                n_nodes, w, batch, node_ptr, s);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_d4_image_counts(const double* cell, const uint8_t* pbc, int64_t n_graphs, double cutoff,
                        int32_t* images, xnn_stream_t stream) {
  XNN_REQUIRE(n_graphs >= 0, "negative size");
  XNN_REQUIRE(cutoff >= 0.0, "negative cutoff");
  if (n_graphs == 0) return XNN_OK;
  XNN_REQUIRE(cell && images, "NULL cell or images");
  hipLaunchKernelGGL(d4_image_counts_kernel, dim3((unsigned)((n_graphs + 255) / 256)), dim3(256),
                     0, as_hip(stream), cell, pbc, n_graphs, cutoff, images);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

size_t xnn_d4_plan_bytes(int64_t n_nodes, int64_t n_graphs) {
  if (n_nodes < 0 || n_graphs < 1) return 0;
  return plan_bytes(n_nodes, n_graphs);
}

int xnn_d4_plan(const double* pos, int64_t n_nodes, const int64_t* node_ptr, int64_t n_graphs,
                const double* cell, const int32_t* images, int32_t* plan, size_t plan_bytes_given,
                xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_graphs >= 1, "negative size or no structure");
  XNN_REQUIRE(n_nodes < (int64_t(1) << 31), "more than 2^31 atoms");
  XNN_REQUIRE(node_ptr && plan, "NULL node_ptr or plan");
  XNN_REQUIRE(n_nodes == 0 || pos, "NULL positions");
  XNN_REQUIRE(cell == nullptr || images != nullptr, "a cell needs the image counts");
  const size_t need = plan_bytes(n_nodes, n_graphs);
  XNN_REQUIRE(plan_bytes_given >= need, "plan too small (%zu < %zu)", plan_bytes_given, need);
  build_plan(pos, n_nodes, node_ptr, n_graphs, cell, images, plan,
             plan + ws_align(4 * (size_t)n_nodes) / 4, as_hip(stream));
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

}  // extern "C"
