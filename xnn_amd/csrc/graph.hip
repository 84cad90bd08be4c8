// Radius graph (cell list) and edge plans (receiver/sender CSR), gfx950.
//
// xnn_radius_graph_*          build_neighbor_list (common/data/neighborlist.py:411-506):
//                             full directed list, dist < cutoff in the geometry dtype,
//                             edge (src=j, dst=i), shift = -S + o_j - o_i with o the
//                             wrap offsets (neighborlist.py:472-475, 500-505).
// xnn_radius_graph_molecules_* the molecular branch (neighborlist.py:466-468) for a batch
// xnn_edge_plan               compressed/orderings (common/models/csr.py:20-51)
//
// Cell list: atoms are binned on a grid in fractional coordinates whose bins are at
// least `cutoff` wide along every plane normal, counting-sorted by bin (stable radix
// sort), and every receiver bin stages the atoms of its neighbor bins in LDS. One wave
// tests one receiver against 64 candidates at a time and compacts the hits with a
// ballot + prefix popcount, so edges of a row land in a fixed order (neighbor bin,
// then atom index): two identical passes (count, then fill) without atomics.
#include <math.h>
#include <string.h>

#include <mutex>

#include <hipcub/hipcub.hpp>

#include "common.h"
#include "device.h"

namespace xnn {

constexpr double kBinSlack = 1e-5;       // bins are (1 + slack) * cutoff wide at least
constexpr int64_t kMaxBins = 1 << 22;   // grid size cap (bins merge beyond it)
constexpr int kTile = 1024;             // candidates staged in LDS per pass

struct GridDev {
  int nb[3], reach[3], periodic[3], has_cell;
  double lo[3], width[3], iwidth[3], inv[9];
};

static inline size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

// blocks per receiver bin: one when bins hold a few waves' worth of atoms; with few,
// crowded bins (a cutoff comparable to the cell) the receivers of a bin are spread over
// up to 1024 blocks, 4 receivers per wave on average
static inline int search_split(int64_t n_atoms, int64_t n_bins) {
  const int64_t per_bin = (n_atoms + n_bins - 1) / (n_bins > 0 ? n_bins : 1);
  const int64_t s = (per_bin + 15) / 16;
  return (int)(s < 1 ? 1 : (s > 1024 ? 1024 : s));
}

// workspace layout of the cell list (offsets in bytes); the count step fills it
// and the fill step reads it back, so both must get the same buffer.
struct GridWs {
  size_t bin_key, bin_key_sorted, atom_id, atom_sorted, wpos, offs, wpos_s, offs_s, bin_cnt,
      bin_start, counts, overflow, cursor, cub, cub_bytes, total;
};

// Sizes the count step sorts and scans in one block (a 1024-thread block scans them in a few
// microseconds, with one launch instead of the library's several); larger ones take the
// library's radix sort and scans.
constexpr int64_t kBlockScanMax = 65536;

template <typename G>
static GridWs grid_ws_layout_uncached(int64_t n, int64_t n_bins) {
  GridWs w;
  size_t at = 0;
  w.bin_key = at; at += align_up(sizeof(int32_t) * n);
  w.bin_key_sorted = at; at += align_up(sizeof(int32_t) * n);
  w.atom_id = at; at += align_up(sizeof(int32_t) * n);
  w.atom_sorted = at; at += align_up(sizeof(int32_t) * n);
  w.wpos = at; at += align_up(sizeof(G) * 4 * n);
  w.offs = at; at += align_up(sizeof(int32_t) * 4 * n);
  w.wpos_s = at; at += align_up(sizeof(G) * 4 * n);
  w.offs_s = at; at += align_up(sizeof(int32_t) * 4 * n);
  w.bin_cnt = at; at += align_up(sizeof(int32_t) * (n_bins + 1));
  w.bin_start = at; at += align_up(sizeof(int32_t) * (n_bins + 1));
  w.counts = at; at += align_up(sizeof(int32_t) * (n + 1));
  w.overflow = at; at += align_up(sizeof(int32_t) * 4);
  w.cursor = at; at += align_up(sizeof(int32_t) * (n_bins + 1));
  size_t sort_bytes = 0, scan_bytes = 0, scan2 = 0;
  (void)hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, (int32_t*)nullptr, (int32_t*)nullptr,
                                     (int32_t*)nullptr, (int32_t*)nullptr, (int)n);
  (void)hipcub::DeviceScan::ExclusiveSum(nullptr, scan_bytes, (int32_t*)nullptr, (int32_t*)nullptr,
                                   (int)(n_bins + 1));
  (void)hipcub::DeviceScan::InclusiveSum(nullptr, scan2, (int32_t*)nullptr, (int32_t*)nullptr,
                                   (int)(n + 1));
  w.cub = at;
  w.cub_bytes = align_up(std::max(sort_bytes, std::max(scan_bytes, scan2)) + 256);
  at += w.cub_bytes;
  w.total = at;
  return w;
}

// The layout for (geometry size, atoms, bins), remembered for the last few shapes: the
// temporary-storage queries of the library sort and scans cost tens of microseconds of host
// time, and the plan, count and fill steps of every build need the same layout.
template <typename G>
static GridWs grid_ws_layout(int64_t n, int64_t n_bins) {
  struct Entry {
    int64_t n = -1, n_bins = -1;
    GridWs w;
  };
  constexpr int kSlots = 8;
  static Entry cache[kSlots];
  static int next = 0;
  static std::mutex mu;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
      if (e.n == n && e.n_bins == n_bins) return e.w;
  }
  const GridWs w = grid_ws_layout_uncached<G>(n, n_bins);
  std::lock_guard<std::mutex> lock(mu);
  cache[next] = Entry{n, n_bins, w};
  next = (next + 1) % kSlots;
  return w;
}

template <typename T>
__device__ __host__ inline T* ws_at(void* ws, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

// ---------------------------------------------------------------- binning
// frac = pos @ inv(cell); wrap offsets o = floor(frac) on periodic axes; wrapped
// position w = pos - o @ cell (geometry dtype, as neighborlist.py:472-475); the bin key from
// the unwrapped fractional coordinate minus the offset (Cartesian without a cell), in
// double times the inverse bin width (the bins' slack absorbs its rounding), clamped to the
// grid.
template <typename G>
__device__ __forceinline__ int wrap_and_bin(const G p[3], const G* __restrict__ cell,
                                            const GridDev& g, G w[3], int o[3]) {
  w[0] = p[0];
  w[1] = p[1];
  w[2] = p[2];
  o[0] = o[1] = o[2] = 0;
  int b[3];
  if (g.has_cell) {
    G f[3];
    for (int a = 0; a < 3; ++a)
      f[a] = p[0] * (G)g.inv[0 * 3 + a] + p[1] * (G)g.inv[1 * 3 + a] + p[2] * (G)g.inv[2 * 3 + a];
    for (int a = 0; a < 3; ++a)
      if (g.periodic[a]) o[a] = (int)floor((double)f[a]);
    if (o[0] | o[1] | o[2]) {
      const G ox = (G)o[0], oy = (G)o[1], oz = (G)o[2];
      for (int a = 0; a < 3; ++a) w[a] = p[a] - (ox * cell[a] + oy * cell[3 + a] + oz * cell[6 + a]);
    }
    for (int a = 0; a < 3; ++a) {
      const double fa = (double)f[a] - (double)o[a];
      int k = (int)floor((fa - g.lo[a]) * g.iwidth[a]);
      b[a] = min(max(k, 0), g.nb[a] - 1);
    }
  } else {
    for (int a = 0; a < 3; ++a) {
      int k = (int)floor(((double)p[a] - g.lo[a]) * g.iwidth[a]);
      b[a] = min(max(k, 0), g.nb[a] - 1);
    }
  }
  return (b[2] * g.nb[1] + b[1]) * g.nb[0] + b[0];
}

template <typename G>
__global__ void bin_atoms_kernel(const G* __restrict__ pos, int64_t n, const G* __restrict__ cell,
                                 GridDev g, int32_t* __restrict__ bin_key,
                                 int32_t* __restrict__ atom_id, G* __restrict__ wpos,
                                 int32_t* __restrict__ offs, int32_t* __restrict__ bin_count,
                                 int32_t* __restrict__ nonfinite) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const G p[3] = {pos[3 * i], pos[3 * i + 1], pos[3 * i + 2]};
  // a non-finite coordinate is flagged for the host (xnn_radius_graph_status); the atom is
  // binned like any other (the bin index is clamped), and finds no neighbor
  if (!(isfinite(p[0]) && isfinite(p[1]) && isfinite(p[2]))) *nonfinite = 1;
  G w[3];
  int o[3];
  const int key = wrap_and_bin(p, cell, g, w, o);
  bin_key[i] = key;
  atom_id[i] = (int32_t)i;
  wpos[4 * i + 0] = w[0];
  wpos[4 * i + 1] = w[1];
  wpos[4 * i + 2] = w[2];
  wpos[4 * i + 3] = G(0);
  offs[4 * i + 0] = o[0];
  offs[4 * i + 1] = o[1];
  offs[4 * i + 2] = o[2];
  offs[4 * i + 3] = key;
  atomicAdd(&bin_count[key], 1);
}

// one row of 4 (16- or 32-byte aligned) in 16-byte stores
__device__ __forceinline__ void store_row4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
__device__ __forceinline__ void store_row4(double* p, double a, double b, double c, double d) {
  reinterpret_cast<double2*>(p)[0] = make_double2(a, b);
  reinterpret_cast<double2*>(p)[1] = make_double2(c, d);
}

// positions of atoms (c + k) * THREADS + t, k < CHUNK, loaded together (indices past the
// last atom clamped to it, n >= 1), so that their round trips overlap
template <typename G, int CHUNK, int THREADS>
__device__ __forceinline__ void load_chunk(const G* __restrict__ pos, int n, int c, int t,
                                           G (&p)[CHUNK][3]) {
#pragma unroll
  for (int k = 0; k < CHUNK; ++k) {
    const int i = min((c + k) * THREADS + t, n - 1);
    p[k][0] = pos[3 * i];
    p[k][1] = pos[3 * i + 1];
    p[k][2] = pos[3 * i + 2];
  }
}

// Sizes the count step bins in one workgroup: the bins' counts and starts and the atoms'
// bin lists held in LDS, 4 (bins + 1) + 4 atoms bytes <= 96 KiB.
constexpr int kOneBlockAtoms = 16384, kOneBlockBins = 8191;

// The count step's whole binning in one workgroup of 1024 threads, for up to kOneBlockAtoms
// atoms and kOneBlockBins bins (one launch where the general path takes five): the count
// step's zeroes; every atom's wrap and bin, counted into its bin by an LDS atomic whose old
// value is the atom's arrival in the bin; the bins' starts (exclusive scan in LDS); the bins'
// atoms listed in arrival order; then, per list position, the atom's rank among its bin's
// atoms of lower index (the order a stable sort by bin gives) and its sorted copies written
// at its bin's start plus that rank. The wrap is computed again for the copies rather than
// kept; positions are loaded 8 (float64: 4) atoms at a time so that their round trips
// overlap.
template <typename G>
__global__ __launch_bounds__(1024) void bin_one_block_kernel(
    const G* __restrict__ pos, int n, const G* __restrict__ cell, GridDev g, int nb,
    int32_t* __restrict__ bin_start, int32_t* __restrict__ atom_sorted, G* __restrict__ wpos_s,
    int32_t* __restrict__ offs_s, int32_t* __restrict__ counts, int32_t* __restrict__ overflow,
    int32_t* __restrict__ row_ptr) {
  constexpr int kThreads = 1024, kPer = kOneBlockAtoms / kThreads;
  constexpr int kScanPer = (kOneBlockBins + 1) / kThreads;
  constexpr int kIdBits = 14, kIdMask = (1 << kIdBits) - 1;  // atoms < 2^14, bins < 2^13
  static_assert(kOneBlockAtoms <= (1 << kIdBits) && kOneBlockBins < (1 << (31 - kIdBits)), "packed list entries");
  // atoms per thread whose positions are loaded together
  constexpr int kChunk = sizeof(G) == 4 ? 8 : 4;
  __shared__ int32_t s_start[kOneBlockBins + 1];
  __shared__ int32_t s_list[kOneBlockAtoms];
  __shared__ int32_t s_wsum[kThreads / kWave];
  __shared__ int32_t s_bad;
  const int t = threadIdx.x, lane = t % kWave, wv = t / kWave;
  for (int b = t; b <= nb; b += kThreads) s_start[b] = 0;
  for (int i = t; i <= n; i += kThreads) counts[i] = 0;
  if (t == 0) {
    s_bad = 0;
    row_ptr[0] = 0;
  }
  __syncthreads();
  // key -1: no atom (past the last one, or in a chunk the loop skips)
  int key[kPer], arrival[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    key[k] = -1;
    arrival[k] = 0;
  }
  bool bad = false;
#pragma unroll
  for (int c = 0; c < kPer; c += kChunk) {
    if (c * kThreads >= n) break;
    G p[kChunk][3];
    load_chunk<G, kChunk, kThreads>(pos, n, c, t, p);
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      const int i = (c + k) * kThreads + t;
      if (i < n) {
        bad = bad || !(isfinite(p[k][0]) && isfinite(p[k][1]) && isfinite(p[k][2]));
        G w[3];
        int o[3];
        key[c + k] = wrap_and_bin(p[k], cell, g, w, o);
        arrival[c + k] = atomicAdd(&s_start[key[c + k]], 1);
      }
    }
  }
  if (bad) s_bad = 1;
  __syncthreads();
  // exclusive scan of the nb + 1 counts (the last one zero): thread t sums a run of
  // kScanPer, the runs are scanned by wave shuffles and one wave over the wave totals
  int32_t v[kScanPer];
  int32_t sum = 0;
#pragma unroll
  for (int k = 0; k < kScanPer; ++k) {
    const int b = t * kScanPer + k;
    v[k] = b <= nb ? s_start[b] : 0;
    sum += v[k];
  }
  int32_t x = sum;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int32_t y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  if (lane == kWave - 1) s_wsum[wv] = x;
  __syncthreads();
  if (wv == 0) {
    int32_t w = lane < kThreads / kWave ? s_wsum[lane] : 0;
#pragma unroll
    for (int o = 1; o < kThreads / kWave; o <<= 1) {
      const int32_t y = __shfl_up(w, o, kWave);
      if (lane >= o) w += y;
    }
    if (lane < kThreads / kWave) s_wsum[lane] = w;
  }
  __syncthreads();
  int32_t run = (wv > 0 ? s_wsum[wv - 1] : 0) + x - sum;
#pragma unroll
  for (int k = 0; k < kScanPer; ++k) {
    const int b = t * kScanPer + k;
    if (b <= nb) {
      s_start[b] = run;
      bin_start[b] = run;
    }
    run += v[k];
  }
  __syncthreads();
  // the bins' lists in arrival order, each entry (bin key << kIdBits) | atom
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    if (key[k] >= 0) s_list[s_start[key[k]] + arrival[k]] = (key[k] << kIdBits) | (k * kThreads + t);
  __syncthreads();
  // position q of the lists: its atom's rank among the bin's atoms of lower index (the
  // entries of one bin compare as their atoms do); the lanes of a wave take consecutive
  // positions, a few bins' worth, so that their reads of a bin's list are LDS broadcasts
#pragma unroll
  for (int c = 0; c < kPer; c += kChunk) {
    if (c * kThreads >= n) break;
    int ent[kChunk];
    G p[kChunk][3];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      ent[k] = s_list[min((c + k) * kThreads + t, n - 1)];
      const int i = ent[k] & kIdMask;
      p[k][0] = pos[3 * i];
      p[k][1] = pos[3 * i + 1];
      p[k][2] = pos[3 * i + 2];
    }
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      if ((c + k) * kThreads + t >= n) continue;
      const int b = ent[k] >> kIdBits, i = ent[k] & kIdMask;
      const int b0 = s_start[b], cnt = s_start[b + 1] - b0;
      int rank = 0;
#pragma unroll 4
      for (int j = 0; j < cnt; ++j) rank += s_list[b0 + j] < ent[k] ? 1 : 0;
      const int at = b0 + rank;
      G w[3];
      int o[3];
      (void)wrap_and_bin(p[k], cell, g, w, o);
      atom_sorted[at] = i;
      store_row4(wpos_s + 4 * (int64_t)at, w[0], w[1], w[2], G(0));
      *reinterpret_cast<int4*>(offs_s + 4 * (int64_t)at) = make_int4(o[0], o[1], o[2], b);
    }
  }
  if (t < 4) overflow[t] = t == 3 ? s_bad : 0;
}

// ---------------------------------------------------------------- search
// One block per receiver bin. Neighbor slots enumerate (dz, dy, dx) in
// [-reach, reach]; slot s has bin index nbin[s] (or -1) and image shift S[s].
template <typename G, bool FILL>
__global__ __launch_bounds__(256) void cell_search_kernel(
    const G* __restrict__ wpos, const int32_t* __restrict__ offs,
    const int32_t* __restrict__ atom_sorted, const int32_t* __restrict__ bin_start,
    const G* __restrict__ cell, GridDev g, G cutoff, int self_interaction,
    int32_t* __restrict__ counts, const int32_t* __restrict__ row_ptr, int32_t* __restrict__ src,
    int32_t* __restrict__ dst, int32_t* __restrict__ shift_out, int64_t* __restrict__ ei64,
    int64_t* __restrict__ sh64, int64_t n_edges, int32_t* __restrict__ overflow,
    const int32_t* __restrict__ e_total, int32_t* __restrict__ status,
    const int32_t* __restrict__ nonfinite) {
  constexpr int kMaxSlots = 343;  // reach <= 3 per axis
  __shared__ int s_bin[kMaxSlots];
  __shared__ int s_img[kMaxSlots][3];
  __shared__ G s_vec[kMaxSlots][3];
  __shared__ int s_first[kMaxSlots + 1];
  __shared__ G t_pos[kTile][3];
  __shared__ int t_atom[kTile];
  __shared__ int t_slot[kTile];

  const int bin = blockIdx.x;
  // the fill's status for the host: the number of edges and the non-finite flag
  if (FILL && status != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    status[0] = e_total != nullptr ? *e_total : (int32_t)n_edges;
    status[1] = *nonfinite;
  }
  const int bx = bin % g.nb[0], by = (bin / g.nb[0]) % g.nb[1], bz = bin / (g.nb[0] * g.nb[1]);
  const int r0 = bin_start[bin], r1 = bin_start[bin + 1];
  // the bin's receivers are dealt to gridDim.y blocks, a wave's worth at a time
  const int split_stride = (int)gridDim.y * (int)(blockDim.x / kWave);
  const int split_first = (int)blockIdx.y * (int)(blockDim.x / kWave);
  if (r1 - r0 <= split_first) return;  // uniform: no receivers for this block
  const int wx = 2 * g.reach[0] + 1, wy = 2 * g.reach[1] + 1, wz = 2 * g.reach[2] + 1;
  const int n_slots = wx * wy * wz;

  // neighbor slots and their image shifts
  for (int s = threadIdx.x; s < n_slots; s += blockDim.x) {
    const int d[3] = {s % wx - g.reach[0], (s / wx) % wy - g.reach[1], s / (wx * wy) - g.reach[2]};
    const int c[3] = {bx, by, bz};
    int idx[3], img[3];
    bool ok = true;
    for (int a = 0; a < 3; ++a) {
      const int t = c[a] + d[a];
      if (g.periodic[a]) {
        const int q = (int)floor((double)t / (double)g.nb[a]);
        img[a] = q;
        idx[a] = t - q * g.nb[a];
      } else {
        img[a] = 0;
        idx[a] = t;
        ok = ok && t >= 0 && t < g.nb[a];
      }
    }
    s_bin[s] = ok ? (idx[2] * g.nb[1] + idx[1]) * g.nb[0] + idx[0] : -1;
    // the slot's candidate count (its bin's atoms), loaded by all threads at once
    s_first[s + 1] = ok ? bin_start[s_bin[s] + 1] - bin_start[s_bin[s]] : 0;
    s_img[s][0] = img[0];
    s_img[s][1] = img[1];
    s_img[s][2] = img[2];
    // image offset S @ cell in the geometry dtype (neighborlist.py:481-483)
    if (cell != nullptr) {
      const G fx = (G)img[0], fy = (G)img[1], fz = (G)img[2];
      for (int a = 0; a < 3; ++a) s_vec[s][a] = fx * cell[a] + fy * cell[3 + a] + fz * cell[6 + a];
    } else {
      s_vec[s][0] = s_vec[s][1] = s_vec[s][2] = G(0);
    }
  }
  __syncthreads();
  // s_first = exclusive prefix sums of the slot counts (held in s_first[1..n_slots]): the
  // first wave scans them, each lane a run of consecutive slots
  if (threadIdx.x < kWave) {
    const int lane0 = threadIdx.x;
    const int per = (n_slots + kWave - 1) / kWave;
    const int a0 = min(n_slots, lane0 * per), a1 = min(n_slots, a0 + per);
    int sum = 0;
    for (int q = a0; q < a1; ++q) sum += s_first[q + 1];
    int x = sum;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int y = __shfl_up(x, o, kWave);
      if (lane0 >= o) x += y;
    }
    int run = x - sum;
    for (int q = a0; q < a1; ++q) {
      const int c = s_first[q + 1];
      s_first[q + 1] = run + c;
      run += c;
    }
    if (lane0 == 0) s_first[0] = 0;
  }
  __syncthreads();
  const int n_cand = s_first[n_slots];

  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int n_recv = r1 - r0;
  // the number of edges: given, or (capacity mode, e_total) the count pass's total on the
  // device, written only when it fits the n_edges entries the outputs hold
  const int64_t n_out = (FILL && e_total != nullptr) ? (int64_t)*e_total : n_edges;
  const bool fits = n_out <= n_edges;

  for (int c0 = 0; c0 < n_cand; c0 += kTile) {
    const int c1 = min(n_cand, c0 + kTile);
    // stage candidates [c0, c1) in LDS, in slot order then bin order
    for (int c = c0 + threadIdx.x; c < c1; c += blockDim.x) {
      int lo = 0, hi = n_slots - 1;  // slot with s_first[slot] <= c < s_first[slot+1]
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_first[mid] <= c) lo = mid; else hi = mid - 1;
      }
      const int s = lo;
      const int p = bin_start[s_bin[s]] + (c - s_first[s]);
      t_pos[c - c0][0] = wpos[4 * p + 0];
      t_pos[c - c0][1] = wpos[4 * p + 1];
      t_pos[c - c0][2] = wpos[4 * p + 2];
      t_atom[c - c0] = atom_sorted[p];
      t_slot[c - c0] = s;
    }
    __syncthreads();
    for (int r = split_first + wave; r < n_recv; r += split_stride) {
      const int pr = r0 + r;
      const int i = atom_sorted[pr];
      const G xi = wpos[4 * pr + 0], yi = wpos[4 * pr + 1], zi = wpos[4 * pr + 2];
      // edges of receiver i found in earlier tiles (a receiver stays with its wave): the
      // count pass adds them up from zero; the fill counts the count pass's totals down,
      // so it needs no zeroing and leaves them in place when its outputs have no room
      const int rem = counts[i];
      const int base = FILL ? (row_ptr[i + 1] - row_ptr[i]) - rem : rem;
      int local = 0;
      for (int c = 0; c < c1 - c0; c += kWave) {
        const int t = c + lane;
        bool hit = false;
        int j = -1, s = 0;
        if (t < c1 - c0) {
          j = t_atom[t];
          s = t_slot[t];
          // (pos_j - pos_i) + S @ cell in the geometry dtype; the squares summed in
          // double (exact products: contraction cannot change them), the root
          // rounded back to the geometry dtype before the strict comparison
          const G dx = (t_pos[t][0] - xi) + s_vec[s][0];
          const G dy = (t_pos[t][1] - yi) + s_vec[s][1];
          const G dz = (t_pos[t][2] - zi) + s_vec[s][2];
          const double d2 = (double)dx * (double)dx + (double)dy * (double)dy +
                            (double)dz * (double)dz;
          hit = (G)sqrt(d2) < cutoff;
          if (!self_interaction && j == i && s_img[s][0] == 0 && s_img[s][1] == 0 &&
              s_img[s][2] == 0)
            hit = false;
        }
        const unsigned long long mask = __ballot(hit);
        if (FILL && hit) {
          const int rank = __popcll(mask & ((1ull << lane) - 1ull));
          const int64_t e = (int64_t)row_ptr[i] + base + local + rank;
          if (fits && e < n_out) {
            const int oi0 = offs[4 * pr + 0], oi1 = offs[4 * pr + 1], oi2 = offs[4 * pr + 2];
            // sender offsets live with the sorted copy; find j's through its own slot
            const int pj = bin_start[s_bin[s]] + (t + c0 - s_first[s]);
            const int sx = -s_img[s][0] + offs[4 * pj + 0] - oi0;
            const int sy = -s_img[s][1] + offs[4 * pj + 1] - oi1;
            const int sz = -s_img[s][2] + offs[4 * pj + 2] - oi2;
            if (sx < -512 || sx > 511 || sy < -512 || sy > 511 || sz < -512 || sz > 511)
              atomicOr(overflow, 1);
            if (src) {
              src[e] = j;
              dst[e] = i;
              shift_out[e] = pack_shift(sx, sy, sz);
            }
            if (ei64) {
              ei64[e] = j;
              ei64[n_out + e] = i;
            }
            if (sh64) {
              sh64[3 * e + 0] = sx;
              sh64[3 * e + 1] = sy;
              sh64[3 * e + 2] = sz;
            }
          }
        }
        local += __popcll(mask);
      }
      if (lane == 0) counts[i] = FILL ? (fits ? rem - local : rem) : base + local;
    }
    __syncthreads();
  }
}

__global__ void zero_i32_kernel(int32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// ---------------------------------------------------------------- nearest edges
// max_neighbors (dataset.py:112-120, nearest_edges neighborlist.py:509-552): per receiver,
// keep the k edges of smallest length, ties to the earlier edge; the kept edges come out
// grouped by receiver and ordered by (length, edge index) within each, the order of the
// reference's two stable sorts.
__global__ void nearest_count_kernel(const int32_t* __restrict__ ptr, int64_t n_nodes, int32_t k,
                                     int32_t* __restrict__ kept_ptr) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_nodes) return;
  kept_ptr[i + 1] = min(ptr[i + 1] - ptr[i], k);
}

// (length, edge) of f before that of e in the order of a stable ascending sort: NaN lengths
// after every number (as torch.sort places them), ties and NaNs by edge index
template <typename T>
__device__ __forceinline__ bool sorts_before(T df, int32_t f, T d, int32_t e) {
  const bool nf = df != df, nd = d != d;
  if (nf != nd) return nd;
  return (!nf && df < d) || ((nf || df == d) && f < e);
}

// one wave per receiver: the rank of every edge of the row among the row's edges (every
// rank below the row's length exactly once, NaN lengths included)
template <typename T>
__global__ __launch_bounds__(256) void nearest_fill_kernel(
    const T* __restrict__ dist, const int32_t* __restrict__ ptr, const int32_t* __restrict__ perm,
    int64_t n_nodes, int32_t k, const int32_t* __restrict__ kept_ptr, int64_t* __restrict__ keep) {
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  if (row >= n_nodes) return;
  const int lane = threadIdx.x % 64;
  const int32_t q0 = ptr[row], q1 = ptr[row + 1];
  for (int32_t q = q0 + lane; q < q1; q += 64) {
    const int32_t e = perm ? perm[q] : q;
    const T d = dist[e];
    int32_t rank = 0;
    for (int32_t r = q0; r < q1; ++r) {
      const int32_t f = perm ? perm[r] : r;
      const T df = dist[f];
      rank += sorts_before(df, f, d, e) ? 1 : 0;
    }
    if (rank < k) keep[kept_ptr[row] + rank] = e;
  }
}

__global__ void set_first_zero_kernel(int32_t* p) { p[0] = 0; }

// the edge count row_ptr[n] and the non-finite flag the count step left, side by side
__global__ void grid_status_kernel(const int32_t* __restrict__ row_ptr, int64_t n,
                                   const int32_t* __restrict__ nonfinite,
                                   int32_t* __restrict__ status) {
  status[0] = row_ptr[n];
  status[1] = *nonfinite;
}

// zeroes of the fill step: per-atom counts (nc) and the overflow flag
__global__ void zero_fill_state_kernel(int32_t* __restrict__ counts, int64_t nc,
                                       int32_t* __restrict__ overflow) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < nc) counts[i] = 0;
  if (i == 0) overflow[0] = 0;
}

// One block's scan of m <= kBlockScanMax ints (in and out distinct): out[i] = the sum of
// in[0..i) (exclusive) or in[0..i] (inclusive). Tiles of 8192 values are loaded coalesced
// into LDS (padded: value i at i + i / 32, so that a thread's 8 consecutive values sit in
// distinct banks across the wave), each thread sums its 8, the 1024 sums are scanned by
// wave shuffles and one wave over the 16 wave totals, and the prefix sums go back through
// LDS to coalesced stores; a carry runs across tiles.
template <bool INCLUSIVE>
__global__ __launch_bounds__(1024) void block_scan_kernel(const int32_t* __restrict__ in,
                                                          int32_t* __restrict__ out, int64_t m) {
  constexpr int kPer = 8, kTileN = 1024 * kPer;
  __shared__ int32_t tile[kTileN + kTileN / 32];
  __shared__ int32_t wsum[16];
  const int t = threadIdx.x, lane = t & (kWave - 1), wv = t / kWave;
  int32_t carry = 0;
  for (int64_t base = 0; base < m; base += kTileN) {
    const int cnt = (int)min<int64_t>(kTileN, m - base);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = k * 1024 + t;
      tile[i + (i >> 5)] = i < cnt ? in[base + i] : 0;
    }
    __syncthreads();
    int32_t v[kPer];
    int32_t sum = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = t * kPer + k;
      v[k] = tile[i + (i >> 5)];
      sum += v[k];
    }
    int32_t x = sum;  // inclusive scan of the thread sums within the wave
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int32_t y = __shfl_up(x, o, kWave);
      if (lane >= o) x += y;
    }
    if (lane == kWave - 1) wsum[wv] = x;
    __syncthreads();
    if (wv == 0) {
      int32_t w = lane < 16 ? wsum[lane] : 0;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const int32_t y = __shfl_up(w, o, kWave);
        if (lane >= o) w += y;
      }
      if (lane < 16) wsum[lane] = w;
    }
    __syncthreads();
    int32_t run = carry + (wv > 0 ? wsum[wv - 1] : 0) + x - sum;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = t * kPer + k;
      if (INCLUSIVE) run += v[k];
      tile[i + (i >> 5)] = run;
      if (!INCLUSIVE) run += v[k];
    }
    carry += wsum[15];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = k * 1024 + t;
      if (i < cnt) out[base + i] = tile[i + (i >> 5)];
    }
    __syncthreads();
  }
}

// counting sort, step 1: every atom into its bin's range (bin_start from the exclusive scan
// of the bin counts), in arbitrary order within the bin
__global__ void bin_scatter_kernel(const int32_t* __restrict__ bin_key, int64_t n,
                                   const int32_t* __restrict__ bin_start,
                                   int32_t* __restrict__ cursor, int32_t* __restrict__ unsorted) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int key = bin_key[i];
  unsorted[bin_start[key] + atomicAdd(&cursor[key], 1)] = (int32_t)i;
}

// counting sort, step 2: one wave per bin puts its atoms in index order (each atom's rank
// among the bin's atoms: the order a stable sort by bin gives) and gathers their wrapped
// positions and image offsets into the sorted copies
template <typename G>
__global__ __launch_bounds__(256) void bin_sort_gather_kernel(
    int64_t n_bins, const int32_t* __restrict__ bin_start, const int32_t* __restrict__ unsorted,
    int32_t* __restrict__ atom_sorted, const G* __restrict__ wpos, const int32_t* __restrict__ offs,
    G* __restrict__ wpos_s, int32_t* __restrict__ offs_s) {
  const int64_t bin = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  if (bin >= n_bins) return;
  const int lane = threadIdx.x % kWave;
  const int r0 = bin_start[bin], cnt = bin_start[bin + 1] - r0;
  for (int t = lane; t < cnt; t += kWave) {
    const int32_t id = unsorted[r0 + t];
    int rank = 0;
    for (int j = 0; j < cnt; ++j) rank += unsorted[r0 + j] < id ? 1 : 0;
    const int at = r0 + rank;
    atom_sorted[at] = id;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      wpos_s[4 * (int64_t)at + c] = wpos[4 * (int64_t)id + c];
      offs_s[4 * (int64_t)at + c] = offs[4 * (int64_t)id + c];
    }
  }
}

// zeroes of the count step: bin counts (nb), per-atom counts (nc), 4 overflow flags and
// row_ptr[0] (the inclusive scan writes row_ptr[1..n])
__global__ void zero_count_state_kernel(int32_t* __restrict__ bin_cnt, int64_t nb,
                                        int32_t* __restrict__ counts, int64_t nc,
                                        int32_t* __restrict__ overflow,
                                        int32_t* __restrict__ row_ptr,
                                        int32_t* __restrict__ cursor) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < nb) {
    bin_cnt[i] = 0;
    cursor[i] = 0;
  }
  if (i < nc) counts[i] = 0;
  if (i < 4) overflow[i] = 0;
  if (i == 0) row_ptr[0] = 0;
}

// ---------------------------------------------------------------- molecules
template <typename G, bool FILL>
__global__ __launch_bounds__(256) void molecule_search_kernel(
    const G* __restrict__ pos, int64_t n, const int64_t* __restrict__ node_ptr,
    const int32_t* __restrict__ batch, G cutoff, int self_interaction,
    int32_t* __restrict__ counts, const int32_t* __restrict__ row_ptr, int32_t* __restrict__ src,
    int32_t* __restrict__ dst, int32_t* __restrict__ shift_out, int64_t* __restrict__ ei64,
    int64_t* __restrict__ sh64, int64_t n_edges) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int b = batch[i];
  const int64_t j0 = node_ptr[b], j1 = node_ptr[b + 1];
  const G xi = pos[3 * i], yi = pos[3 * i + 1], zi = pos[3 * i + 2];
  int64_t k = FILL ? row_ptr[i] : 0;
  int cnt = 0;
  for (int64_t j = j0; j < j1; ++j) {
    const G dx = pos[3 * j] - xi, dy = pos[3 * j + 1] - yi, dz = pos[3 * j + 2] - zi;
    const double d2 = (double)dx * (double)dx + (double)dy * (double)dy + (double)dz * (double)dz;
    if (!((G)sqrt(d2) < cutoff)) continue;
    if (!self_interaction && j == i) continue;
    if (FILL && k < n_edges) {
      src[k] = (int32_t)j;
      dst[k] = (int32_t)i;
      shift_out[k] = 0;
      if (ei64) {
        ei64[k] = j;
        ei64[n_edges + k] = i;
      }
      if (sh64) sh64[3 * k] = sh64[3 * k + 1] = sh64[3 * k + 2] = 0;
    }
    ++k;
    ++cnt;
  }
  if (!FILL) counts[i + 1] = cnt;
}

// ---------------------------------------------------------------- edge plan
__global__ void plan_unpack_kernel(const int64_t* __restrict__ ei, const int64_t* __restrict__ sh,
                                   int64_t E, int64_t n, int32_t* __restrict__ src,
                                   int32_t* __restrict__ dst, int32_t* __restrict__ shift,
                                   int32_t* __restrict__ key_src, int32_t* __restrict__ key_dst,
                                   int32_t* __restrict__ iota, int32_t* __restrict__ cnt_dst,
                                   int32_t* __restrict__ cnt_src, int32_t* __restrict__ overflow) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int64_t s = ei[e], d = ei[E + e];
  if (s < 0 || s >= n || d < 0 || d >= n) {
    atomicOr(overflow, 2);
    src[e] = dst[e] = 0;
    key_src[e] = key_dst[e] = 0;
  } else {
    src[e] = (int32_t)s;
    dst[e] = (int32_t)d;
    key_src[e] = (int32_t)s;
    key_dst[e] = (int32_t)d;
    atomicAdd(&cnt_dst[d + 1], 1);
    atomicAdd(&cnt_src[s + 1], 1);
  }
  iota[e] = (int32_t)e;
  int64_t x = 0, y = 0, z = 0;
  if (sh) {
    x = sh[3 * e];
    y = sh[3 * e + 1];
    z = sh[3 * e + 2];
  }
  if (x < -512 || x > 511 || y < -512 || y > 511 || z < -512 || z > 511) atomicOr(overflow, 1);
  shift[e] = pack_shift((int)x, (int)y, (int)z);
}

struct PlanWs {
  size_t key_src, key_dst, iota, keys_out, cnt, cub, cub_bytes, total;
};

static PlanWs plan_ws_layout(int64_t E, int64_t n) {
  PlanWs w;
  size_t at = 0;
  w.key_src = at; at += align_up(sizeof(int32_t) * E);
  w.key_dst = at; at += align_up(sizeof(int32_t) * E);
  w.iota = at; at += align_up(sizeof(int32_t) * E);
  w.keys_out = at; at += align_up(sizeof(int32_t) * E);
  w.cnt = at; at += align_up(sizeof(int32_t) * 2 * (n + 1));
  size_t sort_bytes = 0, scan_bytes = 0;
  (void)hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, (int32_t*)nullptr, (int32_t*)nullptr,
                                     (int32_t*)nullptr, (int32_t*)nullptr, (int)E);
  (void)hipcub::DeviceScan::InclusiveSum(nullptr, scan_bytes, (int32_t*)nullptr, (int32_t*)nullptr,
                                   (int)(n + 1));
  w.cub = at;
  w.cub_bytes = align_up(std::max(sort_bytes, scan_bytes) + 256);
  at += w.cub_bytes;
  w.total = at;
  return w;
}

static int end_bit_for(int64_t n) {
  int b = 1;
  while ((int64_t(1) << b) < n + 1 && b < 31) ++b;
  return b;
}

// sorted copies of the wrapped positions and offsets (candidates stream from them)
template <typename G>
__global__ void gather_sorted_kernel(const int32_t* __restrict__ atom_sorted, int64_t n,
                                     const G* __restrict__ wpos, const int32_t* __restrict__ offs,
                                     G* __restrict__ wpos_s, int32_t* __restrict__ offs_s) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const int64_t i = atom_sorted[p];
  for (int k = 0; k < 4; ++k) {
    wpos_s[4 * p + k] = wpos[4 * i + k];
    offs_s[4 * p + k] = offs[4 * i + k];
  }
}

// The per-axis bounds the grid plan needs, in one block: lo/hi of the Cartesian coordinates
// (cell == NULL) or of the fractional ones f = pos @ inv(cell) (float64, the inverse from
// the adjugate), any non-finite coordinate making all six NaN; then the cell itself as
// float64 (row-major; zeros without a cell), so that one read gives the host everything.
template <typename G>
__global__ __launch_bounds__(1024) void grid_bounds_kernel(const G* __restrict__ pos, int64_t n,
                                                           const G* __restrict__ cell,
                                                           double* __restrict__ out) {
  double c[9], inv[9];
  const bool frac = cell != nullptr;
#pragma unroll
  for (int k = 0; k < 9; ++k) c[k] = frac ? (double)cell[k] : 0.0;
  if (frac) {
    inv[0] = c[4] * c[8] - c[5] * c[7];
    inv[1] = c[2] * c[7] - c[1] * c[8];
    inv[2] = c[1] * c[5] - c[2] * c[4];
    inv[3] = c[5] * c[6] - c[3] * c[8];
    inv[4] = c[0] * c[8] - c[2] * c[6];
    inv[5] = c[2] * c[3] - c[0] * c[5];
    inv[6] = c[3] * c[7] - c[4] * c[6];
    inv[7] = c[1] * c[6] - c[0] * c[7];
    inv[8] = c[0] * c[4] - c[1] * c[3];
    const double id = 1.0 / (c[0] * inv[0] + c[1] * inv[3] + c[2] * inv[6]);
#pragma unroll
    for (int k = 0; k < 9; ++k) inv[k] *= id;
  }
  double lo[3] = {INFINITY, INFINITY, INFINITY}, hi[3] = {-INFINITY, -INFINITY, -INFINITY};
  bool bad = false;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    double x = (double)pos[3 * i], y = (double)pos[3 * i + 1], z = (double)pos[3 * i + 2];
    if (frac) {
      const double fx = x * inv[0] + y * inv[3] + z * inv[6];
      const double fy = x * inv[1] + y * inv[4] + z * inv[7];
      const double fz = x * inv[2] + y * inv[5] + z * inv[8];
      x = fx;
      y = fy;
      z = fz;
    }
    bad = bad || !isfinite(x) || !isfinite(y) || !isfinite(z);
    lo[0] = fmin(lo[0], x);
    lo[1] = fmin(lo[1], y);
    lo[2] = fmin(lo[2], z);
    hi[0] = fmax(hi[0], x);
    hi[1] = fmax(hi[1], y);
    hi[2] = fmax(hi[2], z);
  }
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      lo[a] = fmin(lo[a], __shfl_xor(lo[a], m, kWave));
      hi[a] = fmax(hi[a], __shfl_xor(hi[a], m, kWave));
    }
  }
  __shared__ double red[1024 / kWave][6];
  __shared__ int any_bad;
  if (threadIdx.x == 0) any_bad = 0;
  __syncthreads();
  if (bad) any_bad = 1;
  if (threadIdx.x % kWave == 0) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      red[threadIdx.x / kWave][a] = lo[a];
      red[threadIdx.x / kWave][3 + a] = hi[a];
    }
  }
  __syncthreads();
  if (threadIdx.x < 6) {
    const int q = threadIdx.x;
    double v = red[0][q];
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w)
      v = q < 3 ? fmin(v, red[w][q]) : fmax(v, red[w][q]);
    out[q] = any_bad ? NAN : v;
  }
  if (threadIdx.x >= kWave && threadIdx.x < kWave + 9) out[6 + threadIdx.x - kWave] = c[threadIdx.x - kWave];
}

static GridDev grid_dev(const xnn_grid_plan* plan) {
  GridDev g;
  for (int a = 0; a < 3; ++a) {
    g.nb[a] = plan->nbins[a];
    g.reach[a] = plan->reach[a];
    g.periodic[a] = plan->periodic[a];
    g.lo[a] = plan->lo[a];
    g.width[a] = plan->width[a];
    g.iwidth[a] = 1.0 / plan->width[a];
  }
  g.has_cell = plan->has_cell;
  for (int k = 0; k < 9; ++k) g.inv[k] = plan->inv_cell[k];
  return g;
}

// count step: bin, sort, search (counting), scan into row_ptr
template <typename G>
static int grid_count(const void* pos_v, int64_t n, const void* cell_v, double cutoff,
                      int self_interaction, const xnn_grid_plan* plan, void* ws,
                      int32_t* row_ptr, hipStream_t stream) {
  const G* pos = (const G*)pos_v;
  const G* cell = (const G*)cell_v;
  const GridDev g = grid_dev(plan);
  const GridWs w = grid_ws_layout<G>(n, plan->n_bins);
  XNN_REQUIRE(w.total <= plan->workspace_bytes, "workspace smaller than the plan's");
  int32_t* bin_key = ws_at<int32_t>(ws, w.bin_key);
  int32_t* bin_key_sorted = ws_at<int32_t>(ws, w.bin_key_sorted);
  int32_t* atom_id = ws_at<int32_t>(ws, w.atom_id);
  int32_t* atom_sorted = ws_at<int32_t>(ws, w.atom_sorted);
  G* wpos = ws_at<G>(ws, w.wpos);
  int32_t* offs = ws_at<int32_t>(ws, w.offs);
  G* wpos_s = ws_at<G>(ws, w.wpos_s);
  int32_t* offs_s = ws_at<int32_t>(ws, w.offs_s);
  int32_t* bin_cnt = ws_at<int32_t>(ws, w.bin_cnt);
  int32_t* bin_start = ws_at<int32_t>(ws, w.bin_start);
  int32_t* counts = ws_at<int32_t>(ws, w.counts);
  int32_t* overflow = ws_at<int32_t>(ws, w.overflow);
  void* cub = ws_at<char>(ws, w.cub);
  size_t cub_bytes = w.cub_bytes;

  const int64_t nb1 = plan->n_bins + 1;
  const bool small = nb1 <= kBlockScanMax && n + 1 <= kBlockScanMax;
  if (n <= kOneBlockAtoms && plan->n_bins <= kOneBlockBins) {
    // the zeroes, the wrap, the bins and the stable sort by bin in one workgroup
    hipLaunchKernelGGL((bin_one_block_kernel<G>), dim3(1), dim3(1024), 0, stream, pos, (int)n,
                       cell, g, (int)plan->n_bins, bin_start, atom_sorted, wpos_s, offs_s, counts,
                       overflow, row_ptr);
    XNN_LAUNCH_CHECK();
  } else {
    // the bin counts, the per-atom counts, the overflow flags and row_ptr[0] in one launch
    int32_t* cursor = ws_at<int32_t>(ws, w.cursor);
    hipLaunchKernelGGL(zero_count_state_kernel, dim3(grid_1d(std::max(nb1, n + 1), 256)),
                       dim3(256), 0, stream, bin_cnt, nb1, counts, n + 1, overflow, row_ptr,
                       cursor);
    hipLaunchKernelGGL((bin_atoms_kernel<G>), dim3(grid_1d(n, 256)), dim3(256), 0, stream, pos,
                       n, cell, g, bin_key, atom_id, wpos, offs, bin_cnt, overflow + 3);
    XNN_LAUNCH_CHECK();
    if (small) {
      // atoms of one bin in ascending index order: a counting sort by bin
      hipLaunchKernelGGL(block_scan_kernel<false>, dim3(1), dim3(1024), 0, stream, bin_cnt,
                         bin_start, nb1);
      hipLaunchKernelGGL(bin_scatter_kernel, dim3(grid_1d(n, 256)), dim3(256), 0, stream,
                         bin_key, n, bin_start, cursor, bin_key_sorted);
      hipLaunchKernelGGL((bin_sort_gather_kernel<G>), dim3(grid_1d(plan->n_bins, 4)), dim3(256),
                         0, stream, plan->n_bins, bin_start, bin_key_sorted, atom_sorted, wpos,
                         offs, wpos_s, offs_s);
      XNN_LAUNCH_CHECK();
    } else {
      XNN_HIP_CHECK(hipcub::DeviceScan::ExclusiveSum(cub, cub_bytes, bin_cnt, bin_start,
                                                     (int)nb1, stream));
      // stable: atoms of one bin keep ascending index order
      XNN_HIP_CHECK(hipcub::DeviceRadixSort::SortPairs(cub, cub_bytes, bin_key, bin_key_sorted,
                                                       atom_id, atom_sorted, (int)n, 0,
                                                       end_bit_for(plan->n_bins), stream));
      hipLaunchKernelGGL((gather_sorted_kernel<G>), dim3(grid_1d(n, 256)), dim3(256), 0, stream,
                         atom_sorted, n, wpos, offs, wpos_s, offs_s);
    }
  }
  hipLaunchKernelGGL((cell_search_kernel<G, false>),
                     dim3(plan->n_bins, search_split(n, plan->n_bins)), dim3(256), 0, stream,
                     wpos_s, offs_s, atom_sorted, bin_start, cell, g, (G)cutoff, self_interaction,
                     counts, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, (int64_t)0,
                     overflow, nullptr, nullptr, nullptr);
  XNN_LAUNCH_CHECK();
  // row_ptr[1..n] = inclusive scan of the per-atom counts; row_ptr[0] = 0
  if (small) {
    hipLaunchKernelGGL(block_scan_kernel<true>, dim3(1), dim3(1024), 0, stream, counts,
                       row_ptr + 1, n);
    XNN_LAUNCH_CHECK();
  } else {
    XNN_HIP_CHECK(hipcub::DeviceScan::InclusiveSum(cub, cub_bytes, counts, row_ptr + 1, (int)n,
                                                   stream));
  }
  return XNN_OK;
}

// fill step: the same search over the binned atoms left in the workspace
template <typename G>
static int grid_fill(const void* pos_v, int64_t n, const void* cell_v, double cutoff,
                     int self_interaction, const xnn_grid_plan* plan, void* ws,
                     const int32_t* row_ptr, int64_t n_edges, int32_t* src, int32_t* dst,
                     int32_t* shift, int64_t* ei64, int64_t* sh64, int32_t* overflow_out,
                     hipStream_t stream, const int32_t* e_total = nullptr,
                     int32_t* status = nullptr) {
  (void)pos_v;
  const G* cell = (const G*)cell_v;
  const GridDev g = grid_dev(plan);
  const GridWs w = grid_ws_layout<G>(n, plan->n_bins);
  XNN_REQUIRE(w.total <= plan->workspace_bytes, "workspace smaller than the plan's");
  int32_t* counts = ws_at<int32_t>(ws, w.counts);
  int32_t* ws_overflow = ws_at<int32_t>(ws, w.overflow);
  int32_t* overflow = overflow_out ? overflow_out : ws_overflow;
  // the workspace's shift-overflow flag was cleared by the count step; a caller's flag is
  // cleared here
  if (overflow_out != nullptr)
    hipLaunchKernelGGL(zero_fill_state_kernel, dim3(1), dim3(64), 0, stream, counts, (int64_t)0,
                       overflow_out);
  hipLaunchKernelGGL((cell_search_kernel<G, true>),
                     dim3(plan->n_bins, search_split(n, plan->n_bins)), dim3(256), 0, stream,
                     ws_at<G>(ws, w.wpos_s), ws_at<int32_t>(ws, w.offs_s),
                     ws_at<int32_t>(ws, w.atom_sorted), ws_at<int32_t>(ws, w.bin_start), cell, g,
                     (G)cutoff, self_interaction, counts, row_ptr, src, dst, shift, ei64, sh64,
                     n_edges, overflow, e_total, status, ws_overflow + 3);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

}  // namespace xnn

using namespace xnn;

extern "C" {

int xnn_radius_graph_plan(int64_t n_nodes, const double* cell, const int32_t* pbc, double cutoff,
                          const double* lo, const double* hi, xnn_grid_plan* plan) {
  XNN_REQUIRE(plan != nullptr && pbc != nullptr, "NULL plan or pbc");
  XNN_REQUIRE(n_nodes >= 0 && n_nodes < (int64_t(1) << 30), "atom count out of range");
  XNN_REQUIRE(cutoff > 0 && isfinite(cutoff), "cutoff must be positive and finite");
  memset(plan, 0, sizeof(*plan));
  const double cut = cutoff * (1.0 + kBinSlack);
  double spacing[3] = {1.0, 1.0, 1.0};
  plan->has_cell = cell != nullptr;
  if (cell != nullptr) {
    const double* m = cell;
    const double det = m[0] * (m[4] * m[8] - m[5] * m[7]) - m[1] * (m[3] * m[8] - m[5] * m[6]) +
                       m[2] * (m[3] * m[7] - m[4] * m[6]);
    XNN_REQUIRE(fabs(det) > 1e-12, "the cell is singular");
    double* v = plan->inv_cell;
    v[0] = (m[4] * m[8] - m[5] * m[7]) / det;
    v[1] = (m[2] * m[7] - m[1] * m[8]) / det;
    v[2] = (m[1] * m[5] - m[2] * m[4]) / det;
    v[3] = (m[5] * m[6] - m[3] * m[8]) / det;
    v[4] = (m[0] * m[8] - m[2] * m[6]) / det;
    v[5] = (m[2] * m[3] - m[0] * m[5]) / det;
    v[6] = (m[3] * m[7] - m[4] * m[6]) / det;
    v[7] = (m[1] * m[6] - m[0] * m[7]) / det;
    v[8] = (m[0] * m[4] - m[1] * m[3]) / det;
    // interplanar spacing along axis a: 1 / |column a of inv(cell)| (neighborlist.py:96-98)
    for (int a = 0; a < 3; ++a) {
      const double c0 = v[a], c1 = v[3 + a], c2 = v[6 + a];
      spacing[a] = 1.0 / sqrt(c0 * c0 + c1 * c1 + c2 * c2);
    }
  }
  int64_t total = 1;
  for (int a = 0; a < 3; ++a) {
    const bool per = plan->has_cell && pbc[a] != 0;
    plan->periodic[a] = per ? 1 : 0;
    double extent;  // coordinate range covered by the grid (fractional or Cartesian)
    if (per) {
      plan->lo[a] = 0.0;
      extent = 1.0;
    } else {
      XNN_REQUIRE(lo != nullptr && hi != nullptr, "non-periodic axes need the coordinate range");
      XNN_REQUIRE(isfinite(lo[a]) && isfinite(hi[a]), "the positions are not finite");
      plan->lo[a] = lo[a];
      extent = hi[a] - lo[a];
    }
    const double length = extent * spacing[a];  // the range as a distance
    double nb = floor(length / cut);
    if (nb < 1) nb = 1;
    if (nb > (double)kMaxBins) nb = (double)kMaxBins;
    plan->nbins[a] = (int)nb;
  }
  // merge bins on the largest axes while the grid is too large
  for (;;) {
    total = (int64_t)plan->nbins[0] * plan->nbins[1] * plan->nbins[2];
    if (total <= kMaxBins) break;
    int a = 0;
    for (int k = 1; k < 3; ++k)
      if (plan->nbins[k] > plan->nbins[a]) a = k;
    plan->nbins[a] = (plan->nbins[a] + 1) / 2;
  }
  for (int a = 0; a < 3; ++a) {
    const double extent = plan->periodic[a] ? 1.0 : (hi[a] - lo[a]);
    double w = extent / plan->nbins[a];
    if (!(w > 0)) w = 1.0;  // a flat axis: one bin of any width
    plan->width[a] = w;
    const double wdist = w * spacing[a];
    int reach = plan->periodic[a] ? (int)ceil(cut / wdist) : 1;
    if (!plan->periodic[a] && plan->nbins[a] == 1) reach = 0;
    plan->reach[a] = reach;
    XNN_REQUIRE(reach <= 3,
                "cutoff %.4g exceeds 3 cell spacings along axis %d (spacing %.4g): "
                "too many periodic images for the cell list",
                cutoff, a, spacing[a]);
  }
  plan->n_bins = total;
  plan->workspace_bytes = grid_ws_layout<double>(n_nodes, total).total;
  return XNN_OK;
}

int xnn_radius_graph_bounds(int geom_dtype, const void* pos, int64_t n_nodes, const void* cell,
                            double* out, xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0, "negative size");
  XNN_REQUIRE(out != nullptr && (n_nodes == 0 || pos != nullptr), "NULL input or output");
  hipStream_t st = as_hip(stream);
  if (geom_dtype == XNN_F32)
    hipLaunchKernelGGL(grid_bounds_kernel<float>, dim3(1), dim3(1024), 0, st, (const float*)pos,
                       n_nodes, (const float*)cell, out);
  else if (geom_dtype == XNN_F64)
    hipLaunchKernelGGL(grid_bounds_kernel<double>, dim3(1), dim3(1024), 0, st,
                       (const double*)pos, n_nodes, (const double*)cell, out);
  else
    XNN_REQUIRE(false, "unsupported geometry dtype %d", geom_dtype);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_radius_graph_count(int geom_dtype, const void* pos, int64_t n_nodes, const void* cell,
                           double cutoff, int32_t self_interaction, const xnn_grid_plan* plan,
                           void* workspace, int32_t* row_ptr, xnn_stream_t stream) {
  XNN_REQUIRE(plan && row_ptr, "NULL plan or row_ptr");
  XNN_REQUIRE(plan->has_cell == 0 || cell != nullptr, "the plan has a cell: pass it");
  if (n_nodes == 0) {
    hipLaunchKernelGGL(set_first_zero_kernel, dim3(1), dim3(1), 0, as_hip(stream), row_ptr);
    XNN_LAUNCH_CHECK();
    return XNN_OK;
  }
  XNN_REQUIRE(pos && workspace, "NULL positions or workspace");
  if (geom_dtype == XNN_F32)
    return grid_count<float>(pos, n_nodes, cell, cutoff, self_interaction, plan, workspace,
                             row_ptr, as_hip(stream));
  if (geom_dtype == XNN_F64)
    return grid_count<double>(pos, n_nodes, cell, cutoff, self_interaction, plan, workspace,
                              row_ptr, as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

int xnn_radius_graph_status(int geom_dtype, int64_t n_nodes, const xnn_grid_plan* plan,
                            const void* workspace, const int32_t* row_ptr, int32_t* status,
                            xnn_stream_t stream) {
  XNN_REQUIRE(plan && row_ptr && status, "NULL plan, row_ptr or status");
  XNN_REQUIRE(n_nodes >= 0, "negative size");
  XNN_REQUIRE(geom_dtype == XNN_F32 || geom_dtype == XNN_F64, "unsupported geometry dtype %d",
              geom_dtype);
  if (n_nodes == 0) {
    hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(64), 0, as_hip(stream), status, (int64_t)2);
    XNN_LAUNCH_CHECK();
    return XNN_OK;
  }
  XNN_REQUIRE(workspace != nullptr, "NULL workspace");
  const GridWs w = geom_dtype == XNN_F32 ? grid_ws_layout<float>(n_nodes, plan->n_bins)
                                         : grid_ws_layout<double>(n_nodes, plan->n_bins);
  XNN_REQUIRE(w.total <= plan->workspace_bytes, "workspace smaller than the plan's");
  const int32_t* overflow = ws_at<const int32_t>(const_cast<void*>(workspace), w.overflow);
  hipLaunchKernelGGL(grid_status_kernel, dim3(1), dim3(1), 0, as_hip(stream), row_ptr, n_nodes,
                     overflow + 3, status);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_radius_graph_fill(int geom_dtype, const void* pos, int64_t n_nodes, const void* cell,
                          double cutoff, int32_t self_interaction, const xnn_grid_plan* plan,
                          void* workspace, const int32_t* row_ptr, int64_t n_edges, int32_t* src,
                          int32_t* dst, int32_t* shift, int64_t* edge_index64, int64_t* shifts64,
                          int32_t* overflow, xnn_stream_t stream) {
  XNN_REQUIRE(plan && row_ptr, "NULL plan or row_ptr");
  if (n_nodes == 0 || n_edges == 0) return XNN_OK;
  XNN_REQUIRE(pos && workspace, "NULL input");
  XNN_REQUIRE((src && dst && shift) || (!src && !dst && !shift && edge_index64 && shifts64),
              "src, dst and shift: all three, or none with both int64 outputs");
  XNN_REQUIRE(plan->has_cell == 0 || cell != nullptr, "the plan has a cell: pass it");
  if (geom_dtype == XNN_F32)
    return grid_fill<float>(pos, n_nodes, cell, cutoff, self_interaction, plan, workspace, row_ptr,
                            n_edges, src, dst, shift, edge_index64, shifts64, overflow,
                            as_hip(stream));
  if (geom_dtype == XNN_F64)
    return grid_fill<double>(pos, n_nodes, cell, cutoff, self_interaction, plan, workspace,
                             row_ptr, n_edges, src, dst, shift, edge_index64, shifts64, overflow,
                             as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

int xnn_radius_graph_fill_capacity(int geom_dtype, const void* pos, int64_t n_nodes,
                                   const void* cell, double cutoff, int32_t self_interaction,
                                   const xnn_grid_plan* plan, void* workspace,
                                   const int32_t* row_ptr, int64_t capacity,
                                   int64_t* edge_index64, int64_t* shifts64, int32_t* status,
                                   xnn_stream_t stream) {
  XNN_REQUIRE(plan && row_ptr, "NULL plan or row_ptr");
  XNN_REQUIRE(capacity >= 0, "negative capacity");
  if (n_nodes == 0) {
    if (status != nullptr) {
      hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(64), 0, as_hip(stream), status,
                         (int64_t)2);
      XNN_LAUNCH_CHECK();
    }
    return XNN_OK;
  }
  XNN_REQUIRE(pos && workspace, "NULL input");
  XNN_REQUIRE(capacity == 0 || (edge_index64 && shifts64), "NULL output");
  XNN_REQUIRE(plan->has_cell == 0 || cell != nullptr, "the plan has a cell: pass it");
  if (geom_dtype == XNN_F32)
    return grid_fill<float>(pos, n_nodes, cell, cutoff, self_interaction, plan, workspace, row_ptr,
                            capacity, nullptr, nullptr, nullptr, edge_index64, shifts64, nullptr,
                            as_hip(stream), row_ptr + n_nodes, status);
  if (geom_dtype == XNN_F64)
    return grid_fill<double>(pos, n_nodes, cell, cutoff, self_interaction, plan, workspace,
                             row_ptr, capacity, nullptr, nullptr, nullptr, edge_index64, shifts64,
                             nullptr, as_hip(stream), row_ptr + n_nodes, status);
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

size_t xnn_scan_workspace_bytes(int64_t n) {
  size_t bytes = 0;
  (void)hipcub::DeviceScan::InclusiveSum(nullptr, bytes, (int32_t*)nullptr, (int32_t*)nullptr,
                                   (int)(n + 1));
  return align_up(bytes + 256) + align_up(sizeof(int32_t) * (n + 1));
}

int xnn_scan_counts(int32_t* row_ptr, int64_t n, void* workspace, xnn_stream_t stream) {
  XNN_REQUIRE(row_ptr != nullptr, "NULL row_ptr");
  hipStream_t s = as_hip(stream);
  if (n > 0) {
    XNN_REQUIRE(workspace != nullptr, "NULL workspace");
    size_t bytes = 0;
    (void)hipcub::DeviceScan::InclusiveSum(nullptr, bytes, (int32_t*)nullptr, (int32_t*)nullptr,
                                     (int)(n + 1));
    size_t cub_bytes = align_up(bytes + 256);
    int32_t* tmp = ws_at<int32_t>(workspace, cub_bytes);
    XNN_HIP_CHECK(hipMemcpyAsync(tmp, row_ptr + 1, sizeof(int32_t) * n, hipMemcpyDeviceToDevice, s));
    XNN_HIP_CHECK(hipcub::DeviceScan::InclusiveSum(workspace, cub_bytes, tmp, row_ptr + 1, (int)n, s));
  }
  hipLaunchKernelGGL(set_first_zero_kernel, dim3(1), dim3(1), 0, s, row_ptr);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_radius_graph_molecules_count(int geom_dtype, const void* pos, int64_t n_nodes,
                                     const int64_t* node_ptr, const int32_t* batch,
                                     int64_t n_graphs, double cutoff, int32_t self_interaction,
                                     int32_t* row_ptr, xnn_stream_t stream) {
  XNN_REQUIRE(row_ptr != nullptr, "NULL row_ptr");
  if (n_nodes == 0) {
    hipLaunchKernelGGL(set_first_zero_kernel, dim3(1), dim3(1), 0, as_hip(stream), row_ptr);
    XNN_LAUNCH_CHECK();
    return XNN_OK;
  }
  XNN_REQUIRE(pos && node_ptr && batch, "NULL input");
  XNN_REQUIRE(cutoff > 0, "cutoff must be positive");
  const dim3 grid(grid_1d(n_nodes, 256)), block(256);
  if (geom_dtype == XNN_F32)
    hipLaunchKernelGGL((molecule_search_kernel<float, false>), grid, block, 0, as_hip(stream),
                       (const float*)pos, n_nodes, node_ptr, batch, (float)cutoff,
                       self_interaction, row_ptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                       nullptr, 0);
  else if (geom_dtype == XNN_F64)
    hipLaunchKernelGGL((molecule_search_kernel<double, false>), grid, block, 0, as_hip(stream),
                       (const double*)pos, n_nodes, node_ptr, batch, cutoff, self_interaction,
                       row_ptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0);
  else {
    set_error("unsupported geometry dtype %d", geom_dtype);
    return XNN_EINVAL;
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_radius_graph_molecules_fill(int geom_dtype, const void* pos, int64_t n_nodes,
                                    const int64_t* node_ptr, const int32_t* batch,
                                    int64_t n_graphs, double cutoff, int32_t self_interaction,
                                    const int32_t* row_ptr, int64_t n_edges, int32_t* src,
                                    int32_t* dst, int32_t* shift, int64_t* edge_index64,
                                    int64_t* shifts64, xnn_stream_t stream) {
  if (n_nodes == 0 || n_edges == 0) return XNN_OK;
  XNN_REQUIRE(pos && node_ptr && batch && row_ptr && src && dst && shift, "NULL input");
  const dim3 grid(grid_1d(n_nodes, 256)), block(256);
  if (geom_dtype == XNN_F32)
    hipLaunchKernelGGL((molecule_search_kernel<float, true>), grid, block, 0, as_hip(stream),
                       (const float*)pos, n_nodes, node_ptr, batch, (float)cutoff,
                       self_interaction, nullptr, row_ptr, src, dst, shift, edge_index64,
                       shifts64, n_edges);
  else if (geom_dtype == XNN_F64)
    hipLaunchKernelGGL((molecule_search_kernel<double, true>), grid, block, 0, as_hip(stream),
                       (const double*)pos, n_nodes, node_ptr, batch, cutoff, self_interaction,
                       nullptr, row_ptr, src, dst, shift, edge_index64, shifts64, n_edges);
  else {
    set_error("unsupported geometry dtype %d", geom_dtype);
    return XNN_EINVAL;
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

size_t xnn_edge_plan_workspace_bytes(int64_t n_edges, int64_t n_nodes) {
  return plan_ws_layout(n_edges, n_nodes).total;
}

int xnn_edge_plan(const int64_t* edge_index, const int64_t* cell_shifts, int64_t n_edges,
                  int64_t n_nodes, int32_t* src, int32_t* dst, int32_t* shift, int32_t* ptr_dst,
                  int32_t* perm_dst, int32_t* ptr_src, int32_t* perm_src, int32_t* overflow,
                  void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  XNN_REQUIRE(n_edges >= 0 && n_nodes >= 0, "negative size");
  XNN_REQUIRE(n_edges < (int64_t(1) << 31) && n_nodes < (int64_t(1) << 31),
              "int32 indices: at most 2^31 - 1 edges and atoms");
  XNN_REQUIRE(ptr_dst && ptr_src && overflow, "NULL output");
  const PlanWs w = plan_ws_layout(n_edges, n_nodes);
  XNN_REQUIRE(workspace_bytes >= w.total, "workspace too small: %zu < %zu", workspace_bytes,
              w.total);
  hipStream_t s = as_hip(stream);
  int32_t* key_src = ws_at<int32_t>(workspace, w.key_src);
  int32_t* key_dst = ws_at<int32_t>(workspace, w.key_dst);
  int32_t* iota = ws_at<int32_t>(workspace, w.iota);
  int32_t* keys_out = ws_at<int32_t>(workspace, w.keys_out);
  int32_t* cnt = ws_at<int32_t>(workspace, w.cnt);
  void* cub = ws_at<char>(workspace, w.cub);
  size_t cub_bytes = w.cub_bytes;
  hipLaunchKernelGGL(zero_i32_kernel, dim3(grid_1d(2 * (n_nodes + 1), 256)), dim3(256), 0, s,
                     cnt, 2 * (n_nodes + 1));
  hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(64), 0, s, overflow, (int64_t)1);
  if (n_edges > 0) {
    XNN_REQUIRE(edge_index && src && dst && shift && perm_dst && perm_src, "NULL input");
    hipLaunchKernelGGL(plan_unpack_kernel, dim3(grid_1d(n_edges, 256)), dim3(256), 0, s,
                       edge_index, cell_shifts, n_edges, n_nodes, src, dst, shift, key_src,
                       key_dst, iota, cnt, cnt + (n_nodes + 1), overflow);
    XNN_LAUNCH_CHECK();
    const int eb = end_bit_for(n_nodes);
    XNN_HIP_CHECK(hipcub::DeviceRadixSort::SortPairs(cub, cub_bytes, key_dst, keys_out, iota,
                                                     perm_dst, (int)n_edges, 0, eb, s));
    XNN_HIP_CHECK(hipcub::DeviceRadixSort::SortPairs(cub, cub_bytes, key_src, keys_out, iota,
                                                     perm_src, (int)n_edges, 0, eb, s));
  }
  XNN_HIP_CHECK(hipcub::DeviceScan::InclusiveSum(cub, cub_bytes, cnt, ptr_dst, (int)(n_nodes + 1), s));
  XNN_HIP_CHECK(hipcub::DeviceScan::InclusiveSum(cub, cub_bytes, cnt + (n_nodes + 1), ptr_src,
                                                 (int)(n_nodes + 1), s));
  return XNN_OK;
}


int xnn_nearest_edges_count(const int32_t* ptr_dst, int64_t n_nodes, int32_t k, int32_t* kept_ptr,
                            xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && k >= 0, "negative size");
  XNN_REQUIRE(kept_ptr && (n_nodes == 0 || ptr_dst), "NULL CSR");
  if (n_nodes > 0) {
    hipLaunchKernelGGL(nearest_count_kernel, dim3(grid_1d(n_nodes, 256)), dim3(256), 0,
                       as_hip(stream), ptr_dst, n_nodes, k, kept_ptr);
    XNN_LAUNCH_CHECK();
  }
  return XNN_OK;
}

int xnn_nearest_edges_fill(int dtype, const void* dist, int64_t n_edges, const int32_t* ptr_dst,
                           const int32_t* perm_dst, int64_t n_nodes, int32_t k,
                           const int32_t* kept_ptr, int64_t* keep, xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_edges >= 0 && k >= 0, "negative size");
  XNN_REQUIRE(dtype == XNN_F32 || dtype == XNN_F64, "dtype must be XNN_F32 or XNN_F64");
  if (n_nodes == 0 || n_edges == 0 || k == 0) return XNN_OK;
  XNN_REQUIRE(dist && ptr_dst && kept_ptr && keep, "NULL input or output");
  XNN_REQUIRE(n_edges < (int64_t(1) << 31), "at most 2^31 - 1 edges");
  const dim3 grid((unsigned)grid_1d(n_nodes, 4));
  if (dtype == XNN_F64)
    hipLaunchKernelGGL(nearest_fill_kernel<double>, grid, dim3(256), 0, as_hip(stream),
                       static_cast<const double*>(dist), ptr_dst, perm_dst, n_nodes, k, kept_ptr,
                       keep);
  else
    hipLaunchKernelGGL(nearest_fill_kernel<float>, grid, dim3(256), 0, as_hip(stream),
                       static_cast<const float*>(dist), ptr_dst, perm_dst, n_nodes, k, kept_ptr,
                       keep);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

}  // extern "C"
