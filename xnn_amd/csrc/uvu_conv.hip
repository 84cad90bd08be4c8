// The message step of an equivariant convolution: gather the sender features, take the
// uvu tensor product with the edge harmonics under per-edge weights, and sum onto the
// receivers (gfx950, wave64, fp32). Deterministic: every sum walks a CSR row in order.
//
// xnn_uvu_conv: for the instructions p = (l1, l2, l3) of a tensor product whose paths are
// all uvu, whose second operand has one copy per block and whose outputs are distinct
// (ConvTensorProduct.conv, gnn/fast/conv.py:93-143: gather_rows (common/models/ops.py:494),
// the e3nn TensorProduct, scatter_sum (ops.py:403), the message divisor),
//   out[i, p, u, k] = c_p sum_{e: dst(e) = i} w[row(e), p, u]
//                     sum_{a, b} C^{l1 l2 l3}[a, b, k] h[src(e), in1(p), u, a] Y[e, in2(p), b]
// with C the real Wigner 3j tensor (cg_tables.h) and c_p the path's normalization
// divided by the message divisor; row(e) = weight_index[e] or e.
//
// Work is split by (node, node-feature block): a wave owns one block of the node rows
// (degree l1) for one node, its lanes the channels u; when the block has at most 32
// channels, each half-wave takes every other edge of the node's row and the halves' sums
// are added at the end. Per edge it reads the sender's block and the
// edge's harmonics once and expands every path that reads the block: the paths of a block
// differ only in (l2, l3), whose combinations for a given l1 are few and known at compile
// time, so the code for each l1 (and largest l2) unrolls all of them, keeps their sums in
// registers, expands each product over the nonzero entries of C only, and skips the
// combinations the tensor product does not have. The second operand's blocks must have
// distinct degrees (one block per l2, as the harmonics have).
//
// xnn_uvu_conv_backward, given d out, over the same waves and the receivers' rows (each
// receiver's d out read once):
//   d w[e, p, u] per edge (the caller sums the rows of shared weights);
//   the channel sums of each block's share of d Y[e], kept per block in the workspace and
//   added up by a last pass;
//   each edge's share of d h at its sender, d h_e[block, u, a] =
//     sum_{p reads block} c_p w[row(e), p, u] sum_{b, k} C[a, b, k] Y[e, b] d out[dst(e), p, u, k],
//   in the workspace in node-row layout, summed over each sender's row by a last pass
//   (deterministic; a walk over the senders' rows would gather d out once per edge).
#include <algorithm>
#include <cstdint>

#include "cg_tables.h"
#include "common.h"
#include "device.h"
#include "fork_join.h"

namespace xnn {

constexpr int kConvWaves = 4;
constexpr int kConvMaxPaths = 48;
constexpr int kConvMaxL = 3;
constexpr int kConvMaxDim2 = 16;   // entries of the edge attribute rows
constexpr int kConvMaxBlocks = 16;  // node-feature blocks
constexpr int kConvCombos = 12;     // (l2, l3) combinations of one l1 (at most 11)

// ------------------------------------------------------------------ (l1, l2, l3) tables
struct Triple {
  int a, b, c;
};
#define XNN_TRIPLE_ENTRY(a, b, c) Triple{a, b, c},
constexpr Triple kTriples[] = {XNN_CG_TRIPLES(XNN_TRIPLE_ENTRY)};
#undef XNN_TRIPLE_ENTRY
constexpr int kNumTriples = (int)(sizeof(kTriples) / sizeof(kTriples[0]));

// position of (l2, l3) among the combinations of l1 (table order), or -1
__host__ __device__ constexpr int combo_index(int l1, int l2, int l3) {
  int n = 0;
  for (int t = 0; t < kNumTriples; ++t) {
    if (kTriples[t].a != l1) continue;
    if (kTriples[t].b == l2 && kTriples[t].c == l3) return n;
    ++n;
  }
  return -1;
}

// first register of combination (l2, l3) among the 2 l3 + 1 sums of every combination of l1
__host__ __device__ constexpr int combo_offset(int l1, int l2, int l3) {
  int off = 0;
  for (int t = 0; t < kNumTriples; ++t) {
    if (kTriples[t].a != l1) continue;
    if (kTriples[t].b == l2 && kTriples[t].c == l3) return off;
    off += 2 * kTriples[t].c + 1;
  }
  return -1;
}

__host__ __device__ constexpr int combo_width(int l1) {
  int off = 0;
  for (int t = 0; t < kNumTriples; ++t)
    if (kTriples[t].a == l1) off += 2 * kTriples[t].c + 1;
  return off;
}

// ------------------------------------------------------------------ arguments
struct ConvCombo {
  int32_t off_w;    // < 0: the product has no such path
  int32_t off_out;
  float coef;
};

struct ConvBlock {
  int32_t l1;       // < 0: no path reads the block
  int32_t mul;
  int32_t off1;
  int32_t pad;
  ConvCombo c[kConvCombos];
};

// The scalar fields, copied into registers at kernel entry and handed to the helpers (a
// reference to the by-value kernel argument that escapes into them makes the compiler
// copy all of it to scratch memory).
struct ConvView {
  const float* h;       // (N, d1)
  const float* y;       // (E, d2)
  const float* w;       // (n_w_rows, dw)
  const int32_t* widx;
  const int32_t* src;
  const int32_t* dst;
  const int32_t* ptr;   // CSR of the walk: the receivers
  const int32_t* perm;
  const float* g_out;   // (N, dout) backward
  float* out;           // forward: (N, dout)
  float* g_w;           // (E, dw) per edge
  float* parts;         // (E, n_blocks, d2): per block channel sums of d Y
  float* dh_edge;       // (E, dh_stride): each edge's share of d h at its sender, node-row
                        // layout (summed over the senders' rows afterwards)
  int64_t dh_stride;
  int64_t n_nodes, n_edges, n_w_rows;
  int32_t d1, d2, dw, dout, n_blocks, ls;
  int32_t off2[kConvMaxL + 1];  // column of the edge-attribute block of degree l (< 0: none)
};

struct ConvArgs {
  ConvView v;
  ConvBlock blocks[kConvMaxBlocks];
  int32_t ids[kConvMaxBlocks];  // the blocks of one launch (one degree l1)
  int32_t n_ids;
};

__device__ __forceinline__ int64_t conv_row(const ConvView& V, int64_t e) {
  return V.widx ? (int64_t)V.widx[e] : e;
}

// The lanes of a wave on its node: all 64 over the channels (in chunks of 64), or, for a
// block of at most 32 channels, two halves of 32 over the channels, each half walking every
// other edge of the node's row (twice the independent gathers in flight per wave; the two
// halves' sums are added once per node).
struct ConvLanes {
  int64_t node;      // the wave's node (>= n_nodes: no work)
  int sub;           // lane within its half (split) or the wave
  int width;         // channels per chunk (64 or 32)
  int half;          // split: the half (0 or 1) whose edges are 2 it + half; else 0
  int step;          // edges per trip: 2 (split) or 1
  int32_t q0, len;   // the node's CSR range
  int32_t trips;     // uniform: trips over the row
};

__device__ __forceinline__ ConvLanes conv_lanes(const ConvView& V, int64_t group, bool split,
                                                int lane) {
  ConvLanes L;
  L.width = split ? 32 : kWave;
  L.sub = split ? (lane & 31) : lane;
  L.half = split ? (lane >> 5) : 0;
  L.step = split ? 2 : 1;
  L.node = group;
  L.q0 = 0;
  L.len = 0;
  if (L.node < V.n_nodes) {
    L.q0 = V.ptr[L.node];
    L.len = V.ptr[L.node + 1] - L.q0;
  }
  L.trips = __builtin_amdgcn_readfirstlane((L.len + L.step - 1) / L.step);
  return L;
}

// a split wave's two halves added (every lane gets the node's total); unchanged otherwise
__device__ __forceinline__ float conv_halves_sum(float v, bool split) {
  return split ? add_xor32(v) : v;
}

// sum over the lanes of one node's group (32 or 64 lanes), on every lane of the group: DPP
// steps inside each 16-lane row, then the row-swap permutes (vector ALU, no LDS round trip)
__device__ __forceinline__ float conv_group_sum(float v, bool pair) {
  v = add_xor16(row_sum16(v));
  return pair ? v : add_xor32(v);
}

// the edge's harmonics of degree <= LS into yv[l^2 + m] (zeros where absent); e must be a
// valid edge
template <int LS>
__device__ __forceinline__ void conv_load_y(const ConvView& V, int64_t e, float* yv) {
  const float* yrow = V.y + e * V.d2;
#pragma unroll
  for (int l = 0; l <= LS; ++l) {
    const int o = V.off2[l];
    // an absent degree loads the row's first value (a valid address) and uses zero: every
    // load is issued unconditionally, so the wait counts of the edge loops stay exact
#pragma unroll
    for (int m = 0; m < 2 * l + 1; ++m) {
      const float v = yrow[o >= 0 ? o + m : 0];
      yv[l * l + m] = o >= 0 ? v : 0.f;
    }
  }
}

// the edge of step `it` of a lane's CSR range
struct ConvEdge {
  int64_t e, other, row;
  bool on, row_ok;
};

// The indices of up to 64 edges of a wave's node row, one edge per lane (lane j: the
// chunk's edge j; past the row's end, its last edge), loaded once per chunk: in the edge
// loops an edge's indices come from a lane exchange, so the loops issue no index loads and
// one edge's operand loads stay in flight across the previous edge's arithmetic.
struct ConvChunk {
  int32_t e, other, row;  // this lane's edge of the chunk
  int32_t cnt, trips;     // the chunk's edges and trips over them (uniform)
};

__device__ __forceinline__ ConvChunk conv_chunk(const ConvView& V, const ConvLanes& L,
                                                int32_t base, int lane,
                                                const int32_t* __restrict__ other_of) {
  ConvChunk K;
  K.cnt = min(kWave, L.len - base);
  K.trips = (K.cnt + L.step - 1) / L.step;
  const int32_t q = L.q0 + base + min(lane, K.cnt - 1);
  K.e = V.perm ? V.perm[q] : q;
  K.other = other_of[K.e];
  K.row = V.widx ? V.widx[K.e] : K.e;
  return K;
}

// the edge of trip `it` of chunk K for a lane: position it * step + half of the chunk (a
// position past the chunk gives its last edge, `on` false)
__device__ __forceinline__ ConvEdge conv_edge_at(const ConvView& V, const ConvChunk& K,
                                                 const ConvLanes& L, int32_t it) {
  const int32_t k = it * L.step + L.half;
  const int src_lane = min(k, K.cnt - 1);
  ConvEdge E;
  E.e = __shfl(K.e, src_lane, kWave);
  E.other = __shfl(K.other, src_lane, kWave);
  E.row = __shfl(K.row, src_lane, kWave);
  E.on = k < K.cnt;
  E.row_ok = E.on && E.row >= 0 && E.row < V.n_w_rows;
  return E;
}

// ------------------------------------------------------------------ operand fetch
// One edge's operands for one lane: the sender's block h[src(e), block, u, :], the edge's
// harmonics and the weight of every path of the block. The edge loops keep two of them,
// fetched one trip ahead of the arithmetic in alternation (no copies between them), so the
// gathers of the next edge are in flight while this one is expanded. Every lane loads, from
// a valid address (a lane without an edge reads the chunk's last edge, a channel past the
// block channel 0, a weight row out of range row 0, an absent path the row's first weight),
// and `use` says whether the operands are the lane's: the arithmetic runs under it, and
// with no branch around a load the wait before each use counts exactly the loads after it.
template <int L1, int LS>
struct ConvFetch {
  float hv[2 * L1 + 1];
  float yv[(LS + 1) * (LS + 1)];
  float wv[kConvCombos];
  bool use;
};

template <int L1, int LS>
__device__ __forceinline__ void conv_fetch(const ConvView& V, const ConvBlock& B,
                                           const ConvEdge& E, int u, bool chan, bool want_h,
                                           ConvFetch<L1, LS>& F) {
  constexpr int D1 = 2 * L1 + 1;
  F.use = E.row_ok && chan;
  const int us = chan ? u : 0;
  // row pointers formed once per edge (the per-path loads add uniform offsets)
  if (want_h) {
    const float* hrow = V.h + E.other * V.d1 + B.off1 + us * D1;
#pragma unroll
    for (int a = 0; a < D1; ++a) F.hv[a] = hrow[a];
  }
  conv_load_y<LS>(V, E.e, F.yv);
  const bool have_w = V.n_w_rows > 0;
  // without weight rows any valid address (no lane uses the values: row_ok is false)
  const float* wrow = have_w ? V.w + (E.row_ok ? E.row : 0) * V.dw + us : V.y;
#define XNN_CONV_FETCH_W(P1_, P2_, P3_)                                               \
  if constexpr (P1_ == L1 && P2_ <= LS) {                                             \
    constexpr int ci = combo_index(P1_, P2_, P3_);                                    \
    F.wv[ci] = wrow[(B.c[ci].off_w >= 0 && have_w) ? B.c[ci].off_w : 0];              \
  }
  XNN_CG_TRIPLES(XNN_CONV_FETCH_W)
#undef XNN_CONV_FETCH_W
}

// ------------------------------------------------------------------ forward
template <int L1, int LS>
__device__ __forceinline__ void conv_fwd_block(const ConvView& V, const ConvBlock& B,
                                               const ConvLanes& L) {
  constexpr int NA = combo_width(L1);
  const int lane = threadIdx.x % kWave;
  for (int u0 = 0; u0 < B.mul; u0 += L.width) {
    const int u = u0 + L.sub;
    const bool chan = u < B.mul;
    float acc[NA];
#pragma unroll
    for (int k = 0; k < NA; ++k) acc[k] = 0.f;
    auto edge = [&](const ConvFetch<L1, LS>& C) {
      if (!C.use) return;
      // the products h_a Y_b, shared by every path of the block that reads them
      float hy[(2 * L1 + 1) * (LS + 1) * (LS + 1)];
#pragma unroll
      for (int a = 0; a < 2 * L1 + 1; ++a)
#pragma unroll
        for (int b = 0; b < (LS + 1) * (LS + 1); ++b)
          hy[a * (LS + 1) * (LS + 1) + b] = C.hv[a] * C.yv[b];
#define XNN_CONV_COMBO(P1_, P2_, P3_)                                                     \
  if constexpr (P1_ == L1 && P2_ <= LS) {                                                 \
    constexpr int ci = combo_index(P1_, P2_, P3_), ao = combo_offset(P1_, P2_, P3_);      \
    using T = CGTable<P1_, P2_, P3_>;                                                     \
    if (B.c[ci].off_w >= 0) {                                                             \
      float t[2 * P3_ + 1];                                                               \
      _Pragma("unroll") for (int k = 0; k < 2 * P3_ + 1; ++k) t[k] = -0.f;                \
      _Pragma("unroll") for (int n = 0; n < T::n; ++n)                                    \
          t[T::e[n].k] += T::e[n].c *                                                     \
                          hy[T::e[n].i * (LS + 1) * (LS + 1) + P2_ * P2_ + T::e[n].j];    \
      _Pragma("unroll") for (int k = 0; k < 2 * P3_ + 1; ++k)                             \
          acc[ao + k] += C.wv[ci] * t[k];                                                 \
    }                                                                                     \
  }
      XNN_CG_TRIPLES(XNN_CONV_COMBO)
#undef XNN_CONV_COMBO
    };
    for (int32_t base = 0; base < L.len; base += kWave) {
      const ConvChunk K = conv_chunk(V, L, base, lane, V.src);
      ConvFetch<L1, LS> F0, F1;
      conv_fetch<L1, LS>(V, B, conv_edge_at(V, K, L, 0), u, chan, true, F0);
      conv_fetch<L1, LS>(V, B, conv_edge_at(V, K, L, 1), u, chan, true, F1);
      for (int32_t it = 0; it < K.trips; it += 2) {
        edge(F0);
        conv_fetch<L1, LS>(V, B, conv_edge_at(V, K, L, it + 2), u, chan, true, F0);
        if (it + 1 < K.trips) edge(F1);
        conv_fetch<L1, LS>(V, B, conv_edge_at(V, K, L, it + 3), u, chan, true, F1);
      }
    }
#pragma unroll
    for (int k = 0; k < NA; ++k) acc[k] = conv_halves_sum(acc[k], L.step == 2);
    if (chan && L.half == 0 && L.node < V.n_nodes) {
      float* o = V.out + L.node * V.dout;
#define XNN_CONV_STORE(P1_, P2_, P3_)                                                     \
  if constexpr (P1_ == L1 && P2_ <= LS) {                                                 \
    constexpr int ci = combo_index(P1_, P2_, P3_), ao = combo_offset(P1_, P2_, P3_);      \
    if (B.c[ci].off_w >= 0) {                                                             \
      _Pragma("unroll") for (int k = 0; k < 2 * P3_ + 1; ++k)                             \
          o[B.c[ci].off_out + u * (2 * P3_ + 1) + k] = B.c[ci].coef * acc[ao + k];        \
    }                                                                                     \
  }
      XNN_CG_TRIPLES(XNN_CONV_STORE)
#undef XNN_CONV_STORE
    }
  }
}

// ------------------------------------------------------------------ backward, edge part
// With DH, also each edge's share of d h at its sender,
//   d h_e[u, a] = sum_p c_p w[e, p, u] sum_{b, k} C[a, b, k] Y[e, b] d out[dst(e), p, u, k],
// from the receiver's output gradient already in registers (the receiver walk reads it once
// per node, where a walk over the senders' rows would gather it once per edge).
template <int L1, int LS, bool DH>
__device__ __forceinline__ void conv_bwd_edge_block(const ConvView& V, const ConvBlock& B,
                                                    const ConvLanes& L, bool pair, int blk) {
  constexpr int NA = combo_width(L1), NY = (LS + 1) * (LS + 1), D1 = 2 * L1 + 1;
  const int lane = threadIdx.x % kWave;
  for (int u0 = 0; u0 < B.mul; u0 += L.width) {
    const int u = u0 + L.sub;
    const bool chan = u < B.mul && L.node < V.n_nodes;
    // the receiver's output gradient of every path of the block, once per node
    float gk[NA];
#pragma unroll
    for (int k = 0; k < NA; ++k) gk[k] = 0.f;
    if (chan) {
      const float* g = V.g_out + L.node * V.dout;
#define XNN_CONV_LOADG(P1_, P2_, P3_)                                                     \
  if constexpr (P1_ == L1 && P2_ <= LS) {                                                 \
    constexpr int ci = combo_index(P1_, P2_, P3_), ao = combo_offset(P1_, P2_, P3_);      \
    if (B.c[ci].off_w >= 0) {                                                             \
      _Pragma("unroll") for (int k = 0; k < 2 * P3_ + 1; ++k)                             \
          gk[ao + k] = g[B.c[ci].off_out + u * (2 * P3_ + 1) + k];                        \
    }                                                                                     \
  }
      XNN_CG_TRIPLES(XNN_CONV_LOADG)
#undef XNN_CONV_LOADG
    }
    auto edge = [&](const ConvFetch<L1, LS>& C, const ConvEdge& E) {
      float dyt[NY], dh[D1];
#pragma unroll
      for (int j = 0; j < NY; ++j) dyt[j] = -0.f;
#pragma unroll
      for (int a = 0; a < D1; ++a) dh[a] = 0.f;
      // a lane whose operands are not its own (no edge, channel past the block, weight row
      // out of range) writes zero weight gradients for an edge it has and adds nothing
      if (C.use) {
#define XNN_CONV_EDGE(P1_, P2_, P3_)                                                      \
  if constexpr (P1_ == L1 && P2_ <= LS) {                                                 \
    constexpr int ci = combo_index(P1_, P2_, P3_), ao = combo_offset(P1_, P2_, P3_);      \
    using T = CGTable<P1_, P2_, P3_>;                                                     \
    if (B.c[ci].off_w >= 0) {                                                             \
      float dw = -0.f, dy[2 * P2_ + 1], dhp[D1];                                          \
      _Pragma("unroll") for (int j = 0; j < 2 * P2_ + 1; ++j) dy[j] = -0.f;               \
      _Pragma("unroll") for (int a = 0; a < D1; ++a) dhp[a] = -0.f;                       \
      _Pragma("unroll") for (int n = 0; n < T::n; ++n) {                                  \
        const float cg = T::e[n].c * gk[ao + T::e[n].k];                                  \
        const float hg = cg * C.hv[T::e[n].i];                                            \
        dw += hg * C.yv[P2_ * P2_ + T::e[n].j];                                           \
        dy[T::e[n].j] += hg;                                                              \
        if (DH) dhp[T::e[n].i] += cg * C.yv[P2_ * P2_ + T::e[n].j];                       \
      }                                                                                   \
      if (V.g_w) V.g_w[E.e * V.dw + B.c[ci].off_w + u] = B.c[ci].coef * dw;              \
      const float sc = B.c[ci].coef * C.wv[ci];                                           \
      _Pragma("unroll") for (int j = 0; j < 2 * P2_ + 1; ++j)                             \
          dyt[P2_ * P2_ + j] += sc * dy[j];                                               \
      if (DH) {                                                                           \
        _Pragma("unroll") for (int a = 0; a < D1; ++a) dh[a] = fmaf(sc, dhp[a], dh[a]);   \
      }                                                                                   \
    }                                                                                     \
  }
        XNN_CG_TRIPLES(XNN_CONV_EDGE)
#undef XNN_CONV_EDGE
      } else if (V.g_w && E.on && u < B.mul) {
#define XNN_CONV_EDGE_ZERO(P1_, P2_, P3_)                                                 \
  if constexpr (P1_ == L1 && P2_ <= LS) {                                                 \
    constexpr int ci = combo_index(P1_, P2_, P3_);                                        \
    if (B.c[ci].off_w >= 0) V.g_w[E.e * V.dw + B.c[ci].off_w + u] = 0.f;                  \
  }
        XNN_CG_TRIPLES(XNN_CONV_EDGE_ZERO)
#undef XNN_CONV_EDGE_ZERO
      }
      if (DH && E.on && u < B.mul) {
        // zeros from a lane whose operands are not its own (dh stays 0)
        float* hr = V.dh_edge + E.e * V.dh_stride + B.off1 + (int64_t)u * D1;
#pragma unroll
        for (int a = 0; a < D1; ++a) hr[a] = dh[a];
      }
      if (V.parts) {
        // this block's share of d Y[e], every column of the present edge blocks
        float* row = V.parts + (E.e * V.n_blocks + blk) * V.d2;
#pragma unroll
        for (int l = 0; l <= LS; ++l) {
          const int o = V.off2[l];
          if (o < 0) continue;
#pragma unroll
          for (int m = 0; m < 2 * l + 1; ++m) {
            const float s = conv_group_sum(dyt[l * l + m], pair);
            if (E.on && L.sub == 0) row[o + m] = u0 == 0 ? s : row[o + m] + s;
          }
        }
      }
    };
    for (int32_t base = 0; base < L.len; base += kWave) {
      const ConvChunk K = conv_chunk(V, L, base, lane, V.src);
      ConvEdge E0 = conv_edge_at(V, K, L, 0), E1 = conv_edge_at(V, K, L, 1);
      ConvFetch<L1, LS> F0, F1;
      conv_fetch<L1, LS>(V, B, E0, u, chan, true, F0);
      conv_fetch<L1, LS>(V, B, E1, u, chan, true, F1);
      for (int32_t it = 0; it < K.trips; it += 2) {
        edge(F0, E0);
        E0 = conv_edge_at(V, K, L, it + 2);
        conv_fetch<L1, LS>(V, B, E0, u, chan, true, F0);
        if (it + 1 < K.trips) edge(F1, E1);
        E1 = conv_edge_at(V, K, L, it + 3);
        conv_fetch<L1, LS>(V, B, E1, u, chan, true, F1);
      }
    }
  }
}

// d Y[e, j] = the sum of the blocks' shares
__global__ void uvu_conv_dy_finish(ConvArgs K, float* __restrict__ g_y) {
  const ConvView V = K.v;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= V.n_edges * V.d2) return;
  const int64_t e = t / V.d2;
  const int j = (int)(t % V.d2);
  float v = 0.f;
  for (int b = 0; b < V.n_blocks; ++b)
    if (K.blocks[b].l1 >= 0) v += V.parts[(e * V.n_blocks + b) * V.d2 + j];
  g_y[t] = v;
}

// d h[s] = the sum of the edge shares over the sender's row, in row order; one wave per
// node, lanes over the columns, NC chunks of 64 columns per pass: each edge's index loaded
// once per pass and its NC loads independent, two edges in flight.
template <int NC>
__global__ __launch_bounds__(256) void uvu_conv_dh_sum(const float* __restrict__ dh_edge,
                                                       int64_t stride, const int32_t* __restrict__ ptr,
                                                       const int32_t* __restrict__ perm,
                                                       int64_t n_nodes, float* __restrict__ out,
                                                       int64_t out_stride) {
  const int lane = threadIdx.x % kWave;
  const int64_t node = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (node >= n_nodes) return;
  const int32_t q0 = ptr[node], q1 = ptr[node + 1];
  for (int64_t f0 = 0; f0 < stride; f0 += NC * kWave) {
    float acc[NC];
    bool in[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      acc[c] = 0.f;
      in[c] = f0 + c * kWave + lane < stride;
    }
    int32_t q = q0;
    for (; q + 1 < q1; q += 2) {
      const int64_t e0 = perm ? (int64_t)perm[q] : (int64_t)q;
      const int64_t e1 = perm ? (int64_t)perm[q + 1] : (int64_t)(q + 1);
      const float* r0 = dh_edge + e0 * stride + f0 + lane;
      const float* r1 = dh_edge + e1 * stride + f0 + lane;
      float v0[NC], v1[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        v0[c] = in[c] ? r0[c * kWave] : 0.f;
        v1[c] = in[c] ? r1[c * kWave] : 0.f;
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) acc[c] = (acc[c] + v0[c]) + v1[c];
    }
    if (q < q1) {
      const int64_t e0 = perm ? (int64_t)perm[q] : (int64_t)q;
      const float* r0 = dh_edge + e0 * stride + f0 + lane;
#pragma unroll
      for (int c = 0; c < NC; ++c) acc[c] += in[c] ? r0[c * kWave] : 0.f;
    }
    float* o = out + node * out_stride + f0 + lane;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (in[c]) o[c * kWave] = acc[c];
  }
}

__global__ __launch_bounds__(256) void uvu_conv_zero(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// ------------------------------------------------------------------ kernels
// the backward's edge part without (1) or with (2) the edges' shares of d h
enum ConvPass { kConvForward = 0, kConvEdgePart = 1, kConvEdgePartDh = 2 };

template <int PASS, int L1, int LS>
__device__ __forceinline__ void conv_pass(const ConvView& V, const ConvBlock& B,
                                          const ConvLanes& L, bool pair, int blk) {
  if constexpr (PASS == kConvForward) conv_fwd_block<L1, LS>(V, B, L);
  else conv_bwd_edge_block<L1, LS, PASS == kConvEdgePartDh>(V, B, L, pair, blk);
}

// One launch per node-block degree l1 (each specialization gets its own register budget):
// wave w takes block ids[w % n_ids] of the node group w / n_ids, the blocks laid out over the
// XCDs (xcd_slot): each XCD walks one contiguous run of receivers, whose senders (their
// neighbours, in a spatial atom order) it gathers from its own L2.
template <int PASS, int L1, int LS>
__global__ __launch_bounds__(kConvWaves * kWave) void uvu_conv_kernel(ConvArgs K) {
  const ConvView V = K.v;
  const int64_t w = xcd_slot() * kConvWaves + wave_in_block();
  const int blk = K.ids[w % K.n_ids];
  const ConvBlock B = K.blocks[blk];
  const bool split = B.mul <= 32;
  const int64_t group = w / K.n_ids;
  if (group >= V.n_nodes) return;
  const ConvLanes L = conv_lanes(V, group, split, threadIdx.x % kWave);
  conv_pass<PASS, L1, LS>(V, B, L, split, blk);
}

// ------------------------------------------------------------------ host
static int conv_setup(ConvArgs& A, const float* h, int64_t n_nodes, int32_t d1, const float* y,
                      int32_t d2, const float* w, int64_t n_w_rows, int32_t dw,
                      const int32_t* widx, const int32_t* src, const int32_t* dst,
                      int64_t n_edges, const xnn_uvu_path* paths, int32_t n_paths,
                      int32_t dout) {
  XNN_REQUIRE(n_nodes >= 0 && n_edges >= 0 && n_w_rows >= 0, "negative size");
  XNN_REQUIRE(n_paths >= 1 && n_paths <= kConvMaxPaths, "1 to %d paths", kConvMaxPaths);
  XNN_REQUIRE(paths != nullptr, "NULL paths");
  XNN_REQUIRE(d1 > 0 && d2 > 0 && d2 <= kConvMaxDim2 && dw > 0 && dout > 0,
              "row widths must be positive, edge attributes at most %d", kConvMaxDim2);
  XNN_REQUIRE(n_nodes < (int64_t(1) << 26) && n_edges < (int64_t(1) << 31),
              "at most 2^26 nodes and 2^31 - 1 edges");
  A = ConvArgs{};
  ConvView& V = A.v;
  V.h = h;
  V.y = y;
  V.w = w;
  V.widx = widx;
  V.src = src;
  V.dst = dst;
  V.n_nodes = n_nodes;
  V.n_edges = n_edges;
  V.n_w_rows = n_w_rows;
  V.d1 = d1;
  V.d2 = d2;
  V.dw = dw;
  V.dout = dout;
  for (int l = 0; l <= kConvMaxL; ++l) V.off2[l] = -1;
  for (int b = 0; b < kConvMaxBlocks; ++b) {
    A.blocks[b].l1 = -1;
    for (int c = 0; c < kConvCombos; ++c) A.blocks[b].c[c].off_w = -1;
  }
  int n_blocks = 0, ls = 0;
  for (int p = 0; p < n_paths; ++p) {
    const xnn_uvu_path& P = paths[p];
    XNN_REQUIRE(P.l1 >= 0 && P.l2 >= 0 && P.l3 >= 0 && P.l1 <= kConvMaxL && P.l2 <= kConvMaxL &&
                    P.l3 <= kConvMaxL,
                "path %d: degrees 0 to %d", p, kConvMaxL);
    XNN_REQUIRE(P.l3 >= std::abs(P.l1 - P.l2) && P.l3 <= P.l1 + P.l2,
                "path %d violates the triangle rule", p);
    XNN_REQUIRE(P.mul >= 1, "path %d: no channels", p);
    XNN_REQUIRE(P.off1 >= 0 && (int64_t)P.off1 + (int64_t)P.mul * (2 * P.l1 + 1) <= d1,
                "path %d: node block outside the row", p);
    XNN_REQUIRE(P.off2 >= 0 && P.off2 + 2 * P.l2 + 1 <= d2, "path %d: edge block outside the row", p);
    XNN_REQUIRE(P.off_out >= 0 && (int64_t)P.off_out + (int64_t)P.mul * (2 * P.l3 + 1) <= dout,
                "path %d: output block outside the row", p);
    XNN_REQUIRE(P.off_w >= 0 && (int64_t)P.off_w + P.mul <= dw, "path %d: weights outside the row", p);
    XNN_REQUIRE(P.block >= 0 && P.block < kConvMaxBlocks, "path %d: node block index 0 to %d", p,
                kConvMaxBlocks - 1);
    XNN_REQUIRE(V.off2[P.l2] < 0 || V.off2[P.l2] == P.off2,
                "path %d: the edge attributes have two blocks of degree %d", p, P.l2);
    V.off2[P.l2] = P.off2;
    ls = std::max(ls, (int)P.l2);
    ConvBlock& B = A.blocks[P.block];
    if (B.l1 < 0) {
      B.l1 = P.l1;
      B.mul = P.mul;
      B.off1 = P.off1;
    }
    XNN_REQUIRE(B.l1 == P.l1 && B.mul == P.mul && B.off1 == P.off1,
                "path %d: block %d read with another degree, channel count or offset", p, P.block);
    const int ci = combo_index(P.l1, P.l2, P.l3);
    XNN_REQUIRE(ci >= 0 && ci < kConvCombos, "path %d: no table entry", p);
    XNN_REQUIRE(B.c[ci].off_w < 0, "two paths read block %d with degrees (%d, %d)", P.block,
                P.l2, P.l3);
    for (int q = 0; q < p; ++q)
      XNN_REQUIRE(paths[q].off_out != P.off_out, "paths %d and %d write one output block", q, p);
    B.c[ci].off_w = P.off_w;
    B.c[ci].off_out = P.off_out;
    B.c[ci].coef = P.coef;
    n_blocks = std::max(n_blocks, (int)P.block + 1);
  }
  V.n_blocks = n_blocks;
  V.ls = ls;
  return XNN_OK;
}

template <int PASS, int L1>
static int conv_launch_l1(ConvArgs& A, hipStream_t stream) {
  A.n_ids = 0;
  for (int b = 0; b < A.v.n_blocks; ++b)
    if (A.blocks[b].l1 == L1) A.ids[A.n_ids++] = b;
  if (A.n_ids == 0) return XNN_OK;
  const int64_t waves = A.v.n_nodes * (int64_t)A.n_ids;
  const dim3 grid((unsigned)xcd_blocks(grid_1d(waves, kConvWaves))), block(kConvWaves * kWave);
  switch (A.v.ls) {
    case 0: hipLaunchKernelGGL((uvu_conv_kernel<PASS, L1, 0>), grid, block, 0, stream, A); break;
    case 1: hipLaunchKernelGGL((uvu_conv_kernel<PASS, L1, 1>), grid, block, 0, stream, A); break;
    case 2: hipLaunchKernelGGL((uvu_conv_kernel<PASS, L1, 2>), grid, block, 0, stream, A); break;
    default: hipLaunchKernelGGL((uvu_conv_kernel<PASS, L1, 3>), grid, block, 0, stream, A); break;
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

// The launches of the node-block degrees are independent (distinct blocks of the node
// rows, distinct output columns and weight columns): degree l goes to stream si[l] of the
// fork.
template <int PASS>
static int conv_launch(const ConvArgs& args, ForkJoin& fj, const int (&si)[4]) {
  ConvArgs A = args;
  int rc = conv_launch_l1<PASS, 0>(A, fj.stream(si[0]));
  if (rc == XNN_OK) rc = conv_launch_l1<PASS, 1>(A, fj.stream(si[1]));
  if (rc == XNN_OK) rc = conv_launch_l1<PASS, 2>(A, fj.stream(si[2]));
  if (rc == XNN_OK) rc = conv_launch_l1<PASS, 3>(A, fj.stream(si[3]));
  return rc;
}

// The backward's workspace: the per-block d Y shares (E, n_blocks, d2), then the edges'
// d h shares (E, dh_stride) with dh_stride the last node-row column a path reads.
struct ConvWsLayout {
  size_t parts, dh, total;
  int64_t dh_stride;
  bool dh_gaps;  // some columns below dh_stride are read by no path (zeroed before use)
};

static ConvWsLayout conv_ws_layout(int64_t n_edges, int32_t dim2, const xnn_uvu_path* paths,
                                   int32_t n_paths) {
  ConvWsLayout L{};
  int32_t n_blocks = 0;
  int64_t stride = 0;
  for (int p = 0; p < n_paths; ++p) {
    n_blocks = std::max(n_blocks, paths[p].block + 1);
    stride = std::max<int64_t>(stride, (int64_t)paths[p].off1 +
                                           (int64_t)paths[p].mul * (2 * paths[p].l1 + 1));
  }
  // columns read by some path (the blocks may leave gaps)
  int64_t covered = 0;
  for (int b = 0; b < n_blocks; ++b) {
    for (int p = 0; p < n_paths; ++p) {
      if (paths[p].block != b) continue;
      covered += (int64_t)paths[p].mul * (2 * paths[p].l1 + 1);
      break;
    }
  }
  L.dh_stride = stride;
  L.dh_gaps = covered != stride;
  const auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  L.parts = 0;
  L.dh = align((size_t)n_edges * (size_t)n_blocks * (size_t)dim2 * sizeof(float));
  L.total = L.dh + (size_t)n_edges * (size_t)stride * sizeof(float);
  return L;
}

}  // namespace xnn

using namespace xnn;

extern "C" {

size_t xnn_uvu_conv_workspace_bytes(int64_t n_edges, int32_t dim2, const xnn_uvu_path* paths,
                                    int32_t n_paths) {
  if (n_edges <= 0 || dim2 <= 0 || paths == nullptr || n_paths <= 0) return 0;
  const ConvWsLayout L = conv_ws_layout(n_edges, dim2, paths, n_paths);
  return L.total;
}

int xnn_uvu_conv(const float* node_feats, int64_t n_nodes, int32_t dim1, const float* edge_attrs,
                 int32_t dim2, const float* weights, int64_t n_weight_rows, int32_t dim_w,
                 const int32_t* weight_index, const int32_t* src, int64_t n_edges,
                 const int32_t* ptr_dst, const int32_t* perm_dst, const xnn_uvu_path* paths,
                 int32_t n_paths, float* out, int32_t dim_out, xnn_stream_t stream) {
  ConvArgs A;
  const int rc = conv_setup(A, node_feats, n_nodes, dim1, edge_attrs, dim2, weights, n_weight_rows,
                            dim_w, weight_index, src, nullptr, n_edges, paths, n_paths, dim_out);
  if (rc != XNN_OK) return rc;
  if (n_nodes == 0) return XNN_OK;
  XNN_REQUIRE(out && ptr_dst, "NULL output or CSR");
  XNN_REQUIRE(n_edges == 0 || (node_feats && edge_attrs && weights && src), "NULL input");
  A.v.ptr = ptr_dst;
  A.v.perm = perm_dst;
  A.v.out = out;
  ForkJoin fj(as_hip(stream));
  const int rc2 = conv_launch<kConvForward>(A, fj, {0, 1, 2, 3});
  XNN_HIP_CHECK(fj.join());
  return rc2;
}

int xnn_uvu_conv_backward(const float* node_feats, int64_t n_nodes, int32_t dim1,
                          const float* edge_attrs, int32_t dim2, const float* weights,
                          int64_t n_weight_rows, int32_t dim_w, const int32_t* weight_index,
                          const int32_t* src, const int32_t* dst, int64_t n_edges,
                          const int32_t* ptr_dst, const int32_t* perm_dst,
                          const int32_t* ptr_src, const int32_t* perm_src,
                          const xnn_uvu_path* paths, int32_t n_paths, const float* grad_out,
                          int32_t dim_out, float* grad_node_feats, float* grad_edge_attrs,
                          float* grad_weights, void* workspace, size_t workspace_bytes,
                          xnn_stream_t stream) {
  ConvArgs A;
  const int rc = conv_setup(A, node_feats, n_nodes, dim1, edge_attrs, dim2, weights, n_weight_rows,
                            dim_w, weight_index, src, dst, n_edges, paths, n_paths, dim_out);
  if (rc != XNN_OK) return rc;
  if (n_nodes == 0) return XNN_OK;
  XNN_REQUIRE(grad_out, "NULL output gradient");
  XNN_REQUIRE(n_edges == 0 || (node_feats && edge_attrs && weights && src), "NULL input");
  A.v.g_out = grad_out;
  const hipStream_t s = as_hip(stream);
  const ConvWsLayout W = conv_ws_layout(n_edges, dim2, paths, n_paths);
  if (grad_node_feats) {
    XNN_REQUIRE(ptr_src && (n_edges == 0 || dst), "NULL sender CSR or receivers");
    if (n_edges == 0) {
      // no edge: every column of the path-read blocks is zero
      hipLaunchKernelGGL(uvu_conv_zero, dim3((unsigned)grid_1d(n_nodes * dim1, 256)), dim3(256), 0,
                         s, grad_node_feats, n_nodes * (int64_t)dim1);
      XNN_LAUNCH_CHECK();
      return XNN_OK;
    }
  }
  if (n_edges == 0 || !(grad_edge_attrs || grad_weights || grad_node_feats)) return XNN_OK;
  XNN_REQUIRE(ptr_dst, "NULL receiver CSR");
  const bool need_ws = grad_edge_attrs || grad_node_feats;
  XNN_REQUIRE(!need_ws || (workspace != nullptr && workspace_bytes >= W.total),
              "workspace of %zu bytes needed (xnn_uvu_conv_workspace_bytes)", W.total);
  ConvArgs B = A;
  B.v.ptr = ptr_dst;
  B.v.perm = perm_dst;
  B.v.g_w = grad_weights;
  if (grad_edge_attrs) B.v.parts = reinterpret_cast<float*>(static_cast<char*>(workspace) + W.parts);
  if (grad_node_feats) {
    B.v.dh_edge = reinterpret_cast<float*>(static_cast<char*>(workspace) + W.dh);
    B.v.dh_stride = W.dh_stride;
    if (W.dh_gaps) {
      hipLaunchKernelGGL(uvu_conv_zero, dim3((unsigned)grid_1d(n_edges * W.dh_stride, 256)),
                         dim3(256), 0, s, B.v.dh_edge, n_edges * W.dh_stride);
      XNN_LAUNCH_CHECK();
    }
  }
  {
    // one edge part over the receivers' rows (the node-block degrees side by side), then the
    // finishes: d Y from the blocks' shares, d h from the edges' shares over the senders
    ForkJoin fj(s);
    const int rc2 = grad_node_feats ? conv_launch<kConvEdgePartDh>(B, fj, {0, 1, 2, 3})
                                    : conv_launch<kConvEdgePart>(B, fj, {0, 1, 2, 3});
    if (rc2 != XNN_OK) return rc2;
    XNN_HIP_CHECK(fj.join());
  }
  if (grad_edge_attrs) {
    hipLaunchKernelGGL(uvu_conv_dy_finish, dim3((unsigned)grid_1d(n_edges * dim2, 256)),
                       dim3(256), 0, s, B, grad_edge_attrs);
    XNN_LAUNCH_CHECK();
  }
  if (grad_node_feats) {
    const dim3 grid((unsigned)grid_1d(n_nodes * kWave, 256));
    if (W.dh_stride <= 4 * kWave)
      hipLaunchKernelGGL(uvu_conv_dh_sum<4>, grid, dim3(256), 0, s, B.v.dh_edge, W.dh_stride,
                         ptr_src, perm_src, n_nodes, grad_node_feats, (int64_t)dim1);
    else
      hipLaunchKernelGGL(uvu_conv_dh_sum<8>, grid, dim3(256), 0, s, B.v.dh_edge, W.dh_stride,
                         ptr_src, perm_src, n_nodes, grad_node_feats, (int64_t)dim1);
    XNN_LAUNCH_CHECK();
  }
  return XNN_OK;
}

}  // extern "C"
