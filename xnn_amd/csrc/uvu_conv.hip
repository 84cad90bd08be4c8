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
// Work is split by (node, path): a wave owns one path of one node (of two nodes, one per
// half-wave, when the path has at most 32 channels), its lanes the channels u. The path is
// uniform over the wave, so each wave runs code specialized for its (l1, l2, l3) that keeps
// the 2 l3 + 1 sums of a channel in registers and expands the product over the nonzero
// entries of C only. The waves of one node are neighbours in the grid, so its rows of h,
// Y and w are shared through the caches.
//
// xnn_uvu_conv_backward, given d out:
//   edge part, waves by (receiver, path) as in the forward: d w[e, p, u] per edge (the
//   caller sums the rows of shared weights) and the channel sums of path p's share of
//   d Y[e], kept per path in the workspace and added up by a last pass;
//   node part, waves by (sender, node block): d h[s, block, u, a] =
//     sum_{p reads block} c_p sum_{e: src(e) = s} w[row(e), p, u]
//                         sum_{b, k} C[a, b, k] Y[e, b] d out[dst(e), p, u, k].
#include <algorithm>
#include <cstdint>

#include "cg_tables.h"
#include "common.h"
#include "device.h"

namespace xnn {

constexpr int kConvWaves = 4;
constexpr int kConvMaxPaths = 48;
constexpr int kConvMaxL = 3;
constexpr int kConvMaxDim2 = 16;  // entries of the edge attribute rows

// The scalar fields of the arguments, copied into registers at kernel entry: the helpers
// take this view, not the kernel argument (a reference to the by-value argument that
// escapes into the specialized paths makes the compiler copy all of it, path table
// included, to scratch memory).
struct ConvView {
  const float* h;
  const float* y;
  const float* w;
  const int32_t* widx;
  const int32_t* src;
  const int32_t* dst;
  const int32_t* ptr;
  const int32_t* perm;
  const float* g_out;
  float* out;
  float* g_w;
  float* parts;
  int64_t n_nodes, n_edges, n_w_rows;
  int32_t d1, d2, dw, dout, n_paths, n_slots;
};

struct ConvArgs {
  const float* h;     // (N, d1)
  const float* y;     // (E, d2)
  const float* w;     // (n_w_rows, dw)
  const int32_t* widx;
  const int32_t* src;
  const int32_t* dst;
  const int32_t* ptr;   // CSR of the walk: receivers (forward, edge part) or senders
  const int32_t* perm;
  const float* g_out;   // (N, dout) backward
  float* out;           // forward: (N, dout); node part: d h (N, d1)
  float* g_w;           // (E, dw) per edge
  float* parts;         // (E, n_slots): per path channel sums of d Y
  int64_t n_nodes, n_edges, n_w_rows;
  int32_t d1, d2, dw, dout, n_paths, n_slots;
  xnn_uvu_path paths[kConvMaxPaths];
  int32_t slot[kConvMaxPaths];  // first column of path p's d Y share in `parts`
};

__device__ __forceinline__ ConvView conv_view(const ConvArgs& A) {
  return ConvView{A.h,     A.y,       A.w,       A.widx,     A.src, A.dst, A.ptr,
                  A.perm,  A.g_out,   A.out,     A.g_w,      A.parts, A.n_nodes,
                  A.n_edges, A.n_w_rows, A.d1, A.d2, A.dw,   A.dout, A.n_paths, A.n_slots};
}

__device__ __forceinline__ int64_t conv_row(const ConvView& A, int64_t e) {
  return A.widx ? (int64_t)A.widx[e] : e;
}

// The nodes of a wave: one (channels in chunks of 64) or two (32 lanes each).
struct ConvLanes {
  int64_t node;      // this lane's node (>= n_nodes: no work)
  int sub;           // lane within its node's group
  int width;         // channels per chunk (64 or 32)
  int32_t q0, len;   // this lane's node's CSR range
  int32_t trips;     // uniform: the longest range of the wave
};

__device__ __forceinline__ ConvLanes conv_lanes(const ConvView& A, int64_t group, bool pair,
                                                int lane) {
  ConvLanes L;
  L.width = pair ? 32 : kWave;
  L.sub = pair ? (lane & 31) : lane;
  L.node = pair ? 2 * group + (lane >> 5) : group;
  L.q0 = 0;
  L.len = 0;
  if (L.node < A.n_nodes) {
    L.q0 = A.ptr[L.node];
    L.len = A.ptr[L.node + 1] - L.q0;
  }
  int32_t t = L.len;
  if (pair) t = std::max(__builtin_amdgcn_readlane(L.len, 0), __builtin_amdgcn_readlane(L.len, 32));
  L.trips = __builtin_amdgcn_readfirstlane(t);
  return L;
}

// sum over the lanes of one node's group (32 or 64 lanes)
__device__ __forceinline__ float conv_group_sum(float v, bool pair) {
  if (!pair) v += __shfl_xor(v, 32);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 1);
  return v;
}

// ------------------------------------------------------------------ forward
template <int L1, int L2, int L3>
__device__ __forceinline__ void conv_fwd_path(const ConvView& A, const xnn_uvu_path& P,
                                              const ConvLanes& L) {
  using T = CGTable<L1, L2, L3>;
  constexpr int D1 = 2 * L1 + 1, D2 = 2 * L2 + 1, D3 = 2 * L3 + 1;
  for (int u0 = 0; u0 < P.mul; u0 += L.width) {
    const int u = u0 + L.sub;
    const bool chan = u < P.mul;
    float acc[D3];
#pragma unroll
    for (int k = 0; k < D3; ++k) acc[k] = 0.f;
    for (int32_t it = 0; it < L.trips; ++it) {
      const bool on = it < L.len;
      int64_t e = 0, s = 0, row = -1;
      if (on) {
        const int32_t q = L.q0 + it;
        e = A.perm ? (int64_t)A.perm[q] : (int64_t)q;
        s = A.src[e];
        row = conv_row(A, e);
      }
      const bool use = on && chan && row >= 0 && row < A.n_w_rows;
      float yv[D2], hv[D1];
#pragma unroll
      for (int b = 0; b < D2; ++b) yv[b] = use ? A.y[e * A.d2 + P.off2 + b] : 0.f;
#pragma unroll
      for (int a = 0; a < D1; ++a) hv[a] = use ? A.h[s * A.d1 + P.off1 + u * D1 + a] : 0.f;
      const float wv = use ? A.w[row * A.dw + P.off_w + u] : 0.f;
      float t[D3];
#pragma unroll
      for (int k = 0; k < D3; ++k) t[k] = 0.f;
#pragma unroll
      for (int n = 0; n < T::n; ++n) t[T::e[n].k] += T::e[n].c * hv[T::e[n].i] * yv[T::e[n].j];
#pragma unroll
      for (int k = 0; k < D3; ++k) acc[k] += wv * t[k];
    }
    if (chan && L.node < A.n_nodes) {
#pragma unroll
      for (int k = 0; k < D3; ++k)
        A.out[L.node * A.dout + P.off_out + u * D3 + k] = P.coef * acc[k];
    }
  }
}

// wave w: path w % n_paths of the node group w / n_paths
__global__ __launch_bounds__(kConvWaves * kWave) void uvu_conv_fwd(ConvArgs K) {
  const ConvView A = conv_view(K);
  const int64_t w = (int64_t)blockIdx.x * kConvWaves + wave_in_block();
  const int p = (int)(w % A.n_paths);
  const xnn_uvu_path P = K.paths[p];
  const bool pair = P.mul <= 32;
  const int64_t group = w / A.n_paths;
  if (group * (pair ? 2 : 1) >= A.n_nodes) return;
  const ConvLanes L = conv_lanes(A, group, pair, threadIdx.x % kWave);
  switch (P.l1 * 16 + P.l2 * 4 + P.l3) {
#define XNN_CONV_CASE(a, b, c) \
  case a * 16 + b * 4 + c: conv_fwd_path<a, b, c>(A, P, L); break;
    XNN_CG_TRIPLES(XNN_CONV_CASE)
#undef XNN_CONV_CASE
    default: break;
  }
}

// ------------------------------------------------------------------ backward, edge part
template <int L1, int L2, int L3>
__device__ __forceinline__ void conv_bwd_edge_path(const ConvView& A, const xnn_uvu_path& P,
                                                   int slot, const ConvLanes& L, bool pair) {
  using T = CGTable<L1, L2, L3>;
  constexpr int D1 = 2 * L1 + 1, D2 = 2 * L2 + 1, D3 = 2 * L3 + 1;
  for (int32_t it = 0; it < L.trips; ++it) {
    const bool on = it < L.len;
    int64_t e = 0, s = 0, row = -1;
    if (on) {
      const int32_t q = L.q0 + it;
      e = A.perm ? (int64_t)A.perm[q] : (int64_t)q;
      s = A.src[e];
      row = conv_row(A, e);
    }
    const bool row_ok = on && row >= 0 && row < A.n_w_rows;
    float yv[D2], dyt[D2];
#pragma unroll
    for (int b = 0; b < D2; ++b) {
      yv[b] = row_ok ? A.y[e * A.d2 + P.off2 + b] : 0.f;
      dyt[b] = 0.f;
    }
    for (int u0 = 0; u0 < P.mul; u0 += L.width) {
      const int u = u0 + L.sub;
      const bool use = row_ok && u < P.mul;
      float hv[D1], gk[D3];
#pragma unroll
      for (int a = 0; a < D1; ++a) hv[a] = use ? A.h[s * A.d1 + P.off1 + u * D1 + a] : 0.f;
#pragma unroll
      for (int k = 0; k < D3; ++k)
        gk[k] = use ? A.g_out[L.node * A.dout + P.off_out + u * D3 + k] : 0.f;
      const float wv = use ? A.w[row * A.dw + P.off_w + u] : 0.f;
      float dw = 0.f, dy[D2];
#pragma unroll
      for (int b = 0; b < D2; ++b) dy[b] = 0.f;
#pragma unroll
      for (int n = 0; n < T::n; ++n) {
        const float hg = T::e[n].c * hv[T::e[n].i] * gk[T::e[n].k];
        dw += hg * yv[T::e[n].j];
        dy[T::e[n].j] += hg;
      }
      if (A.g_w && on && u < P.mul) A.g_w[e * A.dw + P.off_w + u] = P.coef * dw;
#pragma unroll
      for (int b = 0; b < D2; ++b) dyt[b] += P.coef * wv * dy[b];
    }
    if (A.parts) {
#pragma unroll
      for (int b = 0; b < D2; ++b) {
        const float v = conv_group_sum(dyt[b], pair);
        if (on && L.sub == 0) A.parts[e * A.n_slots + slot + b] = v;
      }
    }
  }
}

__global__ __launch_bounds__(kConvWaves * kWave) void uvu_conv_bwd_edge(ConvArgs K) {
  const ConvView A = conv_view(K);
  const int64_t w = (int64_t)blockIdx.x * kConvWaves + wave_in_block();
  const int p = (int)(w % A.n_paths);
  const xnn_uvu_path P = K.paths[p];
  const int slot = K.slot[p];
  const bool pair = P.mul <= 32;
  const int64_t group = w / A.n_paths;
  if (group * (pair ? 2 : 1) >= A.n_nodes) return;
  const ConvLanes L = conv_lanes(A, group, pair, threadIdx.x % kWave);
  switch (P.l1 * 16 + P.l2 * 4 + P.l3) {
#define XNN_CONV_CASE(a, b, c) \
  case a * 16 + b * 4 + c: conv_bwd_edge_path<a, b, c>(A, P, slot, L, pair); break;
    XNN_CG_TRIPLES(XNN_CONV_CASE)
#undef XNN_CONV_CASE
    default: break;
  }
}

// d Y[e, j] = the sum of the paths' shares that land on column j
__global__ void uvu_conv_dy_finish(ConvArgs A, float* __restrict__ g_y) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= A.n_edges * A.d2) return;
  const int64_t e = t / A.d2;
  const int j = (int)(t % A.d2);
  float v = 0.f;
  for (int p = 0; p < A.n_paths; ++p) {
    const int b = j - A.paths[p].off2;
    if (b >= 0 && b < 2 * A.paths[p].l2 + 1) v += A.parts[e * A.n_slots + A.slot[p] + b];
  }
  g_y[t] = v;
}

// ------------------------------------------------------------------ backward, node part
template <int L1, int L2, int L3>
__device__ __forceinline__ void conv_bwd_node_path(const ConvView& A, const xnn_uvu_path& P,
                                                   const ConvLanes& L, int u, float* acc) {
  using T = CGTable<L1, L2, L3>;
  constexpr int D1 = 2 * L1 + 1, D2 = 2 * L2 + 1, D3 = 2 * L3 + 1;
  float part[D1];
#pragma unroll
  for (int a = 0; a < D1; ++a) part[a] = 0.f;
  for (int32_t it = 0; it < L.trips; ++it) {
    const bool on = it < L.len;
    int64_t e = 0, d = 0, row = -1;
    if (on) {
      const int32_t q = L.q0 + it;
      e = A.perm ? (int64_t)A.perm[q] : (int64_t)q;
      d = A.dst[e];
      row = conv_row(A, e);
    }
    const bool use = on && u < P.mul && row >= 0 && row < A.n_w_rows;
    float yv[D2], gk[D3];
#pragma unroll
    for (int b = 0; b < D2; ++b) yv[b] = use ? A.y[e * A.d2 + P.off2 + b] : 0.f;
#pragma unroll
    for (int k = 0; k < D3; ++k) gk[k] = use ? A.g_out[d * A.dout + P.off_out + u * D3 + k] : 0.f;
    const float wv = use ? A.w[row * A.dw + P.off_w + u] : 0.f;
    float t[D1];
#pragma unroll
    for (int a = 0; a < D1; ++a) t[a] = 0.f;
#pragma unroll
    for (int n = 0; n < T::n; ++n) t[T::e[n].i] += T::e[n].c * yv[T::e[n].j] * gk[T::e[n].k];
#pragma unroll
    for (int a = 0; a < D1; ++a) part[a] += wv * t[a];
  }
#pragma unroll
  for (int a = 0; a < D1; ++a) acc[a] += P.coef * part[a];
}

// every path that reads node block `blk` (all of degree L1), chunk by chunk of channels
template <int L1>
__device__ __forceinline__ void conv_bwd_node_block(const ConvArgs& K, const ConvView& A, int blk,
                                                    const ConvLanes& L, int mul, int off1) {
  constexpr int D1 = 2 * L1 + 1;
  for (int u0 = 0; u0 < mul; u0 += L.width) {
    const int u = u0 + L.sub;
    float acc[D1];
#pragma unroll
    for (int a = 0; a < D1; ++a) acc[a] = 0.f;
    for (int p = 0; p < A.n_paths; ++p) {
      const xnn_uvu_path P = K.paths[p];
      if (P.block != blk) continue;
      switch (P.l1 * 16 + P.l2 * 4 + P.l3) {
#define XNN_CONV_CASE(a, b, c)                                           \
  case a * 16 + b * 4 + c:                                               \
    if constexpr (a == L1) conv_bwd_node_path<a, b, c>(A, P, L, u, acc); \
    break;
        XNN_CG_TRIPLES(XNN_CONV_CASE)
#undef XNN_CONV_CASE
        default: break;
      }
    }
    if (u < mul && L.node < A.n_nodes) {
#pragma unroll
      for (int a = 0; a < D1; ++a) A.out[L.node * A.d1 + off1 + u * D1 + a] = acc[a];
    }
  }
}

// wave w: node block w % n_blocks of the sender group w / n_blocks
__global__ __launch_bounds__(kConvWaves * kWave) void uvu_conv_bwd_node(ConvArgs K,
                                                                        int32_t n_blocks) {
  const ConvView A = conv_view(K);
  const int64_t w = (int64_t)blockIdx.x * kConvWaves + wave_in_block();
  const int blk = (int)(w % n_blocks);
  int first = -1;
  for (int p = 0; p < A.n_paths; ++p) {
    if (K.paths[p].block == blk) {
      first = p;
      break;
    }
  }
  if (first < 0) return;
  const xnn_uvu_path P = K.paths[first];
  const bool pair = P.mul <= 32;
  const int64_t group = w / n_blocks;
  if (group * (pair ? 2 : 1) >= A.n_nodes) return;
  const ConvLanes L = conv_lanes(A, group, pair, threadIdx.x % kWave);
  switch (P.l1) {
    case 0: conv_bwd_node_block<0>(K, A, blk, L, P.mul, P.off1); break;
    case 1: conv_bwd_node_block<1>(K, A, blk, L, P.mul, P.off1); break;
    case 2: conv_bwd_node_block<2>(K, A, blk, L, P.mul, P.off1); break;
    case 3: conv_bwd_node_block<3>(K, A, blk, L, P.mul, P.off1); break;
    default: break;
  }
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
  A.h = h;
  A.y = y;
  A.w = w;
  A.widx = widx;
  A.src = src;
  A.dst = dst;
  A.n_nodes = n_nodes;
  A.n_edges = n_edges;
  A.n_w_rows = n_w_rows;
  A.d1 = d1;
  A.d2 = d2;
  A.dw = dw;
  A.dout = dout;
  A.n_paths = n_paths;
  int slots = 0;
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
    XNN_REQUIRE(P.block >= 0 && P.block < kConvMaxPaths, "path %d: node block index", p);
    for (int q = 0; q < p; ++q) {
      if (paths[q].block == P.block)
        XNN_REQUIRE(paths[q].l1 == P.l1 && paths[q].mul == P.mul && paths[q].off1 == P.off1,
                    "paths %d and %d share block %d but not its degree, channels and offset", q,
                    p, P.block);
      XNN_REQUIRE(paths[q].off_out != P.off_out, "paths %d and %d write one output block", q, p);
    }
    A.paths[p] = P;
    A.slot[p] = slots;
    slots += 2 * P.l2 + 1;
  }
  A.n_slots = slots;
  return XNN_OK;
}

}  // namespace xnn

using namespace xnn;

extern "C" {

size_t xnn_uvu_conv_workspace_bytes(int64_t n_edges, const xnn_uvu_path* paths, int32_t n_paths) {
  if (n_edges <= 0 || paths == nullptr || n_paths <= 0) return 0;
  int64_t slots = 0;
  for (int p = 0; p < n_paths; ++p) slots += 2 * (int64_t)paths[p].l2 + 1;
  return (size_t)(n_edges * slots) * sizeof(float);
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
  A.ptr = ptr_dst;
  A.perm = perm_dst;
  A.out = out;
  hipLaunchKernelGGL(uvu_conv_fwd, dim3((unsigned)grid_1d(n_nodes * n_paths, kConvWaves)),
                     dim3(kConvWaves * kWave), 0, as_hip(stream), A);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
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
  A.g_out = grad_out;
  if ((grad_edge_attrs || grad_weights) && n_edges > 0) {
    XNN_REQUIRE(ptr_dst, "NULL receiver CSR");
    ConvArgs B = A;
    B.ptr = ptr_dst;
    B.perm = perm_dst;
    B.g_w = grad_weights;
    if (grad_edge_attrs) {
      const size_t need = xnn_uvu_conv_workspace_bytes(n_edges, paths, n_paths);
      XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need,
                  "workspace of %zu bytes needed (xnn_uvu_conv_workspace_bytes)", need);
      B.parts = static_cast<float*>(workspace);
    }
    hipLaunchKernelGGL(uvu_conv_bwd_edge, dim3((unsigned)grid_1d(n_nodes * n_paths, kConvWaves)),
                       dim3(kConvWaves * kWave), 0, as_hip(stream), B);
    XNN_LAUNCH_CHECK();
    if (grad_edge_attrs) {
      hipLaunchKernelGGL(uvu_conv_dy_finish, dim3((unsigned)grid_1d(n_edges * dim2, 256)),
                         dim3(256), 0, as_hip(stream), B, grad_edge_attrs);
      XNN_LAUNCH_CHECK();
    }
  }
  if (grad_node_feats) {
    XNN_REQUIRE(ptr_src && (n_edges == 0 || dst), "NULL sender CSR or receivers");
    ConvArgs B = A;
    B.ptr = ptr_src;
    B.perm = perm_src;
    B.out = grad_node_feats;
    int32_t n_blocks = 0;
    for (int p = 0; p < n_paths; ++p) n_blocks = std::max(n_blocks, paths[p].block + 1);
    hipLaunchKernelGGL(uvu_conv_bwd_node, dim3((unsigned)grid_1d(n_nodes * n_blocks, kConvWaves)),
                       dim3(kConvWaves * kWave), 0, as_hip(stream), B, n_blocks);
    XNN_LAUNCH_CHECK();
  }
  return XNN_OK;
}

}  // extern "C"
