// Edge -> atom message sums through the radial features, with the linear layer applied
// per atom (gfx950, wave64, fp32 MFMA).
//
// The sum the reference forms edge by edge,
//   A_i[c, lm] = sum_{dst(e)=i} phi_e[c] Y_lm(sign r_e),   phi_e = h_e W,
// (the uvu product of scalar per-edge weights with the edge harmonics followed by
// scatter_sum, gnn/fast/conv.py:137-143 and ops.py:403-448, with phi the last linear layer
// of the radial weights) is linear in h_e, so it equals
//   A_i = W^T B_i,   B_i[k, lm] = sum_{dst(e)=i} h_e[k] Y_lm(sign r_e),
// the same double sum with its two contractions taken in the other order. B_i is K x L
// (8 x 16) per atom where an edge's message is C x L (128 x 16): a receiver row costs one
// 16 x 16 x 4 matrix-core product per four edges plus 2 T products for W^T B_i, and the
// forward is bounded by writing the (N, C, L) rows. The backward reads the rows' cotangent
// G_i = dE/dA_i (any (N, C, L) tensor), forms dB_i = W G_i on the matrix cores (K = C),
// and per edge
//   d h_e[k] = sum_lm dB_i[k, lm] Y_lm(e),   dY_e[lm] = sum_k h_e[k] dB_i[k, lm],
// chained to the edge vector through the harmonics and, when the kernel evaluates the
// radial features itself (RAD), through the enveloped radial basis of |r_e|.
//
// Work mapping: one wave per receiver row (persistent waves). Each lane evaluates one
// edge's harmonics and radial row into LDS; the products read them back in operand layout.
//   B = H^T Y:  M = 16 rows standing for the radial features (row m holds feature
//               2 (m / 4) + m % 4 when m % 4 < 2, zeros otherwise), N = lm, K = 4 edges a
//               step. Result register i < 2 of lane l is then B[2 (l / 16) + i][l % 16].
//   A^T = B^T W per 16-channel tile t: M = lm, N = channel 16 t + l % 16, K = feature
//               2 (l / 16) + s at step s = 0, 1: the A operand is B's result register s
//               unchanged, and result register i is A[16 t + l % 16][4 (l / 16) + i] --
//               four consecutive floats of one channel row, a 1 KB run per tile.
//   dB = W G:   M = the same 16 feature rows, N = lm, K = channel 4 s + l / 16 at step s
//               (the G operand a run of 64 floats per step); result register i < 2 of
//               lane l is dB[2 (l / 16) + i][l % 16], staged through LDS for the edges.
#include <algorithm>
#include <cstdint>

#include "common.h"
#include "device.h"
#include "message.h"
#include "radial_row.h"

namespace xnn {

// The radial feature held by M row m of the feature-row products (-1: a zero row).
__device__ __forceinline__ int basis_row_feature(int m) {
  return (m & 3) < 2 ? 2 * (m >> 2) + (m & 3) : -1;
}

template <typename G>
__device__ __forceinline__ const G* row_cell(const G* __restrict__ cell, int64_t n_graphs,
                                             const int32_t* __restrict__ batch, int64_t row) {
  if (cell == nullptr) return nullptr;
  return (n_graphs <= 1 || batch == nullptr) ? cell : cell + 9 * (int64_t)batch[row];
}

// A given feature row h_e (K <= kLinKMax) into the lane's LDS row, zeros past K and for a
// lane without an edge.
__device__ __forceinline__ void load_h_row(const float* __restrict__ h, int K, bool valid,
                                           int64_t e, float* __restrict__ row) {
#pragma unroll
  for (int k = 0; k < kLinKMax; ++k) row[k] = (valid && k < K) ? h[e * K + k] : 0.f;
}

template <typename G, int LMAX, int T, bool RAD>
__global__ __launch_bounds__(256) void basis_msg_fwd_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, float sign, int K,
    const float* __restrict__ h, Radial<float> R, const float* __restrict__ W,
    float* __restrict__ out) {
  constexpr int L = ShDims<LMAX>::L;
  constexpr int C = 16 * T;
  __shared__ float sY[kWavesPerBlock][kWave * kSY];
  __shared__ float sH[kWavesPerBlock][kWave * kSH];
  __shared__ float sTab[kLinKMax];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int lo = lane & 15, hi = lane >> 4;
  float* ys = sY[wave];
  float* hs = sH[wave];
  const RadialTab tab = RAD ? load_radial_tab(R, sTab) : RadialTab{};
  // B operand of A^T = B^T W for channel tile t at k-step s: W[2 hi + s][16 t + lo]
  float wb[T][2];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int k = 2 * hi + s;
      wb[t][s] = k < K ? W[k * C + 16 * t + lo] : 0.f;
    }
  __syncthreads();  // the radial table
  const int feat = basis_row_feature(lo);
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave;
  // with given edge vectors, the first batch of the wave's next row is loaded a row ahead
  float px = 0.f, py = 0.f, pz = 0.f;
  if (vec != nullptr && row < n_nodes) load_first_vec(vec, perm, ptr[row], ptr[row + 1], lane, px, py, pz);
  for (; row < n_nodes; row += n_waves) {
    const G* cl = row_cell(cell, n_graphs, batch, row);
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    const int b0 = ptr[row], b1 = ptr[row + 1];
    const float cx = px, cy = py, cz = pz;
    if (vec != nullptr && row + n_waves < n_nodes)
      load_first_vec(vec, perm, ptr[row + n_waves], ptr[row + n_waves + 1], lane, px, py, pz);
    for (int base = b0; base < b1; base += kWave) {
      const int cnt = min(kWave, b1 - base);
      const int my_e = lane < cnt ? (perm ? perm[base + lane] : base + lane) : 0;
      float ux, uy, uz, inv, len;
      if (vec != nullptr && base == b0)
        batch_harmonics_xyz<LMAX>(cx, cy, cz, sign, lane, cnt, ys, ux, uy, uz, inv, len);
      else
        batch_harmonics<G, LMAX>(vec, pos, cl, src, shift, (int)row, sign, lane, cnt, my_e, ys,
                                 ux, uy, uz, inv, len);
      if constexpr (RAD)
        radial_row(R, tab, lane < cnt, len, hs + lane * kSH);
      else
        load_h_row(h, K, lane < cnt, my_e, hs + lane * kSH);
      wave_sync();
      // B += H^T Y over groups of four edges (rows past the batch's end are zero)
      const int ngrp = (cnt + 3) >> 2;
#pragma unroll 2
      for (int q = 0; q < ngrp; ++q) {
        const int e = 4 * q + hi;
        const float a = feat >= 0 ? hs[e * kSH + feat] : 0.f;
        acc = mfma_16x16x4(a, ys[e * kSY + lo], acc);
      }
      wave_sync();  // the rows are rewritten by the next batch
    }
    // acc[i] = B[2 hi + i][lo] for i < 2; A^T = B^T W tile by tile
    float* o = out + row * (int64_t)(C * L);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      floatx4 d = floatx4{0.f, 0.f, 0.f, 0.f};
      d = mfma_16x16x4(acc[0], wb[t][0], d);
      d = mfma_16x16x4(acc[1], wb[t][1], d);
      float* oc = o + (16 * t + lo) * L;  // d[i] = A[16 t + lo][4 hi + i]
      if constexpr (L == 16) {
        *reinterpret_cast<float4*>(oc + 4 * hi) = make_float4(d[0], d[1], d[2], d[3]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * hi + i < L) oc[4 * hi + i] = d[i];
      }
    }
  }
}

// d_h (given h, !RAD): the feature rows' gradient (E, K); g_vec (may be NULL when only d_h
// is wanted): the edge vectors' gradient (E, 3), through the harmonics and (RAD) the
// radial row.
template <typename G, int LMAX, int T, bool RAD>
__global__ __launch_bounds__(256) void basis_msg_bwd_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, float sign, int K,
    const float* __restrict__ h, Radial<float> R, const float* __restrict__ W,
    const float* __restrict__ d_out, float* __restrict__ d_h, float* __restrict__ g_vec) {
  constexpr int L = ShDims<LMAX>::L;
  constexpr int C = 16 * T;
  constexpr int NS = C / 4;  // k-steps of dB = W G over the channels
  __shared__ float sY[kWavesPerBlock][kWave * kSY];
  __shared__ float sH[kWavesPerBlock][kWave * kSH];
  __shared__ __align__(16) float sB[kWavesPerBlock][kLinKMax * 16];
  __shared__ float sTab[kLinKMax];
  // W in LDS, rows padded to C + 4 floats: the A operand of dB = W G at k-step s is
  // W[feature of M row lo][channel 4 s + hi] (32 distinct banks for the 8 x 4 addresses)
  constexpr int SWS = C + 4;
  __shared__ float sW[kLinKMax * SWS];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int lo = lane & 15, hi = lane >> 4;
  float* ys = sY[wave];
  float* hs = sH[wave];
  float* sb = sB[wave];
  const RadialTab tab = RAD ? load_radial_tab(R, sTab) : RadialTab{};
  for (int i = threadIdx.x; i < kLinKMax * C; i += blockDim.x)
    sW[(i / C) * SWS + i % C] = i < K * C ? W[i] : 0.f;
  __syncthreads();
  const int feat = basis_row_feature(lo);
  const float* wrow = sW + (feat >= 0 ? feat : 0) * SWS + hi;
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave; row < n_nodes;
       row += n_waves) {
    const int b0 = ptr[row], b1 = ptr[row + 1];
    if (b0 == b1) continue;
    {
      // dB = W G with the row's cotangent in the B operand layout, G[4 s + hi][lo] (a run
      // of 64 floats a step); two accumulators halve the dependent chain
      const float* gr = d_out + row * (int64_t)(C * L);
      float ga[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) ga[s] = lo < L ? gr[(4 * s + hi) * L + lo] : 0.f;
      floatx4 db0 = floatx4{0.f, 0.f, 0.f, 0.f}, db1 = db0;
#pragma unroll
      for (int s = 0; s < NS; s += 2) {
        db0 = mfma_16x16x4(feat >= 0 ? wrow[4 * s] : 0.f, ga[s], db0);
        db1 = mfma_16x16x4(feat >= 0 ? wrow[4 * s + 4] : 0.f, ga[s + 1], db1);
      }
      // dB[2 hi + i][lo] for i < 2, rows in LDS for the edges' lanes
      sb[(2 * hi) * 16 + lo] = db0[0] + db1[0];
      sb[(2 * hi + 1) * 16 + lo] = db0[1] + db1[1];
    }
    const G* cl = row_cell(cell, n_graphs, batch, row);
    for (int base = b0; base < b1; base += kWave) {
      const int cnt = min(kWave, b1 - base);
      const int my_e = lane < cnt ? (perm ? perm[base + lane] : base + lane) : 0;
      float ux, uy, uz, inv, len;
      batch_harmonics<G, LMAX>(vec, pos, cl, src, shift, (int)row, sign, lane, cnt, my_e, ys,
                               ux, uy, uz, inv, len);
      RadialCache rcache;
      if constexpr (RAD)
        radial_row(R, tab, lane < cnt, len, hs + lane * kSH, &rcache);
      else
        load_h_row(h, K, lane < cnt, my_e, hs + lane * kSH);
      wave_sync();  // dB and the batch's rows
      if (lane < cnt) {
        // two passes over dB, so that few per-edge arrays are live together: d h_e first
        // (against the harmonics), then dY_e (against the radial row)
        float du[kLinKMax];
        {
          float Y[16];
#pragma unroll
          for (int m = 0; m < 16; ++m) Y[m] = ys[lane * kSY + m];
#pragma unroll
          for (int k = 0; k < kLinKMax; ++k) {
            du[k] = 0.f;
            if (k < K) {
              const float4* bk = reinterpret_cast<const float4*>(sb + k * 16);
#pragma unroll
              for (int q = 0; q < (L + 3) / 4; ++q) {
                const float4 b = bk[q];
                const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                  if (4 * q + j < L) du[k] = fmaf(bv[j], Y[4 * q + j], du[k]);
              }
            }
          }
        }
        float dl = 0.f;
        if constexpr (RAD) {
          dl = radial_dot(R, tab, rcache, du);
        } else {
#pragma unroll
          for (int k = 0; k < kLinKMax; ++k)
            if (k < K) d_h[(int64_t)my_e * K + k] = du[k];
        }
        if (g_vec != nullptr) {
          float dY[16];
#pragma unroll
          for (int m = 0; m < 16; ++m) dY[m] = 0.f;
#pragma unroll
          for (int k = 0; k < kLinKMax; ++k) {
            if (k < K) {
              const float hk = hs[lane * kSH + k];
              const float4* bk = reinterpret_cast<const float4*>(sb + k * 16);
#pragma unroll
              for (int q = 0; q < (L + 3) / 4; ++q) {
                const float4 b = bk[q];
                const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                  if (4 * q + j < L) dY[4 * q + j] = fmaf(hk, bv[j], dY[4 * q + j]);
              }
            }
          }
          float Gx, Gy, Gz, vx, vy, vz;
          sh_grad<LMAX, float>(ux, uy, uz, dY, Gx, Gy, Gz);
          sh_chain<float>(ux, uy, uz, inv, Gx, Gy, Gz, vx, vy, vz);
          if constexpr (RAD) {
            // + d|r| r / |r|, with r / |r| = sign (ux, uy, uz)
            vx += dl * ux;
            vy += dl * uy;
            vz += dl * uz;
          }
          g_vec[3 * (int64_t)my_e + 0] = sign * vx;
          g_vec[3 * (int64_t)my_e + 1] = sign * vy;
          g_vec[3 * (int64_t)my_e + 2] = sign * vz;
        }
      }
      wave_sync();  // the rows are rewritten by the next batch
    }
  }
}

template <typename G, bool RAD>
static void basis_msg_launch(bool backward, const float* vec, const void* pos, int64_t n_nodes,
                             const void* cell, int64_t n_graphs, const int32_t* batch,
                             const int32_t* src, const int32_t* shift, const int32_t* ptr,
                             const int32_t* perm, int l_max, int sign, int K, int C,
                             const float* h, const Radial<float>& R, const float* W,
                             const float* d_out, float* out_or_dh, float* g_vec,
                             hipStream_t stream) {
  const int64_t blocks_needed = grid_1d(n_nodes, kWavesPerBlock);
  const dim3 block(kWavesPerBlock * kWave);
  const float sg = (float)sign;
#define XNN_BASIS(LM, TT)                                                                      \
  do {                                                                                         \
    if (backward) {                                                                            \
      auto k = basis_msg_bwd_kernel<G, LM, TT, RAD>;                                           \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, blocks_needed));      \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, sg, K, h, R, W,       \
                         d_out, out_or_dh, g_vec);                                              \
    } else {                                                                                   \
      auto k = basis_msg_fwd_kernel<G, LM, TT, RAD>;                                           \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, blocks_needed));      \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, sg, K, h, R, W,       \
                         out_or_dh);                                                            \
    }                                                                                          \
  } while (0)
#define XNN_BASIS_L(TT)                   \
  switch (l_max) {                        \
    case 1: XNN_BASIS(1, TT); break;      \
    case 2: XNN_BASIS(2, TT); break;      \
    default: XNN_BASIS(3, TT); break;     \
  }
  switch (C) {
    case 32: XNN_BASIS_L(2); break;
    case 64: XNN_BASIS_L(4); break;
    default: XNN_BASIS_L(8); break;
  }
#undef XNN_BASIS_L
#undef XNN_BASIS
}

// R == nullptr: h is given (E, K); else h is evaluated in the kernels from R (K = R->K).
template <typename G>
static int basis_msg(bool backward, const float* vec, const void* pos, int64_t n_nodes,
                     const void* cell, int64_t n_graphs, const int32_t* batch,
                     const int32_t* src, const int32_t* shift, const int32_t* ptr,
                     const int32_t* perm, int l_max, int sign, int K, int C, const float* h,
                     const Radial<float>* R, const float* W, const float* d_out,
                     float* out_or_dh, float* g_vec, hipStream_t stream) {
  if (n_nodes == 0) return XNN_OK;
  if (R != nullptr)
    basis_msg_launch<G, true>(backward, vec, pos, n_nodes, cell, n_graphs, batch, src, shift,
                              ptr, perm, l_max, sign, R->K, C, nullptr, *R, W, d_out, out_or_dh,
                              g_vec, stream);
  else
    basis_msg_launch<G, false>(backward, vec, pos, n_nodes, cell, n_graphs, batch, src, shift,
                               ptr, perm, l_max, sign, K, C, h, Radial<float>{}, W, d_out,
                               out_or_dh, g_vec, stream);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

static int basis_check(int64_t n_nodes, int64_t n_edges, int32_t l_max, int32_t sh_sign,
                       int32_t K, int32_t C) {
  XNN_REQUIRE(n_nodes >= 0 && n_edges >= 0, "negative size");
  XNN_REQUIRE(l_max >= 1 && l_max <= 3, "l_max must be in [1, 3], got %d", l_max);
  XNN_REQUIRE(sh_sign == 1 || sh_sign == -1, "sh_sign must be +1 or -1");
  XNN_REQUIRE(K >= 1 && K <= kLinKMax, "n_features must be in [1, %d], got %d", kLinKMax, K);
  XNN_REQUIRE(C == 32 || C == 64 || C == 128, "n_channels must be 32, 64 or 128, got %d", C);
  return XNN_OK;
}

}  // namespace xnn

using namespace xnn;

extern "C" {

int xnn_sh_linear_message_sum(int geom_dtype, const float* vec_in, const void* pos,
                              int64_t n_nodes, const void* cell, int64_t n_graphs,
                              const int32_t* batch, const int32_t* src, const int32_t* shift,
                              int64_t n_edges, const int32_t* ptr_dst, const int32_t* perm_dst,
                              int32_t l_max, int32_t sh_sign, int32_t n_features,
                              int32_t n_channels, const float* h, const float* W, float* out,
                              xnn_stream_t stream) {
  const int st = basis_check(n_nodes, n_edges, l_max, sh_sign, n_features, n_channels);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && out && W), "NULL CSR, weights or output");
  XNN_REQUIRE(aligned16(out), "out must be 16-byte aligned");
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && shift)) && h), "NULL edge input");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  if (geom_dtype == XNN_F32)
    return basis_msg<float>(false, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                            ptr_dst, perm_dst, l_max, sh_sign, n_features, n_channels, h, nullptr,
                            W, nullptr, out, nullptr, as_hip(stream));
  if (geom_dtype == XNN_F64)
    return basis_msg<double>(false, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                             ptr_dst, perm_dst, l_max, sh_sign, n_features, n_channels, h,
                             nullptr, W, nullptr, out, nullptr, as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

int xnn_sh_linear_message_sum_backward(int geom_dtype, const float* vec_in, const void* pos,
                                       int64_t n_nodes, const void* cell, int64_t n_graphs,
                                       const int32_t* batch, const int32_t* src,
                                       const int32_t* shift, int64_t n_edges,
                                       const int32_t* ptr_dst, const int32_t* perm_dst,
                                       int32_t l_max, int32_t sh_sign, int32_t n_features,
                                       int32_t n_channels, const float* h, const float* W,
                                       const float* d_out, float* d_h, float* g_vec,
                                       xnn_stream_t stream) {
  const int st = basis_check(n_nodes, n_edges, l_max, sh_sign, n_features, n_channels);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && d_out && W), "NULL CSR, weights or d_out");
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && shift)) && d_h && h),
              "NULL edge input or output");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  if (geom_dtype == XNN_F32)
    return basis_msg<float>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                            ptr_dst, perm_dst, l_max, sh_sign, n_features, n_channels, h, nullptr,
                            W, d_out, d_h, g_vec, as_hip(stream));
  if (geom_dtype == XNN_F64)
    return basis_msg<double>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                             ptr_dst, perm_dst, l_max, sh_sign, n_features, n_channels, h,
                             nullptr, W, d_out, d_h, g_vec, as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

int xnn_sh_radial_message_sum(int geom_dtype, const float* vec_in, const void* pos,
                              int64_t n_nodes, const void* cell, int64_t n_graphs,
                              const int32_t* batch, const int32_t* src, const int32_t* shift,
                              int64_t n_edges, const int32_t* ptr_dst, const int32_t* perm_dst,
                              const xnn_featurize_params* prm, const float* rbf_table,
                              int32_t n_channels, const float* W, float* out,
                              xnn_stream_t stream) {
  Radial<float> R;
  int st = make_radial<float>(prm, rbf_table, R);
  if (st != XNN_OK) return st;
  st = basis_check(n_nodes, n_edges, prm->l_max, prm->sh_sign, prm->n_rbf, n_channels);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && out && W), "NULL CSR, weights or output");
  XNN_REQUIRE(aligned16(out), "out must be 16-byte aligned");
  XNN_REQUIRE(n_edges == 0 || vec_in || (pos && src && shift), "NULL edge input");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  if (geom_dtype == XNN_F32)
    return basis_msg<float>(false, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                            ptr_dst, perm_dst, prm->l_max, prm->sh_sign, R.K, n_channels, nullptr,
                            &R, W, nullptr, out, nullptr, as_hip(stream));
  if (geom_dtype == XNN_F64)
    return basis_msg<double>(false, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                             ptr_dst, perm_dst, prm->l_max, prm->sh_sign, R.K, n_channels,
                             nullptr, &R, W, nullptr, out, nullptr, as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

int xnn_sh_radial_message_sum_backward(int geom_dtype, const float* vec_in, const void* pos,
                                       int64_t n_nodes, const void* cell, int64_t n_graphs,
                                       const int32_t* batch, const int32_t* src,
                                       const int32_t* shift, int64_t n_edges,
                                       const int32_t* ptr_dst, const int32_t* perm_dst,
                                       const xnn_featurize_params* prm, const float* rbf_table,
                                       int32_t n_channels, const float* W, const float* d_out,
                                       float* g_vec, xnn_stream_t stream) {
  Radial<float> R;
  int st = make_radial<float>(prm, rbf_table, R);
  if (st != XNN_OK) return st;
  st = basis_check(n_nodes, n_edges, prm->l_max, prm->sh_sign, prm->n_rbf, n_channels);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && d_out && W), "NULL CSR, weights or d_out");
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && shift)) && g_vec),
              "NULL edge input or output");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  if (geom_dtype == XNN_F32)
    return basis_msg<float>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                            ptr_dst, perm_dst, prm->l_max, prm->sh_sign, R.K, n_channels, nullptr,
                            &R, W, d_out, nullptr, g_vec, as_hip(stream));
  if (geom_dtype == XNN_F64)
    return basis_msg<double>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                             ptr_dst, perm_dst, prm->l_max, prm->sh_sign, R.K, n_channels,
                             nullptr, &R, W, d_out, nullptr, g_vec, as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

}  // extern "C"
