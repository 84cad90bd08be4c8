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

// The lane's edge features in registers: unit vector, 1/|r|, |r|, the harmonics (zeros past
// L) and the feature row (zeros past K): the enveloped radial basis evaluated from R (RAD,
// with the state its derivative reuses) or the given row h_e (NULL h: zeros).
template <typename G, int LMAX, bool RAD = true>
__device__ __forceinline__ void edge_features(const float* __restrict__ vec, int64_t e,
                                              const G* __restrict__ pos, const G* __restrict__ cl,
                                              const int32_t* __restrict__ src,
                                              const int32_t* __restrict__ shift, int row,
                                              float sign, const Radial<float>& R,
                                              const RadialTab& tab, float& ux, float& uy,
                                              float& uz, float& inv, float& len, float* Y,
                                              float* hk, RadialCache& rc,
                                              const float* __restrict__ h = nullptr, int K = 0) {
  constexpr int L = ShDims<LMAX>::L;
  edge_unit(vec, e, pos, cl, src, shift, row, sign, ux, uy, uz, inv, len);
  sh_eval<LMAX, float>(ux, uy, uz, Y);
#pragma unroll
  for (int m = L; m < 16; ++m) Y[m] = 0.f;
  if constexpr (RAD)
    radial_row(R, tab, true, len, hk, &rc);
  else
    load_h_row(h, K, h != nullptr, e, hk);
}

// d_h (given h, !RAD): the feature rows' gradient (E, K); g_vec (may be NULL when only d_h
// is wanted): the edge vectors' gradient (E, 3), through the harmonics and (RAD) the
// radial row. Each lane keeps its own edge's features in registers (no other lane reads
// them), so LDS holds only dB and W, and 5 waves per SIMD fit (96 VGPRs, no spills; at 6
// the compiler spills and the kernel is slower).
template <typename G, int LMAX, int T, bool RAD>
__global__ __launch_bounds__(256, 5) void basis_msg_bwd_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, float sign, int K,
    const float* __restrict__ h, Radial<float> R, const float* __restrict__ W,
    const float* __restrict__ d_out, float* __restrict__ d_h, float* __restrict__ g_vec) {
  constexpr int L = ShDims<LMAX>::L;
  constexpr int C = 16 * T;
  constexpr int NS = C / 4;  // k-steps of dB = W G over the channels
  __shared__ __align__(16) float sB[kWavesPerBlock][kLinKMax * 16];
  __shared__ float sTab[kLinKMax];
  // W in LDS, rows padded to C + 4 floats: the A operand of dB = W G at k-step s is
  // W[feature of M row lo][channel 4 s + hi] (32 distinct banks for the 8 x 4 addresses)
  constexpr int SWS = C + 4;
  __shared__ float sW[kLinKMax * SWS];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int lo = lane & 15, hi = lane >> 4;
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
    wave_sync();  // dB
    // every lane works on its own edge: features in registers, dB read from LDS
    for (int base = b0; base < b1; base += kWave) {
      if (lane < b1 - base) {
        const int64_t my_e = perm ? perm[base + lane] : base + lane;
        float ux, uy, uz, inv, len, Y[16], hk[kLinKMax];
        RadialCache rcache;
        edge_features<G, LMAX, RAD>(vec, my_e, pos, cl, src, shift, (int)row, sign, R, tab, ux,
                                    uy, uz, inv, len, Y, hk, rcache, h, K);
        // two passes over dB, so that few per-edge arrays are live together: d h_e first
        // (against the harmonics), then dY_e (against the radial row)
        float du[kLinKMax];
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
        float dl = 0.f;
        if constexpr (RAD) {
          dl = radial_dot(R, tab, rcache, du);
        } else {
#pragma unroll
          for (int k = 0; k < kLinKMax; ++k)
            if (k < K) d_h[my_e * K + k] = du[k];
        }
        if (g_vec != nullptr) {
          float dY[16];
#pragma unroll
          for (int m = 0; m < 16; ++m) dY[m] = 0.f;
#pragma unroll
          for (int k = 0; k < kLinKMax; ++k) {
            if (k < K) {
              const float4* bk = reinterpret_cast<const float4*>(sb + k * 16);
#pragma unroll
              for (int q = 0; q < (L + 3) / 4; ++q) {
                const float4 b = bk[q];
                const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                  if (4 * q + j < L) dY[4 * q + j] = fmaf(hk[k], bv[j], dY[4 * q + j]);
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

// ------------------------------------------------------------------ the readout in the kernels
// With a linear readout of the rows, E_i = <U, A_i> + bias[z_i], the same reassociation
// gives E_i = sum_{dst(e)=i} h_e^T P Y_e + bias[z_i] with P = W U (K x L, formed once per
// block): each edge's share of its receiver's energy is a K x L bilinear form, and its
// gradient for a cotangent g_i of E_i is g_i (P Y_e, P^T h_e) in (d h_e, dY_e). No (C, L)
// work remains per edge or per atom.

// P = W U into LDS rows of 16 doubles (zeros past K and L), two threads per element, the
// halves' sums added in a fixed order: every block forms the same P. P is kept in float64:
// one rounding of P to float32 would enter every edge's share alike, and those errors add
// up coherently over all the edges of a structure (at 72k edges past 1e-6 of the energy).
// On gfx950 a float64 FMA issues at the rate of an unpacked float32 one.
__device__ __forceinline__ void form_readout_product(const float* __restrict__ W,
                                                     const float* __restrict__ U, int K, int C,
                                                     int L, double* __restrict__ sP) {
  const int t = threadIdx.x;  // blockDim.x = 256 = 2 x 8 x 16
  const int i = t >> 1, half = t & 1;
  const int k = i >> 4, lm = i & 15;
  double p = 0.0;
  if (k < K && lm < L) {
    const int c0 = half * (C / 2), c1 = c0 + C / 2;
    for (int c = c0; c < c1; ++c) p = fma((double)W[k * C + c], (double)U[c * L + lm], p);
  }
  p += __shfl_xor(p, 1);
  if (half == 0) sP[i] = p;
}

// The per-edge contractions against P's rows in LDS (k < K): dk[k] = P[k] . Y in float64
// (the edge's energy share is h . dk) and (when DY) dY[lm] = sum_k h[k] P[k][lm] in float32
// (a gradient: a systematic relative error of P's rounding, 6e-8, is far below its bar),
// both in one pass over P.
template <int L, bool DY>
__device__ __forceinline__ void contract_rows(const double* __restrict__ M, int K,
                                              const float* Y, const float* h, double* dk,
                                              float* dY) {
  if constexpr (DY) {
#pragma unroll
    for (int m = 0; m < 16; ++m) dY[m] = 0.f;
  }
#pragma unroll
  for (int k = 0; k < kLinKMax; ++k) {
    dk[k] = 0.0;
    if (k < K) {
      const double2* mk = reinterpret_cast<const double2*>(M + k * 16);
#pragma unroll
      for (int q = 0; q < (L + 1) / 2; ++q) {
        const double2 b = mk[q];
        const double bv[2] = {b.x, b.y};
#pragma unroll
        for (int j = 0; j < 2; ++j)
          if (2 * q + j < L) {
            dk[k] = fma(bv[j], (double)Y[2 * q + j], dk[k]);
            if constexpr (DY) dY[2 * q + j] = fmaf(h[k], (float)bv[j], dY[2 * q + j]);
          }
      }
    }
  }
}

// Node energies: a wave per receiver row, each lane's shares summed over the row's batches,
// then across the wave by a fixed butterfly.
template <typename G, int LMAX>
__global__ __launch_bounds__(256) void basis_energy_fwd_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, float sign, Radial<float> R,
    const float* __restrict__ W, const float* __restrict__ U, int C,
    const int64_t* __restrict__ z, const float* __restrict__ bias, int64_t n_bias,
    float* __restrict__ out) {
  constexpr int L = ShDims<LMAX>::L;
  __shared__ __align__(16) double sP[kLinKMax * 16];
  __shared__ float sTab[kLinKMax];
  const int lane = threadIdx.x % kWave;
  const RadialTab tab = load_radial_tab(R, sTab);
  form_readout_product(W, U, R.K, C, L, sP);
  __syncthreads();
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave_in_block(); row < n_nodes;
       row += n_waves) {
    // P is read from LDS where it is used: hoisted out of the loop, its 128 values would
    // take registers for the whole kernel
    asm volatile("" ::: "memory");
    const G* cl = row_cell(cell, n_graphs, batch, row);
    double part = 0.0;
    const int b0 = ptr[row], b1 = ptr[row + 1];
    for (int base = b0; base < b1; base += kWave) {
      asm volatile("" ::: "memory");
      if (lane < b1 - base) {
        const int64_t e = perm ? perm[base + lane] : base + lane;
        float ux, uy, uz, inv, len, Y[16], hk[kLinKMax];
        double dk[kLinKMax];
        RadialCache rc;
        edge_features<G, LMAX>(vec, e, pos, cl, src, shift, (int)row, sign, R, tab, ux, uy, uz,
                               inv, len, Y, hk, rc);
        contract_rows<L, false>(sP, R.K, Y, hk, dk, nullptr);
#pragma unroll
        for (int k = 0; k < kLinKMax; ++k) part = fma((double)hk[k], dk[k], part);
      }
    }
    part = group_sum<kWave>(part);
    if (lane == 0) {
      float b = 0.f;
      if (bias != nullptr) {
        const int64_t zz = z[row];
        b = (zz >= 0 && zz < n_bias) ? bias[zz] : __builtin_nanf("");
      }
      out[row] = (float)part + b;
    }
  }
}

// Edge-vector gradients for the cotangent g of the node energies (and, EE, each edge's
// unscaled share of its receiver's energy): a wave takes 64 consecutive CSR slots, whatever
// rows they belong to; each lane finds its receiver when it needs the receiver's cotangent
// or geometry.
template <typename G, int LMAX, bool EE>
__global__ __launch_bounds__(256) void basis_energy_bwd_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, float sign, Radial<float> R,
    const float* __restrict__ W, const float* __restrict__ U, int C,
    const float* __restrict__ g, int64_t g_stride, float* __restrict__ g_vec,
    float* __restrict__ edge_energy) {
  constexpr int L = ShDims<LMAX>::L;
  __shared__ __align__(16) double sP[kLinKMax * 16];
  __shared__ float sTab[kLinKMax];
  const int lane = threadIdx.x % kWave;
  const RadialTab tab = load_radial_tab(R, sTab);
  form_readout_product(W, U, R.K, C, L, sP);
  __syncthreads();
  const int64_t n_slots = ptr[n_nodes];
  const int64_t n_items = (n_slots + kWave - 1) / kWave;
  const bool need_row = g_stride != 0 || vec == nullptr;
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t item = (int64_t)blockIdx.x * kWavesPerBlock + wave_in_block(); item < n_items;
       item += n_waves) {
    asm volatile("" ::: "memory");  // P stays in LDS (see the forward)
    const int64_t b0 = item * kWave;
    const int64_t slot = b0 + lane;
    int64_t row = 0;
    if (need_row) {
      // the receiver of the item's first slot (binary search, uniform), then each lane
      // steps to its own (64 slots span a few rows)
      int64_t lo_r = 0, hi_r = n_nodes;  // ptr[lo_r] <= b0 < ptr[hi_r]
      while (hi_r - lo_r > 1) {
        const int64_t mid = (lo_r + hi_r) >> 1;
        if (ptr[mid] <= b0) lo_r = mid; else hi_r = mid;
      }
      row = lo_r;
      const int64_t q = min(slot, n_slots - 1);
      while (row + 1 < n_nodes && ptr[row + 1] <= q) ++row;
    }
    if (slot < n_slots) {
      const int64_t e = perm ? perm[slot] : slot;
      const G* cl = row_cell(cell, n_graphs, batch, row);
      float ux, uy, uz, inv, len, Y[16], hk[kLinKMax];
      double dkd[kLinKMax];
      float dY[16];
      RadialCache rc;
      edge_features<G, LMAX>(vec, e, pos, cl, src, shift, (int)row, sign, R, tab, ux, uy, uz,
                             inv, len, Y, hk, rc);
      contract_rows<L, true>(sP, R.K, Y, hk, dkd, dY);
      if constexpr (EE) {
        double se = 0.0;
#pragma unroll
        for (int k = 0; k < kLinKMax; ++k) se = fma((double)hk[k], dkd[k], se);
        edge_energy[e] = (float)se;
      }
      float dk[kLinKMax];
#pragma unroll
      for (int k = 0; k < kLinKMax; ++k) dk[k] = (float)dkd[k];
      const float dl = radial_dot(R, tab, rc, dk);
      float Gx, Gy, Gz, vx, vy, vz;
      sh_grad<LMAX, float>(ux, uy, uz, dY, Gx, Gy, Gz);
      sh_chain<float>(ux, uy, uz, inv, Gx, Gy, Gz, vx, vy, vz);
      // + d|r| r / |r|, with r / |r| = sign (ux, uy, uz); everything is linear in g_i
      const float gs = g[row * g_stride];
      g_vec[3 * e + 0] = gs * (sign * (vx + dl * ux));
      g_vec[3 * e + 1] = gs * (sign * (vy + dl * uy));
      g_vec[3 * e + 2] = gs * (sign * (vz + dl * uz));
    }
  }
}

// The readout arguments of the energy kernels
struct Readout {
  const float* U = nullptr;      // (C, L)
  const int64_t* z = nullptr;    // forward: per-atom bias index
  const float* bias = nullptr;   // forward: per-index bias (may be NULL)
  int64_t n_bias = 0;
  const float* g = nullptr;      // backward: per-atom cotangent of E_i
  int64_t g_stride = 1;
  float* edge_energy = nullptr;  // backward: each edge's share of its receiver's energy
};

// mode 0: node energies; 1: edge-vector gradients; 2: gradients and the edges' shares
template <typename G>
static int basis_energy(int mode, const float* vec, const void* pos, int64_t n_nodes,
                        const void* cell, int64_t n_graphs, const int32_t* batch,
                        const int32_t* src, const int32_t* shift, const int32_t* ptr,
                        const int32_t* perm, int l_max, int sign, int C, const Radial<float>& R,
                        const float* W, float* out, float* g_vec, const Readout& ro,
                        int64_t n_edges, hipStream_t stream) {
  if (n_nodes == 0 || (mode != 0 && n_edges == 0)) return XNN_OK;
  const dim3 block(kWavesPerBlock * kWave);
  const float sg = (float)sign;
  const int64_t needed = mode == 0 ? grid_1d(n_nodes, kWavesPerBlock)
                                   : grid_1d((n_edges + kWave - 1) / kWave, kWavesPerBlock);
#define XNN_ENERGY(LM)                                                                         \
  do {                                                                                         \
    if (mode == 0) {                                                                           \
      auto k = basis_energy_fwd_kernel<G, LM>;                                                 \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, needed));             \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, sg, R, W, ro.U, C,    \
                         ro.z, ro.bias, ro.n_bias, out);                                        \
    } else if (mode == 1) {                                                                    \
      auto k = basis_energy_bwd_kernel<G, LM, false>;                                          \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, needed));             \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, sg, R, W, ro.U, C,    \
                         ro.g, ro.g_stride, g_vec, nullptr);                                    \
    } else {                                                                                   \
      auto k = basis_energy_bwd_kernel<G, LM, true>;                                           \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, needed));             \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, sg, R, W, ro.U, C,    \
                         ro.g, ro.g_stride, g_vec, ro.edge_energy);                             \
    }                                                                                          \
  } while (0)
  switch (l_max) {
    case 1: XNN_ENERGY(1); break;
    case 2: XNN_ENERGY(2); break;
    default: XNN_ENERGY(3); break;
  }
#undef XNN_ENERGY
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
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && shift)) && d_h && (h || !g_vec)),
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

int xnn_sh_radial_message_energy(int geom_dtype, const float* vec_in, const void* pos,
                                 int64_t n_nodes, const void* cell, int64_t n_graphs,
                                 const int32_t* batch, const int32_t* src, const int32_t* shift,
                                 int64_t n_edges, const int32_t* ptr_dst, const int32_t* perm_dst,
                                 const xnn_featurize_params* prm, const float* rbf_table,
                                 int32_t n_channels, const float* W, const float* U,
                                 const int64_t* z, const float* bias, int64_t n_bias,
                                 float* node_energy, xnn_stream_t stream) {
  Radial<float> R;
  int st = make_radial<float>(prm, rbf_table, R);
  if (st != XNN_OK) return st;
  st = basis_check(n_nodes, n_edges, prm->l_max, prm->sh_sign, prm->n_rbf, n_channels);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && node_energy && W && U), "NULL CSR, weights or output");
  XNN_REQUIRE(bias == nullptr || (z != nullptr && n_bias > 0), "bias needs z and n_bias > 0");
  XNN_REQUIRE(n_edges == 0 || vec_in || (pos && src && shift), "NULL edge input");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  Readout ro;
  ro.U = U;
  ro.z = z;
  ro.bias = bias;
  ro.n_bias = n_bias;
  if (geom_dtype == XNN_F32)
    return basis_energy<float>(0, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                               ptr_dst, perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W,
                               node_energy, nullptr, ro, n_edges, as_hip(stream));
  if (geom_dtype == XNN_F64)
    return basis_energy<double>(0, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                                ptr_dst, perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W,
                                node_energy, nullptr, ro, n_edges, as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

static int energy_backward_entry(int mode, int geom_dtype, const float* vec_in,
                                 const void* pos, int64_t n_nodes, const void* cell,
                                 int64_t n_graphs, const int32_t* batch, const int32_t* src,
                                 const int32_t* shift, int64_t n_edges, const int32_t* ptr_dst,
                                 const int32_t* perm_dst, const xnn_featurize_params* prm,
                                 const float* rbf_table, int32_t n_channels, const float* W,
                                 const float* U, const float* g, int64_t g_stride, float* g_vec,
                                 float* edge_energy, xnn_stream_t stream) {
  Radial<float> R;
  int st = make_radial<float>(prm, rbf_table, R);
  if (st != XNN_OK) return st;
  st = basis_check(n_nodes, n_edges, prm->l_max, prm->sh_sign, prm->n_rbf, n_channels);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && g && W && U), "NULL CSR, weights or cotangent");
  XNN_REQUIRE(g_stride == 0 || g_stride == 1, "g_stride must be 0 (broadcast) or 1");
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && shift)) && g_vec &&
                               (mode == 1 || edge_energy)),
              "NULL edge input or output");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  Readout ro;
  ro.U = U;
  ro.g = g;
  ro.g_stride = g_stride;
  ro.edge_energy = edge_energy;
  if (geom_dtype == XNN_F32)
    return basis_energy<float>(mode, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                               ptr_dst, perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W,
                               nullptr, g_vec, ro, n_edges, as_hip(stream));
  if (geom_dtype == XNN_F64)
    return basis_energy<double>(mode, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                                ptr_dst, perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W,
                                nullptr, g_vec, ro, n_edges, as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

int xnn_sh_radial_message_energy_backward(int geom_dtype, const float* vec_in, const void* pos,
                                          int64_t n_nodes, const void* cell, int64_t n_graphs,
                                          const int32_t* batch, const int32_t* src,
                                          const int32_t* shift, int64_t n_edges,
                                          const int32_t* ptr_dst, const int32_t* perm_dst,
                                          const xnn_featurize_params* prm,
                                          const float* rbf_table, int32_t n_channels,
                                          const float* W, const float* U, const float* g,
                                          int64_t g_stride, float* g_vec, xnn_stream_t stream) {
  return energy_backward_entry(1, geom_dtype, vec_in, pos, n_nodes, cell, n_graphs, batch, src,
                               shift, n_edges, ptr_dst, perm_dst, prm, rbf_table, n_channels, W,
                               U, g, g_stride, g_vec, nullptr, stream);
}

int xnn_sh_radial_message_energy_forces(int geom_dtype, const float* vec_in, const void* pos,
                                        int64_t n_nodes, const void* cell, int64_t n_graphs,
                                        const int32_t* batch, const int32_t* src,
                                        const int32_t* shift, int64_t n_edges,
                                        const int32_t* ptr_dst, const int32_t* perm_dst,
                                        const xnn_featurize_params* prm,
                                        const float* rbf_table, int32_t n_channels,
                                        const float* W, const float* U, const float* g,
                                        int64_t g_stride, float* g_vec, float* edge_energy,
                                        xnn_stream_t stream) {
  return energy_backward_entry(2, geom_dtype, vec_in, pos, n_nodes, cell, n_graphs, batch, src,
                               shift, n_edges, ptr_dst, perm_dst, prm, rbf_table, n_channels, W,
                               U, g, g_stride, g_vec, edge_energy, stream);
}

}  // extern "C"
