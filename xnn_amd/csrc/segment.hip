// Receiver-CSR segmented reductions (gfx950, wave64), all deterministic:
// every output is summed by one wave in a fixed order, no float atomics.
//
// xnn_sh_message_sum(_backward)  gnn/fast/conv.py:137-143 (uvu TP of scalar weights with Y)
//                                + scatter_sum (common/models/ops.py:403-448), fused: the
//                                message phi[e,c] Y_lm(e) never leaves registers
// xnn_segment_sum / gather_rows  scatter_sum / gather_rows (ops.py:403-448, 494-528)
// xnn_segment_reduce_f64         structure_sum(s) (ops.py:531-569), fp64 accumulation
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <mutex>

#include "common.h"
#include "device.h"
#include "message.h"

namespace xnn {

// CPL consecutive channels of one phi row starting at c0 (vector loads when aligned)
template <int CPL, bool VEC>
__device__ inline void load_channels(const float* __restrict__ row, int c0, int C, float* p) {
  if constexpr (VEC && CPL == 4) {
    const float4 v = *reinterpret_cast<const float4*>(row + c0);
    p[0] = v.x; p[1] = v.y; p[2] = v.z; p[3] = v.w;
  } else if constexpr (VEC && CPL == 2) {
    const float2 v = *reinterpret_cast<const float2*>(row + c0);
    p[0] = v.x; p[1] = v.y;
  } else {
#pragma unroll
    for (int q = 0; q < CPL; ++q) p[q] = (c0 + q < C) ? row[c0 + q] : 0.f;
  }
}

template <int CPL, bool VEC>
__device__ inline void store_channels(float* __restrict__ row, int c0, int C, const float* p) {
  if constexpr (VEC && CPL == 4) {
    *reinterpret_cast<float4*>(row + c0) = make_float4(p[0], p[1], p[2], p[3]);
  } else if constexpr (VEC && CPL == 2) {
    *reinterpret_cast<float2*>(row + c0) = make_float2(p[0], p[1]);
  } else {
#pragma unroll
    for (int q = 0; q < CPL; ++q)
      if (c0 + q < C) row[c0 + q] = p[q];
  }
}

// One wave per receiver row. Lane l owns channels [l*CPL, l*CPL+CPL). Edges are
// processed in batches of 64: lane j evaluates Y for edge j of the batch and parks it
// in LDS (zeros past the row's end), then the whole wave streams the phi rows of the
// batch, kUnroll edges at a time with all their loads in flight (coalesced, one
// contiguous row segment per edge), and accumulates phi[e, c] * Y[e, lm] in registers.
template <typename G, int LMAX, int CPL, bool VEC>
__global__ __launch_bounds__(256) void sh_msg_fwd_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, int C, float sign,
    const float* __restrict__ phi, float* __restrict__ out) {
  constexpr int L = ShDims<LMAX>::L;
  constexpr int kU = 8;  // edges per load group; two groups are in flight
  __shared__ float sY[kWavesPerBlock][kWave][L];
  __shared__ int sE[kWavesPerBlock][kWave];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int c0 = lane * CPL;
  const bool own = c0 < C;
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  // persistent waves: rows are dealt out round robin, so no wave idles at the tail
  for (int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave; row < n_nodes; row += n_waves) {
    const G* cl = cell == nullptr ? nullptr
                                  : (n_graphs <= 1 || batch == nullptr ? cell
                                                                       : cell + 9 * (int64_t)batch[row]);
    float acc[CPL][L];
#pragma unroll
    for (int q = 0; q < CPL; ++q)
#pragma unroll
      for (int k = 0; k < L; ++k) acc[q][k] = 0.f;

    const int b0 = ptr[row], b1 = ptr[row + 1];
    for (int base = b0; base < b1; base += kWave) {
      const int cnt = min(kWave, b1 - base);
      float Y[L];
      int e = -1;
      if (lane < cnt) {
        const int k = base + lane;
        e = perm ? perm[k] : k;
        float ux, uy, uz, inv, len;
        edge_unit(vec, e, pos, cl, src, shift, (int)row, sign, ux, uy, uz, inv, len);
        sh_eval<LMAX, float>(ux, uy, uz, Y);
      } else {
#pragma unroll
        for (int m = 0; m < L; ++m) Y[m] = 0.f;
      }
#pragma unroll
      for (int m = 0; m < L; ++m) sY[wave][lane][m] = Y[m];
      sE[wave][lane] = e;
      wave_sync();
      if (own) {
        float p[kU][CPL], pn[kU][CPL];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          if (u < cnt)
            load_channels<CPL, VEC>(phi + (int64_t)sE[wave][u] * C, c0, C, pn[u]);
          else
#pragma unroll
            for (int q = 0; q < CPL; ++q) pn[u][q] = 0.f;
        }
        for (int j = 0; j < cnt; j += kU) {
#pragma unroll
          for (int u = 0; u < kU; ++u)
#pragma unroll
            for (int q = 0; q < CPL; ++q) p[u][q] = pn[u][q];
          // the next group's loads go out before this group's arithmetic
#pragma unroll
          for (int u = 0; u < kU; ++u) {
            const int t = j + kU + u;
            if (t < cnt)
              load_channels<CPL, VEC>(phi + (int64_t)sE[wave][t] * C, c0, C, pn[u]);
            else
#pragma unroll
              for (int q = 0; q < CPL; ++q) pn[u][q] = 0.f;
          }
#pragma unroll
          for (int u = 0; u < kU; ++u) {
            if (j + u >= kWave) break;
#pragma unroll
            for (int m = 0; m < L; ++m) {
              const float y = sY[wave][j + u][m];
#pragma unroll
              for (int q = 0; q < CPL; ++q) acc[q][m] += p[u][q] * y;
            }
          }
        }
      }
      wave_sync();
    }
    if (own) {
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        if (c0 + q >= C) break;
        float* o = out + ((int64_t)row * C + c0 + q) * L;
        if constexpr (L % 4 == 0) {
#pragma unroll
          for (int m = 0; m < L; m += 4)
            *reinterpret_cast<float4*>(o + m) =
                make_float4(acc[q][m], acc[q][m + 1], acc[q][m + 2], acc[q][m + 3]);
        } else {
#pragma unroll
          for (int m = 0; m < L; ++m) o[m] = acc[q][m];
        }
      }
    }
  }
}

// Sum of p[0..64) over the 64 lanes of a wave; lane l returns the total of entry l.
// Six halving steps, one per lane bit from the top: at the step of width HALF every
// lane keeps the half of its live entries selected by that bit and adds the partner's
// copy of the same half. Cross-row steps (bits 5 and 4) use v_permlane32_swap /
// v_permlane16_swap, which exchange the odd rows of one register with the even rows of
// another, so keep + received is a plain sum of the two swapped registers. In-row steps
// use DPP lane maps that flip the step's bit: row_mirror (l ^ 15), row_half_mirror
// (l ^ 7), quad_perm xor 2 and xor 1. Together they pair every lane with every other
// exactly once (63 exchanges for 64 totals, all independent within a step). Template
// recursion keeps every index a compile-time constant, so p stays in registers.
template <int HALF>
__device__ __forceinline__ void halving_step(float* p, int lane) {
  if constexpr (HALF == 32 || HALF == 16) {
#pragma unroll
    for (int k = 0; k < HALF; ++k) {
      const unsigned a = __float_as_uint(p[k]), b = __float_as_uint(p[k + HALF]);
      unsigned lo, hi;
      if constexpr (HALF == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
        lo = r[0];
        hi = r[1];
      } else {
        const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
        lo = r[0];
        hi = r[1];
      }
      p[k] = __uint_as_float(lo) + __uint_as_float(hi);
    }
  } else {
    // DPP controls whose lane map flips bit HALF (and only lower bits)
    constexpr int ctrl = HALF == 8 ? 0x140 : (HALF == 4 ? 0x141 : (HALF == 2 ? 0x4E : 0xB1));
    const bool upper = (lane & HALF) != 0;
#pragma unroll
    for (int k = 0; k < HALF; ++k) {
      const float keep = upper ? p[k + HALF] : p[k];
      const float send = upper ? p[k] : p[k + HALF];
      p[k] = keep + __uint_as_float(__builtin_amdgcn_update_dpp(
                        0u, __float_as_uint(send), ctrl, 0xF, 0xF, false));
    }
  }
  if constexpr (HALF > 1) halving_step<HALF / 2>(p, lane);
}

__device__ __forceinline__ float wave_transpose_reduce64(float* p, int lane) {
  halving_step<32>(p, lane);
  return p[0];
}

// Backward, one wave per receiver row: d_phi[e, c] = sum_lm d_out[i, c, lm] Y_lm(e)
// (channel-owned lanes, no reduction) and dY[e, lm] = sum_c d_out[i, c, lm] phi[e, c]
// (a reduction over channels, i.e. across lanes). Edges go in groups of GE = 64 / LP:
// their partial sums fill 64 registers that one transpose-reduction turns into one
// (edge, lm) total per lane, parked in LDS; lane j then chains dY of edge j through
// the SH Jacobian to g_vec.
template <typename G, int LMAX, int CPL, bool VEC>
__global__ __launch_bounds__(256) void sh_msg_bwd_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, int C, float sign,
    const float* __restrict__ phi, const float* __restrict__ d_out, float* __restrict__ d_phi,
    float* __restrict__ g_vec) {
  using D = ShDims<LMAX>;
  constexpr int L = D::L;
  constexpr int LP = D::LP;
  constexpr int GE = kWave / LP;            // edges per reduction group
  constexpr int kSub = GE < 4 ? GE : 4;     // edges per load group
  __shared__ float sY[kWavesPerBlock][kWave][L];
  __shared__ float sdY[kWavesPerBlock][kWave][LP];
  __shared__ int sE[kWavesPerBlock][kWave];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int c0 = lane * CPL;
  const bool own = c0 < C;
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave; row < n_nodes; row += n_waves) {
    const G* cl = cell == nullptr ? nullptr
                                  : (n_graphs <= 1 || batch == nullptr ? cell
                                                                       : cell + 9 * (int64_t)batch[row]);
    float g[CPL][L];
#pragma unroll
    for (int q = 0; q < CPL; ++q)
#pragma unroll
      for (int m = 0; m < L; ++m)
        g[q][m] = (own && c0 + q < C) ? d_out[((int64_t)row * C + c0 + q) * L + m] : 0.f;

    const int b0 = ptr[row], b1 = ptr[row + 1];
    for (int base = b0; base < b1; base += kWave) {
      const int cnt = min(kWave, b1 - base);
      float ux = 0.f, uy = 0.f, uz = 0.f, inv = 0.f, len = 0.f;
      int my_e = -1;
      float Y[L];
      if (lane < cnt) {
        const int k = base + lane;
        my_e = perm ? perm[k] : k;
        edge_unit(vec, my_e, pos, cl, src, shift, (int)row, sign, ux, uy, uz, inv, len);
        sh_eval<LMAX, float>(ux, uy, uz, Y);
      } else {
#pragma unroll
        for (int m = 0; m < L; ++m) Y[m] = 0.f;
      }
#pragma unroll
      for (int m = 0; m < L; ++m) sY[wave][lane][m] = Y[m];
      sE[wave][lane] = my_e;
      wave_sync();
      float pn[kSub][CPL];
#pragma unroll
      for (int u = 0; u < kSub; ++u) {
        if (own && u < cnt)
          load_channels<CPL, VEC>(phi + (int64_t)sE[wave][u] * C, c0, C, pn[u]);
        else
#pragma unroll
          for (int q = 0; q < CPL; ++q) pn[u][q] = 0.f;
      }
      for (int j = 0; j < cnt; j += GE) {
        float part[kWave];
#pragma unroll
        for (int u0 = 0; u0 < GE; u0 += kSub) {
          float p[kSub][CPL];
#pragma unroll
          for (int u = 0; u < kSub; ++u)
#pragma unroll
            for (int q = 0; q < CPL; ++q) p[u][q] = pn[u][q];
          // prefetch the next load group (in this reduction group or the next)
#pragma unroll
          for (int u = 0; u < kSub; ++u) {
            const int t = j + u0 + kSub + u;
            if (own && t < cnt)
              load_channels<CPL, VEC>(phi + (int64_t)sE[wave][t] * C, c0, C, pn[u]);
            else
#pragma unroll
              for (int q = 0; q < CPL; ++q) pn[u][q] = 0.f;
          }
#pragma unroll
          for (int u = 0; u < kSub; ++u) {
            float dp[CPL];
#pragma unroll
            for (int q = 0; q < CPL; ++q) dp[q] = 0.f;
#pragma unroll
            for (int m = 0; m < LP; ++m) {
              float acc = 0.f;
              if (m < L) {
                const float y = sY[wave][j + u0 + u][m];
#pragma unroll
                for (int q = 0; q < CPL; ++q) {
                  dp[q] += g[q][m] * y;
                  acc += g[q][m] * p[u][q];
                }
              }
              part[(u0 + u) * LP + m] = acc;
            }
            if (own && j + u0 + u < cnt)
              store_channels<CPL, VEC>(d_phi + (int64_t)sE[wave][j + u0 + u] * C, c0, C, dp);
          }
        }
        if (g_vec) {
          const float tot = wave_transpose_reduce64(part, lane);
          sdY[wave][j + lane / LP][lane % LP] = tot;
        }
      }
      wave_sync();
      if (g_vec && lane < cnt) {
        float dY[L];
#pragma unroll
        for (int m = 0; m < L; ++m) dY[m] = sdY[wave][lane][m];
        float Gx, Gy, Gz, vx, vy, vz;
        sh_grad<LMAX, float>(ux, uy, uz, dY, Gx, Gy, Gz);
        sh_chain<float>(ux, uy, uz, inv, Gx, Gy, Gz, vx, vy, vz);
        g_vec[3 * (int64_t)my_e + 0] = sign * vx;
        g_vec[3 * (int64_t)my_e + 1] = sign * vy;
        g_vec[3 * (int64_t)my_e + 2] = sign * vz;
      }
      wave_sync();
    }
  }
}

// ---------------------------------------------------------------- matrix-core message kernels
// Per receiver row both message contractions are small matrix products:
//   forward   A_i^T (L x C)  = Y_i^T (L x E_i) . phi_i (E_i x C)
//   backward  d_phi (E_i x C) = Y_i (E_i x L) . G_i^T (L x C),  dY (E_i x L) = phi_i . G_i
// with G_i = d_out[i] (C x L), on v_mfma_f32_16x16x4_f32. The harmonic dimension is padded
// to 16 with zeros; channel tile t of width 16 holds channels c = 16-row index * T + t,
// which makes every lane's operand and result runs contiguous in memory. C = 16 T.

// phi operand of the forward for k-steps k0 .. k0+KG-1 of a batch: lane l feeds edge
// 4 k + l / 16 with channels [(l % 16) T, (l % 16) T + T)
template <int T, int KG>
__device__ __forceinline__ void fwd_phi_group(const float* __restrict__ phi, int k0, int cnt,
                                              int my_e, int lo, int hi, float (&buf)[KG][T]) {
#pragma unroll
  for (int g = 0; g < KG; ++g) {
    const int j = 4 * (k0 + g) + hi;
    const int ej = __shfl(my_e, j & (kWave - 1));
    if (j < cnt) {
      load_run<T>(phi + (int64_t)ej * (16 * T) + lo * T, buf[g]);
    } else {
#pragma unroll
      for (int t = 0; t < T; ++t) buf[g][t] = 0.f;
    }
  }
}

// Forward: one wave per receiver row (persistent, rows dealt round robin). Per batch of
// 64 edges, lane j evaluates Y of edge j into LDS; then 4 edges per k-step:
// A = Y^T (lm = l % 16, edge l / 16), B = phi (edge l / 16, channel (l % 16) T + t) for
// tile t, so D[lm][channel] leaves each lane 4 consecutive lm of one channel: float4
// stores of the (C, L) row.
template <typename G, int LMAX, int T>
__global__ __launch_bounds__(256) void sh_msg_fwd_mfma_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, float sign,
    const float* __restrict__ phi, float* __restrict__ out) {
  constexpr int L = ShDims<LMAX>::L;
  constexpr int C = 16 * T;
  constexpr int KG = 2;  // k-steps per load group (8 edges); the next group is in flight
  __shared__ float sY[kWavesPerBlock][kWave * kSY];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int lo = lane & 15, hi = lane >> 4;
  float* ys = sY[wave];
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave; row < n_nodes; row += n_waves) {
    const G* cl = cell == nullptr ? nullptr
                                  : (n_graphs <= 1 || batch == nullptr ? cell
                                                                       : cell + 9 * (int64_t)batch[row]);
    floatx4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int b0 = ptr[row], b1 = ptr[row + 1];
    for (int base = b0; base < b1; base += kWave) {
      const int cnt = min(kWave, b1 - base);
      const int my_e = lane < cnt ? (perm ? perm[base + lane] : base + lane) : 0;
      const int nk = (cnt + 3) >> 2;
      float cur[KG][T], nxt[KG][T];
      // the first phi loads go out before the harmonics are evaluated
      fwd_phi_group<T, KG>(phi, 0, cnt, my_e, lo, hi, cur);
      float ux, uy, uz, inv, len;
      batch_harmonics<G, LMAX>(vec, pos, cl, src, shift, (int)row, sign, lane, cnt, my_e, ys, ux,
                               uy, uz, inv, len);
      wave_sync();
      for (int k0 = 0; k0 < nk; k0 += KG) {
        if (k0 + KG < nk) fwd_phi_group<T, KG>(phi, k0 + KG, cnt, my_e, lo, hi, nxt);
#pragma unroll
        for (int g = 0; g < KG; ++g) {
          if (k0 + g < nk) {
            const float a = ys[(4 * (k0 + g) + hi) * kSY + lo];
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = mfma_16x16x4(a, cur[g][t], acc[t]);
          }
        }
#pragma unroll
        for (int g = 0; g < KG; ++g)
#pragma unroll
          for (int t = 0; t < T; ++t) cur[g][t] = nxt[g][t];
      }
      wave_sync();  // ys is rewritten by the next batch
    }
    // lane holds A[row, channel lo T + t, lm 4 hi + r]
    float* o = out + (int64_t)row * C * L;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float* oc = o + (int64_t)(lo * T + t) * L;
      if constexpr (L % 4 == 0) {
        if (4 * hi < L)
          *reinterpret_cast<float4*>(oc + 4 * hi) =
              make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (4 * hi + r < L) oc[4 * hi + r] = acc[t][r];
      }
    }
  }
}

// Backward: one wave per receiver row. The row's G = d_out[i] is staged through LDS into
// two register layouts: gA[t][s] = G[lo T + t][4 s + hi] (A operand of d_phi, K = lm)
// and gB[s] = G[hi Q + s][lo] (B operand of dY, K = channels, Q = C / 4). Per tile of 16
// edges of a 64-edge batch:
//   dY:     A = phi[edge lo][hi Q + s], B = gB[s], Q k-steps -> lane gets
//           dY[edge 4 hi + r][lm lo], parked in LDS for the edge's own lane;
//   d_phi:  A = gA[t][s], B = Y[edge lo][4 s + hi], ceil(L / 4) k-steps per tile t ->
//           lane gets d_phi[edge lo][(4 hi + r) T + t]: channels [32 hi, 32 hi + 32) of
//           one edge when T = 8, stored as float4 runs.
// The next tile's phi loads go out before this tile's d_phi products.
template <typename G, int LMAX, int T>
__global__ __launch_bounds__(256) void sh_msg_bwd_mfma_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, float sign,
    const float* __restrict__ phi, const float* __restrict__ d_out, float* __restrict__ d_phi,
    float* __restrict__ g_vec) {
  constexpr int L = ShDims<LMAX>::L;
  constexpr int C = 16 * T;
  constexpr int Q = C / 4;
  constexpr int KS = (L + 3) / 4;
  static_assert(C * L <= 2 * kWave * kSY, "the staged d_out row must fit the LDS slice");
  __shared__ __align__(16) float sbuf[kWavesPerBlock][2 * kWave * kSY];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int lo = lane & 15, hi = lane >> 4;
  float* ys = sbuf[wave];
  float* sdy = sbuf[wave] + kWave * kSY;
  const bool want_vec = g_vec != nullptr;
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave; row < n_nodes; row += n_waves) {
    const int b0 = ptr[row], b1 = ptr[row + 1];
    if (b0 == b1) continue;  // no edges: nothing to write
    const G* cl = cell == nullptr ? nullptr
                                  : (n_graphs <= 1 || batch == nullptr ? cell
                                                                       : cell + 9 * (int64_t)batch[row]);
    // stage G (C x L, contiguous) through LDS: coalesced float4 loads
    {
      const float4* g4 = reinterpret_cast<const float4*>(d_out + (int64_t)row * C * L);
      float4* s4 = reinterpret_cast<float4*>(sbuf[wave]);
      for (int i = lane; i < C * L / 4; i += kWave) s4[i] = g4[i];
    }
    wave_sync();
    float gA[T][KS], gB[Q];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int lm = 4 * s + hi;
        gA[t][s] = lm < L ? sbuf[wave][(lo * T + t) * L + lm] : 0.f;
      }
#pragma unroll
    for (int s = 0; s < Q; ++s) gB[s] = lo < L ? sbuf[wave][(hi * Q + s) * L + lo] : 0.f;
    wave_sync();  // the staging area becomes ys / sdy

    for (int base = b0; base < b1; base += kWave) {
      const int cnt = min(kWave, b1 - base);
      const int my_e = lane < cnt ? (perm ? perm[base + lane] : base + lane) : 0;
      const int ntile = (cnt + 15) >> 4;
      float pc[Q];
      if (want_vec) {
        const int ej = __shfl(my_e, lo);
        if (lo < cnt) {
          load_run<Q>(phi + (int64_t)ej * C + hi * Q, pc);
        } else {
#pragma unroll
          for (int s = 0; s < Q; ++s) pc[s] = 0.f;
        }
      }
      float ux, uy, uz, inv, len;
      batch_harmonics<G, LMAX>(vec, pos, cl, src, shift, (int)row, sign, lane, cnt, my_e, ys, ux,
                               uy, uz, inv, len);
      wave_sync();
      for (int tau = 0; tau < ntile; ++tau) {
        const int je = 16 * tau + lo;  // this lane's edge column within the batch
        if (want_vec) {
          floatx4 dy = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < Q; ++s) dy = mfma_16x16x4(pc[s], gB[s], dy);
          // lane holds dY[edge 16 tau + 4 hi + r][lm lo]
#pragma unroll
          for (int r = 0; r < 4; ++r) sdy[(16 * tau + 4 * hi + r) * kSY + lo] = dy[r];
          if (tau + 1 < ntile) {
            const int jn = je + 16;
            const int ej = __shfl(my_e, jn & (kWave - 1));
            if (jn < cnt) {
              load_run<Q>(phi + (int64_t)ej * C + hi * Q, pc);
            } else {
#pragma unroll
              for (int s = 0; s < Q; ++s) pc[s] = 0.f;
            }
          }
        }
        floatx4 dp[T];
#pragma unroll
        for (int t = 0; t < T; ++t) dp[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const float b = ys[je * kSY + 4 * s + hi];
#pragma unroll
          for (int t = 0; t < T; ++t) dp[t] = mfma_16x16x4(gA[t][s], b, dp[t]);
        }
        const int ej = __shfl(my_e, je & (kWave - 1));
        if (je < cnt) {
          float* drow = d_phi + (int64_t)ej * C;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v[T];
#pragma unroll
            for (int t = 0; t < T; ++t) v[t] = dp[t][r];
            store_run<T>(drow + (4 * hi + r) * T, v);
          }
        }
      }
      wave_sync();
      if (want_vec && lane < cnt) {
        float dY[L];
#pragma unroll
        for (int m = 0; m < L; ++m) dY[m] = sdy[lane * kSY + m];
        float Gx, Gy, Gz, vx, vy, vz;
        sh_grad<LMAX, float>(ux, uy, uz, dY, Gx, Gy, Gz);
        sh_chain<float>(ux, uy, uz, inv, Gx, Gy, Gz, vx, vy, vz);
        g_vec[3 * (int64_t)my_e + 0] = sign * vx;
        g_vec[3 * (int64_t)my_e + 1] = sign * vy;
        g_vec[3 * (int64_t)my_e + 2] = sign * vz;
      }
      wave_sync();
    }
  }
}

// ---------------------------------------------------------------- generic segment ops
template <typename T, int GROUP>
__global__ __launch_bounds__(256) void segment_sum_kernel(const T* __restrict__ src, int64_t F,
                                                          const int32_t* __restrict__ ptr,
                                                          const int32_t* __restrict__ perm,
                                                          int64_t n_seg, T* __restrict__ out) {
  const int lane = threadIdx.x % GROUP;
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / GROUP;
  if (row >= n_seg) return;
  const int b0 = ptr[row], b1 = ptr[row + 1];
  for (int64_t f = lane; f < F; f += GROUP) {
    T acc = T(0);
    for (int k = b0; k < b1; ++k) {
      const int64_t e = perm ? perm[k] : k;
      acc += src[e * F + f];
    }
    out[row * F + f] = acc;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void gather_rows_kernel(const T* __restrict__ src, int64_t F,
                                                          const int32_t* __restrict__ index,
                                                          int64_t n_rows, T* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_rows * F) return;
  const int64_t e = t / F, f = t - e * F;
  out[t] = src[(int64_t)index[e] * F + f];
}

// One block per segment; every thread sums a strided share of the segment's rows for
// up to 16 features in registers, then a fixed tree (wave shuffles, then one LDS row
// per wave) combines them: deterministic, float64 throughout. With `chunks` > 1 the
// single segment is split into that many contiguous row ranges, one per block, whose
// totals land in `partial` for segment_finish_kernel.
template <typename T, int BLOCK>
__global__ __launch_bounds__(BLOCK) void segment_reduce_f64_kernel(const T* __restrict__ src,
                                                                   int64_t F,
                                                                   const int64_t* __restrict__ seg,
                                                                   int chunks,
                                                                   double* __restrict__ out) {
  constexpr int kF = 16;
  constexpr int kWaves = BLOCK / kWave;
  __shared__ double red[kWaves][kF];
  int64_t b, i0, i1;
  if (chunks > 1) {
    b = blockIdx.x;
    const int64_t s0 = seg[0], s1 = seg[1];
    const int64_t per = (s1 - s0 + chunks - 1) / chunks;
    i0 = min(s1, s0 + b * per);
    i1 = min(s1, i0 + per);
  } else {
    b = blockIdx.x;
    i0 = seg[b];
    i1 = seg[b + 1];
  }
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  for (int64_t f0 = 0; f0 < F; f0 += kF) {
    const int nf = (int)min<int64_t>(kF, F - f0);
    double acc[kF];
#pragma unroll
    for (int q = 0; q < kF; ++q) acc[q] = 0.0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += BLOCK) {
      const T* r = src + i * F + f0;
#pragma unroll
      for (int q = 0; q < kF; ++q)
        if (q < nf) acc[q] += (double)r[q];
    }
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1)
#pragma unroll
      for (int q = 0; q < kF; ++q) acc[q] += __shfl_xor(acc[q], m, kWave);
    if (kWaves > 1) {
      if (lane == 0)
#pragma unroll
        for (int q = 0; q < kF; ++q) red[wave][q] = acc[q];
      __syncthreads();
      if (threadIdx.x < kF) {
        double t = 0.0;
        for (int w = 0; w < kWaves; ++w) t += red[w][threadIdx.x];
        if ((int)threadIdx.x < nf) out[b * F + f0 + threadIdx.x] = t;
      }
      __syncthreads();
    } else if (lane == 0) {
#pragma unroll
      for (int q = 0; q < kF; ++q)
        if (q < nf) out[b * F + f0 + q] = acc[q];
    }
  }
}

// out[f] = sum over chunks k of partial[k, f]: one wave per feature, lane l sums chunks
// l, l + 64, ... in order, then a fixed butterfly (deterministic)
__global__ __launch_bounds__(256) void segment_finish_kernel(const double* __restrict__ partial,
                                                             int chunks, int64_t F,
                                                             double* __restrict__ out) {
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  for (int64_t f = wave; f < F; f += blockDim.x / kWave) {
    double t = 0.0;
    for (int k = lane; k < chunks; k += kWave) t += partial[(int64_t)k * F + f];
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) t += __shfl_xor(t, m, kWave);
    if (lane == 0) out[f] = t;
  }
}

// One segment of rows with F <= kFlatMaxF features, read as a flat array: thread t of a
// block (t < S = F P, P the largest power of two with F P <= 256) adds elements
// t, t + S, ... of the block's chunk, all of feature t % F (chunks start at multiples
// of S), with coalesced loads; an LDS tree over the P threads of each feature then
// gives the chunk's partial sums (fixed order: deterministic).
constexpr int kFlatMaxF = 64;
static_assert(kFlatMaxF <= kWave, "wave 0 holds the flat results");
constexpr int kFlatPerThread = 4;
// a single block of 1024 threads takes arrays up to this many elements (no second kernel)
constexpr int64_t kFlatSingleMax = 16384;
// the energy-and-stress finish takes one block: structures up to this many atoms
constexpr int64_t kEnergyStressMaxNodes = 65536;

static int flat_stride(int64_t F, int block) {
  int64_t S = F;
  while (2 * S <= block) S *= 2;
  return (int)S;
}

// The sum of src[c0, c1) over the F interleaved features by the block: thread t < S adds
// elements c0 + t + k S (S a multiple of F), then a pairwise tree folds the S sums to F.
// Every thread of the block calls it; lane t < F of wave 0 gets feature t's sum.
template <typename T, int BLOCK>
__device__ inline double flat_block_sum(const T* __restrict__ src, int64_t F, int S, int64_t c0,
                                        int64_t c1, double* red) {
  const int t = threadIdx.x;
  // four independent sums per thread, so that four loads are in flight at a time (a
  // single-block launch over a short array is otherwise a chain of load latencies)
  double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
  if (t < S) {
    int64_t i = c0 + t;
    for (; i + 3 * (int64_t)S < c1; i += 4 * (int64_t)S) {
      a0 += (double)src[i];
      a1 += (double)src[i + S];
      a2 += (double)src[i + 2 * (int64_t)S];
      a3 += (double)src[i + 3 * (int64_t)S];
    }
    for (; i < c1; i += S) a0 += (double)src[i];
  }
  red[t] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  // pairwise tree, red[t] += red[t + h F]: steps that read beyond one wave through LDS, the
  // rest by shuffles inside wave 0 (the same pairs in the same order, without a barrier per
  // step; F <= kFlatMaxF = kWave, so wave 0 holds every result)
  int h = S / (int)F / 2;
  for (; h > 0 && 2 * h * (int)F > kWave; h >>= 1) {
    if (t < h * F) red[t] += red[t + h * F];
    __syncthreads();
  }
  double x = 0.0;
  if (t < kWave) {
    x = red[t];
    for (; h > 0; h >>= 1) x += __shfl_down(x, h * (int)F, kWave);
  }
  return x;
}

template <typename T, int BLOCK>
__global__ __launch_bounds__(BLOCK) void flat_reduce_f64_kernel(const T* __restrict__ src,
                                                                int64_t F, int S,
                                                                const int64_t* __restrict__ seg,
                                                                int chunks,
                                                                double* __restrict__ partial) {
  __shared__ double red[BLOCK];
  const int64_t e0 = seg[0] * F, e1 = seg[1] * F;
  // chunk length: a multiple of S covering the segment in `chunks` pieces
  const int64_t per_s = ((e1 - e0 + chunks - 1) / chunks + S - 1) / S;
  const int64_t c0 = min(e1, e0 + (int64_t)blockIdx.x * per_s * S);
  const int64_t c1 = min(e1, c0 + per_s * S);
  const double x = flat_block_sum<T, BLOCK>(src, F, S, c0, c1, red);
  if (threadIdx.x < F) partial[(int64_t)blockIdx.x * F + threadIdx.x] = x;
}

// One structure's energy total and stress in one block: energy = the flat sum of the node
// energies (1024 threads, the same order as flat_reduce_f64_kernel<T, 1024> for one chunk
// of one feature), and stress = scale g / V (stress_entry) by lanes of wave 1.
template <typename T, typename G, typename C>
__global__ __launch_bounds__(1024) void energy_stress_finish_kernel(
    const T* __restrict__ node_energy, int64_t n, const G* __restrict__ g,
    const C* __restrict__ cell, const uint8_t* __restrict__ pbc, double scale,
    double* __restrict__ energy, G* __restrict__ stress) {
  __shared__ double red[1024];
  const double x = flat_block_sum<T, 1024>(node_energy, 1, 1024, 0, n, red);
  if (threadIdx.x == 0) energy[0] = x;
  const int j = (int)threadIdx.x - kWave;
  if (j >= 0 && j < 9) stress[j] = stress_entry(g, cell, pbc, 0, j, scale);
}

// Totals of the 9 virial components over `chunks` partial rows (as segment_finish_kernel),
// then out = sym(total + term) (or total + term) cast to T
template <typename T>
__global__ __launch_bounds__(256) void virial_chunks_finish_kernel(
    const double* __restrict__ partial, int chunks, const double* __restrict__ term,
    int symmetrize, T* __restrict__ out) {
  __shared__ double tot[9];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  for (int f = wave; f < 9; f += blockDim.x / kWave) {
    double v = 0.0;
    for (int k = lane; k < chunks; k += kWave) v += partial[(int64_t)k * 9 + f];
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) v += __shfl_xor(v, m, kWave);
    if (lane == 0) tot[f] = v + (term ? term[f] : 0.0);
  }
  __syncthreads();
  const int j = threadIdx.x;
  if (j < 9) {
    const int r = j / 3, c = j % 3;
    out[j] = (T)(symmetrize ? 0.5 * (tot[j] + tot[3 * c + r]) : tot[j]);
  }
}

constexpr int64_t kChunkRows = 2048;
constexpr int kMaxChunks = 256;

// single segments of few features take the flat kernel
static bool reduce_flat(int64_t n_rows, int64_t n_features, int64_t n_segments) {
  return n_segments == 1 && n_features <= kFlatMaxF &&
         n_rows * n_features >= 2 * (int64_t)flat_stride(n_features, 256) * kFlatPerThread;
}

// one block (no partials) for small flat arrays
static bool reduce_flat_single(int64_t n_rows, int64_t n_features, int64_t n_segments) {
  return reduce_flat(n_rows, n_features, n_segments) && n_rows * n_features <= kFlatSingleMax;
}

static int reduce_chunks(int64_t n_rows, int64_t n_features, int64_t n_segments) {
  if (reduce_flat_single(n_rows, n_features, n_segments)) return 1;
  if (reduce_flat(n_rows, n_features, n_segments)) {
    const int64_t per_chunk = (int64_t)flat_stride(n_features, 256) * kFlatPerThread;
    const int64_t c = (n_rows * n_features + per_chunk - 1) / per_chunk;
    return (int)(c < kMaxChunks ? c : kMaxChunks);
  }
  if (n_segments != 1 || n_rows < 2 * kChunkRows) return 1;
  const int64_t c = (n_rows + kChunkRows - 1) / kChunkRows;
  return (int)(c < kMaxChunks ? c : kMaxChunks);
}

// the partial sums of one structure's (n_rows, F) values in `partial` (chunks x F), by the
// flat kernel; `chunks` as reduce_chunks gives it
static void launch_flat(int dtype, const void* src, int64_t F, const int64_t* seg, int chunks,
                        double* partial, hipStream_t s) {
  if (chunks == 1) {
    const int S = flat_stride(F, 1024);
    if (dtype == XNN_F32)
      hipLaunchKernelGGL((flat_reduce_f64_kernel<float, 1024>), dim3(1), dim3(1024), 0, s,
                         (const float*)src, F, S, seg, 1, partial);
    else
      hipLaunchKernelGGL((flat_reduce_f64_kernel<double, 1024>), dim3(1), dim3(1024), 0, s,
                         (const double*)src, F, S, seg, 1, partial);
    return;
  }
  const int S = flat_stride(F, 256);
  if (dtype == XNN_F32)
    hipLaunchKernelGGL((flat_reduce_f64_kernel<float, 256>), dim3(chunks), dim3(256), 0, s,
                       (const float*)src, F, S, seg, chunks, partial);
  else
    hipLaunchKernelGGL((flat_reduce_f64_kernel<double, 256>), dim3(chunks), dim3(256), 0, s,
                       (const double*)src, F, S, seg, chunks, partial);
}

// blocks of `kernel` that stay resident on the whole device (all CUs), capped at `needed`
int64_t resident_blocks(const void* kernel, int block_threads, int64_t needed) {
  // the occupancy of each kernel is queried once and kept (a handful of instantiations)
  static const void* keys[128] = {nullptr};
  static int values[128] = {0};
  int per_cu = 0;
  for (int i = 0; i < 128; ++i) {
    if (keys[i] == kernel) {
      per_cu = values[i];
      break;
    }
    if (keys[i] == nullptr) {
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block_threads, 0) !=
              hipSuccess ||
          per_cu <= 0)
        per_cu = 2;
      keys[i] = kernel;
      values[i] = per_cu;
      break;
    }
  }
  if (per_cu <= 0) per_cu = 2;
  return std::max<int64_t>(1, std::min<int64_t>(needed, (int64_t)per_cu * device_cu_count()));
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// XNN_AMD_MESSAGE_MFMA=0 in the environment selects the vector-ALU message kernels
// (read at every call, so a process can compare the two)
bool message_mfma_enabled() {
  const char* v = std::getenv("XNN_AMD_MESSAGE_MFMA");
  return !(v != nullptr && v[0] == '0');
}

template <typename G>
static int sh_msg(bool backward, const float* vec, const void* pos, int64_t n_nodes,
                  const void* cell, int64_t n_graphs, const int32_t* batch, const int32_t* src,
                  const int32_t* shift, const int32_t* ptr, const int32_t* perm, int l_max,
                  int sign, int C, const float* phi, const float* d_out, float* out_or_dphi,
                  float* g_vec, hipStream_t stream) {
  if (n_nodes == 0) return XNN_OK;
  const int64_t blocks_needed = grid_1d(n_nodes, kWavesPerBlock);
  const dim3 block(kWavesPerBlock * kWave);
  const float sg = (float)sign;
  int cpl = (C + kWave - 1) / kWave;
  if (cpl == 3) cpl = 4;
  const bool vec_ok = (C % cpl) == 0 && aligned16(phi) && aligned16(out_or_dphi) &&
                      (!backward || aligned16(d_out));
  // persistent waves: exactly as many blocks as stay resident, never more than rows need
#define XNN_MSG(LM, CP, VE)                                                                    \
  do {                                                                                         \
    if (backward) {                                                                            \
      auto k = sh_msg_bwd_kernel<G, LM, CP, VE>;                                               \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, blocks_needed));      \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, C, sg, phi, d_out,    \
                         out_or_dphi, g_vec);                                                  \
    } else {                                                                                   \
      auto k = sh_msg_fwd_kernel<G, LM, CP, VE>;                                               \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, blocks_needed));      \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, C, sg, phi,          \
                         out_or_dphi);                                                         \
    }                                                                                          \
  } while (0)
#define XNN_MSG_L(CP, VE)                 \
  switch (l_max) {                        \
    case 0: XNN_MSG(0, CP, VE); break;    \
    case 1: XNN_MSG(1, CP, VE); break;    \
    case 2: XNN_MSG(2, CP, VE); break;    \
    default: XNN_MSG(3, CP, VE); break;   \
  }
  // matrix-core kernels: C = 16 T with the tile counts instantiated below, 16-byte
  // aligned rows (XNN_AMD_MESSAGE_MFMA=0 selects the vector-ALU kernels instead)
  const int T = C / 16;
  const bool aligned = aligned16(phi) && aligned16(out_or_dphi) && (!backward || aligned16(d_out));
  if (aligned && C % 16 == 0 && (T <= 4 || T == 6 || T == 8) && message_mfma_enabled()) {
#define XNN_MFMA(LM, TT)                                                                       \
  do {                                                                                         \
    if (backward) {                                                                            \
      auto k = sh_msg_bwd_mfma_kernel<G, LM, TT>;                                              \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, blocks_needed));      \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, sg, phi, d_out,       \
                         out_or_dphi, g_vec);                                                  \
    } else {                                                                                   \
      auto k = sh_msg_fwd_mfma_kernel<G, LM, TT>;                                              \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, blocks_needed));      \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, sg, phi,              \
                         out_or_dphi);                                                         \
    }                                                                                          \
  } while (0)
#define XNN_MFMA_L(TT)                    \
  switch (l_max) {                        \
    case 0: XNN_MFMA(0, TT); break;       \
    case 1: XNN_MFMA(1, TT); break;       \
    case 2: XNN_MFMA(2, TT); break;       \
    default: XNN_MFMA(3, TT); break;      \
  }
    switch (T) {
      case 1: XNN_MFMA_L(1); break;
      case 2: XNN_MFMA_L(2); break;
      case 3: XNN_MFMA_L(3); break;
      case 4: XNN_MFMA_L(4); break;
      case 6: XNN_MFMA_L(6); break;
      default: XNN_MFMA_L(8); break;
    }
#undef XNN_MFMA_L
#undef XNN_MFMA
    XNN_LAUNCH_CHECK();
    return XNN_OK;
  }
  switch (cpl) {
    case 1: XNN_MSG_L(1, false); break;
    case 2:
      if (vec_ok) { XNN_MSG_L(2, true); } else { XNN_MSG_L(2, false); }
      break;
    case 4:
      if (vec_ok) { XNN_MSG_L(4, true); } else { XNN_MSG_L(4, false); }
      break;
    default: set_error("n_channels must be <= 256, got %d", C); return XNN_EINVAL;
  }
#undef XNN_MSG_L
#undef XNN_MSG
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

// node_energy[i] = bias[z[i]] + sum over the receiver row i of edge_energy: 16 lanes per
// atom, lane k summing the row's edges k, k + 16, ... in order, then a fixed butterfly over
// the 16 (bitwise reproducible). Every lane of a wave takes part in the exchanges (an atom
// index past the end reads nothing). An index z outside [0, n_bias) gives NaN; no bias: 0.
constexpr int kNodeLanes = 16;

__global__ __launch_bounds__(256) void node_energy_from_edges_kernel(
    const float* __restrict__ edge_energy, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, const int64_t* __restrict__ z,
    const float* __restrict__ bias, int64_t n_bias, float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t i = t / kNodeLanes;
  const int k = (int)(t % kNodeLanes);
  const bool live = i < n_nodes;
  float s = 0.f;
  if (live) {
    const int32_t b = ptr[i], e = ptr[i + 1];
    for (int32_t q = b + k; q < e; q += kNodeLanes) s += edge_energy[perm ? perm[q] : q];
  }
  s = group_sum_f<kNodeLanes>(s);
  if (live && k == 0) {
    float base = 0.f;
    if (bias != nullptr) {
      const int64_t zi = z[i];
      base = (zi >= 0 && zi < n_bias) ? bias[zi] : __builtin_nanf("");
    }
    out[i] = base + s;
  }
}

template <typename T>
static int segment_sum_t(const void* src, int64_t F, const int32_t* ptr, const int32_t* perm,
                         int64_t n_seg, void* out, hipStream_t stream) {
  if (n_seg == 0 || F == 0) return XNN_OK;
  int group = 1;
  while (group < F && group < kWave) group <<= 1;
  const int64_t threads = n_seg * group;
  const dim3 grid(grid_1d(threads, 256)), block(256);
  switch (group) {
#define XNN_SEG(GR)                                                                         \
  case GR:                                                                                  \
    hipLaunchKernelGGL((segment_sum_kernel<T, GR>), grid, block, 0, stream, (const T*)src, F, \
                       ptr, perm, n_seg, (T*)out);                                          \
    break;
    XNN_SEG(1) XNN_SEG(2) XNN_SEG(4) XNN_SEG(8) XNN_SEG(16) XNN_SEG(32) XNN_SEG(64)
#undef XNN_SEG
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

}  // namespace xnn

using namespace xnn;

// ---------------------------------------------------------------- no-allocation variant
// The partial sums of xnn_segment_reduce_f64_noalloc live in this file-scope device
// array (one copy per GPU, held for the life of the process). Host code never passes
// the name itself to a kernel: in host code it is a stand-in, not a device address. Each
// device's address is looked up once, with that device current, and kept here.
constexpr size_t kNoAllocScratchDoubles = 131072;  // 1 MiB
static __device__ __align__(256) double scratch[kNoAllocScratchDoubles];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
double* g_scratch_ptr[kMaxDevices] = {};

// this device's address of `scratch`, looked up on its first use (with it current)
int scratch_for_current_device(double** out) {
  int dev = -1;
  XNN_HIP_CHECK(hipGetDevice(&dev));
  XNN_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d outside the scratch table", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    XNN_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    XNN_REQUIRE(p != nullptr, "no device address for the scratch array");
    g_scratch_ptr[dev] = static_cast<double*>(p);
  }
  *out = g_scratch_ptr[dev];
  return XNN_OK;
}
}  // namespace

extern "C" {

int xnn_sh_message_sum(int geom_dtype, const float* vec_in, const void* pos, int64_t n_nodes,
                       const void* cell,
                       int64_t n_graphs, const int32_t* batch, const int32_t* src,
                       const int32_t* shift, int64_t n_edges, const int32_t* ptr_dst,
                       const int32_t* perm_dst, int32_t l_max, int32_t sh_sign,
                       int32_t n_channels, const float* phi, float* out, xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_edges >= 0, "negative size");
  XNN_REQUIRE(l_max >= 0 && l_max <= 3, "l_max must be in [0, 3]");
  XNN_REQUIRE(sh_sign == 1 || sh_sign == -1, "sh_sign must be +1 or -1");
  XNN_REQUIRE(n_channels >= 1 && n_channels <= 256, "n_channels must be in [1, 256]");
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && out), "NULL CSR or output");
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && shift)) && phi), "NULL edge input");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  if (geom_dtype == XNN_F32)
    return sh_msg<float>(false, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift, ptr_dst,
                         perm_dst, l_max, sh_sign, n_channels, phi, nullptr, out, nullptr,
                         as_hip(stream));
  if (geom_dtype == XNN_F64)
    return sh_msg<double>(false, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift, ptr_dst,
                          perm_dst, l_max, sh_sign, n_channels, phi, nullptr, out, nullptr,
                          as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

int xnn_sh_message_sum_backward(int geom_dtype, const float* vec_in, const void* pos,
                                int64_t n_nodes, const void* cell, int64_t n_graphs, const int32_t* batch,
                                const int32_t* src, const int32_t* shift, int64_t n_edges,
                                const int32_t* ptr_dst, const int32_t* perm_dst, int32_t l_max,
                                int32_t sh_sign, int32_t n_channels, const float* phi,
                                const float* d_out, float* d_phi, float* g_vec,
                                xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_edges >= 0, "negative size");
  XNN_REQUIRE(l_max >= 0 && l_max <= 3, "l_max must be in [0, 3]");
  XNN_REQUIRE(sh_sign == 1 || sh_sign == -1, "sh_sign must be +1 or -1");
  XNN_REQUIRE(n_channels >= 1 && n_channels <= 256, "n_channels must be in [1, 256]");
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && d_out), "NULL CSR or d_out");
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && shift)) && phi && d_phi),
              "NULL edge input");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  if (geom_dtype == XNN_F32)
    return sh_msg<float>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift, ptr_dst,
                         perm_dst, l_max, sh_sign, n_channels, phi, d_out, d_phi, g_vec,
                         as_hip(stream));
  if (geom_dtype == XNN_F64)
    return sh_msg<double>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift, ptr_dst,
                          perm_dst, l_max, sh_sign, n_channels, phi, d_out, d_phi, g_vec,
                          as_hip(stream));
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

int xnn_segment_sum(int dtype, const void* src, int64_t n_rows, int64_t n_features,
                    const int32_t* ptr, const int32_t* perm, int64_t n_segments, void* out,
                    xnn_stream_t stream) {
  XNN_REQUIRE(n_rows >= 0 && n_features >= 0 && n_segments >= 0, "negative size");
  XNN_REQUIRE(n_segments == 0 || (ptr && out), "NULL CSR or output");
  XNN_REQUIRE(n_rows == 0 || src, "NULL src");
  if (dtype == XNN_F32)
    return segment_sum_t<float>(src, n_features, ptr, perm, n_segments, out, as_hip(stream));
  if (dtype == XNN_F64)
    return segment_sum_t<double>(src, n_features, ptr, perm, n_segments, out, as_hip(stream));
  set_error("unsupported dtype %d", dtype);
  return XNN_EINVAL;
}

int xnn_node_energy_from_edges(const float* edge_energy, const int32_t* ptr_dst,
                               const int32_t* perm_dst, int64_t n_nodes, const int64_t* z,
                               const float* bias, int64_t n_bias, float* node_energy,
                               xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_bias >= 0, "negative size");
  if (n_nodes == 0) return XNN_OK;
  XNN_REQUIRE(ptr_dst && node_energy, "NULL CSR or output");
  XNN_REQUIRE(bias == nullptr || z != nullptr, "a bias needs the atoms' indices");
  hipLaunchKernelGGL(node_energy_from_edges_kernel,
                     dim3((unsigned)grid_1d(n_nodes * kNodeLanes, 256)),
                     dim3(256), 0, as_hip(stream), edge_energy, ptr_dst, perm_dst, n_nodes, z,
                     bias, n_bias, node_energy);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_gather_rows(int dtype, const void* src, int64_t n_src_rows, int64_t n_features,
                    const int32_t* index, int64_t n_rows, void* out, xnn_stream_t stream) {
  XNN_REQUIRE(n_rows >= 0 && n_features >= 0 && n_src_rows >= 0, "negative size");
  if (n_rows == 0 || n_features == 0) return XNN_OK;
  XNN_REQUIRE(src && index && out, "NULL pointer");
  const int64_t total = n_rows * n_features;
  const dim3 grid(grid_1d(total, 256)), block(256);
  if (dtype == XNN_F32)
    hipLaunchKernelGGL((gather_rows_kernel<float>), grid, block, 0, as_hip(stream),
                       (const float*)src, n_features, index, n_rows, (float*)out);
  else if (dtype == XNN_F64)
    hipLaunchKernelGGL((gather_rows_kernel<double>), grid, block, 0, as_hip(stream),
                       (const double*)src, n_features, index, n_rows, (double*)out);
  else {
    set_error("unsupported dtype %d", dtype);
    return XNN_EINVAL;
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

size_t xnn_segment_reduce_workspace_bytes(int64_t n_rows, int64_t n_features,
                                          int64_t n_segments) {
  const int chunks = reduce_chunks(n_rows, n_features, n_segments);
  return chunks > 1 ? sizeof(double) * (size_t)chunks * (size_t)n_features : 0;
}

int xnn_segment_reduce_f64(int dtype, const void* src, int64_t n_rows, int64_t n_features,
                           const int64_t* seg_ptr, int64_t n_segments, double* out,
                           void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  XNN_REQUIRE(n_rows >= 0 && n_features >= 0 && n_segments >= 0, "negative size");
  if (n_segments == 0 || n_features == 0) return XNN_OK;
  XNN_REQUIRE(seg_ptr && out && (n_rows == 0 || src), "NULL pointer");
  XNN_REQUIRE(dtype == XNN_F32 || dtype == XNN_F64, "unsupported dtype %d", dtype);
  const int chunks = reduce_chunks(n_rows, n_features, n_segments);
  const size_t need = xnn_segment_reduce_workspace_bytes(n_rows, n_features, n_segments);
  XNN_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need),
              "workspace of %zu bytes needed", need);
  hipStream_t s = as_hip(stream);
  double* dest = chunks > 1 ? static_cast<double*>(workspace) : out;
  if (reduce_flat(n_rows, n_features, n_segments)) {
    launch_flat(dtype, src, n_features, seg_ptr, chunks, dest, s);
    XNN_LAUNCH_CHECK();
    if (chunks > 1) {
      hipLaunchKernelGGL(segment_finish_kernel, dim3(1), dim3(256), 0, s, dest, chunks,
                         n_features, out);
      XNN_LAUNCH_CHECK();
    }
    return XNN_OK;
  }
  const int64_t grid = chunks > 1 ? chunks : n_segments;
  // long segments get 1024 threads, short ones (many small structures) a wave
  const bool wide = chunks > 1 || n_rows >= 1024 * n_segments;
#define XNN_RED(T, B)                                                                     \
  hipLaunchKernelGGL((segment_reduce_f64_kernel<T, B>), dim3(grid), dim3(B), 0, s,         \
                     (const T*)src, n_features, seg_ptr, chunks, dest)
  if (dtype == XNN_F32) {
    if (chunks > 1) XNN_RED(float, 256); else if (wide) XNN_RED(float, 1024); else XNN_RED(float, 64);
  } else {
    if (chunks > 1) XNN_RED(double, 256); else if (wide) XNN_RED(double, 1024); else XNN_RED(double, 64);
  }
#undef XNN_RED
  XNN_LAUNCH_CHECK();
  if (chunks > 1) {
    hipLaunchKernelGGL(segment_finish_kernel, dim3(1), dim3(256), 0, s, dest, chunks, n_features,
                       out);
    XNN_LAUNCH_CHECK();
  }
  return XNN_OK;
}

size_t xnn_virial_reduce_workspace_bytes(int64_t n_rows, int64_t n_graphs) {
  if (n_graphs == 1) {
    const int chunks = reduce_chunks(n_rows, 9, 1);
    return sizeof(double) * 9 * (size_t)chunks;
  }
  return sizeof(double) * 9 * (size_t)std::max<int64_t>(n_graphs, 0) +
         xnn_segment_reduce_workspace_bytes(n_rows, 9, n_graphs);
}

int xnn_virial_reduce(int dtype, const double* partial, int64_t n_rows, const int64_t* seg_ptr,
                      int64_t n_graphs, const double* term, int32_t symmetrize, void* out,
                      void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  XNN_REQUIRE(n_rows >= 0 && n_graphs >= 0, "negative size");
  if (n_graphs == 0) return XNN_OK;
  XNN_REQUIRE(seg_ptr && out && (n_rows == 0 || partial), "NULL pointer");
  XNN_REQUIRE(dtype == XNN_F32 || dtype == XNN_F64, "unsupported dtype %d", dtype);
  const size_t need = xnn_virial_reduce_workspace_bytes(n_rows, n_graphs);
  XNN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace of %zu bytes needed",
              need);
  hipStream_t s = as_hip(stream);
  double* ws = static_cast<double*>(workspace);
  if (n_graphs == 1) {
    const int chunks = reduce_chunks(n_rows, 9, 1);
    if (reduce_flat(n_rows, 9, 1)) {
      launch_flat(XNN_F64, partial, 9, seg_ptr, chunks, ws, s);
    } else {
      // few rows: one block sums them (the per-segment kernel), a single "chunk"
      hipLaunchKernelGGL((segment_reduce_f64_kernel<double, 64>), dim3(1), dim3(64), 0, s,
                         partial, (int64_t)9, seg_ptr, 1, ws);
    }
    XNN_LAUNCH_CHECK();
    const int used = reduce_flat(n_rows, 9, 1) ? chunks : 1;
    if (dtype == XNN_F32)
      hipLaunchKernelGGL(virial_chunks_finish_kernel<float>, dim3(1), dim3(256), 0, s, ws, used,
                         term, (int)symmetrize, (float*)out);
    else
      hipLaunchKernelGGL(virial_chunks_finish_kernel<double>, dim3(1), dim3(256), 0, s, ws, used,
                         term, (int)symmetrize, (double*)out);
    XNN_LAUNCH_CHECK();
    return XNN_OK;
  }
  // several structures: per-structure sums, then the finish per structure
  double* M = ws;
  void* ws2 = ws + 9 * n_graphs;
  const size_t ws2_bytes = workspace_bytes - sizeof(double) * 9 * (size_t)n_graphs;
  int st = xnn_segment_reduce_f64(XNN_F64, partial, n_rows, 9, seg_ptr, n_graphs, M, ws2,
                                  ws2_bytes, stream);
  if (st != XNN_OK) return st;
  return xnn_virial_finish(dtype, M, term, n_graphs, symmetrize, out, stream);
}

int64_t xnn_energy_stress_max_nodes(void) { return kEnergyStressMaxNodes; }

int xnn_energy_stress_finish(int node_dtype, const void* node_energy, int64_t n_nodes, int dtype,
                             const void* strain_grad, int cell_dtype, const void* cell,
                             const uint8_t* pbc, double scale, double* energy, void* stress,
                             xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_nodes <= kEnergyStressMaxNodes,
              "n_nodes must be in [0, %lld], got %lld", (long long)kEnergyStressMaxNodes,
              (long long)n_nodes);
  XNN_REQUIRE(energy && strain_grad && cell && stress && (n_nodes == 0 || node_energy),
              "NULL input or output");
  hipStream_t s = as_hip(stream);
#define XNN_ES(T, G, C)                                                                       \
  hipLaunchKernelGGL((energy_stress_finish_kernel<T, G, C>), dim3(1), dim3(1024), 0, s,         \
                     (const T*)node_energy, n_nodes, (const G*)strain_grad, (const C*)cell, pbc, \
                     scale, energy, (G*)stress)
#define XNN_ES_GC(T)                                                                    \
  if (dtype == XNN_F32 && cell_dtype == XNN_F32) XNN_ES(T, float, float);               \
  else if (dtype == XNN_F32 && cell_dtype == XNN_F64) XNN_ES(T, float, double);         \
  else if (dtype == XNN_F64 && cell_dtype == XNN_F32) XNN_ES(T, double, float);         \
  else if (dtype == XNN_F64 && cell_dtype == XNN_F64) XNN_ES(T, double, double);        \
  else {                                                                                \
    set_error("unsupported dtypes %d / %d", dtype, cell_dtype);                         \
    return XNN_EINVAL;                                                                  \
  }
  if (node_dtype == XNN_F32) {
    XNN_ES_GC(float)
  } else if (node_dtype == XNN_F64) {
    XNN_ES_GC(double)
  } else {
    set_error("unsupported node dtype %d", node_dtype);
    return XNN_EINVAL;
  }
#undef XNN_ES_GC
#undef XNN_ES
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

size_t xnn_segment_reduce_noalloc_max_bytes(void) { return sizeof(scratch); }

int xnn_segment_reduce_f64_noalloc(int dtype, const void* src, int64_t n_rows,
                                   int64_t n_features, const int64_t* seg_ptr,
                                   int64_t n_segments, double* out, xnn_stream_t stream) {
  XNN_REQUIRE(n_rows >= 0 && n_features >= 0 && n_segments >= 0, "negative size");
  if (n_segments == 0 || n_features == 0) return XNN_OK;
  const size_t need = xnn_segment_reduce_workspace_bytes(n_rows, n_features, n_segments);
  XNN_REQUIRE(need <= sizeof(scratch),
              "needs %zu bytes of partial sums, more than the %zu-byte scratch array of the "
              "no-allocation entry point (use xnn_segment_reduce_f64 with a workspace)",
              need, sizeof(scratch));
  double* ws = nullptr;
  if (need > 0) {
    const int st = scratch_for_current_device(&ws);
    if (st != XNN_OK) return st;
  }
  // every partial slot the kernels read is written first in the same call: no clearing
  return xnn_segment_reduce_f64(dtype, src, n_rows, n_features, seg_ptr, n_segments, out, ws,
                                need, stream);
}

}  // extern "C"
