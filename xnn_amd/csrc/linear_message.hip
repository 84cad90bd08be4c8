// Fused edge-weight linear layer + SH message aggregation (gfx950, wave64, fp32 MFMA).
//
// xnn_sh_linear_message_sum(_backward): the per-edge channel weights are the output of
// a linear layer, phi_e = h_e W (h: (E, K) with K <= 8, W: (K, C)), as the last layer of
// the reference's radial weight network; they feed the uvu product with the edge
// harmonics and the receiver sum, A_i[c, lm] = sum_{dst(e)=i} phi_e[c] Y_lm(sign r_e)
// (gnn/fast/conv.py:137-143 with per-edge weights, + scatter_sum, ops.py:403-448).
// phi is formed per 16-edge tile on the matrix cores and consumed in registers: it is
// never stored, and the backward returns d_h = (G_i Y_e) W^T, so d_phi is never stored
// either. Per tile, one wave:
//   forward:  phi (16 x C) = h W   (edges in the M rows, permuted so that result register
//             r of lane l is edge 4 r + l / 16, i.e. exactly the B operand of the next
//             product), then A^T += Y^T phi over 4 k-steps of 4 edges;
//   backward: phi^T = W^T h^T, dY = phi G (K = channels), d_phi = Y G^T, d_h = d_phi W^T
//             (K = channels); dY goes through LDS to the edge's own lane for the SH
//             Jacobian, as in the unfused kernels.
// Channel tile t of width 16 holds channels 16-row index * T + t (C = 16 T).
//
// xnn_sh_radial_message_sum(_backward) go one step further: h is the enveloped radial
// basis of the edge length, h_e = rbf(|r_e|) * envelope(|r_e|) (spherical.py:135-138), and
// each lane evaluates it for its own edge next to the harmonics, into LDS. Featurizer,
// linear layer and message are then one kernel each way; the backward folds
// d|r_e| = sum_k d_h[e, k] d h_k / d|r| into the edge gradient, so neither h nor d_h
// exists in memory.
#include <algorithm>
#include <cstdint>

#include "common.h"
#include "device.h"
#include "message.h"
#include "radial_row.h"

namespace xnn {

// RO (readout): instead of the (C, L) row A_i the kernel writes the atom's energy
// E_i = sum_{c, lm} U[c, lm] A_i[c, lm] + bias[z_i] (bias may be NULL), reduced across the
// wave in a fixed order from the accumulators: A never reaches memory.
template <typename G, int LMAX, int T, bool RAD, bool RO>
__global__ __launch_bounds__(256, 4) void lin_msg_fwd_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, float sign, int K,
    const float* __restrict__ h, Radial<float> R, const float* __restrict__ W,
    float* __restrict__ out, const float* __restrict__ U, const int64_t* __restrict__ z,
    const float* __restrict__ bias, int64_t n_bias) {
  constexpr int L = ShDims<LMAX>::L;
  constexpr int C = 16 * T;
  constexpr int KK = kLinKK;
  __shared__ float sY[kWavesPerBlock][kWave * kSY];
  __shared__ float sH[kWavesPerBlock][RAD ? kWave * kSH : 1];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int lo = lane & 15, hi = lane >> 4;
  float* ys = sY[wave];
  float* hs = sH[wave];
  __shared__ float sTab[kLinKMax];
  const RadialTab tab = RAD ? load_radial_tab(R, sTab) : RadialTab{};
  // W in LDS (rows padded to C + 4 floats, zero rows past K): the B operand of h W for
  // channel tile t, k-step q is W[4 q + hi][lo T + t], a run of T floats
  constexpr int SWS = C + 4;
  __shared__ __align__(16) float sW[kLinKMax * SWS];
  for (int i = threadIdx.x; i < kLinKMax * C; i += blockDim.x)
    sW[(i / C) * SWS + i % C] = i < K * C ? W[i] : 0.f;
  // RO: the readout weights U (C, L), read by every row's epilogue
  __shared__ float sU[RO ? C * L : 1];
  if constexpr (RO)
    for (int i = threadIdx.x; i < C * L; i += blockDim.x) sU[i] = U[i];
  __syncthreads();
  // M row lo of h W stands for edge 4 (lo % 4) + lo / 4 of the tile
  const int hrow = 4 * (lo & 3) + (lo >> 2);
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wave;
  // with given edge vectors, the first batch of the wave's next row is loaded a row ahead
  float px = 0.f, py = 0.f, pz = 0.f;
  if (vec != nullptr && row < n_nodes) load_first_vec(vec, perm, ptr[row], ptr[row + 1], lane, px, py, pz);
  for (; row < n_nodes; row += n_waves) {
    const G* cl = cell == nullptr ? nullptr
                                  : (n_graphs <= 1 || batch == nullptr ? cell
                                                                       : cell + 9 * (int64_t)batch[row]);
    floatx4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int b0 = ptr[row], b1 = ptr[row + 1];
    const float cx = px, cy = py, cz = pz;
    if (vec != nullptr && row + n_waves < n_nodes)
      load_first_vec(vec, perm, ptr[row + n_waves], ptr[row + n_waves + 1], lane, px, py, pz);
    for (int base = b0; base < b1; base += kWave) {
      const int cnt = min(kWave, b1 - base);
      const int my_e = lane < cnt ? (perm ? perm[base + lane] : base + lane) : 0;
      // A operand of h W for tile tau (edge 16 tau + hrow): from global memory with the
      // next tile's in flight while a tile is computed, or evaluated into LDS (RAD)
      float ha[KK], hn[KK];
      if constexpr (!RAD) {
        const int ej = __shfl(my_e, hrow);
#pragma unroll
        for (int q = 0; q < KK; ++q) {
          const int k = 4 * q + hi;
          hn[q] = (hrow < cnt && k < K) ? h[(int64_t)ej * K + k] : 0.f;
        }
      }
      float ux, uy, uz, inv, len;
      if (vec != nullptr && base == b0)
        batch_harmonics_xyz<LMAX>(cx, cy, cz, sign, lane, cnt, ys, ux, uy, uz, inv, len);
      else
        batch_harmonics<G, LMAX>(vec, pos, cl, src, shift, (int)row, sign, lane, cnt, my_e, ys,
                                 ux, uy, uz, inv, len);
      if constexpr (RAD) {
        __builtin_amdgcn_sched_barrier(0);
        radial_row(R, tab, lane < cnt, len, hs + lane * kSH);
      }
      wave_sync();
      const int ntile = (cnt + 15) >> 4;
      // the matrix-core phase runs at a raised wave priority, so that the issue arbiter
      // keeps feeding it while other waves evaluate harmonics or wait on memory
      __builtin_amdgcn_s_setprio(1);
#pragma unroll 1
      for (int tau = 0; tau < ntile; ++tau) {
        if constexpr (RAD) {
#pragma unroll
          for (int q = 0; q < KK; ++q) ha[q] = hs[(16 * tau + hrow) * kSH + 4 * q + hi];
        } else {
#pragma unroll
          for (int q = 0; q < KK; ++q) ha[q] = hn[q];
          const int jn = 16 * (tau + 1) + hrow;
          const int ej = __shfl(my_e, jn & (kWave - 1));
#pragma unroll
          for (int q = 0; q < KK; ++q) {
            const int k = 4 * q + hi;
            hn[q] = (jn < cnt && k < K) ? h[(int64_t)ej * K + k] : 0.f;
          }
        }
        floatx4 ph[T];
#pragma unroll
        for (int t = 0; t < T; ++t) ph[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < KK; ++q) {
          float wb[T];
          load_run<T>(sW + (4 * q + hi) * SWS + lo * T, wb);
#pragma unroll
          for (int t = 0; t < T; ++t) ph[t] = mfma_16x16x4(ha[q], wb[t], ph[t]);
        }
        // ph[t][r] = phi[edge 16 tau + 4 r + hi][channel lo T + t]; rows past the batch's
        // end hold zero harmonics, so the last tile runs whole, without branches that
        // would split the accumulators' live ranges
        float a[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = ys[(16 * tau + 4 * r + hi) * kSY + lo];
        // k-steps past the batch's end are skipped (wave-uniform branches)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (r == 0 || 16 * tau + 4 * r < cnt) {
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = mfma_16x16x4(a[r], ph[t][r], acc[t]);
          }
      }
      __builtin_amdgcn_s_setprio(0);
      wave_sync();  // ys is rewritten by the next batch
    }
    // lane holds A[row, channel lo T + t, lm 4 hi + r]
    if constexpr (RO) {
      float part = 0.f;
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (4 * hi + r < L) part += acc[t][r] * sU[(lo * T + t) * L + 4 * hi + r];
      part = group_sum_f<kWave>(part);
      if (lane == 0) {
        float b = 0.f;
        if (bias != nullptr) {
          const int64_t zz = z[row];
          b = (zz >= 0 && zz < n_bias) ? bias[zz] : __builtin_nanf("");
        }
        out[row] = part + b;
      }
    } else {
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
}

// RO (readout): the cotangent of the row is d_A_i = g_i U (the adjoint of the readout
// E_i = <U, A_i> + bias): U's two operand layouts are loaded once per wave and kept in
// registers, and the row's products are scaled by g_i, so no (C, L) row is read or staged.
template <typename G, int LMAX, int T, bool RAD, bool RO>
__global__ __launch_bounds__(256, 3) void lin_msg_bwd_kernel(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cell,
    int64_t n_graphs, const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ shift, const int32_t* __restrict__ ptr,
    const int32_t* __restrict__ perm, int64_t n_nodes, float sign, int K,
    const float* __restrict__ h, Radial<float> R, const float* __restrict__ W,
    const float* __restrict__ d_out, float* __restrict__ d_h, float* __restrict__ g_vec,
    const float* __restrict__ U, const float* __restrict__ g_node, int64_t g_stride,
    float* __restrict__ edge_energy) {
  constexpr int L = ShDims<LMAX>::L;
  constexpr int C = 16 * T;
  constexpr int KS = (L + 3) / 4;
  constexpr int KK = kLinKK;
  static_assert(C * L <= 2 * kWave * kSY, "the staged d_out row must fit the LDS slice");
  __shared__ __align__(16) float sbuf[kWavesPerBlock][2 * kWave * kSY];
  const int wave = wave_in_block(), lane = threadIdx.x % kWave;
  const int lo = lane & 15, hi = lane >> 4;
  float* ys = sbuf[wave];
  float* sdy = sbuf[wave] + kWave * kSY;
  // RAD: per-edge radial features, overwritten tile by tile with d_h once read
  __shared__ float sH[kWavesPerBlock][RAD ? kWave * kSH : 1];
  float* hs = sH[wave];
  __shared__ float sTab[kLinKMax];
  const RadialTab tab = RAD ? load_radial_tab(R, sTab) : RadialTab{};
  const bool want_vec = RAD || g_vec != nullptr;
  // W in LDS, zero rows past K, twice: rows padded to C + 4 floats for the A operand of
  // phi^T = W^T h^T (k-step q: W[4 q + hi][lo T + t], a run of T floats), and permuted for
  // the B operand of d_h = d_phi W^T on the 4 x 4 x 1 products: sWp[k][hi][t][r] =
  // W[k][(4 hi + r) T + t], the four r of one (k, hi, t) a float4, (k, hi) rows padded to
  // 4 T + 4 floats (spreads the 16 addresses of one read over the banks)
  constexpr int SWS = C + 4;
  constexpr int SWP = 4 * T + 4;
  __shared__ __align__(16) float sW[kLinKMax * SWS];
  __shared__ __align__(16) float sWp[kLinKMax * 4 * SWP];
  for (int i = threadIdx.x; i < kLinKMax * C; i += blockDim.x) {
    const int k = i / C, c = i % C;
    const float w = k < K ? W[i] : 0.f;
    sW[k * SWS + c] = w;
    const int hq = c / (4 * T), rr = (c / T) % 4, tt = c % T;  // c = (4 hq + rr) T + tt
    sWp[(k * 4 + hq) * SWP + 4 * tt + rr] = w;
  }
  __syncthreads();
  // G rows of 16 floats are staged with their 4-float chunks permuted by channel,
  // chunk q of channel c at q ^ ((c / T) & 3), so that the 16 channels lo T + t of one
  // A-operand read fall into different banks
  constexpr bool SWZ = (L == 16);
  auto g_at = [](int c, int lm) {
    return SWZ ? c * 16 + ((((lm >> 2) ^ (c / T)) & 3) << 2) + (lm & 3) : c * L + lm;
  };
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  // the G operands: G[lo T + t][4 s + hi] (A of d_phi) and G[(4 hi + r) T + t][lo] (B of dY)
  float gA[T][KS], gB[T][4];
  if constexpr (RO) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
      for (int ss = 0; ss < KS; ++ss) {
        const int lm = 4 * ss + hi;
        gA[t][ss] = lm < L ? U[(lo * T + t) * L + lm] : 0.f;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) gB[t][r] = lo < L ? U[((4 * hi + r) * T + t) * L + lo] : 0.f;
    }
  }
  // RO: every row's cotangent is a multiple g_i U of the same U, so the tiles need not
  // respect the rows: a wave takes 64 consecutive CSR slots (edges of several receivers),
  // every tile is full, and each edge's gradient is scaled by its receiver's g_i at the
  // end (everything before is linear in it). Otherwise a wave takes one receiver row.
  const int64_t n_slots = RO ? (int64_t)ptr[n_nodes] : 0;
  // the lanes' receivers are needed for their cotangents (one per atom) and, without given
  // edge vectors, for the edge geometry; a broadcast cotangent with given vectors needs none
  const bool need_row = g_stride != 0 || vec == nullptr;
  const int64_t n_items = RO ? (n_slots + kWave - 1) / kWave : n_nodes;
  for (int64_t item = (int64_t)blockIdx.x * kWavesPerBlock + wave; item < n_items;
       item += n_waves) {
    int b0, b1;
    int64_t row;    // the receiver of this lane's slot
    if constexpr (RO) {
      b0 = (int)(item * kWave);
      b1 = (int)min<int64_t>(n_slots, (int64_t)b0 + kWave);
      row = 0;
      if (need_row) {
        // the receiver of the batch's first slot (binary search, uniform), then each lane
        // steps to its own (a batch spans a few rows)
        int64_t lo_r = 0, hi_r = n_nodes;  // ptr[lo_r] <= b0 < ptr[hi_r]
        while (hi_r - lo_r > 1) {
          const int64_t mid = (lo_r + hi_r) >> 1;
          if (ptr[mid] <= b0) lo_r = mid; else hi_r = mid;
        }
        row = lo_r;
        const int q = min(b0 + lane, b1 - 1);
        while (row + 1 < n_nodes && ptr[row + 1] <= q) ++row;
      }
    } else {
      row = item;
      b0 = ptr[row];
      b1 = ptr[row + 1];
      if (b0 == b1) continue;
    }
    // with given edge vectors, the first batch's are loaded before G is staged, so that
    // the two loads' latencies overlap
    float cx = 0.f, cy = 0.f, cz = 0.f;
    if (vec != nullptr) load_first_vec(vec, perm, b0, b1, lane, cx, cy, cz);
    const G* cl = cell == nullptr ? nullptr
                                  : (n_graphs <= 1 || batch == nullptr ? cell
                                                                       : cell + 9 * (int64_t)batch[row]);
    // stage G = d_out[row] (C x L) through LDS into the two operand layouts
    if constexpr (!RO) {
      const float4* g4 = reinterpret_cast<const float4*>(d_out + (int64_t)row * C * L);
      float4* s4 = reinterpret_cast<float4*>(sbuf[wave]);
      for (int i = lane; i < C * L / 4; i += kWave) {
        if constexpr (SWZ)
          s4[(i & ~3) | (((i & 3) ^ ((i >> 2) / T)) & 3)] = g4[i];
        else
          s4[i] = g4[i];
      }
    }
    // RAD: the first batch's vectors wait in the radial rows' LDS (free until the batch
    // starts), not in registers through the operand loads below
    if constexpr (RAD) {
      if (vec != nullptr) {
        hs[3 * lane + 0] = cx;
        hs[3 * lane + 1] = cy;
        hs[3 * lane + 2] = cz;
      }
    }
    wave_sync();
    if constexpr (!RO) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int ss = 0; ss < KS; ++ss) {
          const int lm = 4 * ss + hi;
          gA[t][ss] = lm < L ? sbuf[wave][g_at(lo * T + t, lm)] : 0.f;  // G[lo T + t][4 s + hi]
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)  // G[(4 hi + r) T + t][lo]
          gB[t][r] = lo < L ? sbuf[wave][g_at((4 * hi + r) * T + t, lo)] : 0.f;
      }
      wave_sync();  // the staging area becomes ys / sdy
    }

    for (int base = b0; base < b1; base += kWave) {
      const int cnt = min(kWave, b1 - base);
      const int my_e = lane < cnt ? (perm ? perm[base + lane] : base + lane) : 0;
      // B operand of phi^T for tile tau: h[edge 16 tau + lo][4 q + hi]; from global memory
      // with the next tile's in flight while a tile is computed, or from LDS (RAD)
      float hb[KK], hn[KK];
      if constexpr (!RAD) {
        const int ej = __shfl(my_e, lo);
#pragma unroll
        for (int q = 0; q < KK; ++q) {
          const int k = 4 * q + hi;
          hn[q] = (want_vec && lo < cnt && k < K) ? h[(int64_t)ej * K + k] : 0.f;
        }
      }
      float ux, uy, uz, inv, len;
      if (vec != nullptr && base == b0) {
        if constexpr (RAD) {
          cx = hs[3 * lane + 0];
          cy = hs[3 * lane + 1];
          cz = hs[3 * lane + 2];
        }
        batch_harmonics_xyz<LMAX>(cx, cy, cz, sign, lane, cnt, ys, ux, uy, uz, inv, len);
      } else {
        batch_harmonics<G, LMAX>(vec, pos, cl, src, shift, (int)row, sign, lane, cnt, my_e, ys,
                                 ux, uy, uz, inv, len);
      }
      RadialCache rcache;
      if constexpr (RAD) {
        __builtin_amdgcn_sched_barrier(0);
        radial_row(R, tab, lane < cnt, len, hs + lane * kSH, &rcache);
      }
      wave_sync();
      const int ntile = (cnt + 15) >> 4;
      __builtin_amdgcn_s_setprio(1);  // the matrix-core phase (see the forward)
#pragma unroll 1
      for (int tau = 0; tau < ntile; ++tau) {
        const int je = 16 * tau + lo;
        if constexpr (RAD) {
#pragma unroll
          for (int q = 0; q < KK; ++q) hb[q] = hs[je * kSH + 4 * q + hi];
        } else {
#pragma unroll
          for (int q = 0; q < KK; ++q) hb[q] = hn[q];
          const int jn = je + 16;
          const int ej = __shfl(my_e, jn & (kWave - 1));
#pragma unroll
          for (int q = 0; q < KK; ++q) {
            const int k = 4 * q + hi;
            hn[q] = (want_vec && jn < cnt && k < K) ? h[(int64_t)ej * K + k] : 0.f;
          }
        }
        if (want_vec) {
          // pt[t][r] = phi[edge je][channel (4 hi + r) T + t]
          floatx4 pt[T];
#pragma unroll
          for (int t = 0; t < T; ++t) pt[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int q = 0; q < KK; ++q) {
            float wa[T];
            load_run<T>(sW + (4 * q + hi) * SWS + lo * T, wa);
#pragma unroll
            for (int t = 0; t < T; ++t) pt[t] = mfma_16x16x4(wa[t], hb[q], pt[t]);
          }
          floatx4 dy = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < T; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) dy = mfma_16x16x4(pt[t][r], gB[t][r], dy);
          // dy[r] = dY[edge 16 tau + 4 hi + r][lm lo]
#pragma unroll
          for (int r = 0; r < 4; ++r) sdy[(16 * tau + 4 * hi + r) * kSY + lo] = dy[r];
        }
        // keep phi^T and d_phi from being live together
        __builtin_amdgcn_sched_barrier(0);
        // d_phi per channel tile t, dp[r] = d_phi[edge je][channel (4 hi + r) T + t] on the
        // 16 x 16 x 4 products, consumed at once by d_h = d_phi W^T on the 4 x 4 x 1 products
        // (no padded output columns, unlike the 16 x 16 x 4 form whose N = 16 would hold
        // K = 8 functions): block b = 4 hi + lo / 4 takes edges 4 (lo / 4) + i of the tile
        // (A: the lane's own d_phi) and functions k = 4 kh + j (B: W[k][c]) over the 32
        // channels (4 hi + r) T + t of its quarter hi; lane 4 b + j receives D[b][i][j] in
        // register i
        float yb[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) yb[s] = ys[je * kSY + 4 * s + hi];
        floatx4 dq0 = floatx4{0.f, 0.f, 0.f, 0.f}, dq1 = dq0;
        const float* wp0 = sWp + ((lo & 3) * 4 + hi) * SWP;
        const float* wp1 = wp0 + 16 * SWP;  // k + 4
#pragma unroll
        for (int t = 0; t < T; ++t) {
          floatx4 dp = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < KS; ++s) dp = mfma_16x16x4(gA[t][s], yb[s], dp);
          const float4 w0 = *reinterpret_cast<const float4*>(wp0 + 4 * t);
          const float4 w1 = *reinterpret_cast<const float4*>(wp1 + 4 * t);
          dq0 = mfma_4x4x1(dp[0], w0.x, dq0);
          dq1 = mfma_4x4x1(dp[0], w1.x, dq1);
          dq0 = mfma_4x4x1(dp[1], w0.y, dq0);
          dq1 = mfma_4x4x1(dp[1], w1.y, dq1);
          dq0 = mfma_4x4x1(dp[2], w0.z, dq0);
          dq1 = mfma_4x4x1(dp[2], w1.z, dq1);
          dq0 = mfma_4x4x1(dp[3], w0.w, dq0);
          dq1 = mfma_4x4x1(dp[3], w1.w, dq1);
        }
        // sum the four channel quarters (a fixed butterfly): dq{kh}[i] is then
        // d_h[edge 16 tau + 4 (lo / 4) + i][k = 4 kh + lo % 4] on every hi
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dq0[i] = add_xor16(dq0[i]);
          dq1[i] = add_xor16(dq1[i]);
          dq0[i] = add_xor32(dq0[i]);
          dq1[i] = add_xor32(dq1[i]);
        }
        if constexpr (RAD) {
          wave_sync();  // d_h goes into the rows of this tile, whose h was read above
          if (hi == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float* row_h = hs + (16 * tau + 4 * (lo >> 2) + i) * kSH + (lo & 3);
              row_h[0] = dq0[i];
              row_h[4] = dq1[i];
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = 16 * tau + 4 * (lo >> 2) + i;
            const int ej = __shfl(my_e, j);
            if (hi == 0 && j < cnt) {
              if ((lo & 3) < K) d_h[(int64_t)ej * K + (lo & 3)] = dq0[i];
              if (4 + (lo & 3) < K) d_h[(int64_t)ej * K + 4 + (lo & 3)] = dq1[i];
            }
          }
        }
      }
      __builtin_amdgcn_s_setprio(0);
      wave_sync();
      if (want_vec && lane < cnt) {
        // d|r| from the radial features first, then the harmonics' share (kept apart so
        // that their temporaries are not live together)
        float dl = 0.f;
        if constexpr (RAD) dl = radial_dot(R, tab, rcache, hs + lane * kSH);
        __builtin_amdgcn_sched_barrier(0);
        float dY[L];
#pragma unroll
        for (int m = 0; m < L; ++m) dY[m] = sdy[lane * kSY + m];
        if constexpr (RO) {
          // the edge's share of its receiver's <U, A_i>: (phi_e U) . Y_e, the unscaled dY
          // against the edge's harmonics (still in its LDS row)
          if (edge_energy != nullptr) {
            float se = 0.f;
#pragma unroll
            for (int m = 0; m < L; ++m) se = fmaf(dY[m], ys[lane * kSY + m], se);
            edge_energy[my_e] = se;
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
        if constexpr (RO) {
          // the lane's receiver's cotangent scale (everything above is linear in it)
          const float gs = g_node[row * g_stride];
          vx *= gs;
          vy *= gs;
          vz *= gs;
        }
        g_vec[3 * (int64_t)my_e + 0] = sign * vx;
        g_vec[3 * (int64_t)my_e + 1] = sign * vy;
        g_vec[3 * (int64_t)my_e + 2] = sign * vz;
      }
      wave_sync();
    }
  }
}

// the readout arguments of the RO kernels (all NULL / 0 for the A-row kernels)
struct Readout {
  const float* U = nullptr;       // (C, L)
  const int64_t* z = nullptr;     // forward: per-atom bias index
  const float* bias = nullptr;    // forward: per-index bias (may be NULL)
  int64_t n_bias = 0;
  const float* g = nullptr;       // backward: per-atom cotangent of E_i
  int64_t g_stride = 1;
  float* edge_energy = nullptr;   // backward: each edge's share of <U, A_i> (may be NULL)
};

template <typename G, bool RAD, bool RO>
static void lin_msg_launch(bool backward, const float* vec, const void* pos, int64_t n_nodes,
                           const void* cell, int64_t n_graphs, const int32_t* batch,
                           const int32_t* src, const int32_t* shift, const int32_t* ptr,
                           const int32_t* perm, int l_max, int sign, int K, int C,
                           const float* h, const Radial<float>& R, const float* W,
                           const float* d_out, float* out_or_dh, float* g_vec,
                           const Readout& ro, int64_t n_edges, hipStream_t stream) {
  // a wave per receiver row, or (readout backward) per 64 consecutive CSR slots
  const int64_t blocks_needed =
      backward && RO ? grid_1d(std::max<int64_t>(1, (n_edges + kWave - 1) / kWave), kWavesPerBlock)
                     : grid_1d(n_nodes, kWavesPerBlock);
  const dim3 block(kWavesPerBlock * kWave);
  const float sg = (float)sign;
#define XNN_LIN(LM, TT)                                                                        \
  do {                                                                                         \
    if (backward) {                                                                            \
      auto k = lin_msg_bwd_kernel<G, LM, TT, RAD, RO>;                                         \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, blocks_needed));      \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, sg, K, h, R, W,       \
                         d_out, out_or_dh, g_vec, ro.U, ro.g, ro.g_stride, ro.edge_energy);    \
    } else {                                                                                   \
      auto k = lin_msg_fwd_kernel<G, LM, TT, RAD, RO>;                                         \
      const dim3 grid((unsigned)resident_blocks((const void*)k, block.x, blocks_needed));      \
      hipLaunchKernelGGL(k, grid, block, 0, stream, vec, (const G*)pos, (const G*)cell,        \
                         n_graphs, batch, src, shift, ptr, perm, n_nodes, sg, K, h, R, W,       \
                         out_or_dh, ro.U, ro.z, ro.bias, ro.n_bias);                           \
    }                                                                                          \
  } while (0)
#define XNN_LIN_L(TT)                   \
  switch (l_max) {                      \
    case 1: XNN_LIN(1, TT); break;      \
    case 2: XNN_LIN(2, TT); break;      \
    default: XNN_LIN(3, TT); break;     \
  }
  switch (C) {
    case 32: XNN_LIN_L(2); break;
    case 64: XNN_LIN_L(4); break;
    default: XNN_LIN_L(8); break;
  }
#undef XNN_LIN_L
#undef XNN_LIN
}

// The readout kernels: h is evaluated in the kernels from R (K = R.K).
template <typename G>
static int lin_msg(bool backward, const float* vec, const void* pos, int64_t n_nodes,
                   const void* cell, int64_t n_graphs, const int32_t* batch, const int32_t* src,
                   const int32_t* shift, const int32_t* ptr, const int32_t* perm, int l_max,
                   int sign, int C, const Radial<float>& R, const float* W, float* out,
                   float* g_vec, hipStream_t stream, const Readout& ro, int64_t n_edges = 0) {
  if (n_nodes == 0) return XNN_OK;
  lin_msg_launch<G, true, true>(backward, vec, pos, n_nodes, cell, n_graphs, batch, src, shift,
                                ptr, perm, l_max, sign, R.K, C, nullptr, R, W, nullptr, out,
                                g_vec, ro, n_edges, stream);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

static int lin_check(int64_t n_nodes, int64_t n_edges, int32_t l_max, int32_t sh_sign,
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
  st = lin_check(n_nodes, n_edges, prm->l_max, prm->sh_sign, prm->n_rbf, n_channels);
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
    return lin_msg<float>(false, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift, ptr_dst,
                          perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W, node_energy,
                          nullptr, as_hip(stream), ro);
  if (geom_dtype == XNN_F64)
    return lin_msg<double>(false, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                           ptr_dst, perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W,
                           node_energy, nullptr, as_hip(stream), ro);
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
  Radial<float> R;
  int st = make_radial<float>(prm, rbf_table, R);
  if (st != XNN_OK) return st;
  st = lin_check(n_nodes, n_edges, prm->l_max, prm->sh_sign, prm->n_rbf, n_channels);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && g && W && U), "NULL CSR, weights or cotangent");
  XNN_REQUIRE(g_stride == 0 || g_stride == 1, "g_stride must be 0 (broadcast) or 1");
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && shift)) && g_vec),
              "NULL edge input or output");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  Readout ro;
  ro.U = U;
  ro.g = g;
  ro.g_stride = g_stride;
  if (geom_dtype == XNN_F32)
    return lin_msg<float>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift, ptr_dst,
                          perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W, nullptr, g_vec,
                          as_hip(stream), ro, n_edges);
  if (geom_dtype == XNN_F64)
    return lin_msg<double>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                           ptr_dst, perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W, nullptr,
                           g_vec, as_hip(stream), ro, n_edges);
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
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
  Radial<float> R;
  int st = make_radial<float>(prm, rbf_table, R);
  if (st != XNN_OK) return st;
  st = lin_check(n_nodes, n_edges, prm->l_max, prm->sh_sign, prm->n_rbf, n_channels);
  if (st != XNN_OK) return st;
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && g && W && U), "NULL CSR, weights or cotangent");
  XNN_REQUIRE(g_stride == 0 || g_stride == 1, "g_stride must be 0 (broadcast) or 1");
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && shift)) && g_vec && edge_energy),
              "NULL edge input or output");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  Readout ro;
  ro.U = U;
  ro.g = g;
  ro.g_stride = g_stride;
  ro.edge_energy = edge_energy;
  if (geom_dtype == XNN_F32)
    return lin_msg<float>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift, ptr_dst,
                          perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W, nullptr, g_vec,
                          as_hip(stream), ro, n_edges);
  if (geom_dtype == XNN_F64)
    return lin_msg<double>(true, vec_in, pos, n_nodes, cell, n_graphs, batch, src, shift,
                           ptr_dst, perm_dst, prm->l_max, prm->sh_sign, n_channels, R, W, nullptr,
                           g_vec, as_hip(stream), ro, n_edges);
  set_error("unsupported geometry dtype %d", geom_dtype);
  return XNN_EINVAL;
}

}  // extern "C"
