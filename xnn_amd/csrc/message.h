// Device helpers shared by the message-aggregation kernels (gfx950, wave64).
#pragma once
#include <cstdint>

#include "common.h"
#include "device.h"

namespace xnn {

constexpr int kWavesPerBlock = 4;

// host: compute units of the current device (cached per device id)
int device_cu_count();
// host: blocks of `kernel` that stay resident on the whole device, capped at `needed`
int64_t resident_blocks(const void* kernel, int block_threads, int64_t needed);
// host: NULL or 16-byte aligned
bool aligned16(const void* p);
// host: false when XNN_AMD_MESSAGE_MFMA=0 (vector-ALU message kernels)
bool message_mfma_enabled();

template <int LMAX>
struct ShDims {
  static constexpr int L = (LMAX + 1) * (LMAX + 1);
  // partial sums are reduced across the wave padded to a power of two
  static constexpr int LP = L == 1 ? 1 : (L <= 4 ? 4 : 16);
};

// host: the device form of the edge-embedding parameters (validated)
template <typename T>
inline int make_radial(const xnn_featurize_params* prm, const void* table, Radial<T>& R) {
  XNN_REQUIRE(prm != nullptr, "featurize params are NULL");
  XNN_REQUIRE(prm->n_rbf >= 0 && prm->n_rbf <= kMaxRbf, "n_rbf must be in [0, %d], got %d",
              kMaxRbf, prm->n_rbf);
  XNN_REQUIRE(prm->n_rbf == 0 || table != nullptr, "rbf_table is NULL");
  XNN_REQUIRE(prm->basis == XNN_BASIS_BESSEL || prm->basis == XNN_BASIS_GAUSSIAN,
              "unknown basis %d", prm->basis);
  XNN_REQUIRE(prm->envelope >= XNN_ENV_POLYNOMIAL && prm->envelope <= XNN_ENV_NONE,
              "unknown envelope %d", prm->envelope);
  XNN_REQUIRE(prm->envelope != XNN_ENV_POLYNOMIAL || (prm->poly_p >= 1 && prm->poly_p <= 64),
              "polynomial envelope degree must be in [1, 64], got %d", prm->poly_p);
  XNN_REQUIRE(prm->cutoff > 0, "cutoff must be positive");
  XNN_REQUIRE(prm->l_max >= 0 && prm->l_max <= 3, "l_max must be in [0, 3], got %d",
              prm->l_max);
  XNN_REQUIRE(prm->sh_sign == 1 || prm->sh_sign == -1, "sh_sign must be +1 or -1");
  R.K = prm->n_rbf;
  R.basis = prm->basis;
  R.envelope = prm->envelope;
  R.p = prm->poly_p;
  R.rc = (T)prm->cutoff;
  R.inv_rc = (T)(1.0 / prm->cutoff);
  R.prefactor = (T)prm->rbf_prefactor;
  R.gamma = (T)prm->gaussian_gamma;
  R.table = static_cast<const T*>(table);
  return XNN_OK;
}

// Unit vector of sign * (x, y, z), 1/|(x, y, z)| (0 for a zero vector) and the length
__device__ __forceinline__ void unit_of(float x, float y, float z, float sign, float& ux,
                                        float& uy, float& uz, float& inv, float& r) {
  r = sqrtf(x * x + y * y + z * z);
  inv = r > 0.f ? 1.f / r : 0.f;
  ux = sign * x * inv;
  uy = sign * y * inv;
  uz = sign * z * inv;
}

// Per-lane geometry of one edge: unit vector of sign * r_e, 1/|r_e| and |r_e|; the
// vector is given (vec) or formed from positions.
template <typename G>
__device__ inline void edge_unit(const float* __restrict__ vec, int64_t e,
                                 const G* __restrict__ pos, const G* __restrict__ cell,
                                 const int32_t* __restrict__ src, const int32_t* __restrict__ shift,
                                 int d, float sign, float& ux, float& uy, float& uz, float& inv,
                                 float& r) {
  float x, y, z;
  if (vec != nullptr) {
    x = vec[3 * e + 0];
    y = vec[3 * e + 1];
    z = vec[3 * e + 2];
  } else {
    G gx, gy, gz;
    edge_vector(pos, src[e], d, shift[e], cell, gx, gy, gz);
    x = (float)gx;
    y = (float)gy;
    z = (float)gz;
  }
  unit_of(x, y, z, sign, ux, uy, uz, inv, r);
}

// The lane's given edge vector in the first batch of a receiver row's edges [b0, b1)
// (zeros past the batch's end): loaded a row ahead of its use, so that its latency
// overlaps the previous row's products
__device__ __forceinline__ void load_first_vec(const float* __restrict__ vec,
                                               const int32_t* __restrict__ perm, int b0, int b1,
                                               int lane, float& x, float& y, float& z) {
  x = y = z = 0.f;
  if (lane < min(kWave, b1 - b0)) {
    const int64_t e = perm ? perm[b0 + lane] : b0 + lane;
    x = vec[3 * e + 0];
    y = vec[3 * e + 1];
    z = vec[3 * e + 2];
  }
}

// ---------------------------------------------------------------- matrix-core helpers
// v_mfma_f32_16x16x4_f32 (float32 inputs, float32 accumulation), one wave: per
// 16 x 16 x 4 block, lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and receives
// D[4 (l / 16) + r][l % 16] in register r.
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma_16x16x4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// v_mfma_f32_4x4x1f32, 16 independent 4 x 4 x 1 blocks: lane 4 b + i supplies A[b][i],
// lane 4 b + j supplies B[b][j], and lane 4 b + j receives D[b][i][j] in register i
// (checked on gfx950 with a lane-index probe).
__device__ __forceinline__ floatx4 mfma_4x4x1(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

// N consecutive floats at p (vector accesses: p is 4N-byte aligned within 16 bytes)
template <int N>
__device__ __forceinline__ void load_run(const float* __restrict__ p, float* v) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int q = 0; q < N; q += 4) {
      const float4 x = *reinterpret_cast<const float4*>(p + q);
      v[q] = x.x; v[q + 1] = x.y; v[q + 2] = x.z; v[q + 3] = x.w;
    }
  } else if constexpr (N % 2 == 0) {
#pragma unroll
    for (int q = 0; q < N; q += 2) {
      const float2 x = *reinterpret_cast<const float2*>(p + q);
      v[q] = x.x; v[q + 1] = x.y;
    }
  } else {
#pragma unroll
    for (int q = 0; q < N; ++q) v[q] = p[q];
  }
}

template <int N>
__device__ __forceinline__ void store_run(float* __restrict__ p, const float* v) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int q = 0; q < N; q += 4)
      *reinterpret_cast<float4*>(p + q) = make_float4(v[q], v[q + 1], v[q + 2], v[q + 3]);
  } else if constexpr (N % 2 == 0) {
#pragma unroll
    for (int q = 0; q < N; q += 2) *reinterpret_cast<float2*>(p + q) = make_float2(v[q], v[q + 1]);
  } else {
#pragma unroll
    for (int q = 0; q < N; ++q) p[q] = v[q];
  }
}

constexpr int kSY = 17;  // LDS row stride of per-edge harmonics (spreads the banks)

// Lane's edge of the batch (lanes < cnt), and the harmonics of that edge into ys
// (row `lane`, 16 entries, zeros past l_max and past the batch's end).
template <typename G, int LMAX>
__device__ __forceinline__ void batch_harmonics(
    const float* __restrict__ vec, const G* __restrict__ pos, const G* __restrict__ cl,
    const int32_t* __restrict__ src, const int32_t* __restrict__ shift, int row, float sign,
    int lane, int cnt, int e, float* ys, float& ux, float& uy, float& uz, float& inv, float& r) {
  constexpr int L = ShDims<LMAX>::L;
  float Y[L];
  if (lane < cnt) {
    edge_unit(vec, e, pos, cl, src, shift, row, sign, ux, uy, uz, inv, r);
    sh_eval<LMAX, float>(ux, uy, uz, Y);
  } else {
    ux = uy = uz = inv = r = 0.f;
#pragma unroll
    for (int m = 0; m < L; ++m) Y[m] = 0.f;
  }
#pragma unroll
  for (int m = 0; m < 16; ++m) ys[lane * kSY + m] = m < L ? Y[m] : 0.f;
}

// batch_harmonics of an edge vector already in registers
template <int LMAX>
__device__ __forceinline__ void batch_harmonics_xyz(float x, float y, float z, float sign,
                                                    int lane, int cnt, float* ys, float& ux,
                                                    float& uy, float& uz, float& inv, float& r) {
  constexpr int L = ShDims<LMAX>::L;
  float Y[L];
  if (lane < cnt) {
    unit_of(x, y, z, sign, ux, uy, uz, inv, r);
    sh_eval<LMAX, float>(ux, uy, uz, Y);
  } else {
    ux = uy = uz = inv = r = 0.f;
#pragma unroll
    for (int m = 0; m < L; ++m) Y[m] = 0.f;
  }
#pragma unroll
  for (int m = 0; m < 16; ++m) ys[lane * kSY + m] = m < L ? Y[m] : 0.f;
}

}  // namespace xnn
