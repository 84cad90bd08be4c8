// Per-atom linear readout of node rows and its adjoint (gfx950, wave64).
//
//   out[i]    = bias[z[i]] + sum_f rows[i][f] w[f]        (xnn_node_readout)
//   d_rows[i][f] = g[i * g_stride] w[f]                   (xnn_node_readout_backward)
//
// Both are streams over the (N, F) rows: one wave per row, 16-byte loads / stores, four
// vectors in flight per lane, and the row dot product reduced by a fixed butterfly
// (repeated calls agree bit for bit). The per-atom bias gather is folded into the forward
// (no separate index launch). The loads and stores are ordinary (cached) ones: the rows
// (74 MB at the water box) fit MI355X's 256 MB Infinity Cache, the forward reads the rows
// the message kernel has just written and the message backward reads the cotangent rows
// the backward writes here (non-temporal hints cost 1.8 us of a 95 us step).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "device.h"

namespace xnn {

template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
  typedef float type __attribute__((ext_vector_type(4)));
  static constexpr int n = 4;
};
template <>
struct Vec16<double> {
  typedef double type __attribute__((ext_vector_type(2)));
  static constexpr int n = 2;
};

constexpr int kReadoutRows = 4;  // rows (waves) per 256-thread block

template <typename T>
__device__ inline T vdot(typename Vec16<T>::type a, typename Vec16<T>::type b);
template <>
__device__ inline float vdot<float>(Vec16<float>::type a, Vec16<float>::type b) {
  return (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w);
}
template <>
__device__ inline double vdot<double>(Vec16<double>::type a, Vec16<double>::type b) {
  return a.x * b.x + a.y * b.y;
}

// VEC: rows and w are 16-byte aligned and F is a multiple of the vector width
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void readout_fwd_kernel(
    const T* __restrict__ rows, int64_t n, int64_t F, const T* __restrict__ w,
    const int64_t* __restrict__ z, const T* __restrict__ bias, int64_t n_bias,
    T* __restrict__ out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kReadoutRows + wave_in_block();
  if (row >= n) return;
  // the bias gather (two dependent loads) is issued first, so that its latency passes
  // under the row's stream instead of following it
  T b = 0;
  if (bias != nullptr) {
    const int64_t zz = z[row];
    b = (zz >= 0 && zz < n_bias) ? bias[zz] : (T)__builtin_nan("");
  }
  T acc = 0;
  if (VEC) {
    typedef typename Vec16<T>::type VT;
    const int64_t nv = F / Vec16<T>::n;
    const VT* a = reinterpret_cast<const VT*>(rows + row * F);
    const VT* wv = reinterpret_cast<const VT*>(w);
    T acc1 = 0;
    int64_t v = lane;
    for (; v + 3 * kWave < nv; v += 4 * kWave) {
      const VT a0 = a[v];
      const VT a1 = a[v + kWave];
      const VT a2 = a[v + 2 * kWave];
      const VT a3 = a[v + 3 * kWave];
      acc += vdot<T>(a0, wv[v]) + vdot<T>(a2, wv[v + 2 * kWave]);
      acc1 += vdot<T>(a1, wv[v + kWave]) + vdot<T>(a3, wv[v + 3 * kWave]);
    }
    for (; v < nv; v += kWave) acc += vdot<T>(a[v], wv[v]);
    acc += acc1;
  } else {
    const T* a = rows + row * F;
    for (int64_t f = lane; f < F; f += kWave) acc += a[f] * w[f];
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane == 0) out[row] = b + acc;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void readout_bwd_kernel(const T* __restrict__ g,
                                                          int64_t g_stride, int64_t n,
                                                          int64_t F, const T* __restrict__ w,
                                                          T* __restrict__ d_rows) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kReadoutRows + wave_in_block();
  if (row >= n) return;
  const T gi = g[row * g_stride];
  if (VEC) {
    typedef typename Vec16<T>::type VT;
    const int64_t nv = F / Vec16<T>::n;
    VT* d = reinterpret_cast<VT*>(d_rows + row * F);
    const VT* wv = reinterpret_cast<const VT*>(w);
    for (int64_t v = lane; v < nv; v += kWave) d[v] = gi * wv[v];
  } else {
    T* d = d_rows + row * F;
    for (int64_t f = lane; f < F; f += kWave) d[f] = gi * w[f];
  }
}

template <typename T>
static int readout(const void* rows, int64_t n, int64_t F, const void* w, const int64_t* z,
                   const void* bias, int64_t n_bias, void* out, hipStream_t s) {
  const bool vec = ((uintptr_t)rows % 16 == 0) && ((uintptr_t)w % 16 == 0) &&
                   (F % Vec16<T>::n == 0);
  const dim3 grid(grid_1d(n, kReadoutRows)), block(kReadoutRows * kWave);
  const T* r = static_cast<const T*>(rows);
  const T* wt = static_cast<const T*>(w);
  const T* b = static_cast<const T*>(bias);
  T* o = static_cast<T*>(out);
  if (vec)
    hipLaunchKernelGGL((readout_fwd_kernel<T, true>), grid, block, 0, s, r, n, F, wt, z, b,
                       n_bias, o);
  else
    hipLaunchKernelGGL((readout_fwd_kernel<T, false>), grid, block, 0, s, r, n, F, wt, z, b,
                       n_bias, o);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

template <typename T>
static int readout_bwd(const void* g, int64_t g_stride, int64_t n, int64_t F, const void* w,
                       void* d_rows, hipStream_t s) {
  const bool vec = ((uintptr_t)d_rows % 16 == 0) && ((uintptr_t)w % 16 == 0) &&
                   (F % Vec16<T>::n == 0);
  const dim3 grid(grid_1d(n, kReadoutRows)), block(kReadoutRows * kWave);
  const T* gt = static_cast<const T*>(g);
  const T* wt = static_cast<const T*>(w);
  T* d = static_cast<T*>(d_rows);
  if (vec)
    hipLaunchKernelGGL((readout_bwd_kernel<T, true>), grid, block, 0, s, gt, g_stride, n, F, wt,
                       d);
  else
    hipLaunchKernelGGL((readout_bwd_kernel<T, false>), grid, block, 0, s, gt, g_stride, n, F, wt,
                       d);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

}  // namespace xnn

using namespace xnn;

extern "C" {

int xnn_node_readout(int dtype, const void* rows, int64_t n_rows, int64_t n_features,
                     const void* weights, const int64_t* z, const void* bias, int64_t n_bias,
                     void* out, xnn_stream_t stream) {
  XNN_REQUIRE(dtype == XNN_F32 || dtype == XNN_F64, "dtype must be XNN_F32 or XNN_F64");
  XNN_REQUIRE(n_rows >= 0 && n_features >= 0, "negative size");
  XNN_REQUIRE((bias == nullptr) == (z == nullptr), "bias and z go together");
  XNN_REQUIRE(bias == nullptr || n_bias >= 1, "empty bias table");
  if (n_rows == 0) return XNN_OK;
  XNN_REQUIRE(out != nullptr && (n_features == 0 || (rows && weights)), "NULL input or output");
  XNN_REQUIRE(n_rows <= (int64_t)kReadoutRows * 0x7fffffff, "too many rows");
  hipStream_t s = as_hip(stream);
  return dtype == XNN_F32 ? readout<float>(rows, n_rows, n_features, weights, z, bias, n_bias,
                                           out, s)
                          : readout<double>(rows, n_rows, n_features, weights, z, bias, n_bias,
                                            out, s);
}

int xnn_node_readout_backward(int dtype, const void* g, int64_t g_stride, int64_t n_rows,
                              int64_t n_features, const void* weights, void* d_rows,
                              xnn_stream_t stream) {
  XNN_REQUIRE(dtype == XNN_F32 || dtype == XNN_F64, "dtype must be XNN_F32 or XNN_F64");
  XNN_REQUIRE(n_rows >= 0 && n_features >= 0, "negative size");
  if (n_rows == 0 || n_features == 0) return XNN_OK;
  XNN_REQUIRE(g && weights && d_rows, "NULL input or output");
  XNN_REQUIRE(g_stride == 0 || g_stride == 1, "g_stride must be 0 (one value) or 1");
  XNN_REQUIRE(n_rows <= (int64_t)kReadoutRows * 0x7fffffff, "too many rows");
  hipStream_t s = as_hip(stream);
  return dtype == XNN_F32
             ? readout_bwd<float>(g, g_stride, n_rows, n_features, weights, d_rows, s)
             : readout_bwd<double>(g, g_stride, n_rows, n_features, weights, d_rows, s);
}

}  // extern "C"
