// Fused hidden layers of a per-edge radial network (gfx950, wave64, fp32 MFMA).
//
// xnn_radial_hidden(_backward): the hidden layers s_n = silu(c_n s_{n-1} A_n), n = 1..L
// (L <= 3, s_0 = x of shape (E, K) with K <= 32, widths <= 128, float32 products without
// reduced-precision inputs), in one pass over the edges with the activations in registers
// (gnn/fast/radial_kernels.py:43-58 forward, 61-80 backward; the layers and their scalar
// factors c_n as RadialNet folds them, gnn/models/blocks.py:360-405). The backward
// recomputes the activations and returns only the input gradient
// d x = c_1 (g_1 * silu'(z_1)) A_1^T with g_{n-1} = c_n (g_n * silu'(z_n)) A_n^T.
//
// One wave owns a tile of 16 edges and computes every product transposed,
// z^T (width x 16 edges) = A^T s^T, on v_mfma_f32_16x16x4_f32. A result tile is then the
// B operand of the next product as it stands: register i of lane l holds row 4 (l / 16) + i
// of a 16-row tile for edge l % 16, so k-step (t, i) pairs the k index l / 16 with hidden
// unit 16 t + 4 (l / 16) + i and reads the matching weight. Nothing is transposed or
// exchanged between layers, forward or backward.
//
// The weights sit in LDS, zero-padded to 16 x 16 blocks (padded units stay zero through
// silu and contribute nothing). Each block is stored swizzled, element (a, b) at word
// 64 s + 16 ((a / 4 + s) mod 4) + (b + s) mod 16 with s = a mod 4: the three access
// patterns (a layer's product, the first layer's k-steps and the backward's transposed
// product) then each read 64 distinct banks per instruction.
#include <algorithm>
#include <cstdint>

#include "common.h"
#include "device.h"
#include "message.h"

namespace xnn {

constexpr int kRadWaves = 4;           // waves per block
constexpr int kRadMaxIn = 32;          // input features
constexpr int kRadMaxWidth = 128;      // hidden units per layer
constexpr int kRadMaxLayers = 3;

struct RadialArgs {
  const float* x;        // (E, n_in)
  const float* grad;     // (E, width[L-1]) backward only
  float* out;            // forward: (E, width[L-1]); backward: (E, n_in)
  const float* w[kRadMaxLayers];
  float scale[kRadMaxLayers];
  int width[kRadMaxLayers];
  int n_in;
  int64_t n_rows;
};

__host__ __device__ constexpr int rad_swizzle(int a, int b) {
  return 64 * (a & 3) + 16 * (((a >> 2) + (a & 3)) & 3) + ((b + (a & 3)) & 15);
}

// words of the LDS tables: layer 1 (K0P rounded up to 16 rows) and L - 1 square layers
template <int NL, int K0P, int HP>
struct RadialTables {
  static constexpr int RB1 = (K0P + 15) / 16;
  static constexpr int CB = HP / 16;
  static constexpr int words1 = RB1 * 16 * HP;
  static constexpr int wordsN = HP * HP;
  static constexpr int words = words1 + (NL - 1) * wordsN;
  __device__ static int base(int n) { return n == 0 ? 0 : words1 + (n - 1) * wordsN; }
  // word of element (h, c) of layer n's padded matrix
  __device__ static int at(int n, int h, int c) {
    return base(n) + (((h >> 4) * CB + (c >> 4)) << 8) + rad_swizzle(h & 15, c & 15);
  }
};

template <int NL, int K0P, int HP>
__device__ __forceinline__ void rad_stage(const RadialArgs& A, float* lds) {
  using T = RadialTables<NL, K0P, HP>;
  for (int n = 0; n < NL; ++n) {
    const int rows = n == 0 ? A.n_in : A.width[n - 1];
    const int cols = A.width[n];
    const int rows_p = n == 0 ? T::RB1 * 16 : HP;
    const float* __restrict__ w = A.w[n];
    for (int idx = threadIdx.x; idx < rows_p * HP; idx += blockDim.x) {
      const int h = idx / HP, c = idx % HP;
      lds[T::at(n, h, c)] = (h < rows && c < cols) ? w[(int64_t)h * cols + c] : 0.f;
    }
  }
  __syncthreads();
}

// sigma(z) = 1 / (1 + 2^(-z log2 e)) on the hardware exponential and reciprocal (each about
// 1 ulp; the error of the argument's rounding grows with |z|, ~1e-6 relative at |z| ~ 10).
// The activations cost more vector instructions than the products they follow: the
// library's expf and division would make the kernel vector-ALU bound. Large |z| saturates
// cleanly: 2^(+big) = inf gives sigma = 0, 2^(-big) = 0 gives sigma = 1.
__device__ __forceinline__ float rad_sigmoid(float z) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * z));
}

// silu(z) and silu'(z) = sigma(z) (1 + z (1 - sigma(z)))
__device__ __forceinline__ float rad_silu(float z) { return z * rad_sigmoid(z); }
__device__ __forceinline__ float rad_dsilu(float z) {
  const float s = rad_sigmoid(z);
  return s * (1.f + z * (1.f - s));
}

// z^T of layer 1 for the wave's 16 edges: NT result tiles of 16 hidden rows
template <int NL, int K0P, int HP>
__device__ __forceinline__ void rad_layer1(const RadialArgs& A, const float* lds, int64_t edge,
                                           bool valid, int g, int r, floatx4* acc) {
  using T = RadialTables<NL, K0P, HP>;
  constexpr int NT = HP / 16;
#pragma unroll
  for (int o = 0; o < NT; ++o) acc[o] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < K0P / 4; ++s) {
    const int k = 4 * s + g;
    const float xk = (valid && k < A.n_in) ? A.x[edge * A.n_in + k] : 0.f;
#pragma unroll
    for (int o = 0; o < NT; ++o) acc[o] = mfma_16x16x4(lds[T::at(0, k, 16 * o + r)], xk, acc[o]);
  }
}

// z^T of layer n >= 1 (0-based) from the previous activations s (NT tiles)
template <int NL, int K0P, int HP>
__device__ __forceinline__ void rad_layer(const float* lds, int n, int g, int r,
                                          const floatx4* s, floatx4* acc) {
  using T = RadialTables<NL, K0P, HP>;
  constexpr int NT = HP / 16;
#pragma unroll
  for (int o = 0; o < NT; ++o) acc[o] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 16 * t + 4 * g + i;
#pragma unroll
      for (int o = 0; o < NT; ++o) acc[o] = mfma_16x16x4(lds[T::at(n, h, 16 * o + r)], s[t][i], acc[o]);
    }
  }
}

// (A_n d^T) for the backward: rows are layer n's inputs (RT tiles), k runs over its outputs
template <int NL, int K0P, int HP, int RT>
__device__ __forceinline__ void rad_layer_t(const float* lds, int n, int g, int r,
                                            const floatx4* d, floatx4* acc) {
  using T = RadialTables<NL, K0P, HP>;
  constexpr int NT = HP / 16;
#pragma unroll
  for (int o = 0; o < RT; ++o) acc[o] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 16 * t + 4 * g + i;
#pragma unroll
      for (int o = 0; o < RT; ++o) acc[o] = mfma_16x16x4(lds[T::at(n, 16 * o + r, c)], d[t][i], acc[o]);
    }
  }
}

// row `edge` of a (E, cols) matrix, columns 16 o + 4 g + i of the wave's tiles
template <int NT>
__device__ __forceinline__ void rad_store(float* __restrict__ out, int64_t edge, bool valid,
                                          int cols, int g, const floatx4* v) {
  if (!valid) return;
  float* row = out + edge * cols;
  const bool vec = (cols & 3) == 0;
#pragma unroll
  for (int o = 0; o < NT; ++o) {
    const int c = 16 * o + 4 * g;
    if (c >= cols) continue;
    if (vec) {
      *reinterpret_cast<float4*>(row + c) = make_float4(v[o][0], v[o][1], v[o][2], v[o][3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c + i < cols) row[c + i] = v[o][i];
    }
  }
}

template <int NT>
__device__ __forceinline__ void rad_load(const float* __restrict__ in, int64_t edge, bool valid,
                                         int cols, int g, floatx4* v) {
  const float* row = in + edge * cols;
  const bool vec = (cols & 3) == 0;
#pragma unroll
  for (int o = 0; o < NT; ++o) {
    const int c = 16 * o + 4 * g;
    v[o] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (!valid || c >= cols) continue;
    if (vec) {
      const float4 q = *reinterpret_cast<const float4*>(row + c);
      v[o] = floatx4{q.x, q.y, q.z, q.w};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c + i < cols) v[o][i] = row[c + i];
    }
  }
}

template <int NL, int K0P, int HP>
__global__ __launch_bounds__(kRadWaves * kWave) void radial_hidden_fwd(RadialArgs A) {
  extern __shared__ float rad_lds[];
  constexpr int NT = HP / 16;
  rad_stage<NL, K0P, HP>(A, rad_lds);
  const int lane = threadIdx.x % kWave, g = lane >> 4, r = lane & 15;
  const int64_t n_tiles = (A.n_rows + 15) / 16;
  const int width_out = A.width[NL - 1];
  for (int64_t tile = (int64_t)blockIdx.x * kRadWaves + wave_in_block(); tile < n_tiles;
       tile += (int64_t)gridDim.x * kRadWaves) {
    // the weights are re-read from LDS for every tile: without this the compiler hoists
    // every loop-invariant LDS read out of the tile loop and spills the registers
    asm volatile("" ::: "memory");
    const int64_t edge = tile * 16 + r;
    const bool valid = edge < A.n_rows;
    floatx4 s[NT], acc[NT];
    rad_layer1<NL, K0P, HP>(A, rad_lds, edge, valid, g, r, acc);
#pragma unroll
    for (int o = 0; o < NT; ++o)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[o][i] = rad_silu(A.scale[0] * acc[o][i]);
#pragma unroll
    for (int n = 1; n < NL; ++n) {
      rad_layer<NL, K0P, HP>(rad_lds, n, g, r, s, acc);
#pragma unroll
      for (int o = 0; o < NT; ++o)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[o][i] = rad_silu(A.scale[n] * acc[o][i]);
    }
    rad_store<NT>(A.out, edge, valid, width_out, g, s);
  }
}

template <int NL, int K0P, int HP>
__global__ __launch_bounds__(kRadWaves * kWave) void radial_hidden_bwd(RadialArgs A) {
  extern __shared__ float rad_lds[];
  constexpr int NT = HP / 16;
  constexpr int RT1 = (K0P + 15) / 16;
  rad_stage<NL, K0P, HP>(A, rad_lds);
  const int lane = threadIdx.x % kWave, g = lane >> 4, r = lane & 15;
  const int64_t n_tiles = (A.n_rows + 15) / 16;
  const int width_out = A.width[NL - 1];
  for (int64_t tile = (int64_t)blockIdx.x * kRadWaves + wave_in_block(); tile < n_tiles;
       tile += (int64_t)gridDim.x * kRadWaves) {
    // the weights are re-read from LDS for every tile: without this the compiler hoists
    // every loop-invariant LDS read out of the tile loop and spills the registers
    asm volatile("" ::: "memory");
    const int64_t edge = tile * 16 + r;
    const bool valid = edge < A.n_rows;
    // recompute: s_n and silu'(z_n) of every layer
    floatx4 d[NL][NT], s[NT], acc[NT];
    rad_layer1<NL, K0P, HP>(A, rad_lds, edge, valid, g, r, acc);
#pragma unroll
    for (int o = 0; o < NT; ++o)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float z = A.scale[0] * acc[o][i];
        s[o][i] = rad_silu(z);
        d[0][o][i] = rad_dsilu(z);
      }
#pragma unroll
    for (int n = 1; n < NL; ++n) {
      rad_layer<NL, K0P, HP>(rad_lds, n, g, r, s, acc);
#pragma unroll
      for (int o = 0; o < NT; ++o)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float z = A.scale[n] * acc[o][i];
          if (n + 1 < NL) s[o][i] = rad_silu(z);
          d[n][o][i] = rad_dsilu(z);
        }
    }
    // backward: delta_n = g_n * silu'(z_n), g_{n-1} = c_n A_n delta_n
    floatx4 delta[NT];
    rad_load<NT>(A.grad, edge, valid, width_out, g, delta);
#pragma unroll
    for (int n = NL - 1; n >= 1; --n) {
#pragma unroll
      for (int o = 0; o < NT; ++o)
#pragma unroll
        for (int i = 0; i < 4; ++i) delta[o][i] *= d[n][o][i];
      rad_layer_t<NL, K0P, HP, NT>(rad_lds, n, g, r, delta, acc);
#pragma unroll
      for (int o = 0; o < NT; ++o)
#pragma unroll
        for (int i = 0; i < 4; ++i) delta[o][i] = A.scale[n] * acc[o][i];
    }
#pragma unroll
    for (int o = 0; o < NT; ++o)
#pragma unroll
      for (int i = 0; i < 4; ++i) delta[o][i] *= d[0][o][i];
    floatx4 gx[RT1];
    rad_layer_t<NL, K0P, HP, RT1>(rad_lds, 0, g, r, delta, gx);
#pragma unroll
    for (int o = 0; o < RT1; ++o)
#pragma unroll
      for (int i = 0; i < 4; ++i) gx[o][i] *= A.scale[0];
    rad_store<RT1>(A.out, edge, valid, A.n_in, g, gx);
  }
}

template <int NL, int K0P, int HP>
static int rad_launch(bool backward, const RadialArgs& A, hipStream_t stream) {
  using T = RadialTables<NL, K0P, HP>;
  const size_t lds = sizeof(float) * (size_t)T::words;
  const void* kernel = backward ? reinterpret_cast<const void*>(&radial_hidden_bwd<NL, K0P, HP>)
                                : reinterpret_cast<const void*>(&radial_hidden_fwd<NL, K0P, HP>);
  // the tables of the widest layers exceed 64 KB: ask for the LDS once per instantiation
  static bool configured[2] = {false, false};
  if (!configured[backward]) {
    XNN_HIP_CHECK(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)lds));
    configured[backward] = true;
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kRadWaves * kWave, lds) !=
          hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  const int64_t n_tiles = (A.n_rows + 15) / 16;
  const int64_t needed = (n_tiles + kRadWaves - 1) / kRadWaves;
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(needed, (int64_t)per_cu *
                                                                            device_cu_count()));
  if (backward)
    hipLaunchKernelGGL((radial_hidden_bwd<NL, K0P, HP>), dim3((unsigned)blocks),
                       dim3(kRadWaves * kWave), lds, stream, A);
  else
    hipLaunchKernelGGL((radial_hidden_fwd<NL, K0P, HP>), dim3((unsigned)blocks),
                       dim3(kRadWaves * kWave), lds, stream, A);
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

template <int NL, int K0P>
static int rad_dispatch_hp(bool backward, int hp, const RadialArgs& A, hipStream_t stream) {
  switch (hp) {
    case 32: return rad_launch<NL, K0P, 32>(backward, A, stream);
    case 64: return rad_launch<NL, K0P, 64>(backward, A, stream);
    default: return rad_launch<NL, K0P, 128>(backward, A, stream);
  }
}

template <int NL>
static int rad_dispatch_k(bool backward, int k0p, int hp, const RadialArgs& A,
                          hipStream_t stream) {
  switch (k0p) {
    case 8: return rad_dispatch_hp<NL, 8>(backward, hp, A, stream);
    case 16: return rad_dispatch_hp<NL, 16>(backward, hp, A, stream);
    default: return rad_dispatch_hp<NL, 32>(backward, hp, A, stream);
  }
}

static int radial_hidden(bool backward, const float* x, const float* grad, int64_t n_rows,
                         int n_in, int n_layers, const int32_t* widths,
                         const float* const* weights, const float* scales, float* out,
                         xnn_stream_t stream) {
  XNN_REQUIRE(n_rows >= 0, "negative size");
  XNN_REQUIRE(n_layers >= 1 && n_layers <= kRadMaxLayers, "1 to %d hidden layers",
              kRadMaxLayers);
  XNN_REQUIRE(n_in >= 1 && n_in <= kRadMaxIn, "1 to %d input features", kRadMaxIn);
  XNN_REQUIRE(widths && weights && scales, "NULL widths, weights or scales");
  RadialArgs A{};
  int widest = 0;
  for (int n = 0; n < n_layers; ++n) {
    XNN_REQUIRE(widths[n] >= 1 && widths[n] <= kRadMaxWidth, "layer widths 1 to %d",
                kRadMaxWidth);
    XNN_REQUIRE(weights[n] != nullptr, "NULL weight of layer %d", n);
    A.w[n] = weights[n];
    A.width[n] = widths[n];
    A.scale[n] = scales[n];
    widest = std::max(widest, (int)widths[n]);
  }
  if (n_rows == 0) return XNN_OK;
  XNN_REQUIRE(x && out && (!backward || grad), "NULL input or output");
  XNN_REQUIRE(n_rows <= (int64_t(1) << 40), "too many rows");
  XNN_REQUIRE(aligned16(out) && aligned16(grad) && aligned16(x), "buffers must be 16-byte aligned");
  A.x = x;
  A.grad = grad;
  A.out = out;
  A.n_in = n_in;
  A.n_rows = n_rows;
  const int hp = widest <= 32 ? 32 : widest <= 64 ? 64 : 128;
  const int k0p = n_in <= 8 ? 8 : n_in <= 16 ? 16 : 32;
  const hipStream_t s = as_hip(stream);
  switch (n_layers) {
    case 1: return rad_dispatch_k<1>(backward, k0p, hp, A, s);
    case 2: return rad_dispatch_k<2>(backward, k0p, hp, A, s);
    default: return rad_dispatch_k<3>(backward, k0p, hp, A, s);
  }
}

}  // namespace xnn

using namespace xnn;

extern "C" {

int xnn_radial_hidden(const float* x, int64_t n_rows, int n_in, int n_layers,
                      const int32_t* widths, const float* const* weights, const float* scales,
                      float* out, xnn_stream_t stream) {
  return radial_hidden(false, x, nullptr, n_rows, n_in, n_layers, widths, weights, scales, out,
                       stream);
}

int xnn_radial_hidden_backward(const float* x, const float* grad_out, int64_t n_rows, int n_in,
                               int n_layers, const int32_t* widths, const float* const* weights,
                               const float* scales, float* grad_x, xnn_stream_t stream) {
  return radial_hidden(true, x, grad_out, n_rows, n_in, n_layers, widths, weights, scales,
                       grad_x, stream);
}

}  // extern "C"
