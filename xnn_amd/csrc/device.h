// Device-side building blocks shared by the per-edge kernels (gfx950, wave64).
//
//  * packed integer image shifts
//  * the edge vector r_e = pos[dst] - pos[src] + shift @ cell (atomic_data.py:371-418)
//  * real spherical harmonics l <= 3 in the e3nn convention (component
//    normalization, y is the polar axis; gnn/featurizers/spherical.py:91-93)
//  * Bessel / Gaussian radial bases and polynomial / cosine envelopes with
//    their derivatives (common/featurizers/radial.py, cutoff.py)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "xnn_amd.h"

namespace xnn {

constexpr int kWave = 64;

// MI355X's accelerator dies: workgroups are dispatched to the 8 XCDs in turn (block b to XCD
// b % 8), each XCD with its own L2. A launch of a multiple of 8 blocks that gives block b
// the slot xcd_slot(b) = (b % 8) * (blocks / 8) + b / 8 has each XCD walk one contiguous run
// of slots: with work laid out in a spatial order, the rows a run gathers are shared by the
// XCD's other waves and stay in its L2.
constexpr int kXcds = 8;

__device__ __forceinline__ int64_t xcd_slot() {
  const int64_t per_xcd = ((int64_t)gridDim.x + kXcds - 1) / kXcds;
  return (int64_t)(blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
}

// a block count rounded up to whole XCD rounds (xcd_slot is then a permutation)
inline int64_t xcd_blocks(int64_t blocks) { return ((blocks + kXcds - 1) / kXcds) * kXcds; }

// Wave index within the block, as a wave-uniform (scalar) value: the compiler cannot
// infer that threadIdx.x / 64 is the same on every lane, and values derived from a
// divergent-looking index turn uniform loops and branches into vector control flow.
__device__ __forceinline__ int wave_in_block() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
}

// ---------------------------------------------------------------- shifts
__host__ __device__ inline int32_t pack_shift(int sx, int sy, int sz) {
  return (int32_t)(((uint32_t)sx & 1023u) | (((uint32_t)sy & 1023u) << 10) |
                   (((uint32_t)sz & 1023u) << 20));
}
__host__ __device__ inline void unpack_shift(int32_t p, int& sx, int& sy, int& sz) {
  sx = (int32_t)((uint32_t)p << 22) >> 22;
  sy = (int32_t)((uint32_t)p << 12) >> 22;
  sz = (int32_t)((uint32_t)p << 2) >> 22;
}

// ---------------------------------------------------------------- geometry
template <typename G>
struct Cell {
  G m[9];
};

// r = pos[d] - pos[s] + (sx, sy, sz) @ cell, formed in the geometry dtype in the
// reference's order: the difference first, then the image offset.
template <typename G>
__device__ inline void edge_vector(const G* __restrict__ pos, int s, int d, int32_t shift,
                                   const G* __restrict__ cell, G& x, G& y, G& z) {
  x = pos[3 * d + 0] - pos[3 * s + 0];
  y = pos[3 * d + 1] - pos[3 * s + 1];
  z = pos[3 * d + 2] - pos[3 * s + 2];
  if (cell != nullptr) {
    int sx, sy, sz;
    unpack_shift(shift, sx, sy, sz);
    if ((sx | sy | sz) != 0) {
      const G fx = (G)sx, fy = (G)sy, fz = (G)sz;
      x += fx * cell[0] + fy * cell[3] + fz * cell[6];
      y += fx * cell[1] + fy * cell[4] + fz * cell[7];
      z += fx * cell[2] + fy * cell[5] + fz * cell[8];
    }
  }
}

// ---------------------------------------------------------------- spherical harmonics
// Component-normalized real SH of a unit vector u = (x, y, z) in the e3nn order
// (m = -l..l within each l). They are sqrt(2l+1) times the orthonormal real SH
// without Condon-Shortley phase, taken with the standard polar axis on y:
// (x_s, y_s, z_s) = (z, x, y). Homogeneous of degree l in u.
template <int LMAX, typename T>
__device__ inline void sh_eval(T x, T y, T z, T* __restrict__ Y) {
  Y[0] = T(1);
  if constexpr (LMAX >= 1) {
    const T s3 = T(1.7320508075688772);
    Y[1] = s3 * x;
    Y[2] = s3 * y;
    Y[3] = s3 * z;
  }
  if constexpr (LMAX >= 2) {
    const T s15 = T(3.872983346207417);
    const T s5 = T(2.23606797749979);
    const T x2 = x * x, y2 = y * y, z2 = z * z;
    Y[4] = s15 * x * z;
    Y[5] = s15 * x * y;
    Y[6] = s5 * (y2 - T(0.5) * (x2 + z2));
    Y[7] = s15 * y * z;
    Y[8] = T(0.5) * s15 * (z2 - x2);
  }
  if constexpr (LMAX >= 3) {
    const T a = T(2.091650066335189);   // sqrt(35/8)
    const T b = T(10.246950765959598);  // sqrt(105)
    const T c = T(1.620185174601965);   // sqrt(21/8)
    const T d = T(1.3228756555322954);  // sqrt(7)/2
    const T e = T(5.123475382979799);   // sqrt(105)/2
    const T x2 = x * x, y2 = y * y, z2 = z * z;
    Y[9] = a * x * (T(3) * z2 - x2);
    Y[10] = b * x * y * z;
    Y[11] = c * x * (T(4) * y2 - x2 - z2);
    Y[12] = d * y * (T(2) * y2 - T(3) * x2 - T(3) * z2);
    Y[13] = c * z * (T(4) * y2 - x2 - z2);
    Y[14] = e * y * (z2 - x2);
    Y[15] = a * z * (z2 - T(3) * x2);
  }
}

// G = sum_lm dY[lm] * grad_u Y_lm(u) (not projected onto the sphere).
template <int LMAX, typename T>
__device__ inline void sh_grad(T x, T y, T z, const T* __restrict__ dY, T& gx, T& gy, T& gz) {
  gx = T(0);
  gy = T(0);
  gz = T(0);
  if constexpr (LMAX >= 1) {
    const T s3 = T(1.7320508075688772);
    gx += s3 * dY[1];
    gy += s3 * dY[2];
    gz += s3 * dY[3];
  }
  if constexpr (LMAX >= 2) {
    const T s15 = T(3.872983346207417);
    const T s5 = T(2.23606797749979);
    // Y4 = s15 xz, Y5 = s15 xy, Y6 = s5 (y2 - (x2+z2)/2), Y7 = s15 yz, Y8 = s15/2 (z2 - x2)
    gx += s15 * (dY[4] * z + dY[5] * y - dY[8] * x) - s5 * dY[6] * x;
    gy += s15 * (dY[5] * x + dY[7] * z) + T(2) * s5 * dY[6] * y;
    gz += s15 * (dY[4] * x + dY[7] * y + dY[8] * z) - s5 * dY[6] * z;
  }
  if constexpr (LMAX >= 3) {
    const T a = T(2.091650066335189);
    const T b = T(10.246950765959598);
    const T c = T(1.620185174601965);
    const T d = T(1.3228756555322954);
    const T e = T(5.123475382979799);
    const T x2 = x * x, y2 = y * y, z2 = z * z;
    // Y9  = a (3 x z2 - x3)            grad a (3 z2 - 3 x2, 0, 6 x z)
    // Y10 = b x y z                    grad b (y z, x z, x y)
    // Y11 = c (4 x y2 - x3 - x z2)     grad c (4 y2 - 3 x2 - z2, 8 x y, -2 x z)
    // Y12 = d (2 y3 - 3 x2 y - 3 y z2) grad d (-6 x y, 6 y2 - 3 x2 - 3 z2, -6 y z)
    // Y13 = c (4 y2 z - x2 z - z3)     grad c (-2 x z, 8 y z, 4 y2 - x2 - 3 z2)
    // Y14 = e (y z2 - y x2)            grad e (-2 x y, z2 - x2, 2 y z)
    // Y15 = a (z3 - 3 x2 z)            grad a (-6 x z, 0, 3 z2 - 3 x2)
    gx += a * (dY[9] * (T(3) * z2 - T(3) * x2) - dY[15] * T(6) * x * z) + b * dY[10] * y * z +
          c * (dY[11] * (T(4) * y2 - T(3) * x2 - z2) - dY[13] * T(2) * x * z) -
          d * dY[12] * T(6) * x * y - e * dY[14] * T(2) * x * y;
    gy += b * dY[10] * x * z + c * (dY[11] * T(8) * x * y + dY[13] * T(8) * y * z) +
          d * dY[12] * (T(6) * y2 - T(3) * x2 - T(3) * z2) + e * dY[14] * (z2 - x2);
    gz += a * (dY[9] * T(6) * x * z + dY[15] * (T(3) * z2 - T(3) * x2)) + b * dY[10] * x * y +
          c * (-dY[11] * T(2) * x * z + dY[13] * (T(4) * y2 - x2 - T(3) * z2)) -
          d * dY[12] * T(6) * y * z + e * dY[14] * T(2) * y * z;
  }
}

// dL/dv for Y(v / |v|): the gradient G on the unit sphere projected to its
// tangent plane and divided by |v|. Zero for |v| == 0.
template <typename T>
__device__ inline void sh_chain(T ux, T uy, T uz, T inv_len, T gx, T gy, T gz, T& ox, T& oy,
                                T& oz) {
  const T radial = ux * gx + uy * gy + uz * gz;
  ox = (gx - radial * ux) * inv_len;
  oy = (gy - radial * uy) * inv_len;
  oz = (gz - radial * uz) * inv_len;
}

// ---------------------------------------------------------------- radial
// Butterfly steps across the rows of a wave (a row = 16 lanes) on gfx950's row-swap
// permutes, vector-ALU instructions instead of an LDS round trip. With both operands x,
// v_permlane16_swap returns (x with odd rows replaced by the even rows, x with even rows
// replaced by the odd rows), so their sum is x + x[lane ^ 16] on every lane (the two
// addends in either order: the same bits); v_permlane32_swap does the same for the two
// 32-lane halves. Every lane of the wave must be active.
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the 16 lanes of a row, every lane getting it: two quad permutes and the half-row
// and row mirrors (DPP moves, vector ALU). Every lane of the row must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm(1, 0, 3, 2): lane ^ 1
  v += dpp_move<0x4E>(v);   // quad_perm(2, 3, 0, 1): lane ^ 2
  v += dpp_move<0x141>(v);  // row_half_mirror: lane i <-> 7 - i within 8
  v += dpp_move<0x140>(v);  // row_mirror: lane i <-> 15 - i within 16
  return v;
}

// x of lane ^ M for M = 1, 2 (DPP quad permutes, vector ALU) or 4, 8, 16 (ds_swizzle in
// xor mode: the LDS crossbar without an address computation or memory access), for a
// double; every lane of the wave must be active.
template <int M>
__device__ __forceinline__ double xor_lanes(double v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16, "lane mask");
  const int lo = __double2loint(v), hi = __double2hiint(v);
  int a, b;
  if constexpr (M == 1) {
    a = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, false);  // quad_perm(1, 0, 3, 2)
    b = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, false);
  } else if constexpr (M == 2) {
    a = __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xF, 0xF, false);  // quad_perm(2, 3, 0, 1)
    b = __builtin_amdgcn_mov_dpp(hi, 0x4E, 0xF, 0xF, false);
  } else {
    // bit mode: and_mask 0x1F, or_mask 0, xor_mask M
    a = __builtin_amdgcn_ds_swizzle(lo, 0x1F | (M << 10));
    b = __builtin_amdgcn_ds_swizzle(hi, 0x1F | (M << 10));
  }
  return __hiloint2double(b, a);
}

// v + v[lane ^ M] for a double, on the cheapest exchange for M: the row-swap permutes for 32
// and 16, a DPP row rotation for 8, an xor swizzle for 4, DPP quad permutes for 2 and 1 (the
// same pairs and order as __shfl_xor, so the same bits). Every lane of the wave must be
// active.
template <int M>
__device__ __forceinline__ double add_xor_lanes(double v) {
  const unsigned lo = (unsigned)__double2loint(v), hi = (unsigned)__double2hiint(v);
  if constexpr (M == 32 || M == 16) {
    const auto a = M == 32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                           : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto b = M == 32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                           : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return __hiloint2double((int)b[0], (int)a[0]) + __hiloint2double((int)b[1], (int)a[1]);
  } else if constexpr (M == 4) {
    return v + __hiloint2double(__builtin_amdgcn_ds_swizzle((int)hi, 0x1F | (4 << 10)),
                                __builtin_amdgcn_ds_swizzle((int)lo, 0x1F | (4 << 10)));
  } else {
    static_assert(M == 8 || M == 2 || M == 1, "lane mask");
    constexpr int ctrl = M == 8 ? 0x128 : (M == 2 ? 0x4E : 0xB1);
    return v + __hiloint2double(__builtin_amdgcn_mov_dpp((int)hi, ctrl, 0xF, 0xF, false),
                                __builtin_amdgcn_mov_dpp((int)lo, ctrl, 0xF, 0xF, false));
  }
}

// the sum over aligned groups of GROUP lanes (a power of two up to 64), in every lane
template <int GROUP>
__device__ __forceinline__ double group_sum(double v) {
  if constexpr (GROUP >= 64) v = add_xor_lanes<32>(v);
  if constexpr (GROUP >= 32) v = add_xor_lanes<16>(v);
  if constexpr (GROUP >= 16) v = add_xor_lanes<8>(v);
  if constexpr (GROUP >= 8) v = add_xor_lanes<4>(v);
  if constexpr (GROUP >= 4) v = add_xor_lanes<2>(v);
  if constexpr (GROUP >= 2) v = add_xor_lanes<1>(v);
  return v;
}

// v + v[lane ^ M] and the aligned GROUP-lane sums for a float, as add_xor_lanes / group_sum
template <int M>
__device__ __forceinline__ float add_xor_lanes_f(float v) {
  if constexpr (M == 32) {
    return add_xor32(v);
  } else if constexpr (M == 16) {
    return add_xor16(v);
  } else if constexpr (M == 4) {
    return v + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (4 << 10)));
  } else {
    static_assert(M == 8 || M == 2 || M == 1, "lane mask");
    return v + dpp_move<M == 8 ? 0x128 : (M == 2 ? 0x4E : 0xB1)>(v);
  }
}

template <int GROUP>
__device__ __forceinline__ float group_sum_f(float v) {
  if constexpr (GROUP >= 64) v = add_xor_lanes_f<32>(v);
  if constexpr (GROUP >= 32) v = add_xor_lanes_f<16>(v);
  if constexpr (GROUP >= 16) v = add_xor_lanes_f<8>(v);
  if constexpr (GROUP >= 8) v = add_xor_lanes_f<4>(v);
  if constexpr (GROUP >= 4) v = add_xor_lanes_f<2>(v);
  if constexpr (GROUP >= 2) v = add_xor_lanes_f<1>(v);
  return v;
}

// The wave-wide minimum (MAX = false) or maximum of a double in every lane: row-swap
// permutes for lanes ^ 32 and ^ 16 (the two results of a swap of v with itself hold v and
// its partner's value on every lane), then DPP and an xor swizzle for 8, 4, 2, 1. Every lane
// of the wave must be active.
template <bool MAX>
__device__ __forceinline__ double wave_extreme(double v) {
  auto pick = [](double a, double b) { return MAX ? fmax(a, b) : fmin(a, b); };
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const unsigned lo = (unsigned)__double2loint(v), hi = (unsigned)__double2hiint(v);
    const auto a = half == 0 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                             : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto b = half == 0 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                             : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    v = pick(__hiloint2double((int)b[0], (int)a[0]), __hiloint2double((int)b[1], (int)a[1]));
  }
  auto dpp = [](double x, auto ctrl_tag) {
    constexpr int ctrl = decltype(ctrl_tag)::value;
    return __hiloint2double(__builtin_amdgcn_mov_dpp(__double2hiint(x), ctrl, 0xF, 0xF, false),
                            __builtin_amdgcn_mov_dpp(__double2loint(x), ctrl, 0xF, 0xF, false));
  };
  v = pick(v, dpp(v, std::integral_constant<int, 0x128>{}));  // lane ^ 8 (row_ror:8)
  v = pick(v, __hiloint2double(__builtin_amdgcn_ds_swizzle(__double2hiint(v), 0x1F | (4 << 10)),
                               __builtin_amdgcn_ds_swizzle(__double2loint(v), 0x1F | (4 << 10))));
  v = pick(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // lane ^ 2
  v = pick(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // lane ^ 1
  return v;
}

// entry j of structure b's stress, scale g[b] / V_b for a periodic structure (V_b =
// |det cell_b| > 1e-8 and, with pbc, some periodic direction), zero otherwise
// (outputs.py:227-239); float64 inside
template <typename T, typename C>
__device__ inline T stress_entry(const T* __restrict__ g, const C* __restrict__ cell,
                                 const uint8_t* __restrict__ pbc, int64_t b, int j,
                                 double scale) {
  const C* c = cell + 9 * b;
  const double a0 = c[0], a1 = c[1], a2 = c[2], b0 = c[3], b1 = c[4], b2 = c[5], c0 = c[6],
               c1 = c[7], c2 = c[8];
  // row 0 . (row 1 x row 2)
  const double v = fabs(a0 * (b1 * c2 - b2 * c1) + a1 * (b2 * c0 - b0 * c2) + a2 * (b0 * c1 - b1 * c0));
  bool periodic = v > 1e-8;
  if (pbc != nullptr) periodic = periodic && (pbc[3 * b] | pbc[3 * b + 1] | pbc[3 * b + 2]);
  return periodic ? (T)(scale * (double)g[9 * b + j] / v) : T(0);
}

__device__ inline void dev_sincos(float a, float* s, float* c) { sincosf(a, s, c); }
__device__ inline void dev_sincos(double a, double* s, double* c) { sincos(a, s, c); }
__device__ inline float dev_exp(float a) { return expf(a); }
__device__ inline double dev_exp(double a) { return exp(a); }
__device__ inline float dev_sqrt(float a) { return sqrtf(a); }
__device__ inline double dev_sqrt(double a) { return sqrt(a); }

template <typename T>
struct Radial {
  int K;
  int basis;
  int envelope;
  int p;
  T rc;
  T inv_rc;  // 1 / rc, formed on the host in float64
  T prefactor;
  T gamma;
  const T* __restrict__ table;  // Bessel frequencies or Gaussian centers
};

// envelope value and derivative at distance r; every envelope is zero from the cutoff on
// (the reference's multiply by (r < rc), cutoff.py:41, 125), the unit envelope included, so
// that edges of a list longer than the cutoff contribute nothing
template <typename T>
__device__ inline void envelope_eval(const Radial<T>& R, T r, T& f, T& df) {
  if (!(r < R.rc)) {
    f = T(0);
    df = T(0);
    return;
  }
  if (R.envelope == XNN_ENV_NONE) {
    f = T(1);
    df = T(0);
    return;
  }
  if (R.envelope == XNN_ENV_POLYNOMIAL) {
    // 1 + ((-(p(p+1)/2) x + p(p+2)) x - (p+1)(p+2)/2) x^p  (cutoff.py:119-125)
    const T x = r * R.inv_rc;
    const T pp = (T)R.p;
    const T a = -(pp * (pp + T(1)) / T(2));
    const T b = pp * (pp + T(2));
    const T c = -(pp + T(1)) * (pp + T(2)) / T(2);
    T xpm1 = T(1);
    for (int k = 0; k < R.p - 1; ++k) xpm1 *= x;
    const T xp = xpm1 * x;
    const T tail = (a * x + b) * x + c;
    f = T(1) + tail * xp;
    df = ((T(2) * a * x + b) * xp + pp * tail * xpm1) * R.inv_rc;
  } else {
    // 0.5 (cos(pi r / rc) + 1)  (cutoff.py:40-41)
    const T w = T(3.141592653589793) * R.inv_rc;
    T s, c;
    dev_sincos(w * r, &s, &c);
    f = T(0.5) * (c + T(1));
    df = T(-0.5) * w * s;
  }
}

// Per-edge state of the radial expansion: the envelope f(r), f'(r) and the clamped
// radius, evaluated once; radial_k then gives rbf_k(r) f(r) and its r-derivative one
// basis function at a time (no per-thread arrays, so nothing lands in scratch).
template <typename T>
struct RadialAt {
  T r, rr, inv, f, df;
  bool clamped;
};

template <typename T>
__device__ inline RadialAt<T> radial_at(const Radial<T>& R, T r) {
  RadialAt<T> a;
  a.r = r;
  envelope_eval(R, r, a.f, a.df);
  // Bessel: r clamped at 1e-8 (radial.py:267-268)
  a.clamped = r < T(1e-8);
  a.rr = a.clamped ? T(1e-8) : r;
  a.inv = T(1) / a.rr;
  return a;
}

// basis function k with its table entry tk (Bessel frequency or Gaussian center) given
template <typename T, bool DERIV>
__device__ inline void radial_kv(const Radial<T>& R, const RadialAt<T>& a, T tk, T& u, T& du) {
  if (R.basis == XNN_BASIS_BESSEL) {
    // prefactor * sin(freq * r / rc) / r
    const T w = tk * R.inv_rc;
    T s, c;
    dev_sincos(w * a.rr, &s, &c);
    const T b = R.prefactor * s * a.inv;
    u = b * a.f;
    if constexpr (DERIV) {
      const T db = a.clamped ? T(0) : R.prefactor * (c * w - s * a.inv) * a.inv;
      du = db * a.f + b * a.df;
    }
  } else {
    // exp(-gamma (r - mu_k)^2)  (radial.py:73-75)
    const T dd = a.r - tk;
    const T b = dev_exp(-R.gamma * dd * dd);
    u = b * a.f;
    if constexpr (DERIV) du = T(-2) * R.gamma * dd * b * a.f + b * a.df;
  }
}

template <typename T, bool DERIV>
__device__ inline void radial_k(const Radial<T>& R, const RadialAt<T>& a, int k, T& u, T& du) {
  radial_kv<T, DERIV>(R, a, R.table[k], u, du);
}

constexpr int kMaxRbf = 32;

}  // namespace xnn
