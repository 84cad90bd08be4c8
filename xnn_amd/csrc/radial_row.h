// The enveloped radial row of one edge, evaluated per lane for the message kernels
// (gfx950, wave64): h_k = rbf_k(|r|) envelope(|r|) for k < kLinKMax (radial.py:187-268,
// cutoff.py:10-125, spherical.py:135-138), and d E / d|r| through it for the backward.
#pragma once
#include <cstdint>

#include "common.h"
#include "device.h"

namespace xnn {

constexpr int kLinKMax = 8;  // h features: two k-steps of 4
constexpr int kLinKK = 2;
constexpr int kSH = 9;       // LDS row stride of per-edge radial features

// The radial table (Bessel frequencies or Gaussian centers, k < kLinKMax) is read once per
// block into LDS, and its first entry and the progression test into scalars at kernel
// entry, before any store: there the wave-uniform loads are scalar loads (nothing the
// kernel writes can alias them yet). Read next to the kernel's own stores they would be
// per-lane vector loads whose latency the radial evaluation waits for on every row.
struct RadialTab {
  const float* f;  // the table in LDS
  float f0;
  // frequencies in harmonic progression, f_k = (k + 1) f_0 to 4e-7 (the default
  // BesselRBF frequencies n pi, radial.py:226): then sin((k + 1) theta) and its cosine
  // follow from one sincos by the Chebyshev recurrence x_{k+1} = 2 cos(theta) x_k - x_{k-1}
  // instead of one sincos per function
  bool harmonic;
};

// every thread of the block calls this once; the caller synchronizes the block before the
// table is read
__device__ __forceinline__ RadialTab load_radial_tab(const Radial<float>& R, float* sTab) {
  RadialTab t;
  t.f = sTab;
  t.f0 = R.table[0];
  t.harmonic = R.basis == XNN_BASIS_BESSEL;
  for (int k = 1; k < R.K; ++k) {
    const float fk = R.table[k];
    if (fabsf(fk - (float)(k + 1) * t.f0) > 4e-7f * fabsf(fk)) t.harmonic = false;
  }
  if (threadIdx.x < kLinKMax) sTab[threadIdx.x] = (int)threadIdx.x < R.K ? R.table[threadIdx.x] : 0.f;
  return t;
}

// What the backward's d|r| step reuses of the radial row: the envelope state and, for the
// harmonic Bessel frequencies, sin and cos of the first frequency.
struct RadialCache {
  RadialAt<float> a;
  float s1, c1;
};

// The lane's row of radial features h_k = rbf_k(r) envelope(r), k < kLinKMax (zeros past
// R.K, and the whole row when the lane has no edge); the state the backward needs again goes
// to *keep (when given).
__device__ __forceinline__ void radial_row(const Radial<float>& R, const RadialTab& tab,
                                           bool valid, float r, float* __restrict__ row,
                                           RadialCache* keep = nullptr) {
  if (valid) {
    const RadialAt<float> a = radial_at(R, r);
    if (keep) keep->a = a;
    if (tab.harmonic) {
      float s1, c1;
      dev_sincos(tab.f0 * R.inv_rc * a.rr, &s1, &c1);
      if (keep) {
        keep->s1 = s1;
        keep->c1 = c1;
      }
      const float c2 = 2.f * c1, pf = R.prefactor * a.inv * a.f;
      float sp = 0.f, sk = s1;  // sin(k theta), sin((k + 1) theta)
#pragma unroll
      for (int k = 0; k < kLinKMax; ++k) {
        row[k] = k < R.K ? pf * sk : 0.f;
        const float sn = c2 * sk - sp;
        sp = sk;
        sk = sn;
      }
      return;
    }
#pragma unroll 1
    for (int k = 0; k < kLinKMax; ++k) {
      float u = 0.f, du;
      if (k < R.K) radial_kv<float, false>(R, a, tab.f[k], u, du);
      row[k] = u;
    }
  } else {
#pragma unroll
    for (int k = 0; k < kLinKMax; ++k) row[k] = 0.f;
  }
}

// d E / d r through the radial features of one edge, sum_k d_h[k] d h_k / d r, from the
// state radial_row kept. Harmonic Bessel frequencies, with theta = w0 r, w0 = f0 / rc:
// h_k = P sin((k+1) theta) f / r, so sum_k d_h[k] h_k' = P / r (f (w0 sum_k (k+1) d_h[k]
// cos((k+1) theta) - S / r) + f' S) with S = sum_k d_h[k] sin((k+1) theta) (the sine term
// drops at the clamped radius, where h_k does not vary with r).
__device__ __forceinline__ float radial_dot(const Radial<float>& R, const RadialTab& tab,
                                            const RadialCache& rc,
                                            const float* __restrict__ d_h) {
  const RadialAt<float>& a = rc.a;
  if (tab.harmonic) {
    const float w0 = tab.f0 * R.inv_rc;
    const float c2 = 2.f * rc.c1;
    float sp = 0.f, sk = rc.s1, cp = 1.f, ck = rc.c1;
    float S = 0.f, Cw = 0.f;
#pragma unroll
    for (int k = 0; k < kLinKMax; ++k) {
      if (k < R.K) {
        S += d_h[k] * sk;
        Cw += ((float)(k + 1) * d_h[k]) * ck;
      }
      const float sn = c2 * sk - sp, cn = c2 * ck - cp;
      sp = sk;
      sk = sn;
      cp = ck;
      ck = cn;
    }
    const float rad = a.clamped ? 0.f : a.f * (w0 * Cw - a.inv * S);
    return R.prefactor * a.inv * (rad + a.df * S);
  }
  float dl = 0.f;
#pragma unroll 1
  for (int k = 0; k < R.K; ++k) {
    float u, du;
    radial_kv<float, true>(R, a, tab.f[k], u, du);
    dl += d_h[k] * du;
  }
  return dl;
}

}  // namespace xnn
