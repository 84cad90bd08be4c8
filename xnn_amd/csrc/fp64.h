// float64 helpers of the dispersion kernels: refined reciprocal and reciprocal square
// root, and the quintic switching window.
#pragma once
#include <hip/hip_runtime.h>

namespace xnn {

// 1 / x for positive normal x: the hardware estimate (v_rcp_f64) refined by two
// Newton-Raphson steps y <- y (2 - x y), to about an ulp (the IEEE-exact division costs
// several times more and these terms need no exact rounding)
__device__ __forceinline__ double rcp_nr(double x) {
  double y = __builtin_amdgcn_rcp(x);
  double e = fma(-x, y, 1.0);
  y = fma(y, e, y);
  e = fma(-x, y, 1.0);
  return fma(y, e, y);
}

// 1 / sqrt(x) for positive normal x: v_rsq_f64 refined by two Newton-Raphson steps
// y <- y (3 - x y^2) / 2
__device__ __forceinline__ double rsq_nr(double x) {
  double y = __builtin_amdgcn_rsq(x);
  const double h = 0.5 * x;
  y = y * fma(-h * y, y, 1.5);
  y = y * fma(-h * y, y, 1.5);
  return y;
}

// quintic switch and its r-derivative (dispersion.py:42-67); width <= 0: sharp
__device__ inline void switch_d(double r, double cutoff, double width, double& sw, double& dsw) {
  if (width <= 0.0) {
    sw = 1.0;
    dsw = 0.0;
    return;
  }
  const double w = width < cutoff ? width : cutoff;
  double x = (cutoff - r) / w;
  if (x >= 1.0) {
    sw = 1.0;
    dsw = 0.0;
  } else if (x <= 0.0) {
    sw = 0.0;
    dsw = 0.0;
  } else {
    sw = x * x * x * (10.0 + x * (6.0 * x - 15.0));
    const double om = 1.0 - x;
    dsw = -30.0 * x * x * om * om / w;
  }
}

}  // namespace xnn
