/* Scalar math shared by the HIP kernels and the host-side unit tests (plain C / C++). */
#ifndef M3_MATH_H
#define M3_MATH_H

#include <math.h>

#if defined(__HIPCC__)
#define M3_HD __host__ __device__ __forceinline__
#else
#define M3_HD static inline
#endif

/* 2 pi as the FP32 value torch uses for fmod(x, 2.0 * math.pi) (model.py:230). */
#define M3_TWO_PI_F 6.28318530717958647692f

/*
 * fmodf(x, 2 pi) for |x| < 2^20, without the general-purpose reduction loop and without
 * divergent branches. fmod is odd in x, so reduce |x|: q = trunc(|x| / c) and a single fused
 * multiply-add |x| - q c, which is exact whenever q is the true quotient (the fmod result is
 * representable). A quotient that is one off is corrected by one step of c (selects, not
 * branches), and the sign of x is restored (fmodf(-0) = -0).
 */
M3_HD float m3_fmod_2pi_small(float x) {
  const float c = M3_TWO_PI_F;
  const float ax = fabsf(x);
  const float q = truncf(ax * (1.0f / c));
  float r = fmaf(-q, c, ax);
  r = r < 0.0f ? r + c : r;
  r = r >= c ? r - c : r;
  return copysignf(r, x);
}

/* fmodf(x, 2 pi) for every x: the reduction above, fmodf itself for |x| >= 2^20. */
M3_HD float m3_fmod_2pi(float x) {
  if (!(fabsf(x) < 1048576.0f)) return fmodf(x, M3_TWO_PI_F);
  return m3_fmod_2pi_small(x);
}

#endif /* M3_MATH_H */
