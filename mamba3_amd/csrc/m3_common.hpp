// Shared device helpers for the Mamba-3 HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mamba3_hip.h"

namespace m3 {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr float kPi = 3.14159265358979323846f;     // math.pi as FP32 (model.py:226)
constexpr float kTwoPi = 6.28318530717958647692f;  // 2 * math.pi as FP32 (model.py:230)
constexpr float kAFloor = 1e-4f;                   // model.py:22

// ---------------------------------------------------------------- activation types

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(__bf16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f(_Float16 x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T from_f(float x) { return static_cast<T>(x); }

// Round an FP32 value to the activation type and back (the cast points of the reference).
template <typename T>
__device__ __forceinline__ float rnd(float x) { return to_f(from_f<T>(x)); }
template <>
__device__ __forceinline__ float rnd<float>(float x) { return x; }

// Products and sums the reference evaluates as separate activation-dtype ops: no contraction.
template <typename T>
__device__ __forceinline__ float mul_r(float a, float b) { return rnd<T>(__fmul_rn(a, b)); }
template <typename T>
__device__ __forceinline__ float add_r(float a, float b) { return rnd<T>(__fadd_rn(a, b)); }
template <typename T>
__device__ __forceinline__ float sub_r(float a, float b) { return rnd<T>(__fsub_rn(a, b)); }

// Element load with a runtime dtype (parameters, per-token scalars).
__device__ __forceinline__ float ldx(const void* p, int dtype, int64_t i) {
  if (dtype == M3_F32) return static_cast<const float*>(p)[i];
  if (dtype == M3_BF16) return static_cast<float>(static_cast<const __bf16*>(p)[i]);
  return static_cast<float>(static_cast<const _Float16*>(p)[i]);
}

// A runtime-dtype pointer advanced by `i` elements.
__device__ __forceinline__ const void* offx(const void* p, int dtype, int64_t i) {
  return static_cast<const char*>(p) + i * (dtype == M3_F32 ? 4 : 2);
}

// ---------------------------------------------------------------- scalar math

// torch.nn.functional.softplus with beta = 1, threshold = 20.
__device__ __forceinline__ float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }

// ops.py:28-32.
__device__ __forceinline__ float heavy_tail(float x) {
  return x >= 0.f ? 1.f + x : 1.f / (1.f - fminf(x, 0.f));
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }

// The same with the hardware exp and reciprocal (about 2 ulp), for the scan's per-token stage.
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.f + __expf(-x));
}
__device__ __forceinline__ float heavy_tail_fast(float x) {
  return x >= 0.f ? 1.f + x : __builtin_amdgcn_rcpf(1.f - x);
}
__device__ __forceinline__ float siluf(float x) { return x / (1.f + expf(-x)); }

// x * sigmoid(x) with the hardware exp and reciprocal (about 1 ulp each): the output gate of
// the scan epilogue. exp(-x) = inf gives x * 0 = -0 for large negative x.
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.f + __expf(-x));
}

// dt and adt from the raw projection (model.py:195-198) or as given.
__device__ __forceinline__ void dt_adt(bool raw, float dt_in, float a_in, float dt_bias,
                                       float& dt, float& adt) {
  if (raw) {
    dt = softplus(dt_in + dt_bias);
    float decay = fminf(-heavy_tail(a_in), -kAFloor);
    adt = decay * dt;
  } else {
    dt = dt_in;
    adt = a_in;
  }
}

// fmod(pi * tanh(angle) * dt, 2 pi) (model.py:225-230).
__device__ __forceinline__ float phase_inc(float angle, float dt) {
  return fmodf(__fmul_rn(__fmul_rn(kPi, tanhf(angle)), dt), kTwoPi);
}

// ---------------------------------------------------------------- error reporting (host)

}  // namespace m3
