// Shared device helpers for the Mamba-3 HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mamba3_hip.h"
#include "m3_math.h"

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

// Runtime-dtype loads split into a load of the raw bits, without control flow, and a decode by
// selects: a kernel issues all its small loads first and decodes afterwards, so no load waits for
// another (a load inside a dtype branch, or decoded right away, ends in a full wait). Every
// address stays inside the element (16-bit tensors re-read their first half / first 8 bytes where
// FP32 reads the second).
struct RawX { uint32_t lo, hi; };
struct Raw4 { uint32_t w[4]; };

__device__ __forceinline__ RawX ldraw(const void* p, int dtype, int64_t i) {
  const bool w = dtype == M3_F32;
  const uint16_t* e =
      reinterpret_cast<const uint16_t*>(static_cast<const char*>(p) + i * (w ? 4 : 2));
  return RawX{e[0], e[w ? 1 : 0]};
}

// The same with a 32-bit element index (offsets known to fit 31 bits).
__device__ __forceinline__ RawX ldraw(const void* p, int dtype, int i) {
  const bool w = dtype == M3_F32;
  const uint16_t* e = reinterpret_cast<const uint16_t*>(static_cast<const char*>(p) + i * (w ? 4 : 2));
  return RawX{e[0], e[w ? 1 : 0]};
}

__device__ __forceinline__ float decode_x(uint32_t lo, uint32_t hi, int dtype) {
  const float f32 = __uint_as_float(lo | (hi << 16));
  const float bf = __uint_as_float(lo << 16);
  const float f16 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(lo)));
  return dtype == M3_F32 ? f32 : (dtype == M3_BF16 ? bf : f16);
}

__device__ __forceinline__ float decode(RawX r, int dtype) { return decode_x(r.lo, r.hi, dtype); }

// Four consecutive elements (8-byte aligned for 16-bit types, 16-byte for FP32).
__device__ __forceinline__ Raw4 ldraw4(const m3_tensor& t, int64_t i) {
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  const bool w = t.dtype == M3_F32;
  const char* base = static_cast<const char*>(t.ptr) + i * (w ? 4 : 2);
  const u2 x = *reinterpret_cast<const u2*>(base);
  const u2 y = *reinterpret_cast<const u2*>(base + (w ? 8 : 0));
  return Raw4{{x[0], x[1], y[0], y[1]}};
}

__device__ __forceinline__ f4 decode4(const Raw4& r, int dtype) {
  const uint32_t half[4] = {r.w[0] & 0xffffu, r.w[0] >> 16, r.w[1] & 0xffffu, r.w[1] >> 16};
  f4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = dtype == M3_F32 ? __uint_as_float(r.w[j]) : decode_x(half[j], 0u, dtype);
  }
  return v;
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

// log(1 + y) for y >= 0 with the hardware log, corrected for the rounding of 1 + y (the
// standard u = 1 + y, log(u) * y / (u - 1) form): a few ulp where a plain log(1 + y) loses the
// low bits of small y.
__device__ __forceinline__ float log1p_fast(float y) {
  const float u = 1.f + y;
  const float d = u - 1.f;
  return d == 0.f ? y : __logf(u) * (y * __builtin_amdgcn_rcpf(d));
}

// softplus (beta 1, threshold 20) from the hardware exp and log1p_fast.
__device__ __forceinline__ float softplus_fast(float x) {
  return x > 20.f ? x : log1p_fast(__expf(x));
}

// dt_adt with the hardware exp / log / reciprocal (a few ulp): the per-token scalars of the scan.
__device__ __forceinline__ void dt_adt_fast(bool raw, float dt_in, float a_in, float dt_bias,
                                            float& dt, float& adt) {
  if (raw) {
    dt = softplus_fast(dt_in + dt_bias);
    adt = fminf(-heavy_tail_fast(a_in), -kAFloor) * dt;
  } else {
    dt = dt_in;
    adt = a_in;
  }
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

// fmod(pi * tanh(angle) * dt, 2 pi) (model.py:225-230); m3_fmod_2pi is fmodf's exact result
// without its general reduction loop.
__device__ __forceinline__ float phase_inc(float angle, float dt) {
  return m3_fmod_2pi(__fmul_rn(__fmul_rn(kPi, tanhf(angle)), dt));
}

// ---------------------------------------------------------------- error reporting (host)

}  // namespace m3
