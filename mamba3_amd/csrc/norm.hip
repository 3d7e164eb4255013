// m3_rms_norm: the residual stream between two mixers of a prefill or forward pass.
//
// Between mixers the reference runs three elementwise passes over [B, L, d]: the residual add
// h + mixed (mamba3/model.py:511-512), the next block's RMSNorm (or norm_f, model.py:591, 607)
// and, under autocast, the cast of the normed rows to the projection's dtype. At config 2 these
// move about 1.2 GB per layer in torch. One pass here reads h and mixed once and writes the sum
// (when the caller keeps it) and the normed rows in the dtype their consumer wants.
//
// One wave per row (two rows per wave for dim <= 1024), 4 waves per workgroup; lane l holds the
// 4-element chunks 4 l + 256 j, j < CH = dim / 256, so each load instruction of a wave covers
// 256 consecutive elements. Every row's loads are issued before the first is used; the sum of
// squares is reduced over the wave. Arithmetic: s = x + add in FP32, rounded to x's dtype
// (torch's add of the promoted operands), out = rnd_out((s * rsqrt(mean(s^2) + eps)) *
// rnd_x(weight)) (torch's rms_norm with the weight cast to x's dtype, model.py:48-55).
#include <hip/hip_runtime.h>

#include "m3_common.hpp"
#include "m3_host.hpp"

namespace m3 {
namespace {

struct NormGeom {
  const void* x;
  const void* add;  // null: no add
  const void* w;
  void* sum;        // null: not written
  void* out;
  int64_t x_ld, a_ld, s_ld, o_ld;  // row strides (elements)
  int rows, dim, w_dtype;
  float eps;
};

template <typename T>
__device__ __forceinline__ f4 load4(const void* base, int64_t i) {
  f4 r;
  if constexpr (sizeof(T) == 4) {
    r = *reinterpret_cast<const f4*>(static_cast<const float*>(base) + i);
  } else {
    typedef T t4 __attribute__((ext_vector_type(4)));
    const t4 v = *reinterpret_cast<const t4*>(static_cast<const T*>(base) + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = to_f(v[j]);
  }
  return r;
}

template <typename T>
__device__ __forceinline__ void store4(void* base, int64_t i, f4 x) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<f4*>(static_cast<float*>(base) + i) = x;
  } else {
    typedef T t4 __attribute__((ext_vector_type(4)));
    t4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = from_f<T>(x[j]);
    *reinterpret_cast<t4*>(static_cast<T*>(base) + i) = v;
  }
}

__device__ __forceinline__ float wave_allsum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <typename TX, typename TA, typename TO, int CH>
__global__ __launch_bounds__(256) void rms_norm_kernel(const NormGeom g) {
  constexpr int RPW = CH <= 4 ? 2 : 1;  // rows per wave
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r0 = (static_cast<int>(blockIdx.x) * 4 + w) * RPW;
  const bool has_add = g.add != nullptr;
  f4 xv[RPW][CH], av[RPW][CH];
  // rows past the end re-read the last row; nothing of theirs is stored
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = min(r0 + r, g.rows - 1);
#pragma unroll
    for (int j = 0; j < CH; ++j) xv[r][j] = load4<TX>(g.x, row * g.x_ld + 256 * j + 4 * lane);
  }
  if (has_add) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int64_t row = min(r0 + r, g.rows - 1);
#pragma unroll
      for (int j = 0; j < CH; ++j) av[r][j] = load4<TA>(g.add, row * g.a_ld + 256 * j + 4 * lane);
    }
  }
  f4 wv[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int e = 256 * j + 4 * lane;
    const f4 raw = g.w_dtype == M3_F32 ? load4<float>(g.w, e)
                   : g.w_dtype == M3_BF16 ? load4<__bf16>(g.w, e) : load4<_Float16>(g.w, e);
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[j][i] = rnd<TX>(raw[i]);
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (has_add) xv[r][j][i] = rnd<TX>(xv[r][j][i] + av[r][j][i]);
        ss = fmaf(xv[r][j][i], xv[r][j][i], ss);
      }
    }
    ss = wave_allsum(ss);
    const float rstd = rsqrtf(ss / static_cast<float>(g.dim) + g.eps);
    const int row = r0 + r;
    if (row < g.rows) {
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int e = 256 * j + 4 * lane;
        if (g.sum != nullptr) store4<TX>(g.sum, row * g.s_ld + e, xv[r][j]);
        f4 y;
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = (xv[r][j][i] * rstd) * wv[j][i];
        store4<TO>(g.out, row * g.o_ld + e, y);
      }
    }
  }
}

template <typename TX, typename TA, typename TO>
int launch_ch(const NormGeom& g, hipStream_t stream) {
  const int ch = g.dim / 256;
  const int rpw = ch <= 4 ? 2 : 1;
  const int per_block = 4 * rpw;
  const dim3 grid(static_cast<unsigned>((g.rows + per_block - 1) / per_block)), block(256);
  switch (ch) {
    case 1: hipLaunchKernelGGL((rms_norm_kernel<TX, TA, TO, 1>), grid, block, 0, stream, g); break;
    case 2: hipLaunchKernelGGL((rms_norm_kernel<TX, TA, TO, 2>), grid, block, 0, stream, g); break;
    case 3: hipLaunchKernelGGL((rms_norm_kernel<TX, TA, TO, 3>), grid, block, 0, stream, g); break;
    case 4: hipLaunchKernelGGL((rms_norm_kernel<TX, TA, TO, 4>), grid, block, 0, stream, g); break;
    case 8: hipLaunchKernelGGL((rms_norm_kernel<TX, TA, TO, 8>), grid, block, 0, stream, g); break;
    default: return fail(M3_EUNSUPPORTED, "m3_rms_norm: dim %d not in {256, 512, 768, 1024, 2048}",
                         g.dim);
  }
  return check_launch("m3_rms_norm");
}

template <typename TX, typename TA>
int launch_out(const NormGeom& g, int out_dtype, hipStream_t stream) {
  switch (out_dtype) {
    case M3_F32: return launch_ch<TX, TA, float>(g, stream);
    case M3_BF16: return launch_ch<TX, TA, __bf16>(g, stream);
    default: return launch_ch<TX, TA, _Float16>(g, stream);
  }
}

bool overlaps(const m3_tensor& a, const m3_tensor& b, int64_t rows, int64_t dim) {
  if (a.ptr == nullptr || b.ptr == nullptr) return false;
  const char* a0 = static_cast<const char*>(a.ptr);
  const char* b0 = static_cast<const char*>(b.ptr);
  const char* a1 = a0 + ((rows - 1) * a.stride[0] + dim) * elem_size(a.dtype);
  const char* b1 = b0 + ((rows - 1) * b.stride[0] + dim) * elem_size(b.dtype);
  return a0 < b1 && b0 < a1;
}

int validate(const m3_rms_norm_args& a) {
  if (a.rows < 0 || a.dim <= 0) return fail(M3_EINVAL, "m3_rms_norm: invalid dimensions");
  if (a.rows >= INT32_MAX / 2 || a.dim > 2048 || a.dim % 256 != 0) {
    return fail(M3_EUNSUPPORTED, "m3_rms_norm: dim %lld must be a multiple of 256 up to 2048, "
                "rows below 2^30", static_cast<long long>(a.dim));
  }
  if (!(a.eps >= 0.f)) return fail(M3_EINVAL, "m3_rms_norm: eps must be >= 0");
  int rc;
  if ((rc = check_tensor(a.x, "x", 2, a.dim, true, -1)) ||
      (rc = check_tensor(a.add, "add", 2, a.dim, false, -1)) ||
      (rc = check_tensor(a.weight, "weight", 1, a.dim, true, -1)) ||
      (rc = check_tensor(a.sum_out, "sum_out", 2, a.dim, false, a.x.dtype)) ||
      (rc = check_tensor(a.out, "out", 2, a.dim, true, -1))) {
    return rc;
  }
  if (a.sum_out.ptr != nullptr && a.add.ptr == nullptr) {
    return fail(M3_EINVAL, "m3_rms_norm: sum_out needs add");
  }
  // the dtype combinations of a residual stream: FP32 rows with an add of any dtype, or 16-bit
  // rows with an add of their own dtype
  if (a.add.ptr != nullptr && a.x.dtype != M3_F32 && a.add.dtype != a.x.dtype) {
    return fail(M3_EUNSUPPORTED, "m3_rms_norm: a 16-bit x takes an add of its own dtype");
  }
  if (a.x.dtype != M3_F32 && a.out.dtype != a.x.dtype) {
    return fail(M3_EUNSUPPORTED, "m3_rms_norm: a 16-bit x gives out in its own dtype");
  }
  // 16-byte (FP32) / 8-byte (16-bit) chunks: base pointers and row strides aligned to 4 elements
  for (const m3_tensor* t : {&a.x, &a.add, &a.weight, &a.sum_out, &a.out}) {
    if (t->ptr == nullptr) continue;
    const int es = elem_size(t->dtype);
    if (reinterpret_cast<uintptr_t>(t->ptr) % (4 * es) != 0 || (t != &a.weight && t->stride[0] % 4 != 0)) {
      return fail(M3_EUNSUPPORTED, "m3_rms_norm: rows must be aligned to 4 elements");
    }
  }
  if (overlaps(a.out, a.x, a.rows, a.dim) || overlaps(a.out, a.add, a.rows, a.dim) ||
      overlaps(a.out, a.sum_out, a.rows, a.dim)) {
    return fail(M3_EINVAL, "m3_rms_norm: out overlaps an input or sum_out");
  }
  return M3_OK;
}

}  // namespace
}  // namespace m3

extern "C" int m3_rms_norm(const m3_rms_norm_args* args, hipStream_t stream) {
  using namespace m3;
  clear_error();
  if (args == nullptr) return fail(M3_EINVAL, "m3_rms_norm: NULL args");
  const m3_rms_norm_args& a = *args;
  const int rc = validate(a);
  if (rc != M3_OK) return rc;
  if (a.rows == 0) return M3_OK;
  NormGeom g{a.x.ptr, a.add.ptr, a.weight.ptr, a.sum_out.ptr, a.out.ptr,
             a.x.stride[0], a.add.stride[0], a.sum_out.stride[0], a.out.stride[0],
             static_cast<int>(a.rows), static_cast<int>(a.dim), a.weight.dtype, a.eps};
  const int ad = a.add.ptr != nullptr ? a.add.dtype : a.x.dtype;
  switch (a.x.dtype) {
    case M3_F32:
      switch (ad) {
        case M3_F32: return launch_out<float, float>(g, a.out.dtype, stream);
        case M3_BF16: return launch_out<float, __bf16>(g, a.out.dtype, stream);
        default: return launch_out<float, _Float16>(g, a.out.dtype, stream);
      }
    case M3_BF16: return launch_ch<__bf16, __bf16, __bf16>(g, stream);
    default: return launch_ch<_Float16, _Float16, _Float16>(g, stream);
  }
}
