// Standalone per-chunk state update (m3_chunk_state), the replacement of the reference's
// chunk_state launcher (_triton.py:500-561) for callers that drive the chunk loop themselves.
// The fused scan (scan.hip) carries the state in registers and does not use it.
#include "m3_common.hpp"
#include "m3_host.hpp"

namespace m3 {

constexpr int kCsThreads = 256;
constexpr int kCsRows = 64;   // rows staged in LDS per pass
constexpr int kCsMaxE = 64;   // state elements per thread (P * N <= 16384)

// One chunk's state update (_triton.py:294-413) with the portable path's rounding points:
// ke = rnd(rnd(k * rnd(scale)) * rnd(exp(cum_last - cum))); S' = exp(cum_last) S + V^T ke.
template <typename T>
__global__ __launch_bounds__(kCsThreads) void chunk_state_kernel(const m3_chunk_state_args a) {
  const int H = a.heads, W = a.width, R = a.rank, N = a.d_state, P = a.head_dim;
  const int b = blockIdx.x / H, h = blockIdx.x - (blockIdx.x / H) * H;
  const int tid = threadIdx.x;
  extern __shared__ float cs_smem[];
  float* ke = cs_smem;                 // [kCsRows][N]
  float* vv = cs_smem + kCsRows * N;   // [kCsRows][P]
  const float* cum = static_cast<const float*>(a.cumulative.ptr) + b * a.cumulative.stride[0] +
                     h * a.cumulative.stride[1];
  const float* scl = static_cast<const float*>(a.scale.ptr) + b * a.scale.stride[0] +
                     h * a.scale.stride[1];
  const float cl = cum[(W - 1) * a.cumulative.stride[2]];
  const int rows = W * R, total = P * N;
  float acc[kCsMaxE];
#pragma unroll
  for (int i = 0; i < kCsMaxE; ++i) acc[i] = 0.f;
  for (int r0 = 0; r0 < rows; r0 += kCsRows) {
    __syncthreads();
    for (int idx = tid; idx < kCsRows * N; idx += kCsThreads) {
      const int row = r0 + idx / N, n = idx - (idx / N) * N;
      float v = 0.f;
      if (row < rows) {
        const int t = row / R, r = row - t * R;
        const float k = to_f(static_cast<const T*>(a.k.ptr)[b * a.k.stride[0] + h * a.k.stride[1] +
                                                             t * a.k.stride[2] +
                                                             r * a.k.stride[3] + n]);
        const float sc = rnd<T>(scl[t * a.scale.stride[2]]);
        const float ee = rnd<T>(expf(cl - cum[t * a.cumulative.stride[2]]));
        v = mul_r<T>(mul_r<T>(k, sc), ee);
      }
      ke[idx] = v;
    }
    for (int idx = tid; idx < kCsRows * P; idx += kCsThreads) {
      const int row = r0 + idx / P, p = idx - (idx / P) * P;
      float v = 0.f;
      if (row < rows) {
        const int t = row / R, r = row - t * R;
        v = to_f(static_cast<const T*>(a.value.ptr)[b * a.value.stride[0] + h * a.value.stride[1] +
                                                    t * a.value.stride[2] +
                                                    r * a.value.stride[3] + p]);
      }
      vv[idx] = v;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kCsMaxE; ++i) {
      const int e = tid + kCsThreads * i;
      if (e < total) {
        const int p = e / N, n = e - (e / N) * N;
        float s = 0.f;
        for (int j = 0; j < kCsRows; ++j) s += vv[j * P + p] * ke[j * N + n];
        acc[i] += s;
      }
    }
  }
  const float ecl = expf(cl);
  const float* sin_ = static_cast<const float*>(a.state_in.ptr) + b * a.state_in.stride[0] +
                      h * a.state_in.stride[1];
  float* sout = static_cast<float*>(a.state_out.ptr) + b * a.state_out.stride[0] +
                h * a.state_out.stride[1];
#pragma unroll
  for (int i = 0; i < kCsMaxE; ++i) {
    const int e = tid + kCsThreads * i;
    if (e < total) {
      const int p = e / N, n = e - (e / N) * N;
      const float old = sin_[p * a.state_in.stride[2] + n];
      sout[p * a.state_out.stride[2] + n] = ecl * old + acc[i];
    }
  }
}

}  // namespace m3

extern "C" int m3_chunk_state(const m3_chunk_state_args* args, hipStream_t stream) {
  using namespace m3;
  clear_error();
  if (args == nullptr) return fail(M3_EINVAL, "m3_chunk_state: args is NULL");
  const m3_chunk_state_args& a = *args;
  if (a.batch < 0 || a.width <= 0 || a.heads <= 0 || a.rank <= 0 || a.d_state <= 0 ||
      a.head_dim <= 0) {
    return fail(M3_EINVAL, "m3_chunk_state: invalid dimensions");
  }
  if (!valid_dtype(a.act_dtype)) return fail(M3_EINVAL, "m3_chunk_state: invalid act_dtype");
  if (a.d_state * a.head_dim > kCsThreads * kCsMaxE) {
    return fail(M3_EUNSUPPORTED, "m3_chunk_state: d_state x head_dim > %d", kCsThreads * kCsMaxE);
  }
  const size_t lds = sizeof(float) * kCsRows * (a.d_state + a.head_dim);
  if (lds > 64 * 1024) return fail(M3_EUNSUPPORTED, "m3_chunk_state: d_state + head_dim too large");
  const int act = a.act_dtype, N = a.d_state, P = a.head_dim;
  int rc;
  if ((rc = check_tensor(a.k, "k", 5, N, true, act)) ||
      (rc = check_tensor(a.value, "value", 5, P, true, act)) ||
      (rc = check_tensor(a.cumulative, "cumulative", 3, 1, true, M3_F32)) ||
      (rc = check_tensor(a.scale, "scale", 3, 1, true, M3_F32)) ||
      (rc = check_tensor(a.state_in, "state_in", 4, N, true, M3_F32)) ||
      (rc = check_tensor(a.state_out, "state_out", 4, N, true, M3_F32))) {
    return rc;
  }
  if (a.batch == 0) return M3_OK;
  const dim3 grid(static_cast<unsigned>(a.batch) * a.heads), block(kCsThreads);
  switch (act) {
    case M3_F32: hipLaunchKernelGGL(chunk_state_kernel<float>, grid, block, lds, stream, a); break;
    case M3_BF16: hipLaunchKernelGGL(chunk_state_kernel<__bf16>, grid, block, lds, stream, a); break;
    default: hipLaunchKernelGGL(chunk_state_kernel<_Float16>, grid, block, lds, stream, a); break;
  }
  return check_launch("m3_chunk_state");
}
