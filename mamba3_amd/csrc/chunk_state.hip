// Standalone per-chunk state update (m3_chunk_state), the replacement of the reference's
// chunk_state launcher (_triton.py:500-561) for callers that drive the chunk loop themselves.
// The fused scan (scan.hip) carries the state in registers and does not use it.
#include <type_traits>

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

// The model's shape (N = 128, P = 64) with 16-bit activations, on MFMA: the update V^T ke of
// (b, h) is 32 tiles of S'^T (16 columns n x 16 rows p), accumulated over passes of ROWS
// (token, rank) rows with bf16 / f16 16x16x32 MFMAs (exact products of the rounded operands,
// FP32 sums, as the reference's bmm). Each pass stages ke (the same rounding points as above)
// and v transposed into LDS ([n][row], [p][row]); a lane stores a row pair of 8 columns, with
// the row pairs on consecutive lanes so a store instruction's lanes hit distinct banks. The
// global loads of pass i + 1 are issued before the MFMAs of pass i. Wave w owns rows
// p = 16 (w & 3) .. + 15 and its share of the 8 column tiles; lane l ends with S'[p][n .. n+3]
// of each of its tiles in the MFMA output layout, one 16-byte vector of the state row.
//
// ROWS rows per pass, 4 ROWS threads: 128 where the (b, h) pairs fit one workgroup per CU (2
// passes for a 256-token chunk, 52 KB of LDS), else 64 (27 KB, so more workgroups share a CU and
// overlap their loads with each other's MFMAs). Waves 0 .. 3 of the 128-row form take column
// tiles 0 .. 3 and waves 4 .. 7 tiles 4 .. 7 of the same p tiles.
constexpr long kCmCUs = 256;  // MI355X compute units

template <typename T, int ROWS>
__global__ __launch_bounds__(4 * ROWS) void chunk_state_mma_kernel(const m3_chunk_state_args a) {
  constexpr int N = 128, P = 64, LR = ROWS + 8, NT = N / 16 / (ROWS / 64), RP = ROWS / 2;
  typedef T t8 __attribute__((ext_vector_type(8)));
  const int H = a.heads, W = a.width, R = a.rank;
  const int b = blockIdx.x / H, h = blockIdx.x - (blockIdx.x / H) * H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  __shared__ __align__(16) T KeT[N * LR];
  __shared__ __align__(16) T VT[P * LR];
  const float* cum = static_cast<const float*>(a.cumulative.ptr) + b * a.cumulative.stride[0] +
                     h * a.cumulative.stride[1];
  const float* scl = static_cast<const float*>(a.scale.ptr) + b * a.scale.stride[0] +
                     h * a.scale.stride[1];
  const T* kb = static_cast<const T*>(a.k.ptr) + b * a.k.stride[0] + h * a.k.stride[1];
  const T* vb = static_cast<const T*>(a.value.ptr) + b * a.value.stride[0] + h * a.value.stride[1];
  const float cl = cum[(W - 1) * a.cumulative.stride[2]];
  const int rows = W * R;
  f4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f4{0.f, 0.f, 0.f, 0.f};
  const int rp = tid & (RP - 1), cg = tid / RP;  // row pair and column group of the staging
  const int pt = w & 3, nt0 = NT * (w >> 2);      // this wave's p tile and first column tile
  // the raw operands of one pass: every load issues unconditionally (rows past the end re-read
  // row 0 and stage zeros), so the next pass's loads fly during this pass's MFMAs
  t8 kr[2][2], vr[2];
  float sr[2], cr[2];
  auto load = [&](int r0) __attribute__((always_inline)) {
#pragma unroll
    for (int jr = 0; jr < 2; ++jr) {
      const int row = r0 + 2 * rp + jr;
      const int t = row < rows ? row / R : 0, r = row < rows ? row - t * R : 0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n0 = 8 * (cg + 8 * j);
        kr[j][jr] = *reinterpret_cast<const t8*>(kb + t * a.k.stride[2] + r * a.k.stride[3] + n0);
      }
      vr[jr] = *reinterpret_cast<const t8*>(vb + t * a.value.stride[2] + r * a.value.stride[3] +
                                             8 * cg);
      sr[jr] = scl[t * a.scale.stride[2]];
      cr[jr] = cum[t * a.cumulative.stride[2]];
    }
  };
  load(0);
  for (int r0 = 0; r0 < rows; r0 += ROWS) {
    __syncthreads();  // the previous pass's operands are read
    // ke rows 2 rp, 2 rp + 1, columns 8 cg .. 8 cg + 7 (two column groups per thread), then v
    typedef T t2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n0 = 8 * (cg + 8 * j);
      float ke[2][8];
#pragma unroll
      for (int jr = 0; jr < 2; ++jr) {
        const bool ok = r0 + 2 * rp + jr < rows;
        const float sc = rnd<T>(sr[jr]);
        const float ee = rnd<T>(expf(cl - cr[jr]));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          ke[jr][i] = ok ? mul_r<T>(mul_r<T>(to_f(kr[j][jr][i]), sc), ee) : 0.f;
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        *reinterpret_cast<t2*>(&KeT[(n0 + i) * LR + 2 * rp]) =
            t2{from_f<T>(ke[0][i]), from_f<T>(ke[1][i])};
      }
    }
    {
      const int p0 = 8 * cg;
      const bool ok0 = r0 + 2 * rp < rows, ok1 = r0 + 2 * rp + 1 < rows;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        *reinterpret_cast<t2*>(&VT[(p0 + i) * LR + 2 * rp]) =
            t2{ok0 ? vr[0][i] : from_f<T>(0.f), ok1 ? vr[1][i] : from_f<T>(0.f)};
      }
    }
    // no loads after the last pass: they would add a pass of k / v reads and hold the final
    // state read behind them in the in-order load counter
    if (r0 + ROWS < rows) load(r0 + ROWS);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < ROWS / 32; ++ks) {
      const t8 bv = *reinterpret_cast<const t8*>(&VT[(16 * pt + l16) * LR + 32 * ks + 8 * lg]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const t8 av =
            *reinterpret_cast<const t8*>(&KeT[(16 * (nt0 + nt) + l16) * LR + 32 * ks + 8 * lg]);
        if constexpr (std::is_same<T, __bf16>::value) {
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[nt], 0, 0, 0);
        } else {
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[nt], 0, 0, 0);
        }
      }
    }
  }
  const float ecl = expf(cl);
  const int p = 16 * pt + l16;
  const float* sin_ = static_cast<const float*>(a.state_in.ptr) + b * a.state_in.stride[0] +
                      h * a.state_in.stride[1] + p * a.state_in.stride[2];
  float* sout = static_cast<float*>(a.state_out.ptr) + b * a.state_out.stride[0] +
                h * a.state_out.stride[1] + p * a.state_out.stride[2];
  f4 old[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    old[nt] = *reinterpret_cast<const f4*>(sin_ + 16 * (nt0 + nt) + 4 * lg);
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    f4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = ecl * old[nt][i] + acc[nt][i];
    *reinterpret_cast<f4*>(sout + 16 * (nt0 + nt) + 4 * lg) = o;
  }
}

// The MFMA form's operand conditions: the model's shape, 16-bit k / value with 16-byte aligned
// rows of 8-element groups, 16-byte aligned state rows.
bool chunk_state_mma_ok(const m3_chunk_state_args& a) {
  if (a.act_dtype == M3_F32 || a.d_state != 128 || a.head_dim != 64) return false;
  for (const m3_tensor* t : {&a.k, &a.value}) {
    if (reinterpret_cast<uintptr_t>(t->ptr) % 16 != 0) return false;
    for (int i = 0; i < 4; ++i) {
      if (t->stride[i] % 8 != 0) return false;
    }
  }
  for (const m3_tensor* t : {&a.state_in, &a.state_out}) {
    if (reinterpret_cast<uintptr_t>(t->ptr) % 16 != 0) return false;
    for (int i = 0; i < 3; ++i) {
      if (t->stride[i] % 4 != 0) return false;
    }
  }
  return true;
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
  if (chunk_state_mma_ok(a)) {
    const bool few = static_cast<long>(a.batch) * a.heads <= kCmCUs;
    if (act == M3_BF16 && few) {
      hipLaunchKernelGGL((chunk_state_mma_kernel<__bf16, 128>), grid, dim3(512), 0, stream, a);
    } else if (act == M3_BF16) {
      hipLaunchKernelGGL((chunk_state_mma_kernel<__bf16, 64>), grid, dim3(256), 0, stream, a);
    } else if (few) {
      hipLaunchKernelGGL((chunk_state_mma_kernel<_Float16, 128>), grid, dim3(512), 0, stream, a);
    } else {
      hipLaunchKernelGGL((chunk_state_mma_kernel<_Float16, 64>), grid, dim3(256), 0, stream, a);
    }
    return check_launch("m3_chunk_state");
  }
  switch (act) {
    case M3_F32: hipLaunchKernelGGL(chunk_state_kernel<float>, grid, block, lds, stream, a); break;
    case M3_BF16: hipLaunchKernelGGL(chunk_state_kernel<__bf16>, grid, block, lds, stream, a); break;
    default: hipLaunchKernelGGL(chunk_state_kernel<_Float16>, grid, block, lds, stream, a); break;
  }
  return check_launch("m3_chunk_state");
}
