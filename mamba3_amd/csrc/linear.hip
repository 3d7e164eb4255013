// m3_linear: out[M, N] = x[M, K] * weight[N, K]^T (+ residual) for the few rows of a decode step.
//
// A general GEMM tiles M = 1..256 rows poorly: its large tiles leave most of the 256 CUs idle
// and each streams the weight at a fraction of HBM bandwidth. Five kernels, the MFMA ones on the
// bf16 / f16 16x16x32 (FP32 accumulation); the first that applies runs:
//
// gemv kernel (M <= 4, K a multiple of 512 up to 4096): a weight stream without MFMA. Each wave
// owns RW weight rows whose K range it reads whole, lane l taking the 16-byte chunks
// 8 (l + 64 c): one load instruction covers 1 KB of one row, and all of a lane's chunks are in
// flight at once (K / 512 per row). x goes to LDS once per workgroup (normed as in the rows
// kernel); each wave reduces its rows over its 64 lanes, so no sums cross waves. Measured on the
// decode shapes (N 8672, K 2048: 35.5 MB), this layout streams about 1.6x faster than 16 rows of
// 64-byte pieces per instruction.
//
// wide kernel (M <= 16, K a multiple of 512 up to 4096, N <= 16 x 256): the gemv kernel's
// weight stream feeding MFMA. One workgroup per 16 weight rows, one wave per 512 elements of K;
// each wave loads its 16 row pieces whole (1 KB per instruction), stages them in its own LDS
// region and reads them back as MFMA B operands, with x as the A operands straight from L2.
// Every workgroup reads all of x, so it takes the shapes whose workgroups fit one pass over the
// CUs: the out_proj shape (N 2048, K 4096) in 6.4 us at M = 5 and 8.2 us at M = 16.
//
// stream kernel (M <= 64, K a multiple of 256): a block of 32 or 64 x rows and 16-48 weight
// rows per workgroup, x and weight tiles loaded straight into an LDS ring (no registers held in
// flight), the K steps of a stage split over the waves. Fewer workgroups than the wide kernel
// read x. Timed in a graph of 24 calls with distinct weights: in_proj (N 8672, K 2048)
// 9.4-10.5 us at M = 5-32 and 13.5 us at M = 64, 9.6-11.0 / 14.7 us with the RMSNorm fused,
// against about 14-15.4 us for hipBLASLt and 5 us more for a separate norm; out_proj (N 2048,
// K 4096) 8.4-9.0 us at M = 17-64.
//
// rows kernel (M <= 32 where the kernels above do not apply): a weight stream. The B operand of
// a 16x16x32 MFMA is, per lane, 16 contiguous bytes of one weight row (lane l16 + 16 lg holds
// row l16, elements 8 lg .. 8 lg + 7 of the 32-element step), and the A operand the same of an
// x row, so both are loaded straight into registers: no LDS staging, no barrier in the K loop.
// A workgroup owns 16 * TN columns; its waves split the K range and add their sums through LDS
// at the end.
//
// tile kernel (M > 64, or M > 32 with K not a multiple of 256): one 256-thread workgroup
// (4 waves) owns MT rows x NT columns; x and weight tiles are staged through LDS (double
// buffered, KS elements of K per stage, rows padded by 8 elements so the 16 rows one MFMA
// operand reads fall in distinct 16-byte bank groups).
//
// When the output tiles alone do not fill the GPU, the rows and tile kernels also split the K
// axis over workgroups: FP32 partial sums go to the workspace and a reduce kernel adds them (and
// the residual) and rounds once. Loads go through buffer resources whose extents end at the last
// byte of the last valid row, so nothing outside the operands is ever read.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "m3_common.hpp"
#include "m3_host.hpp"

namespace m3 {
namespace {

constexpr int kStep = 32;           // K elements per MFMA
constexpr int kOff = 0x7ffffff0;    // buffer offset past every extent: the load returns 0

template <typename T> struct LinMma;
template <> struct LinMma<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f4 mma(v8 a, v8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct LinMma<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f4 mma(v8 a, v8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

struct LinGeom {
  const char* x;       // [M, K], row stride x_ld (elements)
  const char* w;       // [N, K], row stride w_ld
  const void* res;     // [M, N] or null, row stride r_ld
  void* out;           // [M, N], row stride o_ld
  float* part;         // [splits, M, N] FP32 partial sums (splits > 1)
  const char* nw;      // [K] RMSNorm weight or null (rows kernel, splits == 1)
  float eps;
  int m, n, k, k_split, splits;
  int x_ld, w_ld, r_ld, o_ld;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t lin_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// Bytes from the start of row 0 to the end of row rows - 1 (K elements used per row).
__device__ __forceinline__ int64_t lin_extent(int rows, int ld, int k) {
  return rows > 0 ? (static_cast<int64_t>(rows - 1) * ld + k) * 2 : 0;
}

// One output element: to the partial sums of this K split, or (unsplit) plus the residual,
// rounded once into out.
template <typename T>
__device__ __forceinline__ void lin_emit(const LinGeom& g, int split, int m, int n, float y) {
  if (g.splits > 1) {
    g.part[(static_cast<int64_t>(split) * g.m + m) * g.n + n] = y;
    return;
  }
  if (g.res != nullptr) {
    y += static_cast<float>(static_cast<const T*>(g.res)[static_cast<int64_t>(m) * g.r_ld + n]);
  }
  static_cast<T*>(g.out)[static_cast<int64_t>(m) * g.o_ld + n] = static_cast<T>(y);
}

// ----------------------------------------------------------------------------- rows kernel

// M <= 16 TM rows; workgroup (blockIdx.x, blockIdx.z) = 16 TN columns x one K split; its WAVES
// waves take equal runs of that split's 32-element steps. Rows past M / N are clamped to the last
// valid row (their sums are never written).
//
// NORM (whole K in one workgroup): x is RMS-normalised on the fly. The A operand is x * nw
// (FP32 product, rounded once to T) and each lane also sums the squares of the x it loads; the
// per-row sums of squares meet in LDS with the products, and each output is scaled by
// rsqrt(sum / K + eps): sum_k (x r nw)_k w_k = r sum_k (x nw)_k w_k.
template <typename T, int TM, int TN, int WAVES, int D, bool NORM>
__global__ __launch_bounds__(64 * WAVES) void linear_rows_kernel(const LinGeom g) {
  using M = LinMma<T>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16 * TN, split = blockIdx.z;
  const int k_begin = split * g.k_split;
  const int all = max(0, min(g.k, k_begin + g.k_split) - k_begin) / kStep;
  const int per = (all + WAVES - 1) / WAVES;
  const int s_begin = min(all, w * per);
  const int nsteps = min(all, s_begin + per) - s_begin;
  const int kb = k_begin + s_begin * kStep;

  const int vn = min(16 * TN, g.n - n0);
  const __amdgpu_buffer_rsrc_t rw =
      lin_rsrc(g.w + static_cast<int64_t>(n0) * g.w_ld * 2, lin_extent(vn, g.w_ld, g.k));
  const __amdgpu_buffer_rsrc_t rx = lin_rsrc(g.x, lin_extent(g.m, g.x_ld, g.k));
  const __amdgpu_buffer_rsrc_t rn = lin_rsrc(g.nw, NORM ? int64_t{2} * g.k : 0);
  int woff[TN], xoff[TM];
#pragma unroll
  for (int j = 0; j < TN; ++j) woff[j] = (min(16 * j + l16, vn - 1) * g.w_ld + 8 * lg + kb) * 2;
#pragma unroll
  for (int i = 0; i < TM; ++i) xoff[i] = (min(16 * i + l16, g.m - 1) * g.x_ld + 8 * lg + kb) * 2;
  const int noff = (8 * lg + kb) * 2;

  u32x4 rb[D][TN], ra[D][TM], rnw[D];
  auto load = [&](int slot, int s) __attribute__((always_inline)) {
    const bool live = s < nsteps;
    if constexpr (NORM) {
      rnw[slot] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                rn, live ? noff + 2 * kStep * s : kOff, 0, 0));
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      // non-temporal (aux bit 1): the weight is streamed once per call
      rb[slot][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rw, live ? woff[j] + 2 * kStep * s : kOff, 0, 2));
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      ra[slot][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rx, live ? xoff[i] + 2 * kStep * s : kOff, 0, 0));
    }
  };
  f4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  }
  float ssq[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) ssq[i] = 0.f;
  auto step = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      typename M::v8 a = __builtin_bit_cast(typename M::v8, ra[slot][i]);
      if constexpr (NORM) {
        const typename M::v8 nv = __builtin_bit_cast(typename M::v8, rnw[slot]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float xf = static_cast<float>(a[e]);
          ssq[i] = fmaf(xf, xf, ssq[i]);
          a[e] = static_cast<T>(xf * static_cast<float>(nv[e]));
        }
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        acc[i][j] = M::mma(a, __builtin_bit_cast(typename M::v8, rb[slot][j]), acc[i][j]);
      }
    }
  };
#pragma unroll
  for (int d = 0; d < D; ++d) load(d, d);
  // whole groups of D steps with no exit inside (the wait counts stay exact across the back
  // edge), then the last nsteps % D steps, which load nothing
  const int nfull = nsteps - nsteps % D;
  for (int s0 = 0; s0 < nfull; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      step(d);
      load(d, s0 + d + D);
      __builtin_amdgcn_sched_barrier(0);  // keep each step's loads right after its MFMAs
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    if (nfull + d < nsteps) step(d);
  }

  // lane holds rows 16 i + 4 lg + r, column n0 + 16 j + l16; the waves' sums meet in LDS (and,
  // with NORM, the sums of squares of rows 16 i + l16, first added over the lane's 4 groups)
  __shared__ float red[WAVES][TM * TN * 4][64];
  __shared__ float red_ssq[NORM ? WAVES : 1][TM][16];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) red[w][(i * TN + j) * 4 + r][lane] = acc[i][j][r];
    }
    if constexpr (NORM) {
      float v = ssq[i] + __shfl_xor(ssq[i], 16);
      v += __shfl_xor(v, 32);
      if (lg == 0) red_ssq[w][i][l16] = v;
    }
  }
  __syncthreads();
  for (int e = tid; e < TM * TN * 256; e += 64 * WAVES) {
    const int q = e >> 6, ln = e & 63;
    float y = 0.f;
#pragma unroll
    for (int v = 0; v < WAVES; ++v) y += red[v][q][ln];
    const int i = q / (4 * TN), j = (q >> 2) % TN, r = q & 3;
    const int m = 16 * i + 4 * (ln >> 4) + r, n = n0 + 16 * j + (ln & 15);
    if constexpr (NORM) {
      float sq = 0.f;
#pragma unroll
      for (int v = 0; v < WAVES; ++v) sq += red_ssq[v][i][4 * (ln >> 4) + r];
      y *= rsqrtf(sq / static_cast<float>(g.k) + g.eps);
    }
    if (m < g.m && n < g.n) lin_emit<T>(g, split, m, n, y);
  }
}

// ----------------------------------------------------------------------------- gemv kernel

constexpr int kGemvRows = 4;  // x rows (M) the gemv kernel takes

// Sum over the 64 lanes of a wave: DPP rotations within each 16-lane row, then the rows.
__device__ __forceinline__ float lin_wave_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128,
                                                             0xf, 0xf, false));  // row_ror:8
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124,
                                                             0xf, 0xf, false));  // row_ror:4
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122,
                                                             0xf, 0xf, false));  // row_ror:2
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121,
                                                             0xf, 0xf, false));  // row_ror:1
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Wave w of workgroup b owns weight rows RW (4 b + w) .. + RW - 1 (rows past N are read as zeros
// through the buffer extent and never written). CH >= K / 512 chunks per lane and row.
template <typename T, int RW, int CH, bool NORM>
__global__ __launch_bounds__(256) void linear_gemv_kernel(const LinGeom g) {
  using V8 = typename LinMma<T>::v8;
  constexpr int XU = (64 * CH + 255) / 256;  // x chunks per thread and row
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = (4 * blockIdx.x + w) * RW;
  const int nk = g.k / 512, xk = g.k / 8;  // chunks per lane and row; chunks per x row

  // x (and the norm weight) first: small, mostly from L2; then every weight chunk of the wave
  const __amdgpu_buffer_rsrc_t rx = lin_rsrc(g.x, lin_extent(g.m, g.x_ld, g.k));
  const __amdgpu_buffer_rsrc_t rn = lin_rsrc(g.nw, NORM ? int64_t{2} * g.k : 0);
  const __amdgpu_buffer_rsrc_t rw = lin_rsrc(g.w, lin_extent(g.n, g.w_ld, g.k));
  u32x4 xv[kGemvRows][XU], nv[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int kc = tid + 256 * u;
#pragma unroll
    for (int m = 0; m < kGemvRows; ++m) {
      xv[m][u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rx, m < g.m && kc < xk ? (m * g.x_ld + 8 * kc) * 2
                                                                      : kOff, 0, 0));
    }
    if constexpr (NORM) {
      nv[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rn, kc < xk ? 16 * kc : kOff, 0, 0));
    }
  }
  u32x4 wv[RW][CH];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const bool live = n0 + r < g.n && c < nk;
      // non-temporal (aux bit 1): each weight byte is read once per call
      wv[r][c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rw, live ? ((n0 + r) * g.w_ld + 8 * (lane + 64 * c)) * 2
                                                        : kOff, 0, 2));
    }
  }

  // x rows to LDS: a = rnd(x * nw) with NORM (the RMS factor is applied to the sums), else x.
  // Branch-free: chunks past M or K were loaded as zeros and land in rows / columns no lane
  // reads (256 XU chunks = 512 CH elements per row), so no load is sunk behind a branch whose
  // wait would also wait for the weight stream.
  __shared__ __attribute__((aligned(16))) T xs[kGemvRows][512 * CH];
  __shared__ float red[4][kGemvRows];
  static_assert(256 * XU * 8 <= 512 * CH, "x chunks fit the LDS rows");
  float ssq[kGemvRows];
#pragma unroll
  for (int m = 0; m < kGemvRows; ++m) {
    ssq[m] = 0.f;
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const int kc = tid + 256 * u;
      V8 a = __builtin_bit_cast(V8, xv[m][u]);
      if constexpr (NORM) {
        const V8 nw = __builtin_bit_cast(V8, nv[u]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float xf = static_cast<float>(a[e]);
          ssq[m] = fmaf(xf, xf, ssq[m]);
          a[e] = static_cast<T>(xf * static_cast<float>(nw[e]));
        }
      }
      *reinterpret_cast<V8*>(&xs[m][8 * kc]) = a;
    }
    if constexpr (NORM) {
      const float v = lin_wave_sum(ssq[m]);
      if (lane == 0) red[w][m] = v;
    }
  }
  __syncthreads();

  float acc[RW][kGemvRows];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int m = 0; m < kGemvRows; ++m) acc[r][m] = 0.f;
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (c < nk) {
#pragma unroll
      for (int m = 0; m < kGemvRows; ++m) {
        if (m < g.m) {
          const V8 a = *reinterpret_cast<const V8*>(&xs[m][8 * (lane + 64 * c)]);
#pragma unroll
          for (int r = 0; r < RW; ++r) {
            const V8 wr = __builtin_bit_cast(V8, wv[r][c]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              acc[r][m] = fmaf(static_cast<float>(a[e]), static_cast<float>(wr[e]), acc[r][m]);
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kGemvRows; ++m) {
    if (m < g.m) {
      float scale = 1.f;
      if constexpr (NORM) {
        scale = rsqrtf((red[0][m] + red[1][m] + red[2][m] + red[3][m]) /
                           static_cast<float>(g.k) + g.eps);
      }
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const float y = lin_wave_sum(acc[r][m]);
        if (lane == 0 && n0 + r < g.n) lin_emit<T>(g, 0, m, n0 + r, y * scale);
      }
    }
  }
}

// ----------------------------------------------------------------------------- wide kernel

// 4 < M <= 16 TM (the plan takes TM = 1), K = 512 WAVES. One workgroup per 16 weight rows; wave w owns K elements
// [512 w, 512 w + 512). Its 16 rows' pieces are loaded whole, one instruction per row (lane l
// taking elements 8 l .. 8 l + 7: 1 KB of contiguous row per instruction, the gemv kernel's
// stream), staged in the wave's own LDS region and read back as the MFMA B operands (row l16,
// elements 32 s + 8 lg of K step s). The wave alone reads its region, and one wave's LDS
// operations complete in order, so no barrier separates the two. The A operands come straight
// from memory (x is small and stays in L2), D steps ahead. The waves' partial sums then meet in
// their own regions. NORM as in the rows kernel.
template <typename T, int TM, int WAVES, bool NORM>
__global__ __launch_bounds__(64 * WAVES) void linear_wide_kernel(const LinGeom g) {
  using M = LinMma<T>;
  constexpr int KW = 512, LDW = KW + 8;  // K per wave; LDS row stride (16-byte reads of 16 rows
                                         // at one column fall in 16 distinct bank groups)
  // K steps per wave; steps of x in flight (all of them when they fit the registers)
  constexpr int NS = KW / kStep, D = TM <= 2 ? NS : 4;
  static_assert(NS % D == 0, "whole rings");
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int kb = w * KW;
  const int vn = min(16, g.n - n0);
  const __amdgpu_buffer_rsrc_t rw =
      lin_rsrc(g.w + static_cast<int64_t>(n0) * g.w_ld * 2, lin_extent(vn, g.w_ld, g.k));
  const __amdgpu_buffer_rsrc_t rx = lin_rsrc(g.x, lin_extent(g.m, g.x_ld, g.k));
  const __amdgpu_buffer_rsrc_t rn = lin_rsrc(g.nw, NORM ? int64_t{2} * g.k : 0);

  // the wave's weight rows first (non-temporal: streamed once per call)
  u32x4 wr[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    wr[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          rw, r < vn ? (r * g.w_ld + kb + 8 * lane) * 2 : kOff, 0,
                                          2));
  }
  // x (and the norm weight) of the first D steps
  int xoff[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) xoff[i] = (min(16 * i + l16, g.m - 1) * g.x_ld + kb + 8 * lg) * 2;
  const int noff = (kb + 8 * lg) * 2;
  u32x4 ra[D][TM], rnw[D];
  auto load = [&](int slot, int s) __attribute__((always_inline)) {
    const bool live = s < NS;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      ra[slot][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rx, live ? xoff[i] + 2 * kStep * s : kOff, 0, 0));
    }
    if constexpr (NORM) {
      rnw[slot] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                rn, live ? noff + 2 * kStep * s : kOff, 0, 0));
    }
  };
#pragma unroll
  for (int d = 0; d < D; ++d) load(d, d);
  __builtin_amdgcn_sched_barrier(0);  // every load above issues before the first wait

  // the weight rows to the wave's LDS region
  __shared__ __attribute__((aligned(16))) T wl[WAVES][16][LDW];
#pragma unroll
  for (int r = 0; r < 16; ++r) *reinterpret_cast<u32x4*>(&wl[w][r][8 * lane]) = wr[r];

  f4 acc[TM];
  float ssq[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    acc[i] = f4{0.f, 0.f, 0.f, 0.f};
    ssq[i] = 0.f;
  }
#pragma unroll
  for (int s0 = 0; s0 < NS; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int s = s0 + d;
      const typename M::v8 b =
          *reinterpret_cast<const typename M::v8*>(&wl[w][l16][kStep * s + 8 * lg]);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        typename M::v8 a = __builtin_bit_cast(typename M::v8, ra[d][i]);
        if constexpr (NORM) {
          const typename M::v8 nv = __builtin_bit_cast(typename M::v8, rnw[d]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float xf = static_cast<float>(a[e]);
            ssq[i] = fmaf(xf, xf, ssq[i]);
            a[e] = static_cast<T>(xf * static_cast<float>(nv[e]));
          }
        }
        acc[i] = M::mma(a, b, acc[i]);
      }
      load(d, s + D);
    }
  }

  // partial sums: lane holds rows 16 i + 4 lg + r of column n0 + l16; they go to the wave's own
  // region (its reads of it are complete), and with NORM the sums of squares of rows 16 i + l16
  float* red = reinterpret_cast<float*>(&wl[w][0][0]);
  __shared__ float red_ssq[NORM ? WAVES : 1][TM][16];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(i * 4 + r) * 64 + lane] = acc[i][r];
    if constexpr (NORM) {
      float v = ssq[i] + __shfl_xor(ssq[i], 16);
      v += __shfl_xor(v, 32);
      if (lg == 0) red_ssq[w][i][l16] = v;
    }
  }
  static_assert(TM * 4 * 64 * 4 <= 16 * LDW * 2, "partial sums fit a wave's region");
  __syncthreads();
  for (int e = tid; e < TM * 256; e += 64 * WAVES) {
    const int q = e >> 6, ln = e & 63;
    float y = 0.f;
#pragma unroll
    for (int v = 0; v < WAVES; ++v) y += reinterpret_cast<const float*>(&wl[v][0][0])[q * 64 + ln];
    const int i = q >> 2, r = q & 3;
    const int m = 16 * i + 4 * (ln >> 4) + r, n = n0 + (ln & 15);
    if constexpr (NORM) {
      float sq = 0.f;
#pragma unroll
      for (int v = 0; v < WAVES; ++v) sq += red_ssq[v][i][4 * (ln >> 4) + r];
      y *= rsqrtf(sq / static_cast<float>(g.k) + g.eps);
    }
    if (m < g.m && n < g.n) lin_emit<T>(g, 0, m, n, y);
  }
}

// ----------------------------------------------------------------------------- tile kernel

// Workgroup tile MT x NT, WM x WN waves, each wave (MT / WM) x (NT / WN) of 16x16 MFMA tiles;
// KS elements of K per LDS stage. D stages are in flight in registers (a ring indexed statically
// by unrolling the stage loop D times): at stage s the registers of stage s are free (already in
// LDS) and take stage s + D.
template <typename T, int MT, int NT, int WM, int WN, int KS, int D>
__global__ __launch_bounds__(256) void linear_tile_kernel(const LinGeom g) {
  using M = LinMma<T>;
  constexpr int MW = MT / WM, NW = NT / WN, TM = MW / 16, TN = NW / 16;
  static_assert(WM * WN == 4 && TM >= 1 && TN >= 1, "wave tiling");
  static_assert(D % 2 == 0, "the LDS buffer of stage s is s & 1 == d & 1");
  static_assert(KS % kStep == 0 && 512 % KS == 0, "stage width");
  constexpr int RS = KS + 8;  // LDS row stride (elements)

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int wm = w / WN, wn = w - wm * WN;
  const int n_base = blockIdx.x * NT, m_base = blockIdx.y * MT, split = blockIdx.z;
  const int k_begin = split * g.k_split;
  // K is a multiple of 32 but not always of KS: the last stage may be partial. Its 8-element
  // chunks at or past the split's end read zero (they would otherwise read the next row).
  const int range = max(0, min(g.k, k_begin + g.k_split) - k_begin);
  const int nsteps = (range + KS - 1) / KS;

  // A stage's 16-byte chunks are handed out in wave units of 64: RU = 512 / KS tile rows of
  // KS / 8 chunks. Unit u = 4 j + wave holds x rows RU u.. when u < MT / RU, then weight rows;
  // units past the tile are dummies. Each unit loads through its own buffer resource, built from
  // wave-uniform values (rows past M / N and dummy units read zero).
  constexpr int CPR = KS / 8, RU = 64 / CPR, U = (MT + NT) / RU, NCH = (U + 3) / 4;
  static_assert(MT % RU == 0 && NT % RU == 0, "unit rows");
  __shared__ __attribute__((aligned(16))) T sm[2][4 * NCH * RU * RS];
  __amdgpu_buffer_rsrc_t rs[NCH];
  int goff[NCH], loff[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int u = 4 * j + w;
    const bool isx = u < MT / RU;
    const int row0 = isx ? m_base + RU * u : n_base + RU * (u - MT / RU);
    const int rows = u < U ? (isx ? g.m : g.n) : 0;
    const int ld = isx ? g.x_ld : g.w_ld;
    const int valid = max(0, min(RU, rows - row0));
    rs[j] = lin_rsrc((isx ? g.x : g.w) + static_cast<int64_t>(row0) * ld * 2,
                     lin_extent(valid, ld, g.k));
    goff[j] = ((lane / CPR) * ld + 8 * (lane % CPR) + k_begin) * 2;
    loff[j] = (RU * u + lane / CPR) * RS + 8 * (lane % CPR);
  }
  u32x4 rg[D][NCH];
  const int lcol = 8 * (lane % CPR);
  auto load = [&](int slot, int s) __attribute__((always_inline)) {
    const bool live = s < nsteps && KS * s + lcol < range;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      rg[slot][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rs[j], live ? goff[j] + 2 * KS * s : kOff, 0, 0));
    }
  };
  auto store = [&](int slot, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) *reinterpret_cast<u32x4*>(&sm[buf][loff[j]]) = rg[slot][j];
  };

  f4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int d = 0; d < D; ++d) load(d, d);
  store(0, 0);
  __syncthreads();
  // stage s from LDS buffer s & 1 (== d & 1, D even); then the registers of stage s + 1 go to
  // the other buffer (past the last stage: zeros into the idle buffer)
  auto stage = [&](int d) __attribute__((always_inline)) {
    const T* buf = sm[d & 1];
#pragma unroll
    for (int kk = 0; kk < KS / kStep; ++kk) {
      typename M::v8 av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        av[i] = *reinterpret_cast<const typename M::v8*>(
            &buf[(wm * MW + 16 * i + l16) * RS + kStep * kk + 8 * lg]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        bv[j] = *reinterpret_cast<const typename M::v8*>(
            &buf[(MT + wn * NW + 16 * j + l16) * RS + kStep * kk + 8 * lg]);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = M::mma(av[i], bv[j], acc[i][j]);
      }
    }
    store((d + 1) % D, (d & 1) ^ 1);
    __syncthreads();
  };
  // whole groups of D stages with no exit inside, then the last nsteps % D, which load nothing
  const int nfull = nsteps - nsteps % D;
  for (int s0 = 0; s0 < nfull; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      load(d, s0 + d + D);
      stage(d);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    if (nfull + d < nsteps) stage(d);
  }

  // lane holds rows 16 i + 4 lg + r, column 16 j + l16 of its wave tile
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n_base + wn * NW + 16 * j + l16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m_base + wm * MW + 16 * i + 4 * lg + r;
        if (m < g.m && n < g.n) lin_emit<T>(g, split, m, n, acc[i][j][r]);
      }
    }
  }
}

// ----------------------------------------------------------------------------- stream kernel

// Waits until at most N of this wave's vector-memory operations are outstanding. The stream
// kernel's loads write LDS directly and return nothing to registers; the kernel waits for them
// itself, counting its own loads.
template <int N>
__device__ __forceinline__ void lin_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void lin_wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// LDS reads the compiler does not track, with the wait that makes their values usable, in one
// asm statement: no instruction the compiler places can read an output register before the
// wait (early-clobber outputs, so no address register is overwritten while a later read in the
// statement still needs it). The compiler would otherwise wait for all of the wave's loads into
// LDS still in flight before any LDS read, which undoes the ring.
template <int K>
__device__ __forceinline__ void lin_ds_read_all(u32x4 (&v)[K], const uint32_t (&a)[K]) {
  static_assert(K >= 1 && K <= 6, "1 to 6 reads per statement");
  if constexpr (K == 1) {
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v[0]) : "v"(a[0]));
  } else if constexpr (K == 2) {
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]) : "v"(a[0]), "v"(a[1]));
  } else if constexpr (K == 3) {
    asm volatile("ds_read_b128 %0, %3\n\tds_read_b128 %1, %4\n\tds_read_b128 %2, %5\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]) : "v"(a[0]), "v"(a[1]), "v"(a[2]));
  } else if constexpr (K == 4) {
    asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\t"
                 "ds_read_b128 %3, %7\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]));
  } else if constexpr (K == 5) {
    asm volatile("ds_read_b128 %0, %5\n\tds_read_b128 %1, %6\n\tds_read_b128 %2, %7\n\t"
                 "ds_read_b128 %3, %8\n\tds_read_b128 %4, %9\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]));
  } else {
    asm volatile("ds_read_b128 %0, %6\n\tds_read_b128 %1, %7\n\tds_read_b128 %2, %8\n\t"
                 "ds_read_b128 %3, %9\n\tds_read_b128 %4, %10\n\tds_read_b128 %5, %11\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]));
  }
}

__device__ __forceinline__ uint32_t lin_lds_addr(const char* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p));
}

// A buffer load of 16 bytes per lane written straight to LDS: lane l's bytes land at
// dst + 16 l (dst wave-uniform). The builtin exists only in the device pass of the compiler
// (the host pass, which emits the launch stubs, would drop the kernel).
template <int AUX>
__device__ __forceinline__ void lin_load_lds(__amdgpu_buffer_rsrc_t r, char* dst, int voff,
                                             int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16,
                                           voff, soff, 0, AUX);
#else
  (void)r, (void)dst, (void)voff, (void)soff;
#endif
}

// 4 < M <= 64: a block of MT = 32 or 64 x rows (blockIdx.y) and NT weight rows (blockIdx.x) per
// 512-thread workgroup over the whole K range (one rounding, no reduce launch). Stages of KB
// elements of K hold the MT x rows and NT weight rows in LDS, S stages in a ring, loaded straight into LDS (buffer loads
// with the LDS destination): a load unit is one instruction, 64 lanes x 16 bytes = RPU whole
// row pieces, contiguous in memory and in LDS, and the ring keeps S - 1 stages in flight with no
// registers held. Within a row piece the 16-byte chunk c sits at position c ^ (row & 15), so the
// 16 rows one MFMA operand reads at one chunk fall in 16 distinct bank groups. Each wave takes
// every WK-th K step of a stage for TMW of the M tiles and all NT columns; the waves' partial
// sums meet in LDS at the end. NORM (x RMS-normalised, as in the rows kernel): one more unit per
// stage brings that stage's norm weights, the A operands are multiplied by them and the squares
// of x are summed on the way.
template <typename T, int MT, int NT, int KB, int S, bool NORM>
__global__ __launch_bounds__(512) void linear_stream_kernel(const LinGeom g) {
  using M = LinMma<T>;
  constexpr int WAVES = 8;
  constexpr int CPR = KB / 8;                          // 16-byte chunks per row piece
  constexpr int RPU = 64 / CPR;                        // row pieces per load unit
  constexpr int XU = MT / RPU, U = (MT + NT) / RPU;    // x units, x and weight units
  constexpr int UN = U + (NORM ? 1 : 0);               // + the norm-weight unit
  constexpr int UPW = (UN + WAVES - 1) / WAVES;        // units per wave (past UN: dummies)
  constexpr int XJ = XU / WAVES;                       // a wave's first XJ units are x
  constexpr int SB = UN * 1024;                        // stage bytes
  constexpr int KS = KB / kStep;                       // K steps per stage
  constexpr int WK = KS < WAVES ? KS : WAVES;          // waves splitting a stage's K steps
  constexpr int WT = WAVES / WK;                       // wave groups splitting the M tiles
  constexpr int QS = KS / WK;                          // K steps per wave per stage
  constexpr int TMW = MT / 16 / WT, TN = NT / 16;      // a wave's tiles
  constexpr int RB = CPR * 16;                         // LDS bytes per row piece
  static_assert(CPR >= 16 && CPR <= 64 && XU % WAVES == 0, "stage shape");
  static_assert(KS % WK == 0 && (MT / 16) % WT == 0 && TMW >= 1 && TN >= 1, "wave tiling");
  static_assert(S >= 3 && UPW * (S - 2) < 64, "ring depth");
  static_assert(KB <= 512, "a stage's norm weights fit one unit");
  static_assert(WAVES * TMW * TN * 1024 <= S * SB, "partial sums fit the ring");

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int kw = w % WK, tw = w / WK;
  const int n0 = blockIdx.x * NT, m0 = blockIdx.y * MT;
  const int ns = g.k / KB;  // stages (the plan keeps K a multiple of KB)

  __shared__ __attribute__((aligned(1024))) char ring[S][SB];
  __shared__ __attribute__((aligned(1024))) char spare[UPW * WAVES > UN ? 1024 : 16];
  __shared__ float red_ssq[NORM ? WAVES : 1][TMW][16];

  const __amdgpu_buffer_rsrc_t rx = lin_rsrc(g.x, lin_extent(g.m, g.x_ld, g.k));
  const __amdgpu_buffer_rsrc_t rw = lin_rsrc(g.w, lin_extent(g.n, g.w_ld, g.k));
  const __amdgpu_buffer_rsrc_t rn = lin_rsrc(g.nw, NORM ? int64_t{2} * g.k : 0);

  // unit j of this wave is unit j * WAVES + w of the stage; lane offsets at stage 0. Rows past
  // M / N repeat the last valid row (their sums are never written). With NORM, unit U holds the
  // stage's KB norm weights (lane l loads chunk l % CPR). Dummy units (which keep every wave's
  // count of loads per stage equal) and stages past the last read nothing (offsets past every
  // extent); dummies land in one spare KB. So every wave issues UPW loads per stage, and
  // nothing else in the loop touches memory.
  int uoff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; ++j) {
    const int u = j * WAVES + w;
    const int r = u * RPU + lane / CPR, c = (lane % CPR) ^ (r & 15);
    if (j < XJ) {
      uoff[j] = (min(m0 + r, g.m - 1) * g.x_ld + 8 * c) * 2;
    } else if (u < U) {
      uoff[j] = (min(n0 + r - MT, g.n - 1) * g.w_ld + 8 * c) * 2;
    } else if (NORM && u == U) {
      uoff[j] = 16 * (lane % CPR);
    } else {
      uoff[j] = kOff;
    }
  }
  auto issue = [&](int s, int slot) __attribute__((always_inline)) {
    const bool live = s < ns;
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
      const int u = j * WAVES + w;
      char* dst = u < UN ? &ring[slot][1024 * u] : spare;
      if (j < XJ) {
        lin_load_lds<0>(rx, dst, live ? uoff[j] : kOff, 2 * KB * s);
      } else if (u < U) {
        lin_load_lds<2>(rw, dst, live ? uoff[j] : kOff, 2 * KB * s);
      } else if (NORM && u == U) {
        lin_load_lds<0>(rn, dst, live ? uoff[j] : kOff, 2 * KB * s);
      } else {
        lin_load_lds<0>(rx, dst, kOff, 0);
      }
    }
  };

  // lane's LDS offsets within a row piece for its K steps of a stage (chunk 4 ks + lg of row
  // 16 t + l16 sits at position (4 ks + lg) ^ l16)
  int roff[QS];
#pragma unroll
  for (int q = 0; q < QS; ++q) roff[q] = l16 * RB + 16 * ((4 * (kw + WK * q) + lg) ^ l16);

  f4 acc[TMW][TN];
  float ssq[TMW];
#pragma unroll
  for (int i = 0; i < TMW; ++i) {
    ssq[i] = 0.f;
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  }
  auto compute = [&](int slot) __attribute__((always_inline)) {
    const char* base = ring[slot];
#pragma unroll
    for (int q = 0; q < QS; ++q) {
      // the step's operands: TMW x tiles, TN weight tiles, then the norm weights
      constexpr int NR = TMW + TN + (NORM ? 1 : 0);
      uint32_t ad[NR];
      u32x4 rd[NR];
#pragma unroll
      for (int i = 0; i < TMW; ++i) ad[i] = lin_lds_addr(base + (16 * (TMW * tw + i)) * RB + roff[q]);
#pragma unroll
      for (int j = 0; j < TN; ++j) ad[TMW + j] = lin_lds_addr(base + (MT + 16 * j) * RB + roff[q]);
      if constexpr (NORM) ad[NR - 1] = lin_lds_addr(base + 1024 * U + 16 * (4 * (kw + WK * q) + lg));
      lin_ds_read_all<NR>(rd, ad);
      typename M::v8 av[TMW], bv[TN];
#pragma unroll
      for (int i = 0; i < TMW; ++i) av[i] = __builtin_bit_cast(typename M::v8, rd[i]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[j] = __builtin_bit_cast(typename M::v8, rd[TMW + j]);
      if constexpr (NORM) {
        const typename M::v8 nv = __builtin_bit_cast(typename M::v8, rd[NR - 1]);
#pragma unroll
        for (int i = 0; i < TMW; ++i) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float xf = static_cast<float>(av[i][e]);
            ssq[i] = fmaf(xf, xf, ssq[i]);
            av[i][e] = static_cast<T>(xf * static_cast<float>(nv[e]));
          }
        }
      }
#pragma unroll
      for (int i = 0; i < TMW; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = M::mma(av[i], bv[j], acc[i][j]);
      }
    }
  };

  // Stage t sits in slot t % S (the loop is unrolled S times, so slots are constants). It waits
  // for its own loads (the S - 2 stages after it may still be in flight); the barrier then shows
  // every wave's loads, and every wave is done with the slot of stage t - 1, which takes stage
  // t + S - 1.
#pragma unroll
  for (int p = 0; p < S - 1; ++p) issue(p, p);
  for (int t0 = 0; t0 < ns; t0 += S) {
#pragma unroll
    for (int d = 0; d < S; ++d) {
      if (t0 + d < ns) {
        lin_wait_vm<UPW * (S - 2)>();
        lin_wait_lds();
        __builtin_amdgcn_s_barrier();
        issue(t0 + d + S - 1, (d + S - 1) % S);
        compute(d);
      }
    }
  }
  lin_wait_vm<0>();
  lin_wait_lds();
  __syncthreads();

  // partial sums: lane holds rows 16 i + 4 lg + r of column 16 j + l16 of the wave's tiles
  float* red = reinterpret_cast<float*>(&ring[0][0]);
#pragma unroll
  for (int i = 0; i < TMW; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((w * TMW + i) * TN + j) * 256 + r * 64 + lane] = acc[i][j][r];
    }
    if constexpr (NORM) {
      float v = ssq[i] + __shfl_xor(ssq[i], 16);
      v += __shfl_xor(v, 32);
      if (lg == 0) red_ssq[w][i][l16] = v;
    }
  }
  __syncthreads();
  for (int e = tid; e < MT * NT; e += 512) {
    const int m = e / NT, n = e - m * NT;
    const int ig = m >> 4, j = n >> 4, tg = ig / TMW, i = ig - tg * TMW;
    const int ln = (n & 15) + 16 * ((m & 15) >> 2), r = m & 3;
    float y = 0.f;
#pragma unroll
    for (int v = 0; v < WK; ++v) y += red[(((v + WK * tg) * TMW + i) * TN + j) * 256 + r * 64 + ln];
    if constexpr (NORM) {
      float sq = 0.f;
#pragma unroll
      for (int v = 0; v < WK; ++v) sq += red_ssq[v + WK * tg][i][m & 15];
      y *= rsqrtf(sq / static_cast<float>(g.k) + g.eps);
    }
    if (m0 + m < g.m && n0 + n < g.n) lin_emit<T>(g, 0, m0 + m, n0 + n, y);
  }
}

// out = sum over splits of the partial sums (+ residual), rounded once; one thread per element
template <typename T>
__global__ __launch_bounds__(256) void linear_reduce_kernel(const LinGeom g) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= static_cast<int64_t>(g.m) * g.n) return;
  const int m = static_cast<int>(e / g.n), n = static_cast<int>(e - static_cast<int64_t>(m) * g.n);
  float y = 0.f;
  for (int s = 0; s < g.splits; ++s) y += g.part[static_cast<int64_t>(s) * g.m * g.n + e];
  if (g.res != nullptr) {
    y += static_cast<float>(static_cast<const T*>(g.res)[static_cast<int64_t>(m) * g.r_ld + n]);
  }
  static_cast<T*>(g.out)[static_cast<int64_t>(m) * g.o_ld + n] = static_cast<T>(y);
}

// ----------------------------------------------------------------------------- host side

// A launch: the kernel and its shape. rows kernel: cfg = TM, TN, WAVES and ring depth d; tile
// kernel: cfg = MT, NT, KS (wave layout and ring depth follow from them).
struct LinPlan {
  bool rows, gemv, wide, stream;
  int a, b, c, d;     // rows: TM, TN, WAVES, D; tile: MT, NT, KS; gemv: RW, CH; wide: TM, WAVES;
                      // stream: MT, NT, KB, S
  int gx, gy, splits, k_split;
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

constexpr int64_t kCUs = 256;  // compute units of the MI355X

// Splits of K (each a multiple of `unit` elements) so that about `want` workgroups run.
void split_k(LinPlan& p, int64_t k, int64_t tiles, int64_t want, int64_t unit) {
  int64_t s = std::max<int64_t>(1, std::min<int64_t>(cdiv(want, tiles), k / unit));
  int64_t ks = cdiv(cdiv(k, s), unit) * unit;
  p.splits = static_cast<int>(cdiv(k, ks));
  p.k_split = static_cast<int>(ks);
}

LinPlan plan(int64_t m, int64_t n, int64_t k, bool norm) {
  LinPlan p{};
  if (m <= kGemvRows && k % 512 == 0 && k <= 4096) {
    // gemv kernel: two rows per wave while that leaves 1024 or more workgroups, else one
    p.gemv = true;
    p.a = cdiv(n, 8) >= 1024 ? 2 : 1;
    p.b = k <= 2048 ? 4 : 8;
    p.gx = static_cast<int>(cdiv(n, 4 * p.a));
    p.gy = 1;
    p.splits = 1;
    p.k_split = static_cast<int>(k);
    return p;
  }
  if (m <= 16 && k % 512 == 0 && k <= 4096 && cdiv(n, 16) <= kCUs) {
    // wide kernel: 16 weight rows per workgroup, one wave per 512 elements of K; x is read once
    // per workgroup, so it takes the shapes whose workgroups fit one pass over the CUs
    p.wide = true;
    p.a = 1;
    p.b = static_cast<int>(k / 512);
    p.gx = static_cast<int>(cdiv(n, 16));
    p.gy = 1;
    p.splits = 1;
    p.k_split = static_cast<int>(k);
    return p;
  }
  if (m <= 64 && k % 256 == 0) {
    // stream kernel: the smallest workgroup tile (x rows MT + weight rows NT, the bytes each
    // workgroup streams per K step) whose workgroups fit one pass over the CUs; above 32 rows a
    // 32-row tile runs as two row blocks (out_proj at M = 64: 9.0 against 12.1 us with one
    // 64-row block)
    static constexpr int kFew[][2] = {{32, 16}, {32, 32}, {32, 48}};
    static constexpr int kMore[][2] = {{32, 16}, {32, 32}, {64, 16}, {64, 32}, {64, 48}};
    const auto& tiles = m <= 32 ? kFew : kMore;
    const int count = m <= 32 ? 3 : 5;
    p.stream = true;
    p.a = tiles[count - 1][0];  // (the largest, when none fits one pass)
    p.b = tiles[count - 1][1];
    for (int i = 0; i < count; ++i) {
      if (cdiv(m, tiles[i][0]) * cdiv(n, tiles[i][1]) <= kCUs) {
        p.a = tiles[i][0];
        p.b = tiles[i][1];
        break;
      }
    }
    p.gx = static_cast<int>(cdiv(n, p.b));
    p.gy = static_cast<int>(cdiv(m, p.a));
    p.splits = 1;
    p.k_split = static_cast<int>(k);
    return p;
  }
  if (m <= 32) {
    // rows kernel: 16 columns per workgroup, 4 waves splitting K. Measured on the decode shapes
    // (N 8672 / 2048, K 2048 / 4096, cold weights), one launch that keeps K whole beats a K
    // split plus the reduce launch from 128 workgroups up, so K is split only below 64
    // workgroups; the ring holds 8 steps when a wave runs 32 or more, else 4.
    p.rows = true;
    p.a = m <= 16 ? 1 : 2;
    p.b = 1;
    p.c = 4;
    p.gx = static_cast<int>(cdiv(n, 16 * p.b));
    p.gy = 1;
    split_k(p, k, p.gx, norm ? 1 : 64, 4 * kStep * p.c);
    p.d = p.k_split / (kStep * p.c) >= 32 ? 8 : 4;
    return p;
  }
  p.rows = false;
  p.a = m <= 64 ? 64 : 128;
  p.b = 64;
  p.c = 64;
  p.gx = static_cast<int>(cdiv(n, p.b));
  p.gy = static_cast<int>(cdiv(m, p.a));
  split_k(p, k, static_cast<int64_t>(p.gx) * p.gy, 256, 8 * p.c);
  return p;
}

int validate(const m3_linear_args& a) {
  if (a.dtype != M3_BF16 && a.dtype != M3_F16) {
    return fail(M3_EUNSUPPORTED, "m3_linear: dtype %d is not bf16 or f16", a.dtype);
  }
  if (a.m <= 0 || a.n <= 0 || a.k <= 0) return fail(M3_EINVAL, "m3_linear: empty dims");
  if (a.m > 256) return fail(M3_EUNSUPPORTED, "m3_linear: M = %lld > 256", (long long)a.m);
  if (a.k % kStep != 0) return fail(M3_EUNSUPPORTED, "m3_linear: K %% 32 != 0");
  int rc;
  if ((rc = check_tensor(a.x, "x", 2, a.k, true, a.dtype)) != M3_OK) return rc;
  if ((rc = check_tensor(a.weight, "weight", 2, a.k, true, a.dtype)) != M3_OK) return rc;
  if ((rc = check_tensor(a.residual, "residual", 2, a.n, false, a.dtype)) != M3_OK) return rc;
  if ((rc = check_tensor(a.norm_weight, "norm_weight", 1, a.k, false, a.dtype)) != M3_OK) {
    return rc;
  }
  if (a.norm_weight.ptr != nullptr) {
    if (a.m > 64 || (a.m > 32 && a.k % 256 != 0)) {
      return fail(M3_EUNSUPPORTED,
                  "m3_linear: norm_weight needs M <= 32, or M <= 64 with K a multiple of 256");
    }
    if (reinterpret_cast<uintptr_t>(a.norm_weight.ptr) % 16 != 0) {
      return fail(M3_EUNSUPPORTED, "m3_linear: norm_weight must be 16-byte aligned");
    }
    if (!(a.norm_eps >= 0.f)) return fail(M3_EINVAL, "m3_linear: norm_eps must be >= 0");
  }
  if ((rc = check_tensor(a.out, "out", 2, a.n, true, a.dtype)) != M3_OK) return rc;
  for (const m3_tensor* t : {&a.x, &a.weight}) {
    if (reinterpret_cast<uintptr_t>(t->ptr) % 16 != 0 || t->stride[0] % 8 != 0) {
      return fail(M3_EUNSUPPORTED, "m3_linear: x / weight rows must be 16-byte aligned");
    }
  }
  if ((a.m > 1 && a.x.stride[0] < a.k) || a.weight.stride[0] < a.k) {
    return fail(M3_EINVAL, "m3_linear: row stride below K");
  }
  if ((a.m > 1 && a.out.stride[0] < a.n) ||
      (a.m > 1 && a.residual.ptr != nullptr && a.residual.stride[0] < a.n)) {
    return fail(M3_EINVAL, "m3_linear: out / residual row stride below N");
  }
  // 32-bit byte offsets: a 32-row run of x or weight, and every out / residual element
  constexpr int64_t kLdMax = int64_t{1} << 25;
  if (a.x.stride[0] >= kLdMax || a.weight.stride[0] >= kLdMax || a.k >= kLdMax ||
      a.n >= INT32_MAX || a.out.stride[0] >= INT32_MAX || a.residual.stride[0] >= INT32_MAX ||
      a.n * a.weight.stride[0] * 2 >= (int64_t{1} << 31) ||
      a.m * a.x.stride[0] * 2 >= (int64_t{1} << 31)) {
    return fail(M3_EUNSUPPORTED, "m3_linear: operand above 2 GiB or row stride too large");
  }
  return M3_OK;
}

size_t workspace_bytes(const m3_linear_args& a, const LinPlan& p) {
  return p.splits > 1 ? static_cast<size_t>(p.splits) * a.m * a.n * sizeof(float) : 0;
}

LinGeom geometry(const m3_linear_args& a, const LinPlan& p) {
  LinGeom g{};
  g.x = static_cast<const char*>(a.x.ptr);
  g.w = static_cast<const char*>(a.weight.ptr);
  g.res = a.residual.ptr;
  g.out = a.out.ptr;
  g.part = static_cast<float*>(a.workspace);
  g.nw = static_cast<const char*>(a.norm_weight.ptr);
  g.eps = a.norm_eps;
  g.m = static_cast<int>(a.m);
  g.n = static_cast<int>(a.n);
  g.k = static_cast<int>(a.k);
  g.k_split = p.k_split;
  g.splits = p.splits;
  g.x_ld = static_cast<int>(a.x.stride[0]);
  g.w_ld = static_cast<int>(a.weight.stride[0]);
  g.r_ld = a.residual.ptr != nullptr ? static_cast<int>(a.residual.stride[0]) : 0;
  g.o_ld = static_cast<int>(a.out.stride[0]);
  return g;
}

template <typename T, int TM, int TN, int WAVES, int D>
void launch_rows_d(const LinGeom& g, const LinPlan& p, hipStream_t stream) {
  if (g.nw != nullptr) {
    hipLaunchKernelGGL((linear_rows_kernel<T, TM, TN, WAVES, D, true>), dim3(p.gx, 1, p.splits),
                       dim3(64 * WAVES), 0, stream, g);
  } else {
    hipLaunchKernelGGL((linear_rows_kernel<T, TM, TN, WAVES, D, false>), dim3(p.gx, 1, p.splits),
                       dim3(64 * WAVES), 0, stream, g);
  }
}

template <typename T, int TM, int TN, int WAVES>
void launch_rows(const LinGeom& g, const LinPlan& p, hipStream_t stream) {
  if (p.d == 8) {
    launch_rows_d<T, TM, TN, WAVES, 8>(g, p, stream);
  } else {
    launch_rows_d<T, TM, TN, WAVES, 4>(g, p, stream);
  }
}

template <typename T, int MT, int NT, int WM, int WN, int KS, int D>
void launch_tile(const LinGeom& g, const LinPlan& p, hipStream_t stream) {
  hipLaunchKernelGGL((linear_tile_kernel<T, MT, NT, WM, WN, KS, D>), dim3(p.gx, p.gy, p.splits),
                     dim3(256), 0, stream, g);
}

template <typename T, int RW, int CH>
void launch_gemv(const LinGeom& g, const LinPlan& p, hipStream_t stream) {
  if (g.nw != nullptr) {
    hipLaunchKernelGGL((linear_gemv_kernel<T, RW, CH, true>), dim3(p.gx), dim3(256), 0, stream, g);
  } else {
    hipLaunchKernelGGL((linear_gemv_kernel<T, RW, CH, false>), dim3(p.gx), dim3(256), 0, stream, g);
  }
}

template <typename T, int TM, int WAVES>
void launch_wide(const LinGeom& g, const LinPlan& p, hipStream_t stream) {
  if (g.nw != nullptr) {
    hipLaunchKernelGGL((linear_wide_kernel<T, TM, WAVES, true>), dim3(p.gx), dim3(64 * WAVES), 0,
                       stream, g);
  } else {
    hipLaunchKernelGGL((linear_wide_kernel<T, TM, WAVES, false>), dim3(p.gx), dim3(64 * WAVES), 0,
                       stream, g);
  }
}

template <typename T, int TM>
int launch_wide_k(const LinGeom& g, const LinPlan& p, hipStream_t stream) {
  switch (p.b) {
    case 1: launch_wide<T, TM, 1>(g, p, stream); return M3_OK;
    case 2: launch_wide<T, TM, 2>(g, p, stream); return M3_OK;
    case 3: launch_wide<T, TM, 3>(g, p, stream); return M3_OK;
    case 4: launch_wide<T, TM, 4>(g, p, stream); return M3_OK;
    case 5: launch_wide<T, TM, 5>(g, p, stream); return M3_OK;
    case 6: launch_wide<T, TM, 6>(g, p, stream); return M3_OK;
    case 7: launch_wide<T, TM, 7>(g, p, stream); return M3_OK;
    case 8: launch_wide<T, TM, 8>(g, p, stream); return M3_OK;
    default: return fail(M3_EUNSUPPORTED, "m3_linear: no wide kernel for %d waves", p.b);
  }
}

template <typename T, int MT, int NT, int KB, int S>
void launch_stream(const LinGeom& g, const LinPlan& p, hipStream_t stream) {
  if (g.nw != nullptr) {
    hipLaunchKernelGGL((linear_stream_kernel<T, MT, NT, KB, S, true>), dim3(p.gx, p.gy),
                       dim3(512), 0, stream, g);
  } else {
    hipLaunchKernelGGL((linear_stream_kernel<T, MT, NT, KB, S, false>), dim3(p.gx, p.gy),
                       dim3(512), 0, stream, g);
  }
}

// The compiled shapes; a plan naming any other is refused.
template <typename T>
int launch_plan(const LinGeom& g, const LinPlan& p, hipStream_t stream) {
  if (p.stream) {
    if (p.a == 32 && p.b == 48) {
      launch_stream<T, 32, 48, 128, 4>(g, p, stream);
    } else if (p.a == 32 && p.b == 32) {
      launch_stream<T, 32, 32, 128, 4>(g, p, stream);
    } else if (p.a == 32 && p.b == 16) {
      launch_stream<T, 32, 16, 256, 3>(g, p, stream);
    } else if (p.a == 64 && p.b == 48) {
      launch_stream<T, 64, 48, 128, 4>(g, p, stream);
    } else if (p.a == 64 && p.b == 32) {
      launch_stream<T, 64, 32, 128, 4>(g, p, stream);
    } else if (p.a == 64 && p.b == 16) {
      launch_stream<T, 64, 16, 256, 3>(g, p, stream);
    } else {
      return fail(M3_EUNSUPPORTED, "m3_linear: no stream kernel %d/%d", p.a, p.b);
    }
  } else if (p.wide) {
    if (p.a != 1) return fail(M3_EUNSUPPORTED, "m3_linear: no wide kernel for %d row tiles", p.a);
    const int rc = launch_wide_k<T, 1>(g, p, stream);
    if (rc != M3_OK) return rc;
  } else if (p.gemv) {
    if (p.a == 2 && p.b == 4) {
      launch_gemv<T, 2, 4>(g, p, stream);
    } else if (p.a == 2 && p.b == 8) {
      launch_gemv<T, 2, 8>(g, p, stream);
    } else if (p.a == 1 && p.b == 4) {
      launch_gemv<T, 1, 4>(g, p, stream);
    } else if (p.a == 1 && p.b == 8) {
      launch_gemv<T, 1, 8>(g, p, stream);
    } else {
      return fail(M3_EUNSUPPORTED, "m3_linear: no gemv kernel %d/%d", p.a, p.b);
    }
  } else if (p.rows) {
    if (p.a == 1 && p.b == 1 && p.c == 4) {
      launch_rows<T, 1, 1, 4>(g, p, stream);
    } else if (p.a == 2 && p.b == 1 && p.c == 4) {
      launch_rows<T, 2, 1, 4>(g, p, stream);
    } else {
      return fail(M3_EUNSUPPORTED, "m3_linear: no rows kernel %d/%d/%d", p.a, p.b, p.c);
    }
  } else if (p.a == 64 && p.b == 64 && p.c == 64) {
    launch_tile<T, 64, 64, 2, 2, 64, 4>(g, p, stream);
  } else if (p.a == 128 && p.b == 64 && p.c == 64) {
    launch_tile<T, 128, 64, 2, 2, 64, 4>(g, p, stream);
  } else {
    return fail(M3_EUNSUPPORTED, "m3_linear: no tile kernel %d/%d/%d", p.a, p.b, p.c);
  }
  int rc = check_launch("m3_linear");
  if (rc != M3_OK || p.splits == 1) return rc;
  const int64_t total = static_cast<int64_t>(g.m) * g.n;
  hipLaunchKernelGGL((linear_reduce_kernel<T>), dim3(static_cast<unsigned>(cdiv(total, 256))),
                     dim3(256), 0, stream, g);
  return check_launch("m3_linear (reduce)");
}

int run(const m3_linear_args& a, const LinPlan& p, hipStream_t stream) {
  const size_t need = workspace_bytes(a, p);
  if (need > 0 && (a.workspace == nullptr || a.workspace_bytes < need ||
                   reinterpret_cast<uintptr_t>(a.workspace) % 16 != 0)) {
    return fail(M3_EWORKSPACE, "m3_linear: needs a 16-byte aligned workspace of %zu bytes", need);
  }
  const LinGeom g = geometry(a, p);
  return a.dtype == M3_BF16 ? launch_plan<__bf16>(g, p, stream)
                            : launch_plan<_Float16>(g, p, stream);
}

}  // namespace
}  // namespace m3

extern "C" int m3_linear_workspace_size(const m3_linear_args* args, size_t* bytes) {
  m3::clear_error();
  if (args == nullptr || bytes == nullptr) {
    return m3::fail(M3_EINVAL, "m3_linear_workspace_size: NULL");
  }
  const int rc = m3::validate(*args);
  if (rc != M3_OK) return rc;
  *bytes = m3::workspace_bytes(
      *args, m3::plan(args->m, args->n, args->k, args->norm_weight.ptr != nullptr));
  return M3_OK;
}

extern "C" int m3_linear(const m3_linear_args* args, hipStream_t stream) {
  m3::clear_error();
  if (args == nullptr) return m3::fail(M3_EINVAL, "m3_linear: NULL args");
  const int rc = m3::validate(*args);
  if (rc != M3_OK) return rc;
  return m3::run(*args, m3::plan(args->m, args->n, args->k, args->norm_weight.ptr != nullptr),
                 stream);
}
