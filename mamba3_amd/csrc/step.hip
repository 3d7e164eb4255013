// Mamba-3 decode step for CDNA4: one workgroup per (batch, head) streams that head's FP32
// state [P, N] exactly once (16-byte non-temporal loads and stores), fusing the phase advance,
// the rotation of q/k, the trapezoid state update, the readout, the D skip, the SiLU gate and the
// MIMO rank sum. Replaces ops.fused_step (ops.py:87-190) and its Triton kernel
// (_triton.py:564-947), and the portable ops.mamba3_step (ops.py:825-879).
#include <type_traits>

#include "m3_common.hpp"
#include "m3_host.hpp"
#include "m3_math.h"

namespace m3 {

constexpr int kStepThreads = 256;
constexpr int kStepBatch = 8;  // float4 state vectors a thread keeps in flight

template <typename T>
__device__ __forceinline__ float ld_act(const m3_tensor& t, int64_t i) {
  return to_f(static_cast<const T*>(t.ptr)[i]);
}

// Sum over the `width` consecutive lanes of an aligned lane group (width a power of 2 <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <typename T, int R>
__global__ __launch_bounds__(kStepThreads) void step_kernel(const m3_step_args a) {
  const int H = a.heads, N = a.d_state, P = a.head_dim, S = a.num_angles;
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  const int g = h / (H / a.groups);
  const int tid = threadIdx.x;
  const bool norm = a.q_norm_w.ptr != nullptr;
  const bool bias = a.q_bias.ptr != nullptr;
  const bool rotate = a.phase_mode != M3_PHASE_NONE;

  extern __shared__ float lds[];
  float* qx = lds;            // [R][N] normed + biased q (activation values)
  float* kx = qx + R * N;     // [R][N]
  float* qr = kx + R * N;     // [R][N] rotated q
  float* kr = qr + R * N;     // [R][N] rotated k
  float* pk = kr + R * N;     // [R][N] previous rotated k
  float* vr = pk + R * N;     // [R][P] rank values v * mimo_x
  float* pvr = vr + R * P;    // [R][P] previous rank values
  float* zr = pvr + R * P;    // [R][P] rank gates z * mimo_z
  float* mo = zr + R * P;     // [R][P] mimo_out
  float* yp = mo + R * P;     // [R][P] readout q . S'
  float* vv = yp + R * P;     // [P] value of this token
  float* cs = vv + P;         // [S] cos(phase') in the activation dtype
  float* sn = cs + S;         // [S]
  float* phn = sn + S;        // [S] phase'
  float* rstd = phn + S;      // [2R] RMSNorm factors

  // ---- per-(b, h) scalars (every thread computes them; the loads broadcast)
  float dt, adt;
  dt_adt(a.raw_dt, ldx(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0] + h * a.dt.stride[1]),
         ldx(a.a.ptr, a.a.dtype, b * a.a.stride[0] + h * a.a.stride[1]),
         a.raw_dt ? ldx(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]) : 0.f, dt, adt);
  const float trap = sigmoidf(ldx(a.trap.ptr, a.trap.dtype,
                                  b * a.trap.stride[0] + h * a.trap.stride[1]));
  const float alpha = expf(adt);
  const float beta = (1.f - trap) * dt * alpha;
  const float gamma = trap * dt;
  const float Dh = ldx(a.D.ptr, a.D.dtype, h * a.D.stride[0]);

  // ---- prologue: everything this (b, h) reads besides the state goes to LDS
  if (tid < S) {
    const float old = static_cast<const float*>(
        a.phase_in.ptr)[b * a.phase_in.stride[0] + h * a.phase_in.stride[1] +
                        tid * a.phase_in.stride[2]];
    float ph = old;
    if (a.phase_mode == M3_PHASE_ANGLES) {
      const float th = ldx(a.angles.ptr, a.angles.dtype,
                           b * a.angles.stride[0] + tid * a.angles.stride[1]);
      ph = fmodf(__fadd_rn(old, phase_inc(th, dt)), kTwoPi);
    }
    phn[tid] = ph;
    cs[tid] = rnd<T>(cosf(ph));
    sn[tid] = rnd<T>(sinf(ph));
  }
  for (int i = tid; i < R * N; i += kStepThreads) {
    const int r = i / N, n = i - r * N;
    qx[i] = ld_act<T>(a.q, b * a.q.stride[0] + g * a.q.stride[1] + r * a.q.stride[2] + n);
    kx[i] = ld_act<T>(a.k, b * a.k.stride[0] + g * a.k.stride[1] + r * a.k.stride[2] + n);
    pk[i] = ld_act<T>(a.prev_k, b * a.prev_k.stride[0] + h * a.prev_k.stride[1] +
                                    r * a.prev_k.stride[2] + n);
  }
  for (int p = tid; p < P; p += kStepThreads) {
    const float v = ld_act<T>(a.value, b * a.value.stride[0] + h * a.value.stride[1] + p);
    const float z = ld_act<T>(a.gate, b * a.gate.stride[0] + h * a.gate.stride[1] + p);
    const float pv = ld_act<T>(a.prev_value,
                               b * a.prev_value.stride[0] + h * a.prev_value.stride[1] + p);
    vv[p] = v;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (R > 1) {
        const int64_t o = h * a.mimo_x.stride[0] + r * a.mimo_x.stride[1] + p;
        const float mx = rnd<T>(ldx(a.mimo_x.ptr, a.mimo_x.dtype, o));
        const float mz = rnd<T>(ldx(a.mimo_z.ptr, a.mimo_z.dtype,
                                    h * a.mimo_z.stride[0] + r * a.mimo_z.stride[1] + p));
        vr[r * P + p] = mul_r<T>(v, mx);
        pvr[r * P + p] = mul_r<T>(pv, mx);
        zr[r * P + p] = mul_r<T>(z, mz);
        mo[r * P + p] = ldx(a.mimo_out.ptr, a.mimo_out.dtype,
                            h * a.mimo_out.stride[0] + r * a.mimo_out.stride[1] + p);
      } else {
        vr[p] = v;
        pvr[p] = pv;
        zr[p] = z;
        mo[p] = 1.f;
      }
    }
  }
  __syncthreads();

  // RMSNorm of the raw q / k rows (model.py:190-191): one wave per row.
  if (norm) {
    const int wave = tid >> 6, lane = tid & 63;
    for (int row = wave; row < 2 * R; row += kStepThreads / 64) {
      const float* x = row < R ? qx + row * N : kx + (row - R) * N;
      float s = 0.f;
      for (int n = lane; n < N; n += 64) s += x[n] * x[n];
      s = group_sum(s, 64);
      if (lane == 0) rstd[row] = 1.f / sqrtf(s / static_cast<float>(N) + a.norm_eps);
    }
    __syncthreads();
  }
  if (norm || bias) {
    for (int i = tid; i < R * N; i += kStepThreads) {
      const int r = i / N, n = i - r * N;
      float q = qx[i], k = kx[i];
      if (norm) {
        q = rnd<T>(q * rstd[r] * rnd<T>(ldx(a.q_norm_w.ptr, a.q_norm_w.dtype,
                                               n * a.q_norm_w.stride[0])));
        k = rnd<T>(k * rstd[R + r] * rnd<T>(ldx(a.k_norm_w.ptr, a.k_norm_w.dtype,
                                                   n * a.k_norm_w.stride[0])));
      }
      if (bias) {
        q = add_r<T>(q, rnd<T>(ldx(a.q_bias.ptr, a.q_bias.dtype,
                                   h * a.q_bias.stride[0] + r * a.q_bias.stride[1] + n)));
        k = add_r<T>(k, rnd<T>(ldx(a.k_bias.ptr, a.k_bias.dtype,
                                   h * a.k_bias.stride[0] + r * a.k_bias.stride[1] + n)));
      }
      qx[i] = q;
      kx[i] = k;
    }
    __syncthreads();
  }
  // Rotation (ops.py:35-84): SISO pairs (2j, 2j+1), MIMO pairs (j, j + 2S), j < S.
  for (int i = tid; i < R * N; i += kStepThreads) {
    const int r = i / N, n = i - r * N;
    const float* xq = qx + r * N;
    const float* xk = kx + r * N;
    float oq = xq[n], ok = xk[n];
    if (rotate) {
      int j = -1, lo = 0, hi = 0;
      bool second = false;
      if (!a.mimo_rotation) {
        if (n < 2 * S) { j = n >> 1; lo = n & ~1; hi = n | 1; second = n & 1; }
      } else if (n < S) {
        j = n; lo = n; hi = n + 2 * S;
      } else if (n >= 2 * S && n < 3 * S) {
        j = n - 2 * S; lo = j; hi = n; second = true;
      }
      if (j >= 0) {
        const float c = cs[j], s = sn[j];
        if (second) {
          oq = add_r<T>(mul_r<T>(xq[lo], s), mul_r<T>(xq[hi], c));
          ok = add_r<T>(mul_r<T>(xk[lo], s), mul_r<T>(xk[hi], c));
        } else {
          oq = sub_r<T>(mul_r<T>(xq[lo], c), mul_r<T>(xq[hi], s));
          ok = sub_r<T>(mul_r<T>(xk[lo], c), mul_r<T>(xk[hi], s));
        }
      }
    }
    qr[i] = oq;
    kr[i] = ok;
  }
  __syncthreads();

  // ---- small cache outputs (all inputs they may alias were read above)
  if (tid < S) {
    static_cast<float*>(a.phase_out.ptr)[b * a.phase_out.stride[0] + h * a.phase_out.stride[1] +
                                         tid * a.phase_out.stride[2]] = phn[tid];
  }
  for (int i = tid; i < R * N; i += kStepThreads) {
    const int r = i / N, n = i - r * N;
    static_cast<T*>(a.k_out.ptr)[b * a.k_out.stride[0] + h * a.k_out.stride[1] +
                                 r * a.k_out.stride[2] + n] = from_f<T>(kr[i]);
  }
  if (a.value_out.ptr != nullptr) {
    for (int p = tid; p < P; p += kStepThreads) {
      static_cast<T*>(a.value_out.ptr)[b * a.value_out.stride[0] + h * a.value_out.stride[1] + p] =
          from_f<T>(vv[p]);
    }
  }

  // ---- state stream: thread owns columns [4c, 4c + 4) of rows p = f / N4, f = tid + 256 i.
  const int N4 = N >> 2;
  const int total = P * N4;
  const int c = tid & (N4 - 1);
  const int n0 = c << 2;
  const float* sin_ = static_cast<const float*>(a.state_in.ptr) + b * a.state_in.stride[0] +
                      h * a.state_in.stride[1];
  float* sout = static_cast<float*>(a.state_out.ptr) + b * a.state_out.stride[0] +
                h * a.state_out.stride[1];
  const int64_t sp_in = a.state_in.stride[2], sp_out = a.state_out.stride[2];
  float kc[R][4], pkc[R][4], qc[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kc[r][j] = kr[r * N + n0 + j];
      pkc[r][j] = pk[r * N + n0 + j];
      qc[r][j] = qr[r * N + n0 + j];
    }

  for (int f0 = tid; f0 < total; f0 += kStepThreads * kStepBatch) {
    f4 st[kStepBatch];
#pragma unroll
    for (int u = 0; u < kStepBatch; ++u) {
      const int f = f0 + u * kStepThreads;
      if (f < total) {
        const int p = f / N4;
        st[u] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(sin_ + p * sp_in + n0));
      }
    }
#pragma unroll
    for (int u = 0; u < kStepBatch; ++u) {
      const int f = f0 + u * kStepThreads;
      if (f >= total) break;  // uniform across each lane group of N4 lanes
      const int p = f / N4;
      float po[4] = {0.f, 0.f, 0.f, 0.f}, co[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float pv = pvr[r * P + p], cv = vr[r * P + p];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          po[j] += pv * pkc[r][j];
          co[j] += cv * kc[r][j];
        }
      }
      f4 ns;
#pragma unroll
      for (int j = 0; j < 4; ++j) ns[j] = alpha * st[u][j] + beta * po[j] + gamma * co[j];
      __builtin_nontemporal_store(ns, reinterpret_cast<f4*>(sout + p * sp_out + n0));
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) part += rnd<T>(ns[j]) * qc[r][j];
        part = group_sum(part, N4);
        if (c == 0) yp[r * P + p] = part;
      }
    }
  }
  __syncthreads();

  // ---- epilogue: D skip, SiLU gate, MIMO rank sum (ops.py:869-877)
  for (int p = tid; p < P; p += kStepThreads) {
    float y = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float t = (yp[r * P + p] + Dh * vr[r * P + p]) * siluf(zr[r * P + p]);
      y = R > 1 ? y + t * mo[r * P + p] : t;
    }
    static_cast<T*>(a.out.ptr)[b * a.out.stride[0] + h * a.out.stride[1] + p] = from_f<T>(y);
  }
}

// ------------------------------------------------------------------ model shape (N 128, P 64)

// Sum over the 32 lanes of an aligned half-wave; every lane receives it. DPP rotations inside
// each 16-lane row, then the other row of the pair by a lane swizzle (xor 16).
__device__ __forceinline__ float allreduce32(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128,
                                                             0xf, 0xf, false));  // row_ror:8
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124,
                                                             0xf, 0xf, false));  // row_ror:4
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x122,
                                                             0xf, 0xf, false));  // row_ror:2
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x121,
                                                             0xf, 0xf, false));  // row_ror:1
  x += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401f));
  return x;
}

// The value of lane (lane xor 16) (same 32-lane half-wave).
__device__ __forceinline__ float swap16(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401f));
}

// x of another lane of the same 16-lane DPP row (ctrl: row_ror:8 = lane ^ 8, row_half_mirror =
// lane ^ 7 within 8, quad_perm 0xb1 / 0x4e = lane ^ 1 / lane ^ 2).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                               0xf, 0xf, false));
}

// Reduce-scatter of 8 values over a 32-lane half-wave: lane c returns the sum over all 32 lanes
// of v[(c >> 2) & 7]. Halving stages trade half the remaining values with lane c ^ 16 (bit 4),
// c ^ 8 (bit 3) and c ^ 7 (bit 2, same bits 3-4), each lane keeping the half its bit selects;
// the last two stages add over the quad. 9 exchanges where 8 all-reduces take 40.
__device__ __forceinline__ float reduce_scatter8(const float (&v)[8], int c) {
  const bool b4 = (c & 16) != 0, b3 = (c & 8) != 0, b2 = (c & 4) != 0;
  float h4[4], h3[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) h4[i] = (b4 ? v[4 + i] : v[i]) + swap16(b4 ? v[i] : v[4 + i]);
#pragma unroll
  for (int i = 0; i < 2; ++i) h3[i] = (b3 ? h4[2 + i] : h4[i]) + dpp<0x128>(b3 ? h4[i] : h4[2 + i]);
  float h = (b2 ? h3[1] : h3[0]) + dpp<0x141>(b2 ? h3[0] : h3[1]);
  h += dpp<0xb1>(h);
  h += dpp<0x4e>(h);
  return h;
}

// Four consecutive activation elements (one 8-byte load for 16-bit types, 16 bytes for FP32).
template <typename T>
__device__ __forceinline__ f4 ld4(const void* base, int64_t i) {
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
__device__ __forceinline__ void st4(void* base, int64_t i, const float (&x)[4]) {
  if constexpr (sizeof(T) == 4) {
    f4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = x[j];
    *reinterpret_cast<f4*>(static_cast<float*>(base) + i) = v;
  } else {
    typedef T t4 __attribute__((ext_vector_type(4)));
    t4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = from_f<T>(x[j]);
    *reinterpret_cast<t4*>(static_cast<T*>(base) + i) = v;
  }
}

// The model's decode shape (N = 128, P = 64, 32 angles), one workgroup of 32 * 64 / RPT threads
// per (batch, head), with no LDS round trip before the state update: thread (row group
// rg = tid / 32, column group c = tid % 32) owns columns 4c .. 4c+3 of the state rows rg + RG k,
// k < RPT (RG = 64 / RPT). RPT = 8 (256 threads) streams large batches; RPT = 2 (1024 threads)
// shortens the per-row chain of each workgroup when there are few (batch, head) pairs. Its state
// loads are issued first; while they are in flight it computes, for every rank, the normed,
// biased, rotated q / k of its columns (the RMSNorm sums and the MIMO rotation partner by
// cross-lane exchange within its 32-lane half-wave) and the phases of the angles those columns
// use. Per-row rank values and gates go through LDS behind one barrier. The readout sums over a
// half-wave use DPP; lane c = k finishes row rg + RG k. The small cache outputs are written after a
// final barrier, when every thread has consumed the cache inputs they may alias.
//
// FULL: the model's step (q / k norm weights and biases, raw dt, angle phases, MIMO rotation for
// R > 1) with those features fixed at compile time. The prologue is then one basic block: every
// kernel-argument and input load issues before the first wait, where a branch per optional
// input would cost a round trip each.
//
// PIN (few (batch, head) pairs, where each workgroup's latency chain is the step's time): the
// state loads are issued as soon as their own addresses are known, ahead of the other kernel
// arguments' round trips (the compiler otherwise places them after about six of those). With
// many pairs the launch streams and the default order is the faster one (config 4, tokens/s:
// B = 1 2,058 against 2,012 and B = 32 27.25K against 27.04K; B = 64 36.1K either way; B = 256
// 46.3K against 46.8K), so the launch takes it below 2048 (batch, head) pairs.
template <typename T, int R, int RPT, bool FULL, bool PIN = false>
__global__ __launch_bounds__(32 * 64 / RPT) void step128_kernel(const m3_step_args a) {
  constexpr int N = 128, P = 64, S = 32;
  constexpr int RG = P / RPT;  // row groups: thread rows rg + RG k, k < RPT
  const int H = a.heads;
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  const int g = h / (H / a.groups);
  const int tid = threadIdx.x, c = tid & 31, rg = tid >> 5, n0 = 4 * c;
  const bool norm = FULL || a.q_norm_w.ptr != nullptr;
  const bool bias = FULL || a.q_bias.ptr != nullptr;
  const bool rotate = FULL || a.phase_mode != M3_PHASE_NONE;
  const bool angles = FULL || a.phase_mode == M3_PHASE_ANGLES;
  const bool raw_dt = FULL || a.raw_dt != 0;
  const bool mimo = FULL ? R > 1 : a.mimo_rotation != 0;

  __shared__ float s_vr[R][P], s_pvr[R][P], s_zr[R][P], s_mo[R][P];

  // (1) this thread's state rows
  const float* sin_ = static_cast<const float*>(a.state_in.ptr) + b * a.state_in.stride[0] +
                      h * a.state_in.stride[1] + n0;
  float* sout = static_cast<float*>(a.state_out.ptr) + b * a.state_out.stride[0] +
                h * a.state_out.stride[1] + n0;
  const int64_t sp_in = a.state_in.stride[2], sp_out = a.state_out.stride[2];
  f4 st[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    st[k] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(sin_ + (rg + RG * k) * sp_in));
  }
  if constexpr (PIN) __builtin_amdgcn_sched_barrier(0);

  // (3) every small input of the (b, h): raw loads issued together, decoded after
  const RawX dt_r = ldraw(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0] + h * a.dt.stride[1]);
  const RawX a_r = ldraw(a.a.ptr, a.a.dtype, b * a.a.stride[0] + h * a.a.stride[1]);
  const RawX trap_r = ldraw(a.trap.ptr, a.trap.dtype, b * a.trap.stride[0] + h * a.trap.stride[1]);
  const RawX D_r = ldraw(a.D.ptr, a.D.dtype, h * a.D.stride[0]);
  RawX dtb_r{0u, 0u};
  if (raw_dt) dtb_r = ldraw(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]);
  // phase roles: SISO pairs (2j, 2j+1) -> angles 2c, 2c+1 (c < 16); MIMO pairs (j, j + 2S) ->
  // angles n0 .. n0+3 for the first (c < 8) and third (16 <= c < 24) quarters
  int j0 = -1, nj = 0;
  if (rotate) {
    if (!mimo) {
      if (c < S / 2) { j0 = 2 * c; nj = 2; }
    } else if (c < S / 4) {
      j0 = n0; nj = 4;
    } else if (c >= S / 2 && c < 3 * S / 4) {
      j0 = n0 - 2 * S; nj = 4;
    }
  }
  const float* ph_in = static_cast<const float*>(a.phase_in.ptr) + b * a.phase_in.stride[0] +
                       h * a.phase_in.stride[1];
  float old[4] = {0.f, 0.f, 0.f, 0.f};
  RawX th_r[4] = {};
  if (rotate) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = nj > 0 ? j0 + min(i, nj - 1) : 0;  // lanes without angles read angle 0
      old[i] = ph_in[j * a.phase_in.stride[2]];
    }
  }
  if (rotate && angles) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = nj > 0 ? j0 + min(i, nj - 1) : 0;
      th_r[i] = ldraw(a.angles.ptr, a.angles.dtype, b * a.angles.stride[0] + j * a.angles.stride[1]);
    }
  }
  Raw4 wq_r{}, wk_r{}, bq_r[R] = {}, bk_r[R] = {};
  f4 qx[R], kx[R], px[R];
  if (norm) {
    wq_r = ldraw4(a.q_norm_w, n0);  // weights may be FP32 or the activation type
    wk_r = ldraw4(a.k_norm_w, n0);
  }
  if (bias) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      bq_r[r] = ldraw4(a.q_bias, h * a.q_bias.stride[0] + r * a.q_bias.stride[1] + n0);
      bk_r[r] = ldraw4(a.k_bias, h * a.k_bias.stride[0] + r * a.k_bias.stride[1] + n0);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    qx[r] = ld4<T>(a.q.ptr, b * a.q.stride[0] + g * a.q.stride[1] + r * a.q.stride[2] + n0);
    kx[r] = ld4<T>(a.k.ptr, b * a.k.stride[0] + g * a.k.stride[1] + r * a.k.stride[2] + n0);
    px[r] = ld4<T>(a.prev_k.ptr, b * a.prev_k.stride[0] + h * a.prev_k.stride[1] +
                                     r * a.prev_k.stride[2] + n0);
  }
  // (2) per-row rank values and gates of row p = tid % P: every thread loads them with the batch
  // above (no branch around loads), threads tid < P put them in LDS once decoded
  const int pl = tid & (P - 1);
  const float v = ld_act<T>(a.value, b * a.value.stride[0] + h * a.value.stride[1] + pl);
  const float z = ld_act<T>(a.gate, b * a.gate.stride[0] + h * a.gate.stride[1] + pl);
  const float pv = ld_act<T>(a.prev_value,
                             b * a.prev_value.stride[0] + h * a.prev_value.stride[1] + pl);
  RawX mx_r[R], mz_r[R], mo_r[R];
  if constexpr (R > 1) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      mx_r[r] = ldraw(a.mimo_x.ptr, a.mimo_x.dtype,
                      h * a.mimo_x.stride[0] + r * a.mimo_x.stride[1] + pl);
      mz_r[r] = ldraw(a.mimo_z.ptr, a.mimo_z.dtype,
                      h * a.mimo_z.stride[0] + r * a.mimo_z.stride[1] + pl);
      mo_r[r] = ldraw(a.mimo_out.ptr, a.mimo_out.dtype,
                      h * a.mimo_out.stride[0] + r * a.mimo_out.stride[1] + pl);
    }
  }
  if (tid < P) {
    const int p = tid;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (R > 1) {
        const float mx = rnd<T>(decode(mx_r[r], a.mimo_x.dtype));
        const float mz = rnd<T>(decode(mz_r[r], a.mimo_z.dtype));
        s_vr[r][p] = mul_r<T>(v, mx);
        s_pvr[r][p] = mul_r<T>(pv, mx);
        s_zr[r][p] = mul_r<T>(z, mz);
        s_mo[r][p] = decode(mo_r[r], a.mimo_out.dtype);
      } else {
        s_vr[r][p] = v;
        s_pvr[r][p] = pv;
        s_zr[r][p] = z;
        s_mo[r][p] = 1.f;
      }
    }
    // value_out may alias prev_value: only this thread touches index p
    if (a.value_out.ptr != nullptr) {
      static_cast<T*>(a.value_out.ptr)[b * a.value_out.stride[0] + h * a.value_out.stride[1] +
                                       p] = from_f<T>(v);
    }
  }

  const float dt_in = decode(dt_r, a.dt.dtype), a_in = decode(a_r, a.a.dtype);
  const float trap_in = decode(trap_r, a.trap.dtype), Dh = decode(D_r, a.D.dtype);
  const float dtb_in = raw_dt ? decode(dtb_r, a.dt_bias.dtype) : 0.f;
  float th[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) th[i] = decode(th_r[i], a.angles.dtype);
  f4 wq, wk, bq[R], bk[R];
  wq = decode4(wq_r, a.q_norm_w.dtype);
  wk = decode4(wk_r, a.k_norm_w.dtype);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    bq[r] = decode4(bq_r[r], a.q_bias.dtype);
    bk[r] = decode4(bk_r[r], a.k_bias.dtype);
  }

  // per-(b, h) scalars
  float dt, adt;
  // the scan's forms (hardware exp / log / reciprocal, a few ulp): the per-(b, h) scalars head
  // the prologue's dependent chain
  dt_adt_fast(raw_dt, dt_in, a_in, dtb_in, dt, adt);
  const float trap = sigmoid_fast(trap_in);
  const float alpha = __expf(adt);
  const float beta = (1.f - trap) * dt * alpha;
  const float gamma = trap * dt;

  // (4) phases of the angles this thread's columns use
  float phn[4] = {0.f, 0.f, 0.f, 0.f}, cs[4] = {1.f, 1.f, 1.f, 1.f}, sn[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i < nj) {
      float ph = old[i];
      if (angles) ph = m3_fmod_2pi(__fadd_rn(old[i], phase_inc(th[i], dt)));
      phn[i] = ph;
      float sv, cv;
      __sincosf(ph, &sv, &cv);  // ph in [0, 2 pi): the hardware sine / cosine, as in the scan
      cs[i] = rnd<T>(cv);
      sn[i] = rnd<T>(sv);
    }
  }

  // (5) q / k of this thread's columns, every rank: RMSNorm, weight, bias, rotation
  float qr[R][4], kr[R][4], pk[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float q[4], k[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      q[j] = qx[r][j];
      k[j] = kx[r][j];
      pk[r][j] = px[r][j];
    }
    if (norm) {
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sq += q[j] * q[j];
        sk += k[j] * k[j];
      }
      sq = allreduce32(sq);
      sk = allreduce32(sk);
      const float rq = 1.f / sqrtf(sq / static_cast<float>(N) + a.norm_eps);
      const float rk = 1.f / sqrtf(sk / static_cast<float>(N) + a.norm_eps);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        q[j] = rnd<T>(q[j] * rq * rnd<T>(wq[j]));
        k[j] = rnd<T>(k[j] * rk * rnd<T>(wk[j]));
      }
    }
    if (bias) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        q[j] = add_r<T>(q[j], rnd<T>(bq[r][j]));
        k[j] = add_r<T>(k[j], rnd<T>(bk[r][j]));
      }
    }
    if (rotate && !mimo) {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const float lq = q[2 * pp], hq = q[2 * pp + 1], lk = k[2 * pp], hk = k[2 * pp + 1];
        if (nj > 0) {
          q[2 * pp] = sub_r<T>(mul_r<T>(lq, cs[pp]), mul_r<T>(hq, sn[pp]));
          q[2 * pp + 1] = add_r<T>(mul_r<T>(lq, sn[pp]), mul_r<T>(hq, cs[pp]));
          k[2 * pp] = sub_r<T>(mul_r<T>(lk, cs[pp]), mul_r<T>(hk, sn[pp]));
          k[2 * pp + 1] = add_r<T>(mul_r<T>(lk, sn[pp]), mul_r<T>(hk, cs[pp]));
        }
      }
    } else if (rotate) {
      // partner columns n +- 2S = +-64 live in lane c xor 16
      float oq[4], ok[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        oq[j] = swap16(q[j]);
        ok[j] = swap16(k[j]);
      }
      if (nj > 0) {
        const bool first = c < S / 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (first) {
            q[j] = sub_r<T>(mul_r<T>(q[j], cs[j]), mul_r<T>(oq[j], sn[j]));
            k[j] = sub_r<T>(mul_r<T>(k[j], cs[j]), mul_r<T>(ok[j], sn[j]));
          } else {
            q[j] = add_r<T>(mul_r<T>(oq[j], sn[j]), mul_r<T>(q[j], cs[j]));
            k[j] = add_r<T>(mul_r<T>(ok[j], sn[j]), mul_r<T>(k[j], cs[j]));
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qr[r][j] = q[j];
      kr[r][j] = k[j];
    }
  }
  __syncthreads();  // the per-row LDS vectors

  // (6) state update of rows rg + RG k, each lane's part of their readouts, then the readout
  float part[RPT][R];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int p = rg + RG * k;
    float po[4] = {0.f, 0.f, 0.f, 0.f}, co[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float pv = s_pvr[r][p], cv = s_vr[r][p];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        po[j] += pv * pk[r][j];
        co[j] += cv * kr[r][j];
      }
    }
    f4 ns;
#pragma unroll
    for (int j = 0; j < 4; ++j) ns[j] = alpha * st[k][j] + beta * po[j] + gamma * co[j];
    __builtin_nontemporal_store(ns, reinterpret_cast<f4*>(sout + p * sp_out));
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) sum += rnd<T>(ns[j]) * qr[r][j];
      part[k][r] = sum;
    }
  }
  auto epilogue = [&](int p, const float (&tot)[R]) __attribute__((always_inline)) {
    float y = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float t = (tot[r] + Dh * s_vr[r][p]) * siluf(s_zr[r][p]);
      y = R > 1 ? y + t * s_mo[r][p] : t;
    }
    return y;
  };
  if constexpr (RPT == 8) {
    // lane c holds row rg + RG ((c >> 2) & 7); the first lane of each quad stores it
    float tot[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = part[k][r];
      tot[r] = reduce_scatter8(v, c);
    }
    const int p = rg + RG * ((c >> 2) & 7);
    const float y = epilogue(p, tot);
    if ((c & 3) == 0) {
      static_cast<T*>(a.out.ptr)[b * a.out.stride[0] + h * a.out.stride[1] + p] = from_f<T>(y);
    }
  } else {
    float yrow = 0.f;  // lane c = k keeps row rg + RG k's output
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      float tot[R];
#pragma unroll
      for (int r = 0; r < R; ++r) tot[r] = allreduce32(part[k][r]);
      const float y = epilogue(rg + RG * k, tot);
      if (c == k) yrow = y;
    }
    if (c < RPT) {
      const int p = rg + RG * c;
      static_cast<T*>(a.out.ptr)[b * a.out.stride[0] + h * a.out.stride[1] + p] = from_f<T>(yrow);
    }
  }

  // (7) the small cache outputs, after every thread has consumed the inputs they may alias
  __syncthreads();
  if (rg == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      st4<T>(a.k_out.ptr, b * a.k_out.stride[0] + h * a.k_out.stride[1] + r * a.k_out.stride[2] +
                              n0, kr[r]);
    }
    float* ph_out = static_cast<float*>(a.phase_out.ptr) + b * a.phase_out.stride[0] +
                    h * a.phase_out.stride[1];
    if (rotate) {
      // each angle has one writer: SISO c < 16, MIMO the first quarter (c < 8)
      const bool writer = !mimo || c < S / 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (writer && i < nj) ph_out[(j0 + i) * a.phase_out.stride[2]] = phn[i];
      }
    } else if (c < S) {
      ph_out[c * a.phase_out.stride[2]] = ph_in[c * a.phase_in.stride[2]];
    }
  }
}

// The model's decode shape with 16-bit activations and rank R > 1, the readout on MFMA. One
// 256-thread workgroup per (batch, head); wave w owns state rows p in [16 w, 16 w + 16): half-wave
// hw = 0, 1 of the wave holds rows 16 w + 2 k + hw (k < 8), columns 4c .. 4c+3, so one load
// instruction of the wave covers two whole 512-byte rows (16 rows x 64 bytes, the MFMA output
// layout, streams 15% slower).
//   - The update S' = alpha S + beta sum_r pvr_r pk_r + gamma sum_r vr_r k_r runs on the VALU in
//     the order of step128_kernel; k and pk of the lane's columns come from LDS once.
//   - The readout Y[r][p] = q_r . rnd(S'[p]) is a 16x16x32 MFMA per wave over four K steps: the
//     wave's 16 rounded rows go through LDS (each wave reads only the rows it wrote), q is A and
//     the rows are B, so lanes 0-15 end with every rank of row 16 w + lane.
// Prologue: half-wave j computes q / k / previous k of rank j % R for columns 4c .. 4c+3 (RMSNorm
// sums over the half-wave, MIMO partner columns n +- 64 in lane c ^ 16) while the state loads are
// in flight; half-waves j >= R compute duplicates and store nothing.
template <typename T, int R, bool FULL>
__global__ __launch_bounds__(256) void step_mma_kernel(const m3_step_args a) {
  static_assert(sizeof(T) == 2 && (R == 2 || R == 4), "16-bit activations, rank 2 or 4");
  constexpr int N = 128, P = 64, S = 32, RPT = 8;
  constexpr int SBW = N + 8;  // rounded-state rows padded: 16 rows at one column hit 16 bank groups
  typedef T t4 __attribute__((ext_vector_type(4)));
  typedef T t8 __attribute__((ext_vector_type(8)));
  const int H = a.heads;
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  const int g = h / (H / a.groups);
  const int tid = threadIdx.x, c = tid & 31, hw = tid >> 5, n0 = 4 * c;
  const int rk = hw & (R - 1);        // the rank this half-wave computes
  const bool owner = hw < R;          // ... and stores
  const int l = tid & 63, w = tid >> 6, lm = l & 15, lg = l >> 4;
  const bool norm = FULL || a.q_norm_w.ptr != nullptr;
  const bool bias = FULL || a.q_bias.ptr != nullptr;
  const bool rotate = FULL || a.phase_mode != M3_PHASE_NONE;
  const bool angles = FULL || a.phase_mode == M3_PHASE_ANGLES;
  const bool raw_dt = FULL || a.raw_dt != 0;
  const bool mimo = FULL ? true : a.mimo_rotation != 0;

  __shared__ float s_vr[R][P], s_zr[R][P], s_mo[R][P];
  __shared__ __align__(16) float s_vrt[P][R];   // rank values by row: one vector read per row
  __shared__ __align__(16) float s_pvrt[P][R];
  __shared__ __align__(16) float s_k[R][N];
  __shared__ __align__(16) float s_pk[R][N];
  __shared__ __align__(16) T s_q[R][N];
  __shared__ __align__(16) T s_sb[P][SBW];

  // (1) this thread's state rows
  auto prow = [&](int k) { return 16 * w + 2 * k + (hw & 1); };
  const float* sin_ = static_cast<const float*>(a.state_in.ptr) + b * a.state_in.stride[0] +
                      h * a.state_in.stride[1] + n0;
  float* sout = static_cast<float*>(a.state_out.ptr) + b * a.state_out.stride[0] +
                h * a.state_out.stride[1] + n0;
  const int64_t sp_in = a.state_in.stride[2], sp_out = a.state_out.stride[2];
  f4 st[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    st[k] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(sin_ + prow(k) * sp_in));
  }

  // (2) every small input of the (b, h): raw loads issued together, decoded after
  const RawX dt_r = ldraw(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0] + h * a.dt.stride[1]);
  const RawX a_r = ldraw(a.a.ptr, a.a.dtype, b * a.a.stride[0] + h * a.a.stride[1]);
  const RawX trap_r = ldraw(a.trap.ptr, a.trap.dtype, b * a.trap.stride[0] + h * a.trap.stride[1]);
  const RawX D_r = ldraw(a.D.ptr, a.D.dtype, h * a.D.stride[0]);
  RawX dtb_r{0u, 0u};
  if (raw_dt) dtb_r = ldraw(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]);
  // phase roles as in step128_kernel: SISO pairs (2j, 2j+1) -> angles 2c, 2c+1 (c < 16); MIMO
  // pairs (j, j + 2S) -> angles n0 .. n0+3 for the first (c < 8) and third (16 <= c < 24) quarters
  int j0 = -1, nj = 0;
  if (rotate) {
    if (!mimo) {
      if (c < S / 2) { j0 = 2 * c; nj = 2; }
    } else if (c < S / 4) {
      j0 = n0; nj = 4;
    } else if (c >= S / 2 && c < 3 * S / 4) {
      j0 = n0 - 2 * S; nj = 4;
    }
  }
  const float* ph_in = static_cast<const float*>(a.phase_in.ptr) + b * a.phase_in.stride[0] +
                       h * a.phase_in.stride[1];
  float old[4] = {0.f, 0.f, 0.f, 0.f};
  RawX th_r[4] = {};
  if (rotate) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = nj > 0 ? j0 + min(i, nj - 1) : 0;  // lanes without angles read angle 0
      old[i] = ph_in[j * a.phase_in.stride[2]];
    }
  }
  if (rotate && angles) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = nj > 0 ? j0 + min(i, nj - 1) : 0;
      th_r[i] = ldraw(a.angles.ptr, a.angles.dtype, b * a.angles.stride[0] + j * a.angles.stride[1]);
    }
  }
  Raw4 wq_r{}, wk_r{}, bq_r{}, bk_r{};
  if (norm) {
    wq_r = ldraw4(a.q_norm_w, n0);  // weights may be FP32 or the activation type
    wk_r = ldraw4(a.k_norm_w, n0);
  }
  if (bias) {
    bq_r = ldraw4(a.q_bias, h * a.q_bias.stride[0] + rk * a.q_bias.stride[1] + n0);
    bk_r = ldraw4(a.k_bias, h * a.k_bias.stride[0] + rk * a.k_bias.stride[1] + n0);
  }
  const f4 qx = ld4<T>(a.q.ptr, b * a.q.stride[0] + g * a.q.stride[1] + rk * a.q.stride[2] + n0);
  const f4 kx = ld4<T>(a.k.ptr, b * a.k.stride[0] + g * a.k.stride[1] + rk * a.k.stride[2] + n0);
  const f4 px = ld4<T>(a.prev_k.ptr, b * a.prev_k.stride[0] + h * a.prev_k.stride[1] +
                                         rk * a.prev_k.stride[2] + n0);
  // rank values and gates of rank w % R, row p = tid % P: every thread loads them with the batch
  // above (no branch around loads), waves w < R put them in LDS once decoded
  const int pl = tid & (P - 1), rw = w & (R - 1);
  const float v = ld_act<T>(a.value, b * a.value.stride[0] + h * a.value.stride[1] + pl);
  const float z = ld_act<T>(a.gate, b * a.gate.stride[0] + h * a.gate.stride[1] + pl);
  const float pv = ld_act<T>(a.prev_value,
                             b * a.prev_value.stride[0] + h * a.prev_value.stride[1] + pl);
  const RawX mx_r = ldraw(a.mimo_x.ptr, a.mimo_x.dtype,
                          h * a.mimo_x.stride[0] + rw * a.mimo_x.stride[1] + pl);
  const RawX mz_r = ldraw(a.mimo_z.ptr, a.mimo_z.dtype,
                          h * a.mimo_z.stride[0] + rw * a.mimo_z.stride[1] + pl);
  const RawX mo_r = ldraw(a.mimo_out.ptr, a.mimo_out.dtype,
                          h * a.mimo_out.stride[0] + rw * a.mimo_out.stride[1] + pl);
  if (w < R) {
    const float mx = rnd<T>(decode(mx_r, a.mimo_x.dtype));
    const float mz = rnd<T>(decode(mz_r, a.mimo_z.dtype));
    const float vr = mul_r<T>(v, mx);
    s_vr[rw][pl] = vr;
    s_vrt[pl][rw] = vr;
    s_pvrt[pl][rw] = mul_r<T>(pv, mx);
    s_zr[rw][pl] = mul_r<T>(z, mz);
    s_mo[rw][pl] = decode(mo_r, a.mimo_out.dtype);
  }

  const float dt_in = decode(dt_r, a.dt.dtype), a_in = decode(a_r, a.a.dtype);
  const float trap_in = decode(trap_r, a.trap.dtype), Dh = decode(D_r, a.D.dtype);
  const float dtb_in = raw_dt ? decode(dtb_r, a.dt_bias.dtype) : 0.f;
  float th[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) th[i] = decode(th_r[i], a.angles.dtype);
  const f4 wq = decode4(wq_r, a.q_norm_w.dtype), wk = decode4(wk_r, a.k_norm_w.dtype);
  const f4 bq = decode4(bq_r, a.q_bias.dtype), bk = decode4(bk_r, a.k_bias.dtype);

  // per-(b, h) scalars
  float dt, adt;
  // the scan's forms (hardware exp / log / reciprocal, a few ulp): the per-(b, h) scalars head
  // the prologue's dependent chain
  dt_adt_fast(raw_dt, dt_in, a_in, dtb_in, dt, adt);
  const float trap = sigmoid_fast(trap_in);
  const float alpha = __expf(adt);
  const float beta = (1.f - trap) * dt * alpha;
  const float gamma = trap * dt;

  // (3) phases of the angles this thread's columns use
  float phn[4] = {0.f, 0.f, 0.f, 0.f}, cs[4] = {1.f, 1.f, 1.f, 1.f}, sn[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i < nj) {
      float ph = old[i];
      if (angles) ph = m3_fmod_2pi(__fadd_rn(old[i], phase_inc(th[i], dt)));
      phn[i] = ph;
      float sv, cv;
      __sincosf(ph, &sv, &cv);  // ph in [0, 2 pi): the hardware sine / cosine, as in the scan
      cs[i] = rnd<T>(cv);
      sn[i] = rnd<T>(sv);
    }
  }

  // (4) q / k of rank rk, columns n0 .. n0+3: RMSNorm, weight, bias, rotation (the rounding steps
  // of step128_kernel)
  float q[4], k[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    q[j] = qx[j];
    k[j] = kx[j];
  }
  if (norm) {
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sq += q[j] * q[j];
      sk += k[j] * k[j];
    }
    sq = allreduce32(sq);
    sk = allreduce32(sk);
    const float rq = 1.f / sqrtf(sq / static_cast<float>(N) + a.norm_eps);
    const float rk_ = 1.f / sqrtf(sk / static_cast<float>(N) + a.norm_eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      q[j] = rnd<T>(q[j] * rq * rnd<T>(wq[j]));
      k[j] = rnd<T>(k[j] * rk_ * rnd<T>(wk[j]));
    }
  }
  if (bias) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      q[j] = add_r<T>(q[j], rnd<T>(bq[j]));
      k[j] = add_r<T>(k[j], rnd<T>(bk[j]));
    }
  }
  if (rotate && !mimo) {
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const float lq = q[2 * pp], hq = q[2 * pp + 1], lk = k[2 * pp], hk = k[2 * pp + 1];
      if (nj > 0) {
        q[2 * pp] = sub_r<T>(mul_r<T>(lq, cs[pp]), mul_r<T>(hq, sn[pp]));
        q[2 * pp + 1] = add_r<T>(mul_r<T>(lq, sn[pp]), mul_r<T>(hq, cs[pp]));
        k[2 * pp] = sub_r<T>(mul_r<T>(lk, cs[pp]), mul_r<T>(hk, sn[pp]));
        k[2 * pp + 1] = add_r<T>(mul_r<T>(lk, sn[pp]), mul_r<T>(hk, cs[pp]));
      }
    }
  } else if (rotate) {
    // partner columns n +- 2S = +-64 live in lane c xor 16
    float oq[4], ok[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      oq[j] = swap16(q[j]);
      ok[j] = swap16(k[j]);
    }
    if (nj > 0) {
      const bool first = c < S / 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (first) {
          q[j] = sub_r<T>(mul_r<T>(q[j], cs[j]), mul_r<T>(oq[j], sn[j]));
          k[j] = sub_r<T>(mul_r<T>(k[j], cs[j]), mul_r<T>(ok[j], sn[j]));
        } else {
          q[j] = add_r<T>(mul_r<T>(oq[j], sn[j]), mul_r<T>(q[j], cs[j]));
          k[j] = add_r<T>(mul_r<T>(ok[j], sn[j]), mul_r<T>(k[j], cs[j]));
        }
      }
    }
  }
  if (owner) {
    *reinterpret_cast<t4*>(&s_q[rk][n0]) = t4{from_f<T>(q[0]), from_f<T>(q[1]), from_f<T>(q[2]),
                                              from_f<T>(q[3])};
    *reinterpret_cast<f4*>(&s_k[rk][n0]) = f4{k[0], k[1], k[2], k[3]};
    *reinterpret_cast<f4*>(&s_pk[rk][n0]) = px;
    // k_out may alias prev_k: this thread alone read these elements of it (px, above)
    st4<T>(a.k_out.ptr, b * a.k_out.stride[0] + h * a.k_out.stride[1] + rk * a.k_out.stride[2] +
                            n0, k);
  }
  __syncthreads();  // the per-row and per-column LDS vectors
  // value_out may alias prev_value, which every wave read before the barrier
  if (tid < P && a.value_out.ptr != nullptr) {
    static_cast<T*>(a.value_out.ptr)[b * a.value_out.stride[0] + h * a.value_out.stride[1] +
                                     tid] = from_f<T>(v);
  }

  // (5) state update of this thread's rows (the sums of step128_kernel), the rounded rows to LDS
  float kk[R][4], pk[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const f4 kv = *reinterpret_cast<const f4*>(&s_k[r][n0]);
    const f4 pv4 = *reinterpret_cast<const f4*>(&s_pk[r][n0]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kk[r][j] = kv[j];
      pk[r][j] = pv4[j];
    }
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int p = prow(k);
    typedef float fr __attribute__((ext_vector_type(R)));
    const fr pvr = *reinterpret_cast<const fr*>(&s_pvrt[p][0]);
    const fr vr = *reinterpret_cast<const fr*>(&s_vrt[p][0]);
    float po[4] = {0.f, 0.f, 0.f, 0.f}, co[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        po[j] += pvr[r] * pk[r][j];
        co[j] += vr[r] * kk[r][j];
      }
    }
    f4 ns;
#pragma unroll
    for (int j = 0; j < 4; ++j) ns[j] = alpha * st[k][j] + beta * po[j] + gamma * co[j];
    __builtin_nontemporal_store(ns, reinterpret_cast<f4*>(sout + p * sp_out));
    *reinterpret_cast<t4*>(&s_sb[p][n0]) =
        t4{from_f<T>(ns[0]), from_f<T>(ns[1]), from_f<T>(ns[2]), from_f<T>(ns[3])};
  }

  // (6) readout of the wave's rows: A = q (row m holds rank m % R), B = the rounded rows; LDS
  // operations of one wave complete in order, so a wave-level fence orders its writes before its
  // reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int prow_l = 16 * w + lm;
  f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < N / 32; ++s) {
    const t8 av = *reinterpret_cast<const t8*>(&s_q[lm & (R - 1)][32 * s + 8 * lg]);
    const t8 bv = *reinterpret_cast<const t8*>(&s_sb[prow_l][32 * s + 8 * lg]);
    if constexpr (std::is_same<T, __bf16>::value) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
    } else {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
    }
  }
  // lanes l < 16 hold Y[r][16 w + l] in acc[r]; D skip, gate and the rank sum in rank order
  if (lg == 0) {
    const int p = prow_l;
    float y = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float t = (acc[r] + Dh * s_vr[r][p]) * siluf(s_zr[r][p]);
      y = y + t * s_mo[r][p];
    }
    static_cast<T*>(a.out.ptr)[b * a.out.stride[0] + h * a.out.stride[1] + p] = from_f<T>(y);
  }

  // (7) phase_out may alias phase_in, which every half-wave read before the barrier above
  if (hw == 0) {
    float* ph_out = static_cast<float*>(a.phase_out.ptr) + b * a.phase_out.stride[0] +
                    h * a.phase_out.stride[1];
    if (rotate) {
      // each angle has one writer: SISO c < 16, MIMO the first quarter (c < 8)
      const bool writer = !mimo || c < S / 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (writer && i < nj) ph_out[(j0 + i) * a.phase_out.stride[2]] = phn[i];
      }
    } else if (c < S) {
      ph_out[c * a.phase_out.stride[2]] = ph_in[c * a.phase_in.stride[2]];
    }
  }
}

static size_t step_lds_bytes(int R, int N, int P, int S) {
  return sizeof(float) * (static_cast<size_t>(5) * R * N + 5 * R * P + P + 3 * S + 2 * R);
}

// The model's shape with 4-element column vectors aligned for step128_kernel.
static bool step128_ok(const m3_step_args& a) {
  if (a.d_state != 128 || a.head_dim != 64 || a.num_angles != 32) return false;
  for (const m3_tensor* t : {&a.q, &a.k, &a.prev_k, &a.k_out, &a.q_bias, &a.k_bias,
                             &a.q_norm_w, &a.k_norm_w}) {
    if (t->ptr == nullptr) continue;
    const int es = t->dtype == M3_F32 ? 4 : 2;
    if (reinterpret_cast<uintptr_t>(t->ptr) % (4 * es) != 0) return false;
    const int dims = (t == &a.q_norm_w || t == &a.k_norm_w) ? 1 : (t == &a.q_bias ||
                                                                    t == &a.k_bias) ? 3 : 4;
    for (int i = 0; i < dims - 1; ++i) {
      if (t->stride[i] % 4 != 0) return false;
    }
  }
  return true;
}

// The model's step: norm weights, biases, raw dt with its bias, angle phases, MIMO rotation iff
// R > 1 (the FULL form of step128_kernel).
static bool step_full(const m3_step_args& a) {
  return a.q_norm_w.ptr != nullptr && a.k_norm_w.ptr != nullptr && a.q_bias.ptr != nullptr &&
         a.k_bias.ptr != nullptr && a.raw_dt != 0 && a.dt_bias.ptr != nullptr &&
         a.phase_mode == M3_PHASE_ANGLES && a.angles.ptr != nullptr &&
         (a.mimo_rotation != 0) == (a.rank > 1);
}

template <typename T, int R, int RPT>
static void launch128(const m3_step_args& a, dim3 grid, dim3 block, hipStream_t stream,
                      bool pin) {
  if (step_full(a)) {
    if (pin) {
      hipLaunchKernelGGL((step128_kernel<T, R, RPT, true, true>), grid, block, 0, stream, a);
    } else {
      hipLaunchKernelGGL((step128_kernel<T, R, RPT, true>), grid, block, 0, stream, a);
    }
  } else {
    hipLaunchKernelGGL((step128_kernel<T, R, RPT, false>), grid, block, 0, stream, a);
  }
}

template <typename T, int R>
static void launch_mma(const m3_step_args& a, dim3 grid, hipStream_t stream) {
  if (step_full(a)) {
    hipLaunchKernelGGL((step_mma_kernel<T, R, true>), grid, dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL((step_mma_kernel<T, R, false>), grid, dim3(256), 0, stream, a);
  }
}

template <typename T>
static int launch_step(const m3_step_args& a, hipStream_t stream) {
  const size_t lds = step_lds_bytes(a.rank, a.d_state, a.head_dim, a.num_angles);
  const dim3 grid(static_cast<unsigned>(a.batch) * a.heads), block(kStepThreads);
  if constexpr (sizeof(T) == 2) {
    // 16-bit activations, ranks 2 and 4: the update and the readout on MFMA
    if ((a.rank == 2 || a.rank == 4) && step128_ok(a)) {
      if (a.rank == 2) {
        launch_mma<T, 2>(a, grid, stream);
      } else {
        launch_mma<T, 4>(a, grid, stream);
      }
      return check_launch("m3_step");
    }
  }
  // Ranks 1 and 2; rank 4 only below 1024 (batch, head) pairs (with many, its four readout
  // reductions per row make the LDS-staged step_kernel faster; rank 8 always uses that one).
  // The 256-thread form at every batch: at B = 1 its 4 waves start together, where a 1024-
  // thread form's 16 waves start in four groups about 1400 cycles apart and its barrier waits
  // for the last (13.1k against 18.1k cycles per workgroup, measured).
  const int64_t pairs = static_cast<int64_t>(a.batch) * a.heads;
  const bool few = pairs < 1024, pin = pairs < 2048;
  if ((a.rank <= 2 || (a.rank == 4 && few)) && step128_ok(a)) {
    if (a.rank == 1) {
      launch128<T, 1, 8>(a, grid, block, stream, pin);
    } else if (a.rank == 2) {
      launch128<T, 2, 8>(a, grid, block, stream, pin);
    } else {
      launch128<T, 4, 8>(a, grid, block, stream, pin);
    }
    return check_launch("m3_step");
  }
  switch (a.rank) {
    case 1: hipLaunchKernelGGL((step_kernel<T, 1>), grid, block, lds, stream, a); break;
    case 2: hipLaunchKernelGGL((step_kernel<T, 2>), grid, block, lds, stream, a); break;
    case 4: hipLaunchKernelGGL((step_kernel<T, 4>), grid, block, lds, stream, a); break;
    case 8: hipLaunchKernelGGL((step_kernel<T, 8>), grid, block, lds, stream, a); break;
    default: return fail(M3_EUNSUPPORTED, "m3_step: rank %d not in {1, 2, 4, 8}", a.rank);
  }
  return check_launch("m3_step");
}

static bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

}  // namespace m3

extern "C" int m3_step(const m3_step_args* args, hipStream_t stream) {
  using namespace m3;
  clear_error();
  if (args == nullptr) return fail(M3_EINVAL, "m3_step: args is NULL");
  const m3_step_args& a = *args;
  if (a.batch < 0 || a.heads <= 0 || a.groups <= 0 || a.rank <= 0 || a.d_state <= 0 ||
      a.head_dim <= 0 || a.num_angles < 0) {
    return fail(M3_EINVAL, "m3_step: invalid dimensions");
  }
  if (a.heads % a.groups != 0) return fail(M3_EINVAL, "m3_step: heads %% groups != 0");
  if (!valid_dtype(a.act_dtype)) return fail(M3_EINVAL, "m3_step: invalid act_dtype");
  if (a.d_state < 4) return fail(M3_EUNSUPPORTED, "m3_step: d_state %d < 4", a.d_state);
  if (a.phase_mode != M3_PHASE_NONE && a.phase_mode != M3_PHASE_ANGLES) {
    return fail(M3_EINVAL, "m3_step: phase_mode must be NONE or ANGLES");
  }
  if (a.phase_mode != M3_PHASE_NONE &&
      (a.mimo_rotation ? 4 * a.num_angles != a.d_state : 2 * a.num_angles > a.d_state)) {
    return fail(M3_EUNSUPPORTED, "m3_step: num_angles %d does not fit d_state %d (mimo=%d)",
                a.num_angles, a.d_state, a.mimo_rotation);
  }
  // The step kernels take d_state a power of 2 up to 256, head_dim and num_angles up to 256,
  // ranks 1, 2, 4 and 8, within 64 KiB of LDS; other shapes run as a one-token recurrent scan.
  const bool native = pow2(a.d_state) && a.d_state <= 256 && a.head_dim <= 256 &&
                      a.num_angles <= 256 &&
                      (a.rank == 1 || a.rank == 2 || a.rank == 4 || a.rank == 8) &&
                      step_lds_bytes(a.rank, a.d_state, a.head_dim, a.num_angles) <= 64 * 1024;
  if (!native && !rscan_fits(step_as_scan(a))) {
    return fail(M3_EUNSUPPORTED,
                "m3_step: rank %d, d_state %d, head_dim %d, %d angles: the recurrent step's "
                "per-token q / k / value vectors exceed 160 KiB of LDS",
                a.rank, a.d_state, a.head_dim, a.num_angles);
  }
  const int act = a.act_dtype;
  const int N = a.d_state, P = a.head_dim;
  int rc;
  if ((rc = check_tensor(a.q, "q", 4, N, true, act)) ||
      (rc = check_tensor(a.k, "k", 4, N, true, act)) ||
      (rc = check_tensor(a.q_norm_w, "q_norm_w", 1, N, false, -1)) ||
      (rc = check_tensor(a.k_norm_w, "k_norm_w", 1, N, a.q_norm_w.ptr != nullptr, -1)) ||
      (rc = check_tensor(a.q_bias, "q_bias", 3, N, false, -1)) ||
      (rc = check_tensor(a.k_bias, "k_bias", 3, N, a.q_bias.ptr != nullptr, -1)) ||
      (rc = check_tensor(a.value, "value", 3, P, true, act)) ||
      (rc = check_tensor(a.gate, "gate", 3, P, true, act)) ||
      (rc = check_tensor(a.dt, "dt", 2, 1, true, -1)) ||
      (rc = check_tensor(a.a, "a", 2, 1, true, -1)) ||
      (rc = check_tensor(a.dt_bias, "dt_bias", 1, 1, a.raw_dt != 0, -1)) ||
      (rc = check_tensor(a.trap, "trap", 2, 1, true, -1)) ||
      (rc = check_tensor(a.angles, "angles", 2, 1, a.phase_mode == M3_PHASE_ANGLES, -1)) ||
      (rc = check_tensor(a.D, "D", 1, 1, true, -1)) ||
      (rc = check_tensor(a.mimo_x, "mimo_x", 3, P, a.rank > 1, -1)) ||
      (rc = check_tensor(a.mimo_z, "mimo_z", 3, P, a.rank > 1, -1)) ||
      (rc = check_tensor(a.mimo_out, "mimo_out", 3, P, a.rank > 1, -1)) ||
      (rc = check_tensor(a.phase_in, "phase_in", 3, 1, a.num_angles > 0, M3_F32)) ||
      (rc = check_tensor(a.state_in, "state_in", 4, N, true, M3_F32)) ||
      (rc = check_tensor(a.prev_k, "prev_k", 4, N, true, act)) ||
      (rc = check_tensor(a.prev_value, "prev_value", 3, P, true, act)) ||
      (rc = check_tensor(a.out, "out", 3, P, true, act)) ||
      (rc = check_tensor(a.phase_out, "phase_out", 3, 1, a.num_angles > 0, M3_F32)) ||
      (rc = check_tensor(a.state_out, "state_out", 4, N, true, M3_F32)) ||
      (rc = check_tensor(a.k_out, "k_out", 4, N, true, act)) ||
      (rc = check_tensor(a.value_out, "value_out", 3, P, false, act))) {
    return rc;
  }
  if ((a.q_norm_w.ptr == nullptr) != (a.k_norm_w.ptr == nullptr) ||
      (a.q_bias.ptr == nullptr) != (a.k_bias.ptr == nullptr)) {
    return fail(M3_EINVAL, "m3_step: q/k norm weights and biases come in pairs");
  }
  if (a.batch == 0) return M3_OK;
  if (!native) return launch_recurrent_step(a, stream);
  // 16-byte state vectors.
  for (const m3_tensor* t : {&a.state_in, &a.state_out}) {
    if (reinterpret_cast<uintptr_t>(t->ptr) % 16 != 0 || t->stride[0] % 4 != 0 ||
        t->stride[1] % 4 != 0 || t->stride[2] % 4 != 0) {
      return fail(M3_EUNSUPPORTED, "m3_step: state tensors need 16-byte aligned rows");
    }
  }
  switch (act) {
    case M3_F32: return launch_step<float>(a, stream);
    case M3_BF16: return launch_step<__bf16>(a, stream);
    default: return launch_step<_Float16>(a, stream);
  }
}
