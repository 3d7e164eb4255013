// Mamba-3 scan for the shapes the chunked MFMA kernel (scan.hip) does not tile: d_state not a
// power of 2 or above 128, head_dim above 64, more than 32 angles, ranks 3, 5, 6 and 7.
// The reference takes any d_state >= 4 and any rank on its portable path (model.py:545-548,
// ops.py:544-822); this kernel gives those shapes a GPU path.
//
// One workgroup per (batch, head) walks the sequence one token at a time with the exact
// recurrence the chunked scan is a reordering of (ops.py:825-879; the reference's tests check
// step-by-step equals forward, tests/test_model.py:164-184):
//   S_t = alpha_t S_{t-1} + beta_t (v_{t-1} mx)^T k_{t-1} + gamma_t (v_t mx)^T k_t
//   y_t = sum_r mo_r (q_{t,r} . rnd(S_t) + D v_{t,r}) silu(z_{t,r})
// with alpha = exp(adt), beta = (1 - sigmoid(trap)) dt alpha, gamma = sigmoid(trap) dt, the
// endpoint (k_{-1}, v_{-1}) from initial_k / initial_value (ops.py:681-686), and q / k RMS-normed,
// biased and rotated at the reference's activation-dtype cast points (ops.py:35-84, 700-714). The
// bounded phase is the reference's: increments summed within 64-token blocks counted from the
// call's first token, fmod-reduced, on an fmod-reduced carry (model.py:215-256).
//
// The FP32 state lives in LDS when it fits there with the per-token vectors (160 KiB); a larger
// one (d_state 1024 at head_dim 64 is 256 KiB) is updated in place in final_state, where each
// element has one owning thread for the whole call, so it needs no barrier: the first token reads
// initial_state, every later one the row it wrote (through L2). Ranks above 8 add readout passes
// over the updated rows in groups of 8. Each token costs a few barriers, so this path runs at a
// fraction of the MFMA kernel's speed: it exists for coverage of the shapes, not for the
// BASELINE workloads (all of which take the MFMA kernel).
#include <algorithm>

#include "m3_common.hpp"
#include "m3_host.hpp"
#include "m3_math.h"

namespace m3 {

constexpr int kRThreads = 256;
constexpr int kRGroup = 8;  // ranks per readout pass (accumulators per thread)
constexpr size_t kRMaxLds = 160 * 1024;

// LDS floats the kernel needs for a shape (with the state, or with the state in final_state).
static size_t rscan_lds_floats(int R, int N, int P, int S, bool state_in_lds = true) {
  return (state_in_lds ? static_cast<size_t>(P) * N : 0)  // state
         + 7 * static_cast<size_t>(R) * N      // q, k, previous k, biases, two scratch copies
         + 2 * static_cast<size_t>(N)          // norm weights
         + 7 * static_cast<size_t>(R) * P      // v, previous v, z, mimo x / z / out, readout
         + 2 * static_cast<size_t>(P)          // value, previous value
         + 5 * static_cast<size_t>(S)          // cos, sin, phase, block sum, carry
         + 2 * static_cast<size_t>(R) + 8;     // RMSNorm factors, per-token scalars
}

size_t rscan_lds_bytes(int R, int N, int P, int S, bool state_in_lds = true) {
  return 4 * rscan_lds_floats(R, N, P, S, state_in_lds);
}

// Whether the state stays in LDS (else it is updated in final_state).
static bool rscan_state_in_lds(const m3_scan_args& a) {
  return rscan_lds_bytes(a.rank, a.d_state, a.head_dim, a.num_angles) <= kRMaxLds;
}

template <typename T>
__device__ __forceinline__ float ld_el(const m3_tensor& t, int64_t i) {
  return to_f(static_cast<const T*>(t.ptr)[i]);
}

template <typename T>
__global__ __launch_bounds__(kRThreads) void rscan_kernel(const m3_scan_args a, int tpr,
                                                          const m3_tensor value_out,
                                                          int state_in_lds) {
  const int H = a.heads, N = a.d_state, P = a.head_dim, S = a.num_angles, R = a.rank;
  const int L = a.length;
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  const int g = h / (H / a.groups);
  const int tid = threadIdx.x;
  const bool norm = a.q_norm_w.ptr != nullptr;
  const bool bias = a.q_bias.ptr != nullptr;
  const bool angles = a.phase_mode == M3_PHASE_ANGLES;
  const bool rotate = a.phase_mode != M3_PHASE_NONE;
  const bool raw_dt = a.raw_dt != 0;
  const int RN = R * N, RP = R * P;

  extern __shared__ float lds[];
  // [P][N] FP32 state, row stride sps: in LDS, or this (b, h)'s rows of final_state
  float* st = state_in_lds ? lds
                           : static_cast<float*>(a.final_state.ptr) + b * a.final_state.stride[0] +
                                 h * a.final_state.stride[1];
  const int64_t sps = state_in_lds ? N : a.final_state.stride[2];
  const float* st0 = a.initial_state.ptr == nullptr
                         ? nullptr
                         : static_cast<const float*>(a.initial_state.ptr) +
                               b * a.initial_state.stride[0] + h * a.initial_state.stride[1];
  float* qx = state_in_lds ? lds + P * N : lds;  // [R][N] this token's q (normed, biased, rotated)
  float* kx = qx + RN;       // [R][N] this token's k
  float* pk = kx + RN;       // [R][N] the previous token's rotated k
  float* bq = pk + RN;       // [R][N] C_bias of this head (rounded), 0 without biases
  float* bk = bq + RN;       // [R][N] B_bias
  float* sq = bk + RN;       // [R][N] q before the rotation
  float* sk = sq + RN;       // [R][N] k before the rotation
  float* wq = sk + RN;       // [N] C_norm weight (rounded), 1 without
  float* wk = wq + N;        // [N]
  float* vr = wk + N;        // [R][P] rank values v mx_r
  float* pvr = vr + RP;      // [R][P] previous rank values
  float* zr = pvr + RP;      // [R][P] rank gates z mz_r
  float* mxw = zr + RP;      // [R][P] mimo_x (rounded)
  float* mzw = mxw + RP;     // [R][P] mimo_z (rounded)
  float* mow = mzw + RP;     // [R][P] mimo_out
  float* yp = mow + RP;      // [R][P] readout q . rnd(S)
  float* vv = yp + RP;       // [P] this token's value
  float* pv = vv + P;        // [P] the previous token's value
  float* cs = pv + P;        // [S] cos of the phase, rounded
  float* sn = cs + S;        // [S] sin
  float* ph = sn + S;        // [S] this token's phase
  float* blk = ph + S;       // [S] running sum of the current 64-token block's increments
  float* car = blk + S;      // [S] phase carry at the block's start
  float* rstd = car + S;     // [2R] RMSNorm factors of this token's q / k rows
  float* scal = rstd + 2 * R;  // per-token scalars: dt, adt, trap

  const float Dh = ldx(a.D.ptr, a.D.dtype, h * a.D.stride[0]);
  const float dtb = raw_dt ? ldx(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]) : 0.f;

  // ---- per-head constants, initial state and endpoint
  for (int i = tid; i < RN; i += kRThreads) {
    const int r = i / N, n = i - r * N;
    bq[i] = bias ? rnd<T>(ldx(a.q_bias.ptr, a.q_bias.dtype,
                              h * a.q_bias.stride[0] + r * a.q_bias.stride[1] + n))
                 : 0.f;
    bk[i] = bias ? rnd<T>(ldx(a.k_bias.ptr, a.k_bias.dtype,
                              h * a.k_bias.stride[0] + r * a.k_bias.stride[1] + n))
                 : 0.f;
    pk[i] = a.initial_k.ptr != nullptr
                ? ld_el<T>(a.initial_k, b * a.initial_k.stride[0] + h * a.initial_k.stride[1] +
                                            r * a.initial_k.stride[2] + n)
                : 0.f;
  }
  for (int n = tid; n < N; n += kRThreads) {
    wq[n] = norm ? rnd<T>(ldx(a.q_norm_w.ptr, a.q_norm_w.dtype, n * a.q_norm_w.stride[0])) : 1.f;
    wk[n] = norm ? rnd<T>(ldx(a.k_norm_w.ptr, a.k_norm_w.dtype, n * a.k_norm_w.stride[0])) : 1.f;
  }
  for (int i = tid; i < RP; i += kRThreads) {
    const int r = i / P, p = i - r * P;
    if (R > 1) {
      mxw[i] = rnd<T>(ldx(a.mimo_x.ptr, a.mimo_x.dtype,
                          h * a.mimo_x.stride[0] + r * a.mimo_x.stride[1] + p));
      mzw[i] = rnd<T>(ldx(a.mimo_z.ptr, a.mimo_z.dtype,
                          h * a.mimo_z.stride[0] + r * a.mimo_z.stride[1] + p));
      mow[i] = ldx(a.mimo_out.ptr, a.mimo_out.dtype,
                   h * a.mimo_out.stride[0] + r * a.mimo_out.stride[1] + p);
    } else {
      mxw[i] = mzw[i] = mow[i] = 1.f;
    }
  }
  for (int p = tid; p < P; p += kRThreads) {
    pv[p] = a.initial_value.ptr != nullptr
                ? ld_el<T>(a.initial_value, b * a.initial_value.stride[0] +
                                                h * a.initial_value.stride[1] + p)
                : 0.f;
  }
  if (state_in_lds) {
    for (int i = tid; i < P * N; i += kRThreads) {
      const int p = i / N, n = i - p * N;
      st[i] = st0 != nullptr ? st0[p * a.initial_state.stride[2] + n] : 0.f;
    }
  }
  for (int s = tid; s < S; s += kRThreads) {
    blk[s] = 0.f;
    car[s] = a.initial_phase.ptr != nullptr
                 ? static_cast<const float*>(a.initial_phase.ptr)
                       [b * a.initial_phase.stride[0] + h * a.initial_phase.stride[1] +
                        s * a.initial_phase.stride[2]]
                 : 0.f;
    ph[s] = car[s];
  }
  __syncthreads();
  for (int i = tid; i < RP; i += kRThreads) {
    const int p = i % P;
    pvr[i] = R > 1 ? mul_r<T>(pv[p], mxw[i]) : pv[p];
  }

  float log_decay = 0.f;
  for (int t = 0; t < L; ++t) {
    // ---- (1) this token's inputs
    const int64_t tq = b * a.q.stride[0] + t * a.q.stride[1] + g * a.q.stride[2];
    const int64_t tk = b * a.k.stride[0] + t * a.k.stride[1] + g * a.k.stride[2];
    for (int i = tid; i < RN; i += kRThreads) {
      const int r = i / N, n = i - r * N;
      qx[i] = ld_el<T>(a.q, tq + r * a.q.stride[3] + n);
      kx[i] = ld_el<T>(a.k, tk + r * a.k.stride[3] + n);
    }
    for (int p = tid; p < P; p += kRThreads) {
      const float v = ld_el<T>(a.value, b * a.value.stride[0] + t * a.value.stride[1] +
                                            h * a.value.stride[2] + p);
      const float z = ld_el<T>(a.gate, b * a.gate.stride[0] + t * a.gate.stride[1] +
                                           h * a.gate.stride[2] + p);
      vv[p] = v;
      for (int r = 0; r < R; ++r) {
        vr[r * P + p] = R > 1 ? mul_r<T>(v, mxw[r * P + p]) : v;
        zr[r * P + p] = R > 1 ? mul_r<T>(z, mzw[r * P + p]) : z;
      }
    }
    if (tid == 0) {
      float dt, adt;
      dt_adt(raw_dt, ldx(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0] + t * a.dt.stride[1] +
                                                   h * a.dt.stride[2]),
             ldx(a.a.ptr, a.a.dtype, b * a.a.stride[0] + t * a.a.stride[1] + h * a.a.stride[2]),
             dtb, dt, adt);
      scal[0] = dt;
      scal[1] = adt;
      scal[2] = sigmoidf(ldx(a.trap.ptr, a.trap.dtype,
                             b * a.trap.stride[0] + t * a.trap.stride[1] + h * a.trap.stride[2]));
    }
    __syncthreads();
    const float dt = scal[0], adt = scal[1], trap = scal[2];
    log_decay += adt;

    // ---- (2) RMSNorm factors, phase
    if (norm) {
      const int wave = tid >> 6, lane = tid & 63;
      for (int row = wave; row < 2 * R; row += kRThreads / 64) {
        const float* x = row < R ? qx + row * N : kx + (row - R) * N;
        float s = 0.f;
        for (int n = lane; n < N; n += 64) s = fmaf(x[n], x[n], s);
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if (lane == 0) rstd[row] = 1.f / sqrtf(s / static_cast<float>(N) + a.norm_eps);
      }
    }
    if (rotate) {
      for (int s = tid; s < S; s += kRThreads) {
        float p;
        if (angles) {
          const float th = ldx(a.phase.ptr, a.phase.dtype,
                               b * a.phase.stride[0] + t * a.phase.stride[1] + s * a.phase.stride[2]);
          const float bs = (t & 63) == 0 ? phase_inc(th, dt) : __fadd_rn(blk[s], phase_inc(th, dt));
          p = m3_fmod_2pi(__fadd_rn(bs, car[s]));
          blk[s] = bs;
          if ((t & 63) == 63 || t == L - 1) {
            if (a.block_phase.ptr != nullptr) {
              static_cast<float*>(a.block_phase.ptr)[b * a.block_phase.stride[0] +
                                                     h * a.block_phase.stride[1] +
                                                     (t >> 6) * a.block_phase.stride[2] +
                                                     s * a.block_phase.stride[3]] = bs;
            }
            if ((t & 63) == 63) car[s] = m3_fmod_2pi(__fadd_rn(car[s], bs));
          }
        } else {
          p = static_cast<const float*>(a.phase.ptr)[b * a.phase.stride[0] +
                                                     t * a.phase.stride[1] +
                                                     h * a.phase.stride[2] +
                                                     s * a.phase.stride[3]];
        }
        ph[s] = p;
        cs[s] = rnd<T>(cosf(p));
        sn[s] = rnd<T>(sinf(p));
      }
    }
    __syncthreads();

    // ---- (3) q, k: norm, bias (activation-dtype cast points), then the rotation (ops.py:35-84):
    // SISO pairs (2j, 2j+1), MIMO pairs (j, j + 2S), j < S
    for (int i = tid; i < RN; i += kRThreads) {
      const int r = i / N, n = i - r * N;
      float q = qx[i], k = kx[i];
      if (norm) {
        q = rnd<T>(q * rstd[r] * wq[n]);
        k = rnd<T>(k * rstd[R + r] * wk[n]);
      }
      if (bias) {
        q = add_r<T>(q, bq[i]);
        k = add_r<T>(k, bk[i]);
      }
      sq[i] = q;
      sk[i] = k;
    }
    __syncthreads();
    for (int i = tid; i < RN; i += kRThreads) {
      const int r = i / N, n = i - r * N;
      const float* xq = sq + r * N;
      const float* xk = sk + r * N;
      float oq = xq[n], ok = xk[n];
      int j = -1, lo = 0, hi = 0;
      bool second = false;
      if (rotate) {
        if (!a.mimo_rotation) {
          if (n < 2 * S) { j = n >> 1; lo = n & ~1; hi = n | 1; second = n & 1; }
        } else if (n < S) {
          j = n; lo = n; hi = n + 2 * S;
        } else if (n >= 2 * S && n < 3 * S) {
          j = n - 2 * S; lo = j; hi = n; second = true;
        }
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
      qx[i] = oq;
      kx[i] = ok;
    }
    __syncthreads();

    // ---- (4) state update and readout: tpr consecutive lanes share a row p. The thread that
    // updates element (p, n) is the same at every token (the state in final_state relies on it).
    const float alpha = expf(adt);
    const float beta = (1.f - trap) * dt * alpha;
    const float gamma = trap * dt;
    const int rows_per_pass = kRThreads / tpr;
    const int lane_in_row = tid & (tpr - 1);
    const bool first = !state_in_lds && t == 0;  // the state's previous value is initial_state
    for (int p0 = 0; p0 < P; p0 += rows_per_pass) {
      const int p = p0 + tid / tpr;
      float part[kRGroup];
#pragma unroll
      for (int r = 0; r < kRGroup; ++r) part[r] = 0.f;
      if (p < P) {
        for (int n = lane_in_row; n < N; n += tpr) {
          float po = 0.f, co = 0.f;
#pragma unroll
          for (int r = 0; r < kRGroup; ++r) {
            if (r < R) {
              po = fmaf(pvr[r * P + p], pk[r * N + n], po);
              co = fmaf(vr[r * P + p], kx[r * N + n], co);
            }
          }
          for (int r = kRGroup; r < R; ++r) {
            po = fmaf(pvr[r * P + p], pk[r * N + n], po);
            co = fmaf(vr[r * P + p], kx[r * N + n], co);
          }
          const float old = first ? (st0 != nullptr ? st0[p * a.initial_state.stride[2] + n] : 0.f)
                                  : st[p * sps + n];
          const float ns = alpha * old + beta * po + gamma * co;
          st[p * sps + n] = ns;
          const float nr = rnd<T>(ns);
#pragma unroll
          for (int r = 0; r < kRGroup; ++r) {
            if (r < R) part[r] = fmaf(nr, qx[r * N + n], part[r]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < kRGroup; ++r) {
        if (r < R) {
          float v = part[r];
          for (int o = tpr >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o);
          if (p < P && lane_in_row == 0) yp[r * P + p] = v;
        }
      }
      // ranks beyond the first 8: further readout passes over the row this thread just wrote
      for (int r0 = kRGroup; r0 < R; r0 += kRGroup) {
#pragma unroll
        for (int r = 0; r < kRGroup; ++r) part[r] = 0.f;
        if (p < P) {
          for (int n = lane_in_row; n < N; n += tpr) {
            const float nr = rnd<T>(st[p * sps + n]);
#pragma unroll
            for (int r = 0; r < kRGroup; ++r) {
              if (r0 + r < R) part[r] = fmaf(nr, qx[(r0 + r) * N + n], part[r]);
            }
          }
        }
#pragma unroll
        for (int r = 0; r < kRGroup; ++r) {
          if (r0 + r < R) {
            float v = part[r];
            for (int o = tpr >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o);
            if (p < P && lane_in_row == 0) yp[(r0 + r) * P + p] = v;
          }
        }
      }
    }
    __syncthreads();

    // ---- (5) epilogue: D skip, SiLU gate, MIMO rank sum; the endpoint of the next token
    for (int p = tid; p < P; p += kRThreads) {
      float y = 0.f;
      for (int r = 0; r < R; ++r) {
        const float u = (yp[r * P + p] + Dh * vr[r * P + p]) * siluf(zr[r * P + p]);
        y = R > 1 ? y + u * mow[r * P + p] : u;
      }
      static_cast<T*>(a.out.ptr)[b * a.out.stride[0] + t * a.out.stride[1] +
                                 h * a.out.stride[2] + p] = from_f<T>(y);
    }
    for (int i = tid; i < RN; i += kRThreads) pk[i] = kx[i];
    for (int i = tid; i < RP; i += kRThreads) pvr[i] = vr[i];
    __syncthreads();
  }

  // ---- final state (already in place when it lives in final_state, unless L = 0), phase, k,
  // decay
  if (state_in_lds || L == 0) {
    for (int i = tid; i < P * N; i += kRThreads) {
      const int p = i / N, n = i - p * N;
      static_cast<float*>(a.final_state.ptr)[b * a.final_state.stride[0] +
                                             h * a.final_state.stride[1] +
                                             p * a.final_state.stride[2] + n] =
          state_in_lds ? st[i] : (st0 != nullptr ? st0[p * a.initial_state.stride[2] + n] : 0.f);
    }
  }
  if (a.final_phase.ptr != nullptr) {
    for (int s = tid; s < S; s += kRThreads) {
      static_cast<float*>(a.final_phase.ptr)[b * a.final_phase.stride[0] +
                                             h * a.final_phase.stride[1] +
                                             s * a.final_phase.stride[2]] = ph[s];
    }
  }
  if (a.final_k.ptr != nullptr && L > 0) {
    for (int i = tid; i < RN; i += kRThreads) {
      const int r = i / N, n = i - r * N;
      static_cast<T*>(a.final_k.ptr)[b * a.final_k.stride[0] + h * a.final_k.stride[1] +
                                     r * a.final_k.stride[2] + n] = from_f<T>(pk[i]);
    }
  }
  if (a.final_decay.ptr != nullptr && tid == 0) {
    static_cast<float*>(a.final_decay.ptr)[b * a.final_decay.stride[0] +
                                           h * a.final_decay.stride[1]] = log_decay;
  }
  // a decode step's next previous value (the last token's value)
  if (value_out.ptr != nullptr && L > 0) {
    for (int p = tid; p < P; p += kRThreads) {
      static_cast<T*>(value_out.ptr)[b * value_out.stride[0] + h * value_out.stride[1] + p] =
          from_f<T>(vv[p]);
    }
  }
}

bool rscan_fits(const m3_scan_args& a) {
  return a.rank >= 1 &&
         rscan_lds_bytes(a.rank, a.d_state, a.head_dim, a.num_angles, false) <= kRMaxLds;
}

template <typename T>
static int launch_rscan_t(const m3_scan_args& a, const m3_tensor& value_out, hipStream_t stream) {
  const bool in_lds = rscan_state_in_lds(a);
  const size_t lds = rscan_lds_bytes(a.rank, a.d_state, a.head_dim, a.num_angles, in_lds);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&rscan_kernel<T>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kRMaxLds);
    if (e != hipSuccess) {
      return fail(M3_ELAUNCH, "recurrent scan: hipFuncSetAttribute: %s", hipGetErrorString(e));
    }
    attr_set = true;
  }
  // lanes per state row: the largest power of 2 with every row of a pass in one workgroup
  int tpr = 64;
  while (tpr > 1 && kRThreads / tpr < std::min(a.head_dim, kRThreads)) tpr >>= 1;
  hipLaunchKernelGGL((rscan_kernel<T>), dim3(static_cast<unsigned>(a.batch) * a.heads),
                     dim3(kRThreads), lds, stream, a, tpr, value_out, in_lds ? 1 : 0);
  return check_launch("recurrent scan");
}

static int launch_rscan(const m3_scan_args& a, const m3_tensor& value_out, hipStream_t stream) {
  switch (a.act_dtype) {
    case M3_F32: return launch_rscan_t<float>(a, value_out, stream);
    case M3_BF16: return launch_rscan_t<__bf16>(a, value_out, stream);
    default: return launch_rscan_t<_Float16>(a, value_out, stream);
  }
}

int launch_recurrent_scan(const m3_scan_args& a, hipStream_t stream) {
  return launch_rscan(a, m3_tensor{}, stream);
}

// A per-token tensor of the step ([B, X...]) seen as the scan's [B, L = 1, X...].
static m3_tensor one_token(const m3_tensor& t) {
  m3_tensor o = t;
  o.stride[0] = t.stride[0];
  for (int i = 4; i >= 2; --i) o.stride[i] = t.stride[i - 1];
  o.stride[1] = 0;
  return o;
}

// One decode token as a one-token scan from the cache: the phase advance of a one-token scan is
// fmod(phase + increment, 2 pi), its update and readout the step's (ops.py:825-879).
m3_scan_args step_as_scan(const m3_step_args& s) {
  m3_scan_args a{};
  a.batch = s.batch;
  a.length = 1;
  a.heads = s.heads;
  a.groups = s.groups;
  a.rank = s.rank;
  a.d_state = s.d_state;
  a.head_dim = s.head_dim;
  a.num_angles = s.num_angles;
  a.chunk = 1;
  a.act_dtype = s.act_dtype;
  a.mimo_rotation = s.mimo_rotation;
  a.raw_dt = s.raw_dt;
  a.phase_mode = s.phase_mode;
  a.segments = 1;
  a.norm_eps = s.norm_eps;
  a.q = one_token(s.q);
  a.k = one_token(s.k);
  a.q_norm_w = s.q_norm_w;
  a.k_norm_w = s.k_norm_w;
  a.q_bias = s.q_bias;
  a.k_bias = s.k_bias;
  a.value = one_token(s.value);
  a.gate = one_token(s.gate);
  a.dt = one_token(s.dt);
  a.a = one_token(s.a);
  a.dt_bias = s.dt_bias;
  a.trap = one_token(s.trap);
  a.phase = s.phase_mode == M3_PHASE_ANGLES ? one_token(s.angles) : m3_tensor{};
  a.initial_phase = s.phase_in;
  a.D = s.D;
  a.mimo_x = s.mimo_x;
  a.mimo_z = s.mimo_z;
  a.mimo_out = s.mimo_out;
  a.initial_state = s.state_in;
  a.initial_k = s.prev_k;
  a.initial_value = s.prev_value;
  a.out = one_token(s.out);
  a.final_state = s.state_out;
  a.final_phase = s.phase_out;
  a.final_k = s.k_out;
  return a;
}

int launch_recurrent_step(const m3_step_args& s, hipStream_t stream) {
  return launch_rscan(step_as_scan(s), s.value_out, stream);
}

}  // namespace m3
