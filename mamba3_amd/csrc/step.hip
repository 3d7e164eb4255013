// Mamba-3 decode step for CDNA4: one workgroup per (batch, head) streams that head's FP32
// state [P, N] exactly once (16-byte non-temporal loads and stores), fusing the phase advance,
// the rotation of q/k, the trapezoid state update, the readout, the D skip, the SiLU gate and the
// MIMO rank sum. Replaces ops.fused_step (ops.py:87-190) and its Triton kernel
// (_triton.py:564-947), and the portable ops.mamba3_step (ops.py:825-879).
#include "m3_common.hpp"
#include "m3_host.hpp"

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

static size_t step_lds_bytes(int R, int N, int P, int S) {
  return sizeof(float) * (static_cast<size_t>(5) * R * N + 5 * R * P + P + 3 * S + 2 * R);
}

template <typename T>
static int launch_step(const m3_step_args& a, hipStream_t stream) {
  const size_t lds = step_lds_bytes(a.rank, a.d_state, a.head_dim, a.num_angles);
  const dim3 grid(static_cast<unsigned>(a.batch) * a.heads), block(kStepThreads);
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
  if (!pow2(a.d_state) || a.d_state < 4 || a.d_state > 256) {
    return fail(M3_EUNSUPPORTED, "m3_step: d_state %d must be a power of 2 in [4, 256]",
                a.d_state);
  }
  if (a.head_dim > 256) return fail(M3_EUNSUPPORTED, "m3_step: head_dim > 256");
  if (a.phase_mode != M3_PHASE_NONE && a.phase_mode != M3_PHASE_ANGLES) {
    return fail(M3_EINVAL, "m3_step: phase_mode must be NONE or ANGLES");
  }
  if (a.phase_mode != M3_PHASE_NONE &&
      (a.mimo_rotation ? 4 * a.num_angles != a.d_state : 2 * a.num_angles > a.d_state)) {
    return fail(M3_EUNSUPPORTED, "m3_step: num_angles %d does not fit d_state %d (mimo=%d)",
                a.num_angles, a.d_state, a.mimo_rotation);
  }
  if (a.num_angles > 256) return fail(M3_EUNSUPPORTED, "m3_step: num_angles > 256");
  if (step_lds_bytes(a.rank, a.d_state, a.head_dim, a.num_angles) > 64 * 1024) {
    return fail(M3_EUNSUPPORTED, "m3_step: shape needs more than 64 KiB of LDS");
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
  // 16-byte state vectors.
  for (const m3_tensor* t : {&a.state_in, &a.state_out}) {
    if (reinterpret_cast<uintptr_t>(t->ptr) % 16 != 0 || t->stride[0] % 4 != 0 ||
        t->stride[1] % 4 != 0 || t->stride[2] % 4 != 0) {
      return fail(M3_EUNSUPPORTED, "m3_step: state tensors need 16-byte aligned rows");
    }
  }
  if (a.batch == 0) return M3_OK;
  switch (act) {
    case M3_F32: return launch_step<float>(a, stream);
    case M3_BF16: return launch_step<__bf16>(a, stream);
    default: return launch_step<_Float16>(a, stream);
  }
}
