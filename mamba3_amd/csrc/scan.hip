// Chunked Mamba-3 SSD for CDNA4 (gfx950).
//
// One persistent workgroup (4 waves) per (batch, head) walks the sequence in sub-chunks of
// ROWS flattened (token, rank) rows. The FP32 state lives in MFMA accumulator registers for the
// whole sequence, stored transposed (S^T [N, P]) as 16x16 tiles spread over the four waves, so
// the per-chunk state update of the reference (_triton.py:294-413, launched once per chunk by
// ops.py:444-504) is fused into the same kernel and the state never round-trips through HBM.
//
// Per sub-chunk:
//   prologue  per-token dt / adt / trap from the raw projection or given (model.py:195-198),
//             exp-trapezoid scale and diagonal (ops.py:659-671), within-chunk cumsum of adt,
//             bounded phase (model.py:215-256), RMSNorm of raw B/C (model.py:190-191), head
//             bias and rotation in the activation dtype (ops.py:35-84, 700-714), k * scale and
//             k * scale * end_decay (ops.py:743, 806-807), rank values v * mimo_x, z * mimo_z;
//             staged in LDS as MFMA operands.
//   scores    Sc^T = K_s Q^T                    (MFMA, FP32 accumulate)       ops.py:763-765
//   weights   W = rnd(Sc * decay)  masked by token, diagonal gamma / scale     ops.py:770-787
//   intra     W V   (W stays in registers: the K axis is permuted consistently in both operands)
//   inter     Q rnd(S)^T * exp(cum)                                          ops.py:753-759
//   epilogue  (inter + intra + D v) silu(z), MIMO rank sum                   ops.py:792-802
//   carry     S^T = exp(cum_last) S^T + Ke^T V                               ops.py:806-816
//
// Replaces ops._fused_chunk_scan (ops.py:253-367) / its driver (ops.py:370-505) and the Triton
// kernels _chunk_main_kernel (_triton.py:74-291) and _chunk_state_kernel (_triton.py:294-413);
// the same kernel serves the portable entry ops.mamba3_scan (ops.py:544-822).
#include "m3_common.hpp"
#include "m3_host.hpp"

namespace m3 {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kMaxStateTiles = 16;  // 16x16 state tiles per wave (N_pad * P_pad <= 16384)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// MFMA policy per activation type: 16-bit types use 16x16x32 (K = 32, 8 elements per lane),
// FP32 uses 16x16x4 (K = 4, one element per lane). ROWS is the sub-chunk height.
template <typename T> struct Mma;
template <> struct Mma<__bf16> {
  static constexpr int KS = 32, ROWS = 64, PAD = 8;
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  static __device__ __forceinline__ f4 mma(v8 a, v8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<_Float16> {
  static constexpr int KS = 32, ROWS = 64, PAD = 8;
  typedef f16x8 v8;
  typedef f16x4 v4;
  static __device__ __forceinline__ f4 mma(v8 a, v8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<float> {
  static constexpr int KS = 4, ROWS = 32, PAD = 4;
  static __device__ __forceinline__ f4 mma(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

// Geometry shared by host and device.
struct ScanGeom {
  int n_pad, p_pad;      // N rounded up to 32, P rounded up to 16
  int lq;                // row stride (elements) of Qs, Ks, Sb
  int lr;                // row stride (elements) of KeT, VT, ZT
  int tok;               // tokens per sub-chunk (ROWS / R)
  int nt, pt;            // 16-row tiles of N_pad and P_pad
  int xcd_map;           // 1: map blocks so an XCD holds consecutive (b, h)
  // LDS byte offsets
  int o_qs, o_ks, o_ket, o_vt, o_zt, o_sb, o_f;
  int bytes;
};

// Float scratch in LDS, offsets in floats from o_f.
struct FOff {
  int cum, ecum, diag, scale, eend, cs, sn, pbase, poff, mx, mz, mo, ecl;
};

__device__ __forceinline__ FOff f_offsets(int tok, int S, int R, int P) {
  FOff o;
  o.cum = 0;
  o.ecum = o.cum + 64;
  o.diag = o.ecum + 64;
  o.scale = o.diag + 64;
  o.eend = o.scale + 64;
  o.cs = o.eend + 64;
  o.sn = o.cs + tok * S;
  o.pbase = o.sn + tok * S;
  o.poff = o.pbase + S;
  o.mx = o.poff + S;
  o.mz = o.mx + R * P;
  o.mo = o.mz + R * P;
  o.ecl = o.mo + R * P;
  return o;
}

static inline int f_floats(int tok, int S, int R, int P) {
  return 5 * 64 + 2 * tok * S + 2 * S + 3 * R * P + 4;
}

__device__ __forceinline__ f4 zero4() {
  f4 z;
  z[0] = z[1] = z[2] = z[3] = 0.f;
  return z;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ float wave_incl_scan(float v, int lane) {
  for (int o = 1; o < 64; o <<= 1) {
    const float u = __shfl_up(v, o);
    if (lane >= o) v += u;
  }
  return v;
}

template <typename T>
__device__ __forceinline__ T* lds_t(char* base, int off) {
  return reinterpret_cast<T*>(base + off);
}

template <typename T, int R>
__global__ __launch_bounds__(kThreads) void scan_kernel(const m3_scan_args a, const ScanGeom g) {
  using M = Mma<T>;
  constexpr int ROWS = M::ROWS;
  constexpr int RT = ROWS / 16;        // 16-row tiles per sub-chunk
  constexpr int WPR = kWaves / RT;     // waves sharing one query row tile
  const int H = a.heads, L = a.length, N = a.d_state, P = a.head_dim, S = a.num_angles;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;

  // ---- block -> (b, h)
  int bid = blockIdx.x;
  if (g.xcd_map) {
    const int per = gridDim.x >> 3;
    bid = (bid & 7) * per + (bid >> 3);
  }
  const int b = bid / H, h = bid - b * H;
  const int grp = h / (H / a.groups);

  extern __shared__ __attribute__((aligned(16))) char smem[];
  T* Qs = lds_t<T>(smem, g.o_qs);
  T* Ks = lds_t<T>(smem, g.o_ks);
  T* KeT = lds_t<T>(smem, g.o_ket);
  T* VT = lds_t<T>(smem, g.o_vt);
  T* ZT = lds_t<T>(smem, g.o_zt);
  T* Sb = lds_t<T>(smem, g.o_sb);
  float* F = lds_t<float>(smem, g.o_f);
  const FOff fo = f_offsets(g.tok, S, R, P);
  const int LQ = g.lq, LR = g.lr, NP = g.n_pad, PP = g.p_pad, TOK = g.tok;

  const bool norm = a.q_norm_w.ptr != nullptr;
  const bool bias = a.q_bias.ptr != nullptr;
  const bool rotate = a.phase_mode != M3_PHASE_NONE;
  const float Dh = ldx(a.D.ptr, a.D.dtype, h * a.D.stride[0]);

  // ---- one-time LDS setup: zero the padded operand regions, MIMO parameters, phase carry
  for (int i = tid; i < (g.o_f - g.o_qs) / 2; i += kThreads) {
    reinterpret_cast<uint16_t*>(smem + g.o_qs)[i] = 0;
  }
  for (int i = tid; i < R * P; i += kThreads) {
    const int r = i / P, p = i - r * P;
    if (R > 1) {
      F[fo.mx + i] = rnd<T>(ldx(a.mimo_x.ptr, a.mimo_x.dtype,
                                h * a.mimo_x.stride[0] + r * a.mimo_x.stride[1] + p));
      F[fo.mz + i] = rnd<T>(ldx(a.mimo_z.ptr, a.mimo_z.dtype,
                                h * a.mimo_z.stride[0] + r * a.mimo_z.stride[1] + p));
      F[fo.mo + i] = ldx(a.mimo_out.ptr, a.mimo_out.dtype,
                         h * a.mimo_out.stride[0] + r * a.mimo_out.stride[1] + p);
    } else {
      F[fo.mx + i] = 1.f;
      F[fo.mz + i] = 1.f;
      F[fo.mo + i] = 1.f;
    }
  }
  for (int s = tid; s < S; s += kThreads) {
    F[fo.pbase + s] = 0.f;
    F[fo.poff + s] = a.initial_phase.ptr != nullptr
                         ? static_cast<const float*>(a.initial_phase.ptr)
                               [b * a.initial_phase.stride[0] + h * a.initial_phase.stride[1] +
                                s * a.initial_phase.stride[2]]
                         : 0.f;
  }

  // ---- the state: S^T tiles (ni, pj), tile u = w + 4k; lane holds n = 16 ni + 4 lg + i,
  // p = 16 pj + l16.
  const int n_tiles = g.nt * g.pt;
  f4 st[kMaxStateTiles];
#pragma unroll
  for (int k = 0; k < kMaxStateTiles; ++k) {
    st[k] = zero4();
    const int u = w + kWaves * k;
    if (u < n_tiles) {
      const int ni = u / g.pt, pj = u - ni * g.pt;
      const int p = 16 * pj + l16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = 16 * ni + 4 * lg + i;
        if (a.initial_state.ptr != nullptr && p < P && n < N) {
          st[k][i] = static_cast<const float*>(a.initial_state.ptr)
              [b * a.initial_state.stride[0] + h * a.initial_state.stride[1] +
               p * a.initial_state.stride[2] + n];
        }
      }
    }
  }
  // Endpoint continuation (ops.py:681-686): S += dt_0 (1 - trap_0) sum_r (v_prev mx_r) k_prev_r.
  if (a.initial_k.ptr != nullptr && L > 0) {
    float dt0, adt0;
    dt_adt(a.raw_dt, ldx(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0] + h * a.dt.stride[2]),
           ldx(a.a.ptr, a.a.dtype, b * a.a.stride[0] + h * a.a.stride[2]),
           a.raw_dt ? ldx(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]) : 0.f, dt0,
           adt0);
    const float tr0 = sigmoidf(ldx(a.trap.ptr, a.trap.dtype,
                                   b * a.trap.stride[0] + h * a.trap.stride[2]));
    const float c0 = dt0 * (1.f - tr0);
#pragma unroll
    for (int k = 0; k < kMaxStateTiles; ++k) {
      const int u = w + kWaves * k;
      if (u >= n_tiles) continue;
      const int ni = u / g.pt, pj = u - ni * g.pt;
      const int p = 16 * pj + l16;
      if (p >= P) continue;
      const float v0 = to_f(static_cast<const T*>(a.initial_value.ptr)
                                [b * a.initial_value.stride[0] + h * a.initial_value.stride[1] + p]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = 16 * ni + 4 * lg + i;
        if (n >= N) continue;
        float outer = 0.f;
        for (int r = 0; r < R; ++r) {
          const float pv = R > 1 ? mul_r<T>(v0, rnd<T>(ldx(a.mimo_x.ptr, a.mimo_x.dtype,
                                                             h * a.mimo_x.stride[0] +
                                                                 r * a.mimo_x.stride[1] + p)))
                                 : v0;
          const float k0 = to_f(static_cast<const T*>(a.initial_k.ptr)
                                    [b * a.initial_k.stride[0] + h * a.initial_k.stride[1] +
                                     r * a.initial_k.stride[2] + n]);
          outer += pv * k0;
        }
        st[k][i] += c0 * outer;
      }
    }
  }
  __syncthreads();

  // ---- sub-chunk loop
  for (int t0 = 0; t0 < L; t0 += TOK) {
    const int width = min(TOK, L - t0);

    // (1) per-token scalars: every wave computes them for lane = token.
    const int tg = t0 + lane;
    const bool tv = lane < width;
    float dt = 0.f, adt = 0.f, tr = 0.f;
    if (tv) {
      dt_adt(a.raw_dt, ldx(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0] + tg * a.dt.stride[1] +
                                                     h * a.dt.stride[2]),
             ldx(a.a.ptr, a.a.dtype, b * a.a.stride[0] + tg * a.a.stride[1] + h * a.a.stride[2]),
             a.raw_dt ? ldx(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]) : 0.f, dt,
             adt);
      tr = sigmoidf(ldx(a.trap.ptr, a.trap.dtype,
                        b * a.trap.stride[0] + tg * a.trap.stride[1] + h * a.trap.stride[2]));
    }
    if (w == 0) {
      // right trapezoid endpoint of the next token: dt_{t+1} (1 - trap_{t+1}), 0 past the end
      float left = dt * (1.f - tr);
      float right = __shfl_down(left, 1);
      if (lane == TOK - 1 || lane == 63) {
        right = 0.f;
        const int tn = t0 + TOK;
        if (lane == TOK - 1 && tn < L) {
          float dtn, adtn;
          dt_adt(a.raw_dt, ldx(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0] + tn * a.dt.stride[1] +
                                                         h * a.dt.stride[2]),
                 ldx(a.a.ptr, a.a.dtype,
                     b * a.a.stride[0] + tn * a.a.stride[1] + h * a.a.stride[2]),
                 a.raw_dt ? ldx(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]) : 0.f,
                 dtn, adtn);
          const float trn = sigmoidf(ldx(a.trap.ptr, a.trap.dtype,
                                         b * a.trap.stride[0] + tn * a.trap.stride[1] +
                                             h * a.trap.stride[2]));
          right = dtn * (1.f - trn);
        }
      }
      if (!(tg + 1 < L)) right = 0.f;
      const float gamma = dt * tr;
      const float scale = gamma + right;
      const float cum = wave_incl_scan(tv ? adt : 0.f, lane);
      const float cum_last = __shfl(cum, width - 1);
      if (lane < 64) {
        const float c = tv ? cum : cum_last;
        F[fo.cum + lane] = c;
        F[fo.ecum + lane] = tv ? expf(c) : 0.f;
        F[fo.diag + lane] = tv ? gamma / scale : 0.f;
        F[fo.scale + lane] = tv ? rnd<T>(scale) : 0.f;
        F[fo.eend + lane] = tv ? rnd<T>(expf(cum_last - cum)) : 0.f;
      }
      if (lane == 0) F[fo.ecl] = expf(cum_last);
    }

    // (2) phase and its cos / sin per (token, angle), angle s handled by wave s % 4.
    if (rotate) {
      const bool new_block = (t0 & 63) == 0;
      for (int s = w; s < S; s += kWaves) {
        float ph = 0.f;
        if (a.phase_mode == M3_PHASE_GIVEN) {
          if (tv) {
            ph = static_cast<const float*>(a.phase.ptr)[b * a.phase.stride[0] +
                                                        tg * a.phase.stride[1] +
                                                        h * a.phase.stride[2] +
                                                        s * a.phase.stride[3]];
          }
        } else {
          float inc = 0.f;
          if (tv) {
            inc = phase_inc(ldx(a.phase.ptr, a.phase.dtype,
                                b * a.phase.stride[0] + tg * a.phase.stride[1] +
                                    s * a.phase.stride[2]),
                            dt);
          }
          const float loc = wave_incl_scan(inc, lane);
          float base = F[fo.pbase + s], off = F[fo.poff + s];
          if (new_block && t0 > 0) {
            off = fmodf(__fadd_rn(off, base), kTwoPi);
            base = 0.f;
          }
          ph = fmodf(__fadd_rn(__fadd_rn(base, loc), off), kTwoPi);
          const float tot = __shfl(loc, 63);
          if (lane == 0) {
            F[fo.pbase + s] = __fadd_rn(base, tot);
            F[fo.poff + s] = off;
          }
          if (tv && tg == L - 1 && a.final_phase.ptr != nullptr) {
            static_cast<float*>(a.final_phase.ptr)[b * a.final_phase.stride[0] +
                                                   h * a.final_phase.stride[1] +
                                                   s * a.final_phase.stride[2]] = ph;
          }
        }
        if (lane < TOK) {
          F[fo.cs + lane * S + s] = rnd<T>(cosf(ph));
          F[fo.sn + lane * S + s] = rnd<T>(sinf(ph));
        }
      }
    }
    __syncthreads();

    // (3) q / k rows: RMSNorm, bias, rotation, scale -> Qs, Ks, KeT.
    const bool mimo_pairs = a.mimo_rotation != 0;
    for (int row = w; row < ROWS; row += kWaves) {
      const int tt = row / R, r = row - tt * R;
      const int tgr = t0 + tt;
      const bool valid = tt < width;
      const int64_t qo = b * a.q.stride[0] + tgr * a.q.stride[1] + grp * a.q.stride[2] +
                         r * a.q.stride[3];
      const int64_t ko = b * a.k.stride[0] + tgr * a.k.stride[1] + grp * a.k.stride[2] +
                         r * a.k.stride[3];
      const int half = N >> 1;
      // each lane owns pairs j = lane + 64 m
      float q0[2], q1[2], k0[2], k1[2];
      int e0[2], e1[2];
      float ssq = 0.f, ssk = 0.f;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int j = lane + 64 * m;
        e0[m] = mimo_pairs ? j : 2 * j;
        e1[m] = mimo_pairs ? j + half : 2 * j + 1;
        q0[m] = q1[m] = k0[m] = k1[m] = 0.f;
        if (valid && j < half) {
          const T* qp = static_cast<const T*>(a.q.ptr) + qo;
          const T* kp = static_cast<const T*>(a.k.ptr) + ko;
          q0[m] = to_f(qp[e0[m]]);
          q1[m] = to_f(qp[e1[m]]);
          k0[m] = to_f(kp[e0[m]]);
          k1[m] = to_f(kp[e1[m]]);
          ssq += q0[m] * q0[m] + q1[m] * q1[m];
          ssk += k0[m] * k0[m] + k1[m] * k1[m];
        }
      }
      float rq = 1.f, rk = 1.f;
      if (norm) {
        ssq = wave_sum(ssq);
        ssk = wave_sum(ssk);
        rq = 1.f / sqrtf(ssq / static_cast<float>(N) + a.norm_eps);
        rk = 1.f / sqrtf(ssk / static_cast<float>(N) + a.norm_eps);
      }
      const float sc = F[fo.scale + tt];
      const float ee = F[fo.eend + tt];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int j = lane + 64 * m;
        if (j >= half) continue;
        float a0 = q0[m], a1 = q1[m], c0 = k0[m], c1 = k1[m];
        if (valid) {
          if (norm) {
            const float wq0 = rnd<T>(ldx(a.q_norm_w.ptr, a.q_norm_w.dtype,
                                         e0[m] * a.q_norm_w.stride[0]));
            const float wq1 = rnd<T>(ldx(a.q_norm_w.ptr, a.q_norm_w.dtype,
                                         e1[m] * a.q_norm_w.stride[0]));
            const float wk0 = rnd<T>(ldx(a.k_norm_w.ptr, a.k_norm_w.dtype,
                                         e0[m] * a.k_norm_w.stride[0]));
            const float wk1 = rnd<T>(ldx(a.k_norm_w.ptr, a.k_norm_w.dtype,
                                         e1[m] * a.k_norm_w.stride[0]));
            a0 = rnd<T>(a0 * rq * wq0);
            a1 = rnd<T>(a1 * rq * wq1);
            c0 = rnd<T>(c0 * rk * wk0);
            c1 = rnd<T>(c1 * rk * wk1);
          }
          if (bias) {
            const int64_t bo = h * a.q_bias.stride[0] + r * a.q_bias.stride[1];
            const int64_t bk = h * a.k_bias.stride[0] + r * a.k_bias.stride[1];
            a0 = add_r<T>(a0, rnd<T>(ldx(a.q_bias.ptr, a.q_bias.dtype, bo + e0[m])));
            a1 = add_r<T>(a1, rnd<T>(ldx(a.q_bias.ptr, a.q_bias.dtype, bo + e1[m])));
            c0 = add_r<T>(c0, rnd<T>(ldx(a.k_bias.ptr, a.k_bias.dtype, bk + e0[m])));
            c1 = add_r<T>(c1, rnd<T>(ldx(a.k_bias.ptr, a.k_bias.dtype, bk + e1[m])));
          }
          if (rotate && j < S) {
            const float cc = F[fo.cs + tt * S + j], ss = F[fo.sn + tt * S + j];
            const float ra0 = sub_r<T>(mul_r<T>(a0, cc), mul_r<T>(a1, ss));
            const float ra1 = add_r<T>(mul_r<T>(a0, ss), mul_r<T>(a1, cc));
            const float rc0 = sub_r<T>(mul_r<T>(c0, cc), mul_r<T>(c1, ss));
            const float rc1 = add_r<T>(mul_r<T>(c0, ss), mul_r<T>(c1, cc));
            a0 = ra0; a1 = ra1; c0 = rc0; c1 = rc1;
          }
          if (tgr == L - 1 && a.final_k.ptr != nullptr) {
            T* fk = static_cast<T*>(a.final_k.ptr) + b * a.final_k.stride[0] +
                    h * a.final_k.stride[1] + r * a.final_k.stride[2];
            fk[e0[m]] = from_f<T>(c0);
            fk[e1[m]] = from_f<T>(c1);
          }
        }
        const float ks0 = mul_r<T>(c0, sc), ks1 = mul_r<T>(c1, sc);
        Qs[row * LQ + e0[m]] = from_f<T>(a0);
        Qs[row * LQ + e1[m]] = from_f<T>(a1);
        Ks[row * LQ + e0[m]] = from_f<T>(ks0);
        Ks[row * LQ + e1[m]] = from_f<T>(ks1);
        KeT[e0[m] * LR + row] = from_f<T>(mul_r<T>(ks0, ee));
        KeT[e1[m] * LR + row] = from_f<T>(mul_r<T>(ks1, ee));
      }
    }
    // (4) value / gate rows -> VT, ZT (rank values, activation dtype).
    for (int idx = tid; idx < TOK * P; idx += kThreads) {
      const int tt = idx / P, p = idx - tt * P;
      const int tgr = t0 + tt;
      float v = 0.f, z = 0.f;
      if (tt < width) {
        v = to_f(static_cast<const T*>(a.value.ptr)[b * a.value.stride[0] +
                                                    tgr * a.value.stride[1] +
                                                    h * a.value.stride[2] + p]);
        z = to_f(static_cast<const T*>(a.gate.ptr)[b * a.gate.stride[0] +
                                                   tgr * a.gate.stride[1] +
                                                   h * a.gate.stride[2] + p]);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = tt * R + r;
        VT[p * LR + row] = from_f<T>(R > 1 ? mul_r<T>(v, F[fo.mx + r * P + p]) : v);
        ZT[p * LR + row] = from_f<T>(R > 1 ? mul_r<T>(z, F[fo.mz + r * P + p]) : z);
      }
    }
    // (5) the state at the start of this sub-chunk, rounded to the activation dtype -> Sb[p][n].
#pragma unroll
    for (int k = 0; k < kMaxStateTiles; ++k) {
      const int u = w + kWaves * k;
      if (u < n_tiles) {
        const int ni = u / g.pt, pj = u - ni * g.pt;
        T* dst = Sb + (16 * pj + l16) * LQ + 16 * ni + 4 * lg;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = from_f<T>(st[k][i]);
      }
    }
    __syncthreads();

    // (6) outputs for query row tile `it` and P tiles pj = wp, wp + WPR, ...
    {
      const int it = w / WPR, wp = w - it * WPR;
      const int trow = 16 * it + l16;            // query row in D-layout columns
      const int tq = trow / R;
      const float cum_t = F[fo.cum + tq];
      const float diag_t = F[fo.diag + tq];
      // scores^T tiles (sj <= it): rows s = 16 sj + 4 lg + i, column t = trow
      f4 wsc[RT];
#pragma unroll
      for (int sj = 0; sj < RT; ++sj) {
        wsc[sj] = zero4();
        if (sj > it) continue;
        f4 acc = zero4();
        if constexpr (sizeof(T) == 2) {
          for (int kk = 0; kk < NP; kk += 32) {
            const typename M::v8 av =
                *reinterpret_cast<const typename M::v8*>(Ks + (16 * sj + l16) * LQ + kk + 8 * lg);
            const typename M::v8 bv =
                *reinterpret_cast<const typename M::v8*>(Qs + trow * LQ + kk + 8 * lg);
            acc = M::mma(av, bv, acc);
          }
        } else {
          for (int kk = 0; kk < NP; kk += 4) {
            acc = M::mma(Ks[(16 * sj + l16) * LQ + kk + lg], Qs[trow * LQ + kk + lg], acc);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int srow = 16 * sj + 4 * lg + i;
          const int ts = srow / R;
          const float d = tq > ts ? expf(cum_t - F[fo.cum + ts]) : (tq == ts ? diag_t : 0.f);
          wsc[sj][i] = rnd<T>(acc[i] * d);
        }
      }
      for (int pj = wp; pj < g.pt; pj += WPR) {
        const int pcol = 16 * pj + l16;
        f4 yi = zero4(), ye = zero4();
        // intra: W V with the K axis permuted as the D-layout of wsc
        if constexpr (sizeof(T) == 2) {
#pragma unroll
          for (int m = 0; m < (RT + 1) / 2; ++m) {
            if (2 * m > it) continue;
            typename M::v8 av;
            const typename M::v4 b0 =
                *reinterpret_cast<const typename M::v4*>(VT + pcol * LR + 32 * m + 4 * lg);
            const typename M::v4 b1 =
                *reinterpret_cast<const typename M::v4*>(VT + pcol * LR + 32 * m + 16 + 4 * lg);
            typename M::v8 bv;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              av[i] = from_f<T>(wsc[2 * m][i]);
              av[4 + i] = (2 * m + 1 < RT) ? from_f<T>(wsc[2 * m + 1][i]) : from_f<T>(0.f);
              bv[i] = b0[i];
              bv[4 + i] = b1[i];
            }
            yi = M::mma(av, bv, yi);
          }
          for (int kk = 0; kk < NP; kk += 32) {
            const typename M::v8 av =
                *reinterpret_cast<const typename M::v8*>(Qs + (16 * it + l16) * LQ + kk + 8 * lg);
            const typename M::v8 bv =
                *reinterpret_cast<const typename M::v8*>(Sb + pcol * LQ + kk + 8 * lg);
            ye = M::mma(av, bv, ye);
          }
        } else {
#pragma unroll
          for (int sj = 0; sj < RT; ++sj) {
            if (sj > it) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              yi = M::mma(wsc[sj][i], VT[pcol * LR + 16 * sj + 4 * lg + i], yi);
            }
          }
          for (int kk = 0; kk < NP; kk += 4) {
            ye = M::mma(Qs[(16 * it + l16) * LQ + kk + lg], Sb[pcol * LQ + kk + lg], ye);
          }
        }
        // epilogue: rows 16 it + 4 lg + i, column pcol
        if (pcol < P) {
          float y = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int row = 16 * it + 4 * lg + i;
            const int tt = row / R, r = row - tt * R;
            const float v = to_f(VT[pcol * LR + row]);
            const float z = to_f(ZT[pcol * LR + row]);
            float yr = (ye[i] * F[fo.ecum + tt] + yi[i] + Dh * v) * siluf(z);
            if (R > 1) yr *= F[fo.mo + r * P + pcol];
            y = (R > 1 && r > 0) ? y + yr : yr;
            if (r == R - 1 && tt < width) {
              static_cast<T*>(a.out.ptr)[b * a.out.stride[0] + (t0 + tt) * a.out.stride[1] +
                                         h * a.out.stride[2] + pcol] = from_f<T>(y);
            }
          }
        }
      }
    }

    // (7) state carry: S^T = exp(cum_last) S^T + Ke^T V
    {
      const float ecl = F[fo.ecl];
#pragma unroll
      for (int k = 0; k < kMaxStateTiles; ++k) {
        const int u = w + kWaves * k;
        if (u >= n_tiles) continue;
        const int ni = u / g.pt, pj = u - ni * g.pt;
        f4 acc = zero4();
        if constexpr (sizeof(T) == 2) {
#pragma unroll
          for (int kk = 0; kk < ROWS; kk += 32) {
            const typename M::v8 av =
                *reinterpret_cast<const typename M::v8*>(KeT + (16 * ni + l16) * LR + kk + 8 * lg);
            const typename M::v8 bv =
                *reinterpret_cast<const typename M::v8*>(VT + (16 * pj + l16) * LR + kk + 8 * lg);
            acc = M::mma(av, bv, acc);
          }
        } else {
#pragma unroll
          for (int kk = 0; kk < ROWS; kk += 4) {
            acc = M::mma(KeT[(16 * ni + l16) * LR + kk + lg], VT[(16 * pj + l16) * LR + kk + lg],
                         acc);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) st[k][i] = ecl * st[k][i] + acc[i];
      }
    }
    __syncthreads();
  }

  // ---- final state
#pragma unroll
  for (int k = 0; k < kMaxStateTiles; ++k) {
    const int u = w + kWaves * k;
    if (u >= n_tiles) continue;
    const int ni = u / g.pt, pj = u - ni * g.pt;
    const int p = 16 * pj + l16;
    if (p >= P) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = 16 * ni + 4 * lg + i;
      if (n < N) {
        static_cast<float*>(a.final_state.ptr)[b * a.final_state.stride[0] +
                                               h * a.final_state.stride[1] +
                                               p * a.final_state.stride[2] + n] = st[k][i];
      }
    }
  }
}

// ------------------------------------------------------------------ host side

template <typename T>
static ScanGeom make_geom(const m3_scan_args& a) {
  using M = Mma<T>;
  ScanGeom g{};
  const int es = sizeof(T);
  g.n_pad = (a.d_state + 31) / 32 * 32;
  g.p_pad = (a.head_dim + 15) / 16 * 16;
  g.lq = g.n_pad + M::PAD;
  g.lr = M::ROWS + M::PAD;
  g.tok = M::ROWS / a.rank;
  g.nt = g.n_pad / 16;
  g.pt = g.p_pad / 16;
  const int total = a.batch * a.heads;
  g.xcd_map = (total % 8 == 0) ? 1 : 0;
  auto al = [](int x) { return (x + 15) / 16 * 16; };
  g.o_qs = 0;
  g.o_ks = al(g.o_qs + M::ROWS * g.lq * es);
  g.o_ket = al(g.o_ks + M::ROWS * g.lq * es);
  g.o_vt = al(g.o_ket + g.n_pad * g.lr * es);
  g.o_zt = al(g.o_vt + g.p_pad * g.lr * es);
  g.o_sb = al(g.o_zt + g.p_pad * g.lr * es);
  g.o_f = al(g.o_sb + g.p_pad * g.lq * es);
  g.bytes = g.o_f + 4 * f_floats(g.tok, a.num_angles, a.rank, a.head_dim);
  return g;
}

template <typename T, int R>
static int launch_scan_r(const m3_scan_args& a, hipStream_t stream) {
  const ScanGeom g = make_geom<T>(a);
  if (g.nt * g.pt > kWaves * kMaxStateTiles) {
    return fail(M3_EUNSUPPORTED, "m3_scan_fwd: d_state x head_dim too large for the state tiles");
  }
  if (g.bytes > 160 * 1024) {
    return fail(M3_EUNSUPPORTED, "m3_scan_fwd: shape needs %d bytes of LDS", g.bytes);
  }
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_kernel<T, R>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) {
      return fail(M3_ELAUNCH, "m3_scan_fwd: hipFuncSetAttribute: %s", hipGetErrorString(e));
    }
    attr_set = true;
  }
  const dim3 grid(static_cast<unsigned>(a.batch) * a.heads), block(kThreads);
  hipLaunchKernelGGL((scan_kernel<T, R>), grid, block, g.bytes, stream, a, g);
  return check_launch("m3_scan_fwd");
}

template <typename T>
static int launch_scan(const m3_scan_args& a, hipStream_t stream) {
  switch (a.rank) {
    case 1: return launch_scan_r<T, 1>(a, stream);
    case 2: return launch_scan_r<T, 2>(a, stream);
    case 4: return launch_scan_r<T, 4>(a, stream);
    default: return fail(M3_EUNSUPPORTED, "m3_scan_fwd: rank %d not in {1, 2, 4}", a.rank);
  }
}

static bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

static int validate_scan(const m3_scan_args& a) {
  if (a.batch < 0 || a.length < 0 || a.heads <= 0 || a.groups <= 0 || a.rank <= 0 ||
      a.d_state <= 0 || a.head_dim <= 0 || a.num_angles < 0) {
    return fail(M3_EINVAL, "m3_scan_fwd: invalid dimensions");
  }
  if (a.heads % a.groups != 0) return fail(M3_EINVAL, "m3_scan_fwd: heads %% groups != 0");
  if (!valid_dtype(a.act_dtype)) return fail(M3_EINVAL, "m3_scan_fwd: invalid act_dtype");
  if (!pow2(a.d_state) || a.d_state < 4 || a.d_state > 256) {
    return fail(M3_EUNSUPPORTED, "m3_scan_fwd: d_state %d must be a power of 2 in [4, 256]",
                a.d_state);
  }
  if (a.phase_mode < M3_PHASE_NONE || a.phase_mode > M3_PHASE_ANGLES) {
    return fail(M3_EINVAL, "m3_scan_fwd: invalid phase_mode");
  }
  if (a.phase_mode != M3_PHASE_NONE &&
      (a.mimo_rotation ? 4 * a.num_angles != a.d_state : 2 * a.num_angles > a.d_state)) {
    return fail(M3_EUNSUPPORTED, "m3_scan_fwd: num_angles %d does not fit d_state %d (mimo=%d)",
                a.num_angles, a.d_state, a.mimo_rotation);
  }
  const int act = a.act_dtype, N = a.d_state, P = a.head_dim;
  const bool angles = a.phase_mode == M3_PHASE_ANGLES;
  int rc;
  if ((rc = check_tensor(a.q, "q", 5, N, true, act)) ||
      (rc = check_tensor(a.k, "k", 5, N, true, act)) ||
      (rc = check_tensor(a.q_norm_w, "q_norm_w", 1, N, false, -1)) ||
      (rc = check_tensor(a.k_norm_w, "k_norm_w", 1, N, a.q_norm_w.ptr != nullptr, -1)) ||
      (rc = check_tensor(a.q_bias, "q_bias", 3, N, false, -1)) ||
      (rc = check_tensor(a.k_bias, "k_bias", 3, N, a.q_bias.ptr != nullptr, -1)) ||
      (rc = check_tensor(a.value, "value", 4, P, true, act)) ||
      (rc = check_tensor(a.gate, "gate", 4, P, true, act)) ||
      (rc = check_tensor(a.dt, "dt", 3, 1, true, -1)) ||
      (rc = check_tensor(a.a, "a", 3, 1, true, -1)) ||
      (rc = check_tensor(a.dt_bias, "dt_bias", 1, 1, a.raw_dt != 0, -1)) ||
      (rc = check_tensor(a.trap, "trap", 3, 1, true, -1)) ||
      (rc = check_tensor(a.phase, "phase", angles ? 3 : 4, 1, a.phase_mode != M3_PHASE_NONE,
                         a.phase_mode == M3_PHASE_GIVEN ? M3_F32 : -1)) ||
      (rc = check_tensor(a.initial_phase, "initial_phase", 3, 1, false, M3_F32)) ||
      (rc = check_tensor(a.D, "D", 1, 1, true, -1)) ||
      (rc = check_tensor(a.mimo_x, "mimo_x", 3, P, a.rank > 1, -1)) ||
      (rc = check_tensor(a.mimo_z, "mimo_z", 3, P, a.rank > 1, -1)) ||
      (rc = check_tensor(a.mimo_out, "mimo_out", 3, P, a.rank > 1, -1)) ||
      (rc = check_tensor(a.initial_state, "initial_state", 4, N, false, M3_F32)) ||
      (rc = check_tensor(a.initial_k, "initial_k", 4, N, false, act)) ||
      (rc = check_tensor(a.initial_value, "initial_value", 3, P, a.initial_k.ptr != nullptr,
                         act)) ||
      (rc = check_tensor(a.out, "out", 4, P, true, act)) ||
      (rc = check_tensor(a.final_state, "final_state", 4, N, true, M3_F32)) ||
      (rc = check_tensor(a.final_phase, "final_phase", 3, 1, false, M3_F32)) ||
      (rc = check_tensor(a.final_k, "final_k", 4, N, false, act))) {
    return rc;
  }
  if ((a.q_norm_w.ptr == nullptr) != (a.k_norm_w.ptr == nullptr) ||
      (a.q_bias.ptr == nullptr) != (a.k_bias.ptr == nullptr)) {
    return fail(M3_EINVAL, "m3_scan_fwd: q/k norm weights and biases come in pairs");
  }
  if (a.final_phase.ptr != nullptr && !angles) {
    return fail(M3_EINVAL, "m3_scan_fwd: final_phase needs phase_mode ANGLES");
  }
  return M3_OK;
}

}  // namespace m3

extern "C" int m3_scan_workspace_size(const m3_scan_args* args, size_t* bytes) {
  m3::clear_error();
  if (args == nullptr || bytes == nullptr) return m3::fail(M3_EINVAL, "NULL argument");
  *bytes = 0;
  return M3_OK;
}

extern "C" int m3_scan_fwd(const m3_scan_args* args, hipStream_t stream) {
  using namespace m3;
  clear_error();
  if (args == nullptr) return fail(M3_EINVAL, "m3_scan_fwd: args is NULL");
  const m3_scan_args& a = *args;
  int rc = validate_scan(a);
  if (rc != M3_OK) return rc;
  if (a.batch == 0) return M3_OK;
  switch (a.act_dtype) {
    case M3_F32: return launch_scan<float>(a, stream);
    case M3_BF16: return launch_scan<__bf16>(a, stream);
    default: return launch_scan<_Float16>(a, stream);
  }
}

// ------------------------------------------------------------------ standalone chunk state

namespace m3 {

constexpr int kCsRows = 64;   // rows staged in LDS per pass
constexpr int kCsMaxE = 64;   // state elements per thread (P * N <= 16384)

// One chunk's state update (_triton.py:294-413) with the portable path's rounding points:
// ke = rnd(rnd(k * rnd(scale)) * rnd(exp(cum_last - cum))); S' = exp(cum_last) S + V^T ke.
template <typename T>
__global__ __launch_bounds__(kThreads) void chunk_state_kernel(const m3_chunk_state_args a) {
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
    for (int idx = tid; idx < kCsRows * N; idx += kThreads) {
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
    for (int idx = tid; idx < kCsRows * P; idx += kThreads) {
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
      const int e = tid + kThreads * i;
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
    const int e = tid + kThreads * i;
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
  if (a.d_state * a.head_dim > kThreads * kCsMaxE) {
    return fail(M3_EUNSUPPORTED, "m3_chunk_state: d_state x head_dim > %d", kThreads * kCsMaxE);
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
  const dim3 grid(static_cast<unsigned>(a.batch) * a.heads), block(kThreads);
  switch (act) {
    case M3_F32: hipLaunchKernelGGL(chunk_state_kernel<float>, grid, block, lds, stream, a); break;
    case M3_BF16: hipLaunchKernelGGL(chunk_state_kernel<__bf16>, grid, block, lds, stream, a); break;
    default: hipLaunchKernelGGL(chunk_state_kernel<_Float16>, grid, block, lds, stream, a); break;
  }
  return check_launch("m3_chunk_state");
}
