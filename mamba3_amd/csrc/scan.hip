// Chunked Mamba-3 SSD for CDNA4 (gfx950).
//
// Two launches per call:
//   prep_kernel  head-independent per-token work, once per token instead of once per head:
//                the RMSNorm factors of the raw B / C rows (model.py:190-191) and
//                pi * tanh(angle) of the phase increments (model.py:225-228), into a workspace.
//   scan_kernel  one persistent workgroup (8 waves) per (batch, head) walks the sequence in
//                sub-chunks of ROWS flattened (token, rank) rows. The FP32 state lives in MFMA
//                accumulator registers for the whole sequence (stored transposed, S^T [N, P],
//                as 16x16 tiles spread over the waves), so the per-chunk state update that the
//                reference launches once per chunk (_triton.py:294-413 from ops.py:444-504) is
//                fused and the state never round-trips through HBM.
//
// Per sub-chunk of scan_kernel (the global loads of sub-chunk c+1 are issued into registers
// before the MFMA work of sub-chunk c, so their latency hides behind it):
//   scalars  dt, adt, trap from the raw projection or given (model.py:195-198), the
//            exp-trapezoid gamma and scale (ops.py:659-671), within-chunk cumsum of adt.
//   phase    bounded phase (model.py:215-256): 64-token blocks of fmod-reduced increments with
//            an fmod-reduced carry, 4 tokens per lane plus a cross-lane scan; cos / sin.
//   q / k    RMSNorm, head bias, rotation (ops.py:35-84, 700-714) -> Q, K (row-major) and K^T.
//   v / z    rank values v * mimo_x, z * mimo_z, and v * scale * end_decay -> V^T, Vs^T, Z^T.
//   scores   Sc^T = K Q^T                                  (MFMA, FP32 accumulate) ops.py:763
//   weights  W = rnd(Sc * d), d[t,s] = scale_s exp(cum_t - cum_s) for s < t, gamma_t at s = t:
//            the reference's K * scale and diagonal gamma / scale fold (ops.py:743, 770-787).
//   intra    W V   (W stays in registers: the K axis is permuted alike in both operands)
//   inter    Q rnd(S)^T * exp(cum)                                               ops.py:753
//   epilogue (inter + intra + D v) silu(z), MIMO rank sum                    ops.py:792-802
//   carry    S^T = exp(cum_last) S^T + K^T Vs                                ops.py:806-816
//
// Products and sums are evaluated in FP32 and rounded to the activation dtype once, where the
// data become MFMA operands; the reference rounds some intermediates (bias add, rotation,
// k * scale) separately in the activation dtype.
//
// Replaces ops._fused_chunk_scan (ops.py:253-367) / its driver (ops.py:370-505) and the Triton
// kernels _chunk_main_kernel (_triton.py:74-291) and _chunk_state_kernel (_triton.py:294-413);
// the same kernel serves the portable entry ops.mamba3_scan (ops.py:544-822).
#include "m3_common.hpp"
#include "m3_host.hpp"
#include "m3_math.h"

#include <algorithm>
#include <type_traits>

namespace m3 {

constexpr int kThreads = 512;
constexpr int kWaves = 8;
constexpr int kTiles = 4;  // 16x16 state tiles per wave (N_pad * P_pad <= 128 * 64)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// MFMA policy per activation type: 16-bit types use 16x16x32 (K = 32, 8 elements per lane),
// FP32 uses 16x16x4 (K = 4, one element per lane). ROWS is the sub-chunk height.
template <typename T> struct Mma;
template <> struct Mma<__bf16> {
  static constexpr int ROWS = 64, PAD = 8;
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  typedef bf16x2 v2;
  static __device__ __forceinline__ f4 mma(v8 a, v8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<_Float16> {
  static constexpr int ROWS = 64, PAD = 8;
  typedef f16x8 v8;
  typedef f16x4 v4;
  typedef f16x2 v2;
  static __device__ __forceinline__ f4 mma(v8 a, v8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<float> {
  static constexpr int ROWS = 32, PAD = 4;
  typedef float v8;  // unused: FP32 operands are single elements
  typedef f4 v4;
  typedef f32x2 v2;
  static __device__ __forceinline__ f4 mma(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

// Compile-time LDS layout. Operand tiles are padded to N = 128 and P = 64 (the largest shapes
// the kernel takes; every Mamba3 configuration has P <= 64), so every offset and loop bound is a
// constant; smaller shapes run on zero padding.
constexpr int kNPad = 128, kPPad = 64, kSMax = 32, kRMax = 8;
constexpr int kNT = kNPad / 16, kPT = kPPad / 16;  // 16-row tiles of N and P

template <typename T> struct Layout {
  static constexpr int ROWS = Mma<T>::ROWS, PAD = Mma<T>::PAD, ES = sizeof(T);
  static constexpr int LQ = kNPad + PAD;   // row stride (elements) of Qs, Ks, Sb
  static constexpr int LR = ROWS + PAD;    // row stride (elements) of KT, VT
  static constexpr int LP = kPPad + PAD;   // row stride (elements) of VR, ZR
  static constexpr int al(int x) { return (x + 15) / 16 * 16; }
  static constexpr int QS = 0;
  static constexpr int KS = al(QS + ROWS * LQ * ES);
  static constexpr int KT = al(KS + ROWS * LQ * ES);
  static constexpr int VT = al(KT + kNPad * LR * ES);
  static constexpr int VR = al(VT + kPPad * LR * ES);
  static constexpr int ZR = al(VR + ROWS * LP * ES);
  static constexpr int SB = al(ZR + ROWS * LP * ES);
  static constexpr int FB = al(SB + kPPad * LQ * ES);
  // float scratch, offsets in floats from FB, sized for TM = ROWS tokens (rank 1): two side
  // blocks alternating (a sub-chunk's scalar block, ScBlk, then the (q, k) RMSNorm factors of
  // its rows), the angle tile, two cos / sin tables ([token][angle][cos, sin], token stride CST
  // for 16-byte aligned rows)
  static constexpr int TM = ROWS;
  static constexpr int SCB = 5 * TM + 8 + 2 * ROWS, SC0 = 0;
  static constexpr int ANG = SC0 + 2 * SCB;  // [TM / 4][kSMax][4]
  static constexpr int CST = 2 * kSMax + 4, CSB = TM * CST;
  static constexpr int CS0 = ANG + TM * kSMax, PBASE = CS0 + 2 * CSB;
  static constexpr int POFF = PBASE + kSMax, MX = POFF + kSMax, MZ = MX + kRMax * kPPad;
  static constexpr int MO = MZ + kRMax * kPPad;
  static constexpr int BYTES = FB + 4 * (MO + kRMax * kPPad);
};

// Per-token scalar block of one sub-chunk of TOK tokens (floats, token-indexed arrays): dt, the
// within-chunk cumsum of adt, the exp-trapezoid scale, gamma, scale * decay to the end of the
// token's 16-row tile; then the cumsum at each tile end, exp of the last cumsum and the last
// cumsum itself. The prep pass writes them; the scan copies them to LDS (and takes exp(cum) and
// scale * exp(cum_last - cum) from them itself, an exp per lane).
template <int TOK> struct ScBlk {
  static constexpr int DTV = 0, CUM = TOK, SCL = 2 * TOK, GAM = 3 * TOK, BSC = 4 * TOK;
  static constexpr int CEND = 5 * TOK, ECL = 5 * TOK + 4, CL = 5 * TOK + 5;
  static constexpr int SIZE = 5 * TOK + 8;
};

// Per-launch values shared by host and device.
struct ScanGeom {
  int xcd_map;           // 1: map blocks so each XCD holds consecutive (b, h)
  int vec_qk, vec_vz;    // 1: q/k rows and v/z rows may be loaded with 16 / 8-byte vectors
  int vec_nw;            // 1: both norm weights unit-stride and 8-byte aligned (4-element loads)
  int norm_factors;      // 1: prep stores the RMSNorm factors (every scan kernel but the 16-wave
                         // one, which reads the normalized rows instead)
  // prep workspace, float offsets of its regions (-1: absent): RMSNorm factors [B][L][G*R][2]
  // (q, k), pi tanh(angle) [B][L4][S][4] (4 consecutive tokens of one angle together, L4 =
  // ceil(L / 4)), scalar blocks [B*H][nsub][scw] of `tok`-token sub-chunks
  int64_t ws_norm, ws_ang, ws_sc;
  int L4, tok, nsub, scw;
  int ws_bytes;  // workspace bytes when below 2^31 (the projection form addresses it in 32 bits)
  // the model's 16-bit shape at ranks 1 and 4 (scan16_kernel): the RMS-normalized q / k rows
  // [B][L][R][2][N] in the activation dtype, after the regions above (byte offset, -1: absent)
  // and their bytes when below 2^31 (read through a buffer resource of their own)
  int64_t ws_qk;
  int qk_bytes;
  // projection form (the full-shape kernel): q, k, value, gate, dt, a, trap are slices of one
  // projection row; byte offsets of each slice from `proj`, the batch / token strides and the
  // group / rank / head strides of the slices, in bytes
  const char* proj;
  int64_t proj_b, out_b;
  int tok_b, o_q, o_k, o_v, o_z, o_dt, o_a, o_tr, qk_g, qk_r, vz_h, sc_h, out_t, out_h;
  // the output's physical start and the offset of logical token 0 from it (non-zero when the
  // call runs backwards: token strides < 0, logical token t at physical token L - 1 - t)
  const char* out_base;
  int out_o0;
};

__device__ __forceinline__ f4 zero4() {
  f4 z;
  z[0] = z[1] = z[2] = z[3] = 0.f;
  return z;
}

template <typename T>
__device__ __forceinline__ T* lds_t(char* base, int off) {
  return reinterpret_cast<T*>(base + off);
}

// ------------------------------------------------------------------ raw register tiles

// Activation elements held as raw bits until they are used: W8 words hold 8 elements,
// W4 words hold 4 (two 16-bit elements per word, or one FP32 element per word).
template <typename T> struct Words {
  static constexpr int W8 = sizeof(T) == 4 ? 8 : 4;
  static constexpr int W4 = sizeof(T) == 4 ? 4 : 2;
};

__device__ __forceinline__ float bits_to_f(uint32_t bits16, __bf16*) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float bits_to_f(uint32_t bits16, _Float16*) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

template <typename T, int NW>
__device__ __forceinline__ float raw_get(const uint32_t (&w)[NW], int i) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(w[i]);
  } else {
    const uint32_t x = w[i >> 1];
    return bits_to_f((i & 1) ? (x >> 16) : (x & 0xffffu), static_cast<T*>(nullptr));
  }
}

template <typename T>
__device__ __forceinline__ uint32_t elem_bits(const T* p) {
  if constexpr (sizeof(T) == 4) {
    return __float_as_uint(*p);
  } else {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, *p));
  }
}

// Load up to E elements (n valid, the rest zero) into raw words; one vector load when `vec`
// and all E are valid (16 bytes, or 8 bytes for four 16-bit elements).
template <typename T, int E, int NW>
__device__ __forceinline__ void load_words(uint32_t (&w)[NW], const T* p, int n, bool vec) {
  if (vec && n >= E) {
    if constexpr (NW == 2) {
      const uint2 q = *reinterpret_cast<const uint2*>(p);
      w[0] = q.x; w[1] = q.y;
    } else {
#pragma unroll
      for (int j = 0; j < NW; j += 4) {
        const uint4 q = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint32_t*>(p) + j);
        w[j] = q.x; w[j + 1] = q.y; w[j + 2] = q.z; w[j + 3] = q.w;
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NW; ++j) w[j] = 0u;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    if (i < n) {
      const uint32_t e = elem_bits(p + i);
      if constexpr (sizeof(T) == 4) {
        w[i] = e;
      } else {
        w[i >> 1] |= e << (16 * (i & 1));
      }
    }
  }
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Two values rounded to a 16-bit type (round to nearest even) and packed into one word, a
// first: one packed convert for bf16.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  typedef T t2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, t2));
}

// Two adjacent activation values stored with one LDS write.
template <typename T>
__device__ __forceinline__ void st_pair(T* dst, float a, float b) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<f32x2*>(dst) = (f32x2){a, b};
  } else {
    *reinterpret_cast<uint32_t*>(dst) = pack2<T>(a, b);
  }
}

// Four adjacent activation values stored with one LDS write.
template <typename T>
__device__ __forceinline__ void st_quad(T* dst, f4 x) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<f4*>(dst) = x;
  } else {
    *reinterpret_cast<u32x2*>(dst) = (u32x2){pack2<T>(x[0], x[1]), pack2<T>(x[2], x[3])};
  }
}

template <typename T>
__device__ __forceinline__ void st_row8(T* dst, const float* x) {
  if constexpr (sizeof(T) == 4) {
    f4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) { a[i] = x[i]; b[i] = x[4 + i]; }
    reinterpret_cast<f4*>(dst)[0] = a;
    reinterpret_cast<f4*>(dst)[1] = b;
  } else {
    *reinterpret_cast<u32x4*>(dst) = (u32x4){pack2<T>(x[0], x[1]), pack2<T>(x[2], x[3]),
                                             pack2<T>(x[4], x[5]), pack2<T>(x[6], x[7])};
  }
}

// ------------------------------------------------------------------ scan

// Wave-level scans with DPP row shifts (no LDS traffic). row_shr:n = 0x110 + n; lanes whose
// source lies before their 16-lane row read 0.
template <int CTRL>
__device__ __forceinline__ float dpp_shr(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               CTRL, 0xf, 0xf, true));
}

// Inclusive scan within aligned segments of SEG lanes (SEG a power of 2, <= 16). For SEG = 16
// the segment is the DPP row, whose shifts already read 0 before the row's first lane (the
// same +0 the masks add), so no mask is applied.
template <int SEG>
__device__ __forceinline__ float seg_incl_scan(float x, int lane) {
  const int j = lane & (SEG - 1);
  constexpr bool ROW = SEG == 16;
  if constexpr (SEG > 1) { const float u = dpp_shr<0x111>(x); x += (ROW || j >= 1) ? u : 0.f; }
  if constexpr (SEG > 2) { const float u = dpp_shr<0x112>(x); x += (ROW || j >= 2) ? u : 0.f; }
  if constexpr (SEG > 4) { const float u = dpp_shr<0x114>(x); x += (ROW || j >= 4) ? u : 0.f; }
  if constexpr (SEG > 8) { const float u = dpp_shr<0x118>(x); x += (ROW || j >= 8) ? u : 0.f; }
  return x;
}

// Sum over each 16-lane row, in every lane of the row: DPP row rotations by 8, 4, 2 and 1.
__device__ __forceinline__ float row16_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128,
                                                             0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124,
                                                             0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x122,
                                                             0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x121,
                                                             0xf, 0xf, false));
  return x;
}

__device__ __forceinline__ float readlane_f(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

// Inclusive scan over the 64 lanes of a wave.
__device__ __forceinline__ float wave_incl_scan(float x, int lane) {
  x = seg_incl_scan<16>(x, lane);
  const float r0 = readlane_f(x, 15), r1 = readlane_f(x, 31), r2 = readlane_f(x, 47);
  const int row = lane >> 4;
  x += row >= 1 ? r0 : 0.f;
  x += row >= 2 ? r1 : 0.f;
  x += row >= 3 ? r2 : 0.f;
  return x;
}

// Transposed operand tiles ([n or p][row]) XOR-swizzle their 8-row groups by a key taken from
// the tile row (n or p) so that the column-wise stores of the staging spread over the LDS banks;
// every reader applies the same swizzle. Groups of 8 (16-bit: 16 bytes) stay contiguous.
template <int ROWS>
__device__ __forceinline__ int swz(int row, int key) {
  return row ^ (8 * (key & (ROWS / 8 - 1)));
}

// Column col of row row of the Ks tile when swizzled: its 16-byte chunk c sits at c ^ 2 (row & 3)
// (16-bit). The scores' reads of one chunk in 16 consecutive rows (rows 272 bytes apart) still
// cover 16 bank groups, and the carry's transposing reads of 4 rows x 32 bytes no longer overlap.
template <bool PLAIN>
__device__ __forceinline__ int ks_col(int row, int col) {
  if constexpr (PLAIN) {
    return col;
  } else {
    return (((col >> 3) ^ (2 * (row & 3))) << 3) | (col & 7);
  }
}

// Buffer resource over `bytes` bytes from `base` (raw, stride 0): loads at offsets beyond the
// extent return zero, stores there are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), bytes,
                                           0x00020000);
}

// NW raw words (NW in {2, 4, 8}) from a buffer at byte offset `off`.
template <int NW>
__device__ __forceinline__ void bload_words(uint32_t (&w)[NW], __amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (NW == 2) {
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
    w[0] = v[0];
    w[1] = v[1];
  } else {
#pragma unroll
    for (int j = 0; j < NW; j += 4) {
      const u32x4 v =
          __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 4 * j, 0, 0));
      w[j] = v[0];
      w[j + 1] = v[1];
      w[j + 2] = v[2];
      w[j + 3] = v[3];
    }
  }
}

__device__ __forceinline__ float bload_f32(__amdgpu_buffer_rsrc_t r, int off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Four consecutive activation values stored as one vector (8 bytes for 16-bit types).
template <typename T>
__device__ __forceinline__ void bstore_quad(f4 x, __amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), r, off, 0, 0);
  } else {
    typename Mma<T>::v4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = from_f<T>(x[i]);
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, 0);
  }
}

// Global reads of one (batch, head). Per sub-chunk: the q / k and value / gate words of each
// lane's rows, and the side data the block stages through LDS: its scalar block followed by the
// RMSNorm factors of its rows (SIDE floats, one 8-byte word per lane) and its angle tile (4
// consecutive tokens of one angle per 16-byte word, TOK * S floats). FULL: every per-token input
// is a slice of one projection row (host-checked), read at per-lane byte offsets through one
// buffer resource per batch row whose extent ends at token L, so rows of tokens >= L read as
// zero without guards; the workspace likewise through one resource. BUF (the model's shape with
// the generic inputs, host-checked): the same guard-free reads through one resource per input
// tensor and (batch, head), whose extent ends at token L, at 32-bit per-lane offsets. Otherwise
// element pointers with explicit guards.
template <typename T, int R, bool FULL, bool BUF = false>
struct Feed {
  static constexpr int ES = sizeof(T), W8 = Words<T>::W8, W4 = Words<T>::W4;
  static constexpr int ROWS = Mma<T>::ROWS, TOK = ROWS / R;
  static constexpr int VJ = R == 1 ? 2 : 1;  // value / gate tokens per lane
  // FULL
  __amdgpu_buffer_rsrc_t rs_p, rs_w;
  int o_qk, o_vz, d_q1, d_k, d_z, tok_b;  // per-lane byte offsets at token 0, uniform deltas
  int d_hi = 8;  // MIMO projection form: byte offset of a row's second 4-column chunk
  int side_o, side_s, ang_o, ang_s;        // per-lane workspace byte offsets at sub-chunk 0, strides
  // BUF: resources of q, k, value, gate and the given phases; per-lane byte offsets at token 0,
  // the byte strides of a token and the second row's delta
  __amdgpu_buffer_rsrc_t rs_q, rs_k, rs_v, rs_z, rs_x;
  int o_q, o_k, o_v, o_z, o_x, tq_b, tk_b, tv_b, tz_b, tx_b, d_q2, d_k2;
  // generic
  const T *q_row, *k_row, *v_row, *z_row;
  const float *side_p, *ang_p;  // this lane's side / angle word at sub-chunk 0 (null: none)
  const float* ph_row;          // given phases of (b, h): [L][S] with strides ph_t, ph_s
  int64_t side_ps, ang_ps;      // per-sub-chunk strides (floats)
  int q_t, q_r, k_t, k_r, v_t, z_t, ph_t, ph_s, qk_n, vz_n;
  int side_tok, side_lim;       // norm words: token of the word (sub-chunk 0), last valid
  bool vec_qk, vec_vz, given;
  int rp, vp, nsub, L, S, L4;

  __device__ __forceinline__ void init(const m3_scan_args& a, const ScanGeom& g,
                                       const float* prep, int b, int h, int grp, int rp_,
                                       int n0, int vp_, int p0, int N, int P, bool norm) {
    L = a.length;
    S = a.num_angles;
    L4 = g.L4;
    rp = rp_;
    vp = vp_;
    nsub = g.nsub;
    const int GR = a.groups * a.rank, H = a.heads, tid = threadIdx.x;
    const int tt0 = (2 * rp) / R, r0 = (2 * rp) % R;
    const int scw = g.scw;
    // side word of this lane: floats 2 tid, 2 tid + 1 of [scalar block (scw) | norms (2 ROWS)]
    const int q2 = 2 * tid;
    const int64_t sc0 = g.ws_sc + static_cast<int64_t>(b * H + h) * nsub * scw + q2;
    const int nrow = (q2 - scw) >> 1;  // norm word: row of the sub-chunk (token nrow / R)
    if constexpr (FULL) {
      tok_b = g.tok_b;
      rs_p = make_rsrc(g.proj + b * g.proj_b, L * (tok_b < 0 ? -tok_b : tok_b));
      rs_w = make_rsrc(prep, g.ws_bytes);
      o_qk = g.o_q + grp * g.qk_g + r0 * g.qk_r + tt0 * tok_b + n0 * ES;
      o_vz = g.o_v + h * g.vz_h + (R == 1 ? 2 * vp : (2 * vp) / R) * tok_b + p0 * ES;
      d_q1 = R == 1 ? tok_b : g.qk_r;  // row 2rp + 1: the next token (R = 1) or the next rank
      d_k = g.o_k - g.o_q;
      d_z = g.o_z - g.o_v;
      // groups == 1: the norm pairs of a sub-chunk's rows are 2 ROWS contiguous floats
      if (q2 < scw) {
        side_o = static_cast<int>(sc0) * 4;
        side_s = scw * 4;
      } else if (q2 < scw + 2 * ROWS) {
        side_o = static_cast<int>(g.ws_norm + static_cast<int64_t>(b) * L * GR * 2 + q2 - scw) * 4;
        side_s = TOK * GR * 2 * 4;
      } else {
        side_o = side_s = 0;
      }
      ang_o = static_cast<int>(g.ws_ang + static_cast<int64_t>(b) * g.L4 * S * 4 + 4 * tid) * 4;
      ang_s = (TOK / 4) * S * 16;
    } else if constexpr (BUF) {
      rs_w = make_rsrc(prep, g.ws_bytes);
      // every token stride is positive and a token's row ends below the next token's (host),
      // so rows of tokens >= L lie past the extent L * stride and read as zero
      const char* q0 = static_cast<const char*>(a.q.ptr) + b * a.q.stride[0] * ES;
      const char* k0 = static_cast<const char*>(a.k.ptr) + b * a.k.stride[0] * ES;
      const char* v0 = static_cast<const char*>(a.value.ptr) +
                       (b * a.value.stride[0] + h * a.value.stride[2]) * ES;
      const char* z0 = static_cast<const char*>(a.gate.ptr) +
                       (b * a.gate.stride[0] + h * a.gate.stride[2]) * ES;
      tq_b = static_cast<int>(a.q.stride[1]) * ES;
      tk_b = static_cast<int>(a.k.stride[1]) * ES;
      tv_b = static_cast<int>(a.value.stride[1]) * ES;
      tz_b = static_cast<int>(a.gate.stride[1]) * ES;
      rs_q = make_rsrc(q0, L * tq_b);
      rs_k = make_rsrc(k0, L * tk_b);
      rs_v = make_rsrc(v0, L * tv_b);
      rs_z = make_rsrc(z0, L * tz_b);
      const int qr_b = static_cast<int>(a.q.stride[3]) * ES, kr_b = static_cast<int>(a.k.stride[3]) * ES;
      o_q = tt0 * tq_b + r0 * qr_b + n0 * ES;
      o_k = tt0 * tk_b + r0 * kr_b + n0 * ES;
      d_q2 = R == 1 ? tq_b : qr_b;  // row 2rp + 1: the next token (R = 1) or the next rank
      d_k2 = R == 1 ? tk_b : kr_b;
      const int tv = R == 1 ? 2 * vp : (2 * vp) / R;
      o_v = tv * tv_b + p0 * ES;
      o_z = tv * tz_b + p0 * ES;
      // side and angle words as in the projection form (groups == 1); no norm: unused words
      if (q2 < scw) {
        side_o = static_cast<int>(sc0) * 4;
        side_s = scw * 4;
      } else if (q2 < scw + 2 * ROWS && g.ws_norm >= 0) {
        side_o = static_cast<int>(g.ws_norm + static_cast<int64_t>(b) * L * GR * 2 + q2 - scw) * 4;
        side_s = TOK * GR * 2 * 4;
      } else {
        side_o = side_s = 0;
      }
      ang_o = g.ws_ang >= 0
                  ? static_cast<int>(g.ws_ang + static_cast<int64_t>(b) * g.L4 * S * 4 + 4 * tid) * 4
                  : 0;
      ang_s = (TOK / 4) * S * 16;
      given = a.phase_mode == M3_PHASE_GIVEN;
      if (given) {
        // tile word tid = (group, angle): tokens 4 group .. + 3 of that angle
        const char* x0 = static_cast<const char*>(a.phase.ptr) +
                         (b * a.phase.stride[0] + h * a.phase.stride[2]) * 4;
        tx_b = static_cast<int>(a.phase.stride[1]) * 4;
        rs_x = make_rsrc(x0, L * tx_b);
        const int grp4 = tid / S, sa = tid - grp4 * S;
        o_x = 4 * grp4 * tx_b + sa * static_cast<int>(a.phase.stride[3]) * 4;
      }
    } else {
      q_row = static_cast<const T*>(a.q.ptr) + b * a.q.stride[0] + grp * a.q.stride[2] + n0;
      k_row = static_cast<const T*>(a.k.ptr) + b * a.k.stride[0] + grp * a.k.stride[2] + n0;
      q_t = static_cast<int>(a.q.stride[1]);
      q_r = static_cast<int>(a.q.stride[3]);
      k_t = static_cast<int>(a.k.stride[1]);
      k_r = static_cast<int>(a.k.stride[3]);
      v_row = static_cast<const T*>(a.value.ptr) + b * a.value.stride[0] +
              h * a.value.stride[2] + p0;
      z_row = static_cast<const T*>(a.gate.ptr) + b * a.gate.stride[0] + h * a.gate.stride[2] +
              p0;
      v_t = static_cast<int>(a.value.stride[1]);
      z_t = static_cast<int>(a.gate.stride[1]);
      qk_n = max(0, min(8, N - n0));
      vz_n = max(0, min(4, P - p0));
      vec_qk = g.vec_qk;
      vec_vz = g.vec_vz;
      side_p = nullptr;
      side_tok = 0;
      side_lim = INT32_MAX;
      if (q2 < scw) {
        side_p = prep + sc0;
        side_ps = scw;
      } else if (q2 < scw + 2 * ROWS && norm) {
        // rows are (token, rank); a word holds the (q, k) pair of one row
        const int tr = nrow / R, rr = nrow - tr * R;
        side_p = prep + g.ws_norm + (static_cast<int64_t>(b) * L * GR + tr * GR + grp * R + rr) * 2;
        side_ps = static_cast<int64_t>(TOK) * GR * 2;
        side_tok = tr;
        side_lim = L - 1;
      }
      given = a.phase_mode == M3_PHASE_GIVEN;
      ang_p = nullptr;
      ph_row = nullptr;
      if (a.phase_mode == M3_PHASE_ANGLES && 4 * tid < TOK * S) {
        ang_p = prep + g.ws_ang + static_cast<int64_t>(b) * g.L4 * S * 4 + 4 * tid;
        ang_ps = (TOK / 4) * S * 4;
      } else if (given && 4 * tid < TOK * S) {
        ph_row = static_cast<const float*>(a.phase.ptr) + b * a.phase.stride[0] +
                 h * a.phase.stride[2];
        ph_t = static_cast<int>(a.phase.stride[1]);
        ph_s = static_cast<int>(a.phase.stride[3]);
      }
    }
  }

  // q / k rows 2rp, 2rp+1 and the value / gate of rows 2vp, 2vp+1 of the sub-chunk at token t0
  // (nw valid tokens): tokens 2vp, 2vp+1 for R = 1, else token 2vp / R (both rows' ranks)
  __device__ __forceinline__ void words(int t0, int nw, bool qk_on, bool vz_on,
                                        uint32_t (&rq)[2][W8], uint32_t (&rk)[2][W8],
                                        uint32_t (&rv)[2][W4], uint32_t (&rz)[2][W4]) const {
    words_qk(t0, nw, qk_on, rq, rk);
    words_vz(t0, nw, vz_on, rv, rz);
  }

  __device__ __forceinline__ void words_qk(int t0, int nw, bool qk_on, uint32_t (&rq)[2][W8],
                                           uint32_t (&rk)[2][W8]) const {
    if constexpr (FULL && R > 1 && ES == 2) {
      // MIMO: two 4-column chunks per row, d_hi apart (a rotation pair's partners, or adjacent)
      const int tb = t0 * tok_b;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        uint32_t lo[2], hi[2];
        bload_words<2>(lo, rs_p, o_qk + tb + j * d_q1);
        bload_words<2>(hi, rs_p, o_qk + tb + j * d_q1 + d_hi);
        rq[j][0] = lo[0]; rq[j][1] = lo[1]; rq[j][2] = hi[0]; rq[j][3] = hi[1];
        bload_words<2>(lo, rs_p, o_qk + tb + j * d_q1 + d_k);
        bload_words<2>(hi, rs_p, o_qk + tb + j * d_q1 + d_k + d_hi);
        rk[j][0] = lo[0]; rk[j][1] = lo[1]; rk[j][2] = hi[0]; rk[j][3] = hi[1];
      }
    } else if constexpr (FULL) {
      // unconditional, also for lanes without a q/k or v/z role: every offset stays inside a
      // buffer or past its extent, where the load returns zero
      const int tb = t0 * tok_b;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bload_words<W8>(rq[j], rs_p, o_qk + tb + j * d_q1);
        bload_words<W8>(rk[j], rs_p, o_qk + tb + j * d_q1 + d_k);
      }
    } else if constexpr (BUF) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bload_words<W8>(rq[j], rs_q, o_q + t0 * tq_b + j * d_q2);
        bload_words<W8>(rk[j], rs_k, o_k + t0 * tk_b + j * d_k2);
      }
    } else {
      if (qk_on) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int row = 2 * rp + j, tt = row / R, r = row - tt * R;
          const bool ok = tt < nw;
          const int tg = t0 + tt;
          load_words<T, 8>(rq[j], q_row + tg * q_t + r * q_r, ok ? qk_n : 0, vec_qk);
          load_words<T, 8>(rk[j], k_row + tg * k_t + r * k_r, ok ? qk_n : 0, vec_qk);
        }
      }
    }
  }

  __device__ __forceinline__ void words_vz(int t0, int nw, bool vz_on, uint32_t (&rv)[2][W4],
                                           uint32_t (&rz)[2][W4]) const {
    if constexpr (FULL) {
      const int tb = t0 * tok_b;
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        bload_words<W4>(rv[j], rs_p, o_vz + tb + j * tok_b);
        bload_words<W4>(rz[j], rs_p, o_vz + tb + j * tok_b + d_z);
      }
    } else if constexpr (BUF) {
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        bload_words<W4>(rv[j], rs_v, o_v + (t0 + j) * tv_b);
        bload_words<W4>(rz[j], rs_z, o_z + (t0 + j) * tz_b);
      }
    } else {
      if (vz_on) {
#pragma unroll
        for (int j = 0; j < VJ; ++j) {
          const int tt = R == 1 ? 2 * vp + j : (2 * vp) / R;
          const bool ok = tt < nw;
          const int tg = t0 + tt;
          load_words<T, 4>(rv[j], v_row + tg * v_t, ok ? vz_n : 0, vec_vz);
          load_words<T, 4>(rz[j], z_row + tg * z_t, ok ? vz_n : 0, vec_vz);
        }
      }
    }
  }

  // this lane's side word of sub-chunk c (FULL: unconditional; unused words read anything)
  __device__ __forceinline__ float2 side_in(int c) const {
    if constexpr (FULL || BUF) {
      const u32x2 v = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_w, side_o + c * side_s, 0, 0));
      return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
    } else {
      float2 v = make_float2(1.f, 1.f);
      if (side_p != nullptr && c < nsub && side_tok + c * TOK <= side_lim) {
        v = *reinterpret_cast<const float2*>(side_p + c * side_ps);
      }
      return v;
    }
  }

  // this lane's angle word of sub-chunk c: in the tile order [TOK/4][S][4], 4-token group
  // tid / S of angle tid % S
  __device__ __forceinline__ float4 ang_in(int c) const {
    if constexpr (BUF) {
      if (given) {
        const int o = o_x + c * TOK * tx_b;
        return make_float4(bload_f32(rs_x, o), bload_f32(rs_x, o + tx_b),
                           bload_f32(rs_x, o + 2 * tx_b), bload_f32(rs_x, o + 3 * tx_b));
      }
    }
    if constexpr (FULL || BUF) {
      const u32x4 v = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_w, ang_o + c * ang_s, 0, 0));
      return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                         __uint_as_float(v[3]));
    } else {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (c >= nsub) return v;
      if (ang_p != nullptr) {
        if (c * (TOK / 4) + static_cast<int>(threadIdx.x) / S < L4) {  // groups past L4: none
          v = *reinterpret_cast<const float4*>(ang_p + c * ang_ps);
        }
      } else if (ph_row != nullptr) {
        // tile word tid = (group, angle): tokens 4 group .. + 3 of that angle
        const int tid = threadIdx.x;
        const int grp4 = tid / S, sa = tid - grp4 * S;
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = c * TOK + 4 * grp4 + i;
          e[i] = t < L ? ph_row[static_cast<int64_t>(t) * ph_t + sa * ph_s] : 0.f;
        }
        v = make_float4(e[0], e[1], e[2], e[3]);
      }
      return v;
    }
  }
};

// Column of angle `col` in the cos / sin table row of token tt. SWZ (64-token sub-chunks, 32
// angles): blocks of 4 angles are XOR-swizzled by the token's 16-token block, spreading the
// phase stage's column writes over the LDS banks, and the two angle pairs of a block swap places
// in every other token pair, so the 16-byte reads of two token rows 2 apart (136 floats: the
// same banks shifted by 8) fall into different halves of each 8-float group. A reader takes a
// block as two pairs, each at its own cs_col.
template <bool SWZ>
__device__ __forceinline__ int cs_col(int col, int tt) {
  return SWZ ? col ^ (4 * ((tt >> 4) & 3)) ^ (2 * ((tt >> 1) & 1)) : col;
}

// Bounded phase (model.py:215-256) of tokens TPL pg .. TPL pg + TPL-1 of the sub-chunk at t0 for
// angle ps: fmod-reduced increments summed within 64-token blocks, an fmod-reduced carry between
// blocks, the running block sum and carry in pbase / poff; cos / sin into the table of angle ps.
template <int PG, int TPL, int CST, bool SWZ, bool EXACT>
__device__ __forceinline__ void phase_stage(float* tab, int ps, float* pbase, float* poff,
                                            const float* dtv, int t0, int L, int pg, int lane,
                                            bool angles, const float (&pa)[TPL], float* fph,
                                            float* fblk, int64_t blk_stride) {
  float ph[TPL];
  if (angles) {
    float x[TPL];
    float mx = 0.f;  // largest |increment| of the lane (NaN and inf reduce like any x below)
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      x[i] = __fmul_rn(pa[i], dtv[TPL * pg + i]);  // dt is 0 past the sub-chunk's last token
      mx = fmaxf(mx, fabsf(x[i]));
    }
    // fmodf(x, 2 pi) is x itself for |x| < 2 pi (dt < 2, the usual case); the reductions are
    // chosen per wave, so no lane branches on its own elements
    float inc[TPL];
    if (__builtin_amdgcn_ballot_w64(!(mx < M3_TWO_PI_F)) == 0) {
#pragma unroll
      for (int i = 0; i < TPL; ++i) inc[i] = x[i];
    } else if (__builtin_amdgcn_ballot_w64(!(mx < 1048576.0f)) == 0) {
#pragma unroll
      for (int i = 0; i < TPL; ++i) inc[i] = m3_fmod_2pi_small(x[i]);
    } else {
#pragma unroll
      for (int i = 0; i < TPL; ++i) inc[i] = m3_fmod_2pi(x[i]);
    }
    float cpre[TPL];
    float run = 0.f;
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      run = __fadd_rn(run, inc[i]);
      cpre[i] = run;
    }
    const float incl = seg_incl_scan<PG>(run, lane);
    // the previous lane's inclusive sum: sums of earlier tokens only (incl - run would round in
    // the later tokens of this lane's group)
    float excl = dpp_shr<0x111>(incl);
    if (pg == 0) excl = 0.f;
    float base = *pbase, off = *poff;
    if ((t0 & 63) == 0 && t0 > 0) {
      // the block that just ended: its increment sum, when asked for (block_phase)
      if (fblk != nullptr && pg == 0) fblk[((t0 >> 6) - 1) * blk_stride] = base;
      off = m3_fmod_2pi_small(__fadd_rn(off, base));
      base = 0.f;
    }
    // the final phase (token L - 1), when this sub-chunk holds it (wave-uniform test)
    const bool last = fph != nullptr && t0 <= L - 1 && L - 1 - t0 < PG * TPL;
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      // |base|, |excl + cpre| <= 64 * 2 pi and |off| < 2 pi: within the reduction's range.
      // !EXACT (16-bit activations): sin / cos reduce the phase themselves (below 66 turns, the
      // hardware's range), a difference far below the 16-bit rounding of the rotated values.
      const float raw = __fadd_rn(__fadd_rn(base, __fadd_rn(excl, cpre[i])), off);
      ph[i] = EXACT ? m3_fmod_2pi_small(raw) : raw;
    }
    if (last) {  // one wave-uniform branch instead of a lane test per token
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        if (t0 + TPL * pg + i == L - 1) *fph = EXACT ? ph[i] : m3_fmod_2pi_small(ph[i]);
      }
    }
    if (pg == PG - 1) {
      *pbase = __fadd_rn(base, incl);
      *poff = off;
    }
  } else {
#pragma unroll
    for (int i = 0; i < TPL; ++i) ph[i] = pa[i];
  }
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int tt = TPL * pg + i;
    float2 v;
    __sincosf(ph[i], &v.y, &v.x);
    *reinterpret_cast<float2*>(tab + tt * CST + 2 * cs_col<SWZ>(ps, tt)) = v;
  }
}

// ------------------------------------------------------------------ prep

// The scalar block of sub-chunk c of (batch, head) bh (one wave, lane = token): dt, adt, trap
// from the raw projection or given (model.py:195-198), gamma = dt sigmoid(trap), scale = gamma +
// dt' (1 - sigmoid(trap')) of the next token, 0 at the last token (ops.py:659-671), the
// within-chunk cumsum of adt by a wave scan, and the decay products the scan uses.
template <int TOK, int TPT>
__device__ __forceinline__ void scalar_block(const m3_scan_args& a, float* __restrict__ o,
                                             int c, int lane, float dt_bias, float dt_in,
                                             float a_in, float tr_in, float dtn_in,
                                             float trn_in) {
  using B = ScBlk<TOK>;
  const int L = a.length;
  const int tb = c * TOK, t = tb + lane;
  const int wn = min(TOK, L - tb);
  const bool tv = lane < wn;
  const bool nv = lane < TOK && t + 1 < L;
  const bool raw_dt = a.raw_dt != 0;
  float dt = 0.f, adt = 0.f, tr = 0.f;
  if (tv) {
    dt_adt_fast(raw_dt, dt_in, a_in, dt_bias, dt, adt);
    tr = sigmoid_fast(tr_in);
  }
  // right = dt' (1 - sigmoid(trap')) of the next token: lane + 1's; the last lane's from the
  // token after the sub-chunk (dtn_in, trn_in)
  const float own = dt * (1.f - tr);
  float right = __shfl_down(own, 1);
  if (lane == TOK - 1) {
    float dn, an;
    dt_adt_fast(raw_dt, dtn_in, 0.f, dt_bias, dn, an);
    right = dn * (1.f - sigmoid_fast(trn_in));
  }
  if (!nv) right = 0.f;
  const float gamma = dt * tr;
  const float scale = gamma + right;
  const float cum = wave_incl_scan(adt, lane);
  const float cum_last = readlane_f(cum, wn - 1);
  const float cv = tv ? cum : cum_last;
  // cum at the end of this lane's 16-row tile (TPT tokens), clamped to the last valid token
  float cend;
  if constexpr (TPT == 16) {
    const float e0 = readlane_f(cv, 15), e1 = readlane_f(cv, 31), e2 = readlane_f(cv, 47);
    const float e3 = readlane_f(cv, 63);
    const int q = lane >> 4;
    cend = q == 0 ? e0 : (q == 1 ? e1 : (q == 2 ? e2 : e3));
  } else {
    cend = __shfl(cv, min(lane | (TPT - 1), wn - 1));
  }
  if (lane < TOK) {
    o[B::DTV + lane] = dt;
    o[B::CUM + lane] = cv;
    o[B::SCL + lane] = tv ? scale : 0.f;
    o[B::GAM + lane] = gamma;
    o[B::BSC + lane] = tv ? scale * __expf(cend - cv) : 0.f;
    if ((lane & (TPT - 1)) == 0) o[B::CEND + lane / TPT] = cend;
  }
  if (lane == 0) {
    o[B::ECL] = __expf(cum_last);
    o[B::CL] = cum_last;
  }
}

// The same for sub-chunks of TOK <= 16 tokens, 64 / TOK heads per wave: lane = (head lane / TOK,
// token lane % TOK), `o` the lane's head's block, `live` false for lanes past the last head
// (they compute on a valid head's inputs and store nothing). The arithmetic and its order are
// scalar_block's (a segment's scan is the wave scan's first row), so the blocks are identical.
template <int TOK, int TPT>
__device__ __forceinline__ void scalar_block_seg(const m3_scan_args& a, float* __restrict__ o,
                                                 int c, int lane, bool live, float dt_bias,
                                                 float dt_in, float a_in, float tr_in,
                                                 float dtn_in, float trn_in) {
  static_assert(TOK <= 16 && (TOK & (TOK - 1)) == 0, "segments of at most 16 lanes");
  using B = ScBlk<TOK>;
  const int L = a.length;
  const int j = lane & (TOK - 1), s0 = lane - j;  // token in the sub-chunk, segment's lane 0
  const int tb = c * TOK, t = tb + j;
  const int wn = min(TOK, L - tb);
  const bool tv = j < wn;
  const bool nv = t + 1 < L;
  const bool raw_dt = a.raw_dt != 0;
  float dt = 0.f, adt = 0.f, tr = 0.f;
  if (tv) {
    dt_adt_fast(raw_dt, dt_in, a_in, dt_bias, dt, adt);
    tr = sigmoid_fast(tr_in);
  }
  const float own = dt * (1.f - tr);
  float right = __shfl_down(own, 1);
  if (j == TOK - 1) {
    float dn, an;
    dt_adt_fast(raw_dt, dtn_in, 0.f, dt_bias, dn, an);
    right = dn * (1.f - sigmoid_fast(trn_in));
  }
  if (!nv) right = 0.f;
  const float gamma = dt * tr;
  const float scale = gamma + right;
  const float cum = seg_incl_scan<TOK>(adt, lane);
  const float cum_last = __shfl(cum, s0 + wn - 1);
  const float cv = tv ? cum : cum_last;
  const float cend = __shfl(cv, s0 + min(j | (TPT - 1), wn - 1));
  if (live) {
    o[B::DTV + j] = dt;
    o[B::CUM + j] = cv;
    o[B::SCL + j] = tv ? scale : 0.f;
    o[B::GAM + j] = gamma;
    o[B::BSC + j] = tv ? scale * __expf(cend - cv) : 0.f;
    if ((j & (TPT - 1)) == 0) o[B::CEND + j / TPT] = cend;
    if (j == 0) {
      o[B::ECL] = __expf(cum_last);
      o[B::CL] = cum_last;
    }
  }
}

// Head-independent and per-(head, sub-chunk) work ahead of the scan, three block ranges:
//  [0, nb_norm)  one 16-lane group per norm_rows() raw q / k rows (token, group, rank, q|k), 8
//                elements per lane: each row's RMSNorm factor 1 / sqrt(mean(x^2) + eps)
//                (model.py:190-191);
//  [.., +nb_ang) one lane per kAngQuads (4-token group, angle) pairs, tokens padded to a multiple
//                of 4: pi * tanh(angle) (model.py:225-228), 0 in the padding;
// The first two give each workgroup several rows' loads in flight: with one round trip per
// workgroup they were bound by workgroup turnover (the scalar blocks' LDS allows 6 workgroups per
// CU). The scalar blocks, the longest workgroups, are dispatched first.
//  [.., +nb_sc)  one workgroup per (batch, sub-chunk): the dt / a / trap of its TOK tokens and
//                the next sub-chunk's first, every head, loaded with consecutive lanes on
//                consecutive heads (32 heads per pass) into LDS; then one wave per head computes
//                that head's scalar block (sub-chunks of 16 tokens or fewer: one 16- or 8-lane
//                segment per head, 4 or 8 heads per wave).
// q / k rows per 16-lane group of prep_kernel: 16 for the 16-bit single-rank rows (their fewer,
// longer workgroups measured faster at config 2: 37.5 -> 34.8 us per prep), else 8 (16 measured
// slower at rank 4, and FP32 rows would not fit the registers)
template <typename T, int R>
constexpr int norm_rows() {
  return sizeof(T) == 2 && R == 1 ? 16 : 8;
}
constexpr int kAngQuads = 4;  // (4-token group, angle) pairs per lane of prep_kernel

template <typename T, int R>
__global__ __launch_bounds__(256) void prep_kernel(const m3_scan_args a, const ScanGeom g,
                                                   float* __restrict__ ws, int nb_norm,
                                                   int nb_ang) {
  // every index below fits 31 bits (checked by the host)
  constexpr int TOK = Mma<T>::ROWS / R, TPT = 16 / R;
  constexpr int kNormRows = norm_rows<T, R>();
  // the longest-running range (scalar blocks) is dispatched first: block ids [0, nb_sc) map to
  // it, the rest to the norm and angle ranges in order
  const int nb_sc = a.batch * g.nsub;
  const int tid = threadIdx.x;
  const int blk = static_cast<int>(blockIdx.x) < nb_sc ? static_cast<int>(blockIdx.x) + nb_norm + nb_ang
                                                       : static_cast<int>(blockIdx.x) - nb_sc;
  const int L = a.length, tokens = a.batch * L;
  if (blk < nb_norm) {
    // rows blk * 16 kNormRows + (tid >> 4) + 16 k, k < kNormRows: every row's loads first
    const int gr_n = a.groups * a.rank;
    const int nrows = tokens * gr_n * 2;
    const int l16 = tid & 15, row0 = blk * 16 * kNormRows + (tid >> 4);
    const int N = a.d_state;
    const bool in = 8 * l16 < N;  // lanes past column N load column 0 and count zeros
    // Rows (token, group, rank, q | k): a lane's rows row0 + 16 k all have row0's parity, so one
    // tensor (q or k). When 2 gr_n divides 16 they also share its (group, rank), the token
    // advancing by 8 / gr_n per k: the addresses follow from row0's by additions (a division
    // per row and a select per tensor field, unrolled over the rows, were most of this range's
    // instructions). Rows past the end re-read the last batch row's last token.
    const int which = row0 & 1;
    const m3_tensor& xt = which ? a.k : a.q;
    const T* xbase = static_cast<const T*>(xt.ptr) + (in ? 8 * l16 : 0);
    const int64_t xs0 = xt.stride[0], xs1 = xt.stride[1];
    const bool step_rows = 16 % (2 * gr_n) == 0;
    const int dtok = step_rows ? 8 / gr_n : 0;
    int tk = row0 / (2 * gr_n);
    const int gr = (row0 - tk * 2 * gr_n) >> 1;
    const int gi = gr / a.rank, rk = gr - gi * a.rank;
    const T* xgr = xbase + gi * xt.stride[2] + rk * xt.stride[3];
    int bk = tk / L, tt = tk - bk * L;
    auto row_ptr = [&](int k) -> const T* {
      if (step_rows) {
        if (k > 0) {
          tt += dtok;
          while (tt >= L) {
            tt -= L;
            ++bk;
          }
        }
        const bool live = bk < a.batch;
        return xgr + (live ? bk : a.batch - 1) * xs0 + (live ? tt : L - 1) * xs1;
      }
      const int row = min(row0 + 16 * k, nrows - 1);
      const int tok = row / (2 * gr_n);
      const int rem = row - tok * 2 * gr_n;
      const int g2 = rem >> 1, wh = rem & 1;
      const int g2i = g2 / a.rank, r2 = g2 - g2i * a.rank;
      const int b2 = tok / L, t2 = tok - b2 * L;
      const m3_tensor& x = wh ? a.k : a.q;
      return static_cast<const T*>(x.ptr) + b2 * x.stride[0] + t2 * x.stride[1] +
             g2i * x.stride[2] + r2 * x.stride[3] + (in ? 8 * l16 : 0);
    };
    float ss[kNormRows];
    uint32_t w8[kNormRows][Words<T>::W8];
    // the normalized rows' weights for this lane's 8 columns, raw, issued with the rows (after
    // the factor stores below they would be a second round trip)
    const bool rows_out = sizeof(T) == 2 && g.ws_qk >= 0 && g.vec_qk;
    const bool nw_vec = rows_out && g.vec_nw;
    Raw4 nw_r[2][2] = {};
    if (nw_vec) {
      nw_r[0][0] = ldraw4(a.q_norm_w, 8 * l16);
      nw_r[0][1] = ldraw4(a.q_norm_w, 8 * l16 + 4);
      nw_r[1][0] = ldraw4(a.k_norm_w, 8 * l16);
      nw_r[1][1] = ldraw4(a.k_norm_w, 8 * l16 + 4);
    }
    if (g.vec_qk) {
#pragma unroll
      for (int k = 0; k < kNormRows; ++k) {
        // rows past the end re-read an earlier row; their sums are not stored
        const T* p = row_ptr(k);
#pragma unroll
        for (int j = 0; j < Words<T>::W8; j += 4) {
          const uint4 q = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint32_t*>(p) + j);
          w8[k][j] = in ? q.x : 0u;
          w8[k][j + 1] = in ? q.y : 0u;
          w8[k][j + 2] = in ? q.z : 0u;
          w8[k][j + 3] = in ? q.w : 0u;
        }
      }
#pragma unroll
      for (int k = 0; k < kNormRows; ++k) {
        ss[k] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float v = raw_get<T>(w8[k], i);
          ss[k] = fmaf(v, v, ss[k]);
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < kNormRows; ++k) {
        const T* p = row_ptr(k);
        ss[k] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (in && 8 * l16 + i < N) {
            const float v = to_f(p[i]);
            ss[k] = fmaf(v, v, ss[k]);
          }
        }
      }
    }
    float fac[kNormRows];
#pragma unroll
    for (int k = 0; k < kNormRows; ++k) {
      ss[k] = row16_sum(ss[k]);  // the row's 16 lanes
      const int row = row0 + 16 * k;
      fac[k] = 1.f / sqrtf(ss[k] / static_cast<float>(N) + a.norm_eps);
      if (l16 == 0 && row < nrows && g.norm_factors) ws[g.ws_norm + static_cast<int64_t>(row)] = fac[k];
    }
    if constexpr (sizeof(T) == 2) {
      if (rows_out) {
        // the model's shape at ranks 1 and 4 (N = 128, one group, vector rows): the normalized rows
        // themselves, rnd(x * factor * rnd(w)) (model.py:48-55: F.rms_norm with the weight in the
        // activation dtype, the result in it), rows (token, q | k) at N elements each
        // the lane's tensor's weights (every row of the lane is q, or every row k), chosen by
        // bit masks on the raw words: a select between two weight arrays by `which` became a
        // dynamically indexed array in scratch memory
        float wl[8];
        if (nw_vec) {
          const uint32_t msk = 0u - static_cast<uint32_t>(which);
          const int wdt = which ? a.k_norm_w.dtype : a.q_norm_w.dtype;
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            Raw4 r;
#pragma unroll
            for (int j = 0; j < 4; ++j) r.w[j] = (nw_r[0][h2].w[j] & ~msk) | (nw_r[1][h2].w[j] & msk);
            const f4 v4 = decode4(r, wdt);
#pragma unroll
            for (int e = 0; e < 4; ++e) wl[4 * h2 + e] = rnd<T>(v4[e]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float wq = ldx(a.q_norm_w.ptr, a.q_norm_w.dtype, (8 * l16 + i) * a.q_norm_w.stride[0]);
            const float wk = ldx(a.k_norm_w.ptr, a.k_norm_w.dtype, (8 * l16 + i) * a.k_norm_w.stride[0]);
            wl[i] = rnd<T>(which ? wk : wq);
          }
        }
        char* qk = reinterpret_cast<char*>(ws) + g.ws_qk;
#pragma unroll
        for (int k = 0; k < kNormRows; ++k) {
          const int row = row0 + 16 * k;
          if (row >= nrows) continue;
          float x[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = raw_get<T>(w8[k], i) * fac[k] * wl[i];
          st_row8<T>(reinterpret_cast<T*>(qk + (static_cast<int64_t>(row) * N + 8 * l16) * 2), x);
        }
      }
    }
  } else if (blk < nb_norm + nb_ang) {
    // (b, t4, s) quads blk * 256 kAngQuads + tid + 256 k: the angle s of tokens 4 t4 .. 4 t4 + 3,
    // written as the angle region's 4 consecutive elements (b, t4, s, i); 0 past token L - 1
    const int S = a.num_angles;
    const int nq = a.batch * g.L4 * S;
    const int q0 = (blk - nb_norm) * 256 * kAngQuads + tid;
    RawX raw[kAngQuads][4];
#pragma unroll
    for (int k = 0; k < kAngQuads; ++k) {
      const int quad = min(q0 + 256 * k, nq - 1);
      const int sa = quad % S, bt4 = quad / S;
      const int b = bt4 / g.L4, t4 = bt4 - b * g.L4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = min(4 * t4 + i, L - 1);
        raw[k][i] = ldraw(a.phase.ptr, a.phase.dtype,
                          b * a.phase.stride[0] + t * a.phase.stride[1] + sa * a.phase.stride[2]);
      }
    }
#pragma unroll
    for (int k = 0; k < kAngQuads; ++k) {
      const int quad = q0 + 256 * k;
      if (quad >= nq) continue;
      const int bt4 = quad / S;
      const int t4 = bt4 - (bt4 / g.L4) * g.L4;
      float4 v;
      float* vv = reinterpret_cast<float*>(&v);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float th = decode(raw[k][i], a.phase.dtype);
        vv[i] = 4 * t4 + i < L ? __fmul_rn(kPi, tanhf(th)) : 0.f;
      }
      *reinterpret_cast<float4*>(ws + g.ws_ang + 4 * static_cast<int64_t>(quad)) = v;
    }
  } else {
    const int bc = blk - nb_norm - nb_ang;
    if (bc >= a.batch * g.nsub) return;  // whole workgroups leave together
    const int b = bc / g.nsub, c = bc - b * g.nsub;
    constexpr int HG = 32, NE = (TOK + 1) * HG, NIT = (NE + 255) / 256;
    __shared__ float s_in[3][TOK + 1][HG + 1];
    __shared__ float s_db[HG];  // dt_bias of the group's heads
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const char* base_dt = static_cast<const char*>(offx(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0]));
    const char* base_a = static_cast<const char*>(offx(a.a.ptr, a.a.dtype, b * a.a.stride[0]));
    const char* base_tr =
        static_cast<const char*>(offx(a.trap.ptr, a.trap.dtype, b * a.trap.stride[0]));
    const int s1_dt = static_cast<int>(a.dt.stride[1]), s2_dt = static_cast<int>(a.dt.stride[2]);
    const int s1_a = static_cast<int>(a.a.stride[1]), s2_a = static_cast<int>(a.a.stride[2]);
    const int s1_tr = static_cast<int>(a.trap.stride[1]), s2_tr = static_cast<int>(a.trap.stride[2]);
    for (int h0 = 0; h0 < a.heads; h0 += HG) {
      const int hn = min(HG, a.heads - h0);
      // raw loads of every element first (clamped to valid tokens / heads), then decode and store
      RawX rd[NIT], ra[NIT], rt[NIT];
      // dt_bias with the batch (inside the per-head loop below, after its stores, each head's
      // load would be a round trip of its own)
      const RawX rdb = a.raw_dt != 0
                           ? ldraw(a.dt_bias.ptr, a.dt_bias.dtype,
                                   (h0 + min(tid & (HG - 1), hn - 1)) * a.dt_bias.stride[0])
                           : RawX{0u, 0u};
#pragma unroll
      for (int k = 0; k < NIT; ++k) {
        const int e = min(tid + 256 * k, NE - 1);
        const int j = e / HG, hh = e - j * HG;
        const int t = min(c * TOK + j, L - 1), h = h0 + min(hh, hn - 1);
        rd[k] = ldraw(base_dt, a.dt.dtype, t * s1_dt + h * s2_dt);
        ra[k] = ldraw(base_a, a.a.dtype, t * s1_a + h * s2_a);
        rt[k] = ldraw(base_tr, a.trap.dtype, t * s1_tr + h * s2_tr);
      }
#pragma unroll
      for (int k = 0; k < NIT; ++k) {
        const int e = tid + 256 * k;
        if (e < NE) {
          const int j = e / HG, hh = e - j * HG;
          s_in[0][j][hh] = decode(rd[k], a.dt.dtype);
          s_in[1][j][hh] = decode(ra[k], a.a.dtype);
          s_in[2][j][hh] = decode(rt[k], a.trap.dtype);
        }
      }
      if (tid < HG) s_db[tid] = a.raw_dt != 0 ? decode(rdb, a.dt_bias.dtype) : 0.f;
      __syncthreads();
      if constexpr (TOK <= 16) {
        // 64 / TOK heads per wave (one wave per head would leave most lanes idle)
        constexpr int HPW = 64 / TOK;
        const int j = lane & (TOK - 1);
        for (int hb = w * HPW; hb < hn; hb += 4 * HPW) {
          const int hh = hb + lane / TOK, hc = min(hh, hn - 1);
          scalar_block_seg<TOK, TPT>(
              a, ws + g.ws_sc + (static_cast<int64_t>(b * a.heads + h0 + hc) * g.nsub + c) * g.scw,
              c, lane, hh < hn, s_db[hc], s_in[0][j][hc], s_in[1][j][hc], s_in[2][j][hc],
              s_in[0][TOK][hc], s_in[2][TOK][hc]);
        }
      } else {
        for (int hh = w; hh < hn; hh += 4) {
          const int h = h0 + hh, j = min(lane, TOK - 1);
          scalar_block<TOK, TPT>(
              a, ws + g.ws_sc + (static_cast<int64_t>(b * a.heads + h) * g.nsub + c) * g.scw, c,
              lane, s_db[hh], s_in[0][j][hh], s_in[1][j][hh], s_in[2][j][hh], s_in[0][TOK][hh],
              s_in[2][TOK][hh]);
        }
      }
      __syncthreads();
    }
  }
}

// SO (state only, with FULL): the segmented scan's first pass, which needs the end state, log
// decay, last k and phase block sums but no outputs. The stores of Qs, VR, ZR, Sb and the output
// are left out, and with them (dead code) the q math, the scores, the decay weights, the intra
// and inter products and the epilogue; k, the carry tiles and products and the phase remain.
//
// SHAPE (without FULL): the model's shape (N = 128, P = 64, 32 angles when rotating, aligned
// 16-byte rows) with the generic inputs (the hook form): the dimensions and the vector-load
// choice are compile-time constants, the features stay runtime; every read and the output go
// through buffer resources at per-lane offsets, issued unconditionally as in the FULL form.
template <typename T, int R, bool FULL, bool SO = false, bool SHAPE = false>
__global__ __launch_bounds__(kThreads) void scan_kernel(const m3_scan_args a, const ScanGeom g,
                                                        const float* __restrict__ prep) {
  using M = Mma<T>;
  using Lay = Layout<T>;
  constexpr int ROWS = M::ROWS;
  constexpr int RT = ROWS / 16;        // 16-row tiles per sub-chunk
  constexpr int WPR = kWaves / RT;     // waves sharing one query row tile
  constexpr int TOK = ROWS / R;        // tokens per sub-chunk
  constexpr bool F32 = sizeof(T) == 4;
  // the swizzled Ks layout (ks_col): rank 1 in 16 bits (config 2 442 against 445 us); at rank 4
  // it measured within the 1% spread of these comparisons, and the plain rows are kept
  constexpr bool KSW = !F32 && R == 1;
  constexpr int ES = sizeof(T);
  constexpr int LQ = Lay::LQ, LR = Lay::LR, LP = Lay::LP, NP = kNPad, CST = Lay::CST;
  using SB_ = ScBlk<TOK>;
  // SISO model shape: q / k lanes split by column half, waves 0-3 holding the rotated columns;
  // the phase on waves 0-3 only, 8 tokens per lane (their compute interval is the shorter one)
  constexpr bool SPLIT = (FULL || SHAPE) && R == 1 && !F32;
  // MIMO model shape in projection form: q / k lanes split by rotation role as well. Waves 0-3
  // hold the rotated pairs (n, n + 64), n < 32, four pairs per lane (the MIMO rotation pairs
  // quarter 1 with quarter 3, model.py:201-213, ops.py:35-84), waves 4-7 eight consecutive
  // columns of the unrotated quarters 2 and 4: no lane exchanges a partner, and only the rotated
  // half does rotation arithmetic.
  constexpr bool MSPLIT = FULL && R > 1 && !F32;
  constexpr int TPL = SPLIT ? 8 : 4;   // tokens per phase lane
  constexpr int PG = TOK / TPL;        // phase lanes per angle
  // swizzle keys of the FP32 transposed tiles, n >> KSH for KT and p >> VSH for VT
  constexpr int KSH = F32 ? 3 : 4, VSH = F32 ? 2 : 4;
  // 16-bit: no transposed copies. The carry reads K~^T from the row-major Ks and V from the
  // row-major VS (the rank values with each token's scale * end decay, in KT's place), the
  // intra product V^T from VR, all through transposing LDS reads
  constexpr bool KTR = !F32;
  // FULL: the model's shape (N = 128, P = 64, S = 32) in projection form with vector loads
  constexpr bool FIX = FULL || SHAPE;  // the model's shape, fixed at compile time
  const int N = FIX ? kNPad : a.d_state;
  const int P = FIX ? kPPad : a.head_dim;
  const int S = FIX ? kSMax : a.num_angles;
  const bool norm = FULL || g.ws_norm >= 0;
  const bool bias = FULL || a.q_bias.ptr != nullptr;
  const bool rotate = FULL || a.phase_mode != M3_PHASE_NONE;
  const bool angles = FULL || a.phase_mode == M3_PHASE_ANGLES;
  const bool raw_dt = FULL || a.raw_dt != 0;
  const bool mimo_rot = FULL ? (R > 1) : (a.mimo_rotation != 0);
  const int H = a.heads, L = a.length;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index (wave-uniform)
  const int l16 = lane & 15, lg = lane >> 4;

  // ---- block -> (b, h): with xcd_map the blocks of one XCD (blockIdx % 8) take consecutive
  // (b, h), so the heads of one batch row share that XCD's L2 for q, k and the angles.
  int bid = blockIdx.x;
  if (g.xcd_map) {
    const int per = gridDim.x >> 3;
    bid = (bid & 7) * per + (bid >> 3);
  }
  const int b = bid / H, h = bid - b * H;
  const int grp = h / (H / a.groups);

  extern __shared__ __attribute__((aligned(16))) char smem[];
  T* Qs = lds_t<T>(smem, Lay::QS);
  T* Ks = lds_t<T>(smem, Lay::KS);
  T* KT = lds_t<T>(smem, Lay::KT);  // FP32: [n][row] K~, transposed and scaled (carry)
  T* VS = KT;                        // 16-bit: [row][p] rank values scaled per token (carry)
  T* VT = lds_t<T>(smem, Lay::VT);  // FP32: [p][row] rank values v mx_r, transposed
  T* VR = lds_t<T>(smem, Lay::VR);  // [row][p] the same, row-major (epilogue D v)
  T* ZR = lds_t<T>(smem, Lay::ZR);  // [row][p] rank gates z mz_r, row-major (epilogue)
  T* Sb = lds_t<T>(smem, Lay::SB);
  float* F = lds_t<float>(smem, Lay::FB);
  const float Dh = ldx(a.D.ptr, a.D.dtype, h * a.D.stride[0]);

  // ---- lane roles
  // q / k: row pair rp (rows 2rp, 2rp+1), columns n0 .. n0+7 (SPLIT: waves 0-3 columns 0-63,
  // waves 4-7 columns 64-127)
  const int rp = (SPLIT || MSPLIT) ? (tid & 255) >> 3 : tid >> 4;
  const int n0 = SPLIT    ? 64 * (tid >> 8) + 8 * (tid & 7)
                 : MSPLIT ? (tid < 256 ? 4 * (tid & 7)
                                       : ((tid & 7) < 4 ? 32 + 8 * (tid & 7) : 64 + 8 * (tid & 7)))
                          : 8 * (tid & 15);
  // the lane's i-th column (MSPLIT rotated lanes: n0 .. n0+3, then their partners n0+64 ..)
  auto col_of = [&](int i) {
    return (MSPLIT && tid < 256) ? (i < 4 ? n0 + i : n0 + 60 + i) : n0 + i;
  };
  // (SPLIT / MSPLIT: every lane has both roles, 512 threads covering 64 rows x 128 columns and
  // 64 rows x 64 columns)
  const bool qk_on = SPLIT || MSPLIT || (rp < ROWS / 2 && n0 < N);
  // v / z: row pair vp (rows 2vp, 2vp+1; tokens 2vp, 2vp+1 for R = 1), columns p0 .. p0+3
  constexpr int P4 = kPPad / 4;
  const int vp = tid / P4, p0 = 4 * (tid % P4);
  const bool vz_on = SPLIT || (2 * vp < TOK * R && p0 < P);
  // phase: angle ps, token group pg (tokens TPL pg .. TPL pg + TPL-1)
  const int pg = tid % PG, ps = tid / PG;
  const bool ph_on = rotate && ps < S;

  // ---- one-time LDS setup: zero the operand regions (padding), MIMO parameters, phase carry
  for (int i = tid; i < Lay::FB / 4; i += kThreads) reinterpret_cast<uint32_t*>(smem)[i] = 0u;
  for (int i = tid; i < R * P; i += kThreads) {
    const int r = i / P, p = i - r * P;
    const int o = r * kPPad + p;
    if (R > 1) {
      F[Lay::MX + o] = rnd<T>(ldx(a.mimo_x.ptr, a.mimo_x.dtype,
                                  h * a.mimo_x.stride[0] + r * a.mimo_x.stride[1] + p));
      F[Lay::MZ + o] = rnd<T>(ldx(a.mimo_z.ptr, a.mimo_z.dtype,
                                  h * a.mimo_z.stride[0] + r * a.mimo_z.stride[1] + p));
      F[Lay::MO + o] = ldx(a.mimo_out.ptr, a.mimo_out.dtype,
                           h * a.mimo_out.stride[0] + r * a.mimo_out.stride[1] + p);
    } else {
      F[Lay::MX + o] = 1.f;
      F[Lay::MZ + o] = 1.f;
      F[Lay::MO + o] = 1.f;
    }
  }
  for (int s = tid; s < S; s += kThreads) {
    F[Lay::PBASE + s] = 0.f;
    F[Lay::POFF + s] = a.initial_phase.ptr != nullptr
                           ? static_cast<const float*>(a.initial_phase.ptr)
                                 [b * a.initial_phase.stride[0] + h * a.initial_phase.stride[1] +
                                  s * a.initial_phase.stride[2]]
                           : 0.f;
  }

  // per-lane constants of the value / gate role (R > 1): the rounded mimo_x / mimo_z of its rows
  // ranks, (2 vp) % R and the next, at columns p0 .. p0+3, read once here instead of from LDS
  // in every sub-chunk
  float mxl[2][4], mzl[2][4];
#pragma unroll
  for (int jr = 0; jr < 2; ++jr) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (2 * vp + jr) % R, p = min(p0 + i, P - 1);
      mxl[jr][i] = R > 1 ? rnd<T>(ldx(a.mimo_x.ptr, a.mimo_x.dtype,
                                      h * a.mimo_x.stride[0] + r * a.mimo_x.stride[1] + p))
                         : 1.f;
      mzl[jr][i] = R > 1 ? rnd<T>(ldx(a.mimo_z.ptr, a.mimo_z.dtype,
                                      h * a.mimo_z.stride[0] + r * a.mimo_z.stride[1] + p))
                         : 1.f;
    }
  }

  // per-lane constants of the q / k role: rounded norm weights and the biases of its rows
  // (rows 2rp, 2rp+1 have ranks (2rp) % R, (2rp+1) % R: one set suffices when R == 1)
  constexpr int NB = R == 1 ? 1 : 2;
  float wq[8], wk[8], bq[NB][8], bk[NB][8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int n = col_of(i);
    const bool ok = qk_on && n < N;
    wq[i] = (ok && norm) ? rnd<T>(ldx(a.q_norm_w.ptr, a.q_norm_w.dtype, n * a.q_norm_w.stride[0]))
                         : 1.f;
    wk[i] = (ok && norm) ? rnd<T>(ldx(a.k_norm_w.ptr, a.k_norm_w.dtype, n * a.k_norm_w.stride[0]))
                         : 1.f;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int r = (2 * rp + j) % R;
      bq[j][i] = (ok && bias) ? rnd<T>(ldx(a.q_bias.ptr, a.q_bias.dtype,
                                           h * a.q_bias.stride[0] + r * a.q_bias.stride[1] + n))
                              : 0.f;
      bk[j][i] = (ok && bias) ? rnd<T>(ldx(a.k_bias.ptr, a.k_bias.dtype,
                                           h * a.k_bias.stride[0] + r * a.k_bias.stride[1] + n))
                              : 0.f;
    }
  }

  // ---- the state: S^T tiles (ni, pj), tile u = w + 8k; lane holds n = 16 ni + 4 lg + i,
  // p = 16 pj + l16.
  constexpr int n_tiles = kNT * kPT;
  static_assert(n_tiles <= kWaves * kTiles, "state tiles exceed the waves' share");
  constexpr bool all_tiles = n_tiles == kWaves * kTiles;  // every (wave, k) holds a tile
  f4 st[kTiles];
#pragma unroll
  for (int k = 0; k < kTiles; ++k) {
    st[k] = zero4();
    const int u = w + kWaves * k;
    if (u < n_tiles && a.initial_state.ptr != nullptr) {
      const int ni = u / kPT, pj = u - ni * kPT;
      const int p = 16 * pj + l16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = 16 * ni + 4 * lg + i;
        if (p < P && n < N) {
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
    dt_adt(raw_dt, ldx(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0] + h * a.dt.stride[2]),
           ldx(a.a.ptr, a.a.dtype, b * a.a.stride[0] + h * a.a.stride[2]),
           raw_dt ? ldx(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]) : 0.f, dt0,
           adt0);
    const float tr0 = sigmoidf(ldx(a.trap.ptr, a.trap.dtype,
                                   b * a.trap.stride[0] + h * a.trap.stride[2]));
    const float c0 = dt0 * (1.f - tr0);
#pragma unroll
    for (int k = 0; k < kTiles; ++k) {
      const int u = w + kWaves * k;
      if (u >= n_tiles) continue;
      const int ni = u / kPT, pj = u - ni * kPT;
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

  // ---- per-token reads
  Feed<T, R, FULL, SHAPE> fd;
  fd.init(a, g, prep, b, h, grp, rp, n0, vp, p0, N, P, norm);
  if constexpr (MSPLIT) fd.d_hi = (col_of(4) - n0) * ES;
  float* fph = a.final_phase.ptr != nullptr
                   ? static_cast<float*>(a.final_phase.ptr) + b * a.final_phase.stride[0] +
                         h * a.final_phase.stride[1] + ps * a.final_phase.stride[2]
                   : nullptr;
  float* fblk = a.block_phase.ptr != nullptr
                    ? static_cast<float*>(a.block_phase.ptr) + b * a.block_phase.stride[0] +
                          h * a.block_phase.stride[1] + ps * a.block_phase.stride[3]
                    : nullptr;
  const int64_t blk_stride = a.block_phase.stride[2];
  const __amdgpu_buffer_rsrc_t rs_o =
      make_rsrc(FIX ? const_cast<char*>(g.out_base) + b * g.out_b : nullptr,
                FIX ? L * (g.out_t < 0 ? -g.out_t : g.out_t) : 0);
  T* out_row = nullptr;
  int out_t = 0, o_out = 0;
  if constexpr (FIX) {
    out_t = g.out_t;
    o_out = h * g.out_h + g.out_o0;
  } else {
    out_row = static_cast<T*>(a.out.ptr) + b * a.out.stride[0] + h * a.out.stride[2];
    out_t = static_cast<int>(a.out.stride[1]);
  }

  // rotation roles of the q / k lane's 8 columns n0 + i: partner element, cos / sin table
  // column and the sign of the sine term; columns outside the rotated range keep cos 1, sin 0
  int rcol[8];
  float rsgn[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int n = n0 + i;
    if (!mimo_rot) {
      const int jn = n >> 1;
      rcol[i] = min(jn, max(S - 1, 0));
      rsgn[i] = jn < S ? ((i & 1) ? 1.f : -1.f) : 0.f;
    } else {
      const bool first = n < S, third = n >= 2 * S && n < 3 * S;
      rcol[i] = first ? n : (third ? n - 2 * S : 0);
      rsgn[i] = first ? -1.f : (third ? 1.f : 0.f);
    }
  }

  // ---- registers the global data of coming sub-chunks is loaded into
  constexpr int W8 = Words<T>::W8, W4 = Words<T>::W4;
  uint32_t rq[2][W8], rk[2][W8], rv[2][W4], rz[2][W4];
  float2 side;   // this lane's side word of a coming sub-chunk
  float4 ang;    // this lane's angle word of a coming sub-chunk
  const int nsub = g.nsub, scw = g.scw;
  const int side_n = scw + 2 * ROWS;  // floats of a side block
  float* ANG = F + Lay::ANG;
  // angle tile slot (16 bytes) of 4-token group g and angle s: rows of kSMax slots, the angle
  // XOR-keyed by the group's phase lane, so the PG lanes reading one angle and the lanes writing
  // one group hit distinct banks (key < 16, so s ^ key < kSMax)
  static_assert(16 % PG == 0 && 16 / PG * (PG - 1) < kSMax, "angle tile key");
  auto ang_slot = [&](int g, int s) { return g * kSMax + (s ^ ((g / (TPL / 4)) * (16 / PG))); };
  auto ang_store = [&](const float4& v) {
    if (4 * tid < TOK * S) {
      const int g = tid / S;
      *reinterpret_cast<float4*>(ANG + 4 * ang_slot(g, tid - g * S)) = v;
    }
  };
  // the angle inputs of this phase lane's tokens, from the angle tile
  auto angles_of = [&](float (&pa)[TPL]) {
#pragma unroll
    for (int q = 0; q < TPL / 4; ++q) {
      const float4 v = *reinterpret_cast<const float4*>(ANG + 4 * ang_slot((TPL / 4) * pg + q, ps));
      pa[4 * q] = v.x;
      pa[4 * q + 1] = v.y;
      pa[4 * q + 2] = v.z;
      pa[4 * q + 3] = v.w;
    }
  };
  auto scb = [&](int c) { return F + Lay::SC0 + (c & 1) * Lay::SCB; };
  auto csb = [&](int c) { return F + Lay::CS0 + (c & 1) * Lay::CSB; };

  // Pipeline: iteration c stages sub-chunk c into LDS and writes the side block and angle tile of
  // c + 1 there (interval 1), then computes the outputs and state carry of c while the phases of
  // c + 1 are computed and the loads of c + 1 (words) and c + 2 (side, angles) are in flight
  // (interval 2). Side blocks and cos / sin tables alternate between two LDS buffers each.
  // prologue: side block and angle tile of 0 to LDS, phases of 0
  side = fd.side_in(0);
  ang = fd.ang_in(0);
  fd.words(0, min(TOK, L), qk_on, vz_on, rq, rk, rv, rz);
  if (2 * tid < side_n) *reinterpret_cast<float2*>(scb(0) + 2 * tid) = side;
  ang_store(ang);
  side = fd.side_in(1);
  ang = fd.ang_in(1);
  __syncthreads();
  if (ph_on && nsub > 0) {
    float pa[TPL];
    angles_of(pa);
    phase_stage<PG, TPL, CST, SPLIT, F32>(csb(0), ps, F + Lay::PBASE + ps, F + Lay::POFF + ps,
                                     scb(0) + SB_::DTV, 0, L, pg, lane, angles, pa, fph, fblk,
                                     blk_stride);
  }
  __syncthreads();

  float log_decay = 0.f;  // sum of adt so far: the log of the state's decay over the sequence
  for (int c = 0; c < nsub; ++c) {
    const int t0 = c * TOK;
    const int width = min(TOK, L - t0);
    const float* SC = scb(c);
    const float* CSt = csb(c);

    // ---- interval 1: stage sub-chunk c; the scalar block of c + 1 to LDS
    if (c + 1 < nsub) {
      if (2 * tid < side_n) *reinterpret_cast<float2*>(scb(c + 1) + 2 * tid) = side;
      ang_store(ang);
    }
    // q / k rows -> Qs, Ks (row-major), FP32 KT (transposed, swizzled); rows 2rp, 2rp+1.
    // SPLIT: one copy of the code per column half, rotated (waves 0-3) or not, so no values
    // merge between the two.
    auto stage_qk = [&](auto rot_tag) {
      constexpr bool ROT = decltype(rot_tag)::value;
      // (q, k) RMSNorm factors of rows 2rp, 2rp+1
      float fq[2] = {1.f, 1.f}, fk[2] = {1.f, 1.f};
      if (norm) {
        const float4 f = *reinterpret_cast<const float4*>(SC + scw + 4 * rp);
        fq[0] = f.x;
        fk[0] = f.y;
        fq[1] = f.z;
        fk[1] = f.w;
      }
      float kt[2][8];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int row = 2 * rp + j, tt = row / R;
        float q[8], k[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          q[i] = fmaf(raw_get<T>(rq[j], i), fq[j] * wq[i], bq[R == 1 ? 0 : j][i]);
          k[i] = fmaf(raw_get<T>(rk[j], i), fk[j] * wk[i], bk[R == 1 ? 0 : j][i]);
        }
        if constexpr (MSPLIT) {
          // pairs (n0 + i, n0 + 64 + i), angles n0 + i, i < 4 (waves 0-3)
          if (ROT) {
            const float* tr = CSt + tt * CST;
            const f4 c01 = *reinterpret_cast<const f4*>(tr + 2 * n0);
            const f4 c23 = *reinterpret_cast<const f4*>(tr + 2 * n0 + 4);
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const f4& cv = pp < 2 ? c01 : c23;
              const float cc = cv[2 * (pp & 1)], ss = cv[2 * (pp & 1) + 1];
              const float q0 = q[pp], q1 = q[pp + 4];
              const float k0 = k[pp], k1 = k[pp + 4];
              q[pp] = fmaf(q0, cc, -(q1 * ss));
              q[pp + 4] = fmaf(q0, ss, q1 * cc);
              k[pp] = fmaf(k0, cc, -(k1 * ss));
              k[pp + 4] = fmaf(k0, ss, k1 * cc);
            }
          }
        } else if constexpr (SPLIT) {
          // pairs (2j, 2j+1), j = n0/2 .. n0/2+3: the rotated columns are waves 0-3's (SHAPE:
          // when the call rotates)
          if (ROT && (FULL || rotate)) {
            const float* tr = CSt + tt * CST;
            const f4 c01 = *reinterpret_cast<const f4*>(tr + 2 * cs_col<true>(n0 >> 1, tt));
            const f4 c23 = *reinterpret_cast<const f4*>(tr + 2 * cs_col<true>((n0 >> 1) + 2, tt));
            // c01 = c0 s0 c1 s1, c23 = c2 s2 c3 s3
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const f4& cv = pp < 2 ? c01 : c23;
              const float cc = cv[2 * (pp & 1)], ss = cv[2 * (pp & 1) + 1];
              const float q0 = q[2 * pp], q1 = q[2 * pp + 1];
              const float k0 = k[2 * pp], k1 = k[2 * pp + 1];
              q[2 * pp] = fmaf(q0, cc, -(q1 * ss));
              q[2 * pp + 1] = fmaf(q0, ss, q1 * cc);
              k[2 * pp] = fmaf(k0, cc, -(k1 * ss));
              k[2 * pp + 1] = fmaf(k0, ss, k1 * cc);
            }
          }
        } else if (rotate) {
          // x' = x cos + sgn partner sin: SISO pairs (2j, 2j+1), MIMO pairs (n, n + N/2)
          float qp[8], kp[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (!mimo_rot) {
              qp[i] = q[i ^ 1];
              kp[i] = k[i ^ 1];
            } else {
              const int half = N >> 1;
              if (FULL) {
                // N = 128: the partner lane is lane ^ 8, a rotation by 8 in the 16-lane row
                qp[i] = dpp_shr<0x128>(q[i]);
                kp[i] = dpp_shr<0x128>(k[i]);
              } else if (half >= 8) {
                qp[i] = __shfl_xor(q[i], half >> 3, 16);
                kp[i] = __shfl_xor(k[i], half >> 3, 16);
              } else {
                qp[i] = q[i ^ half];
                kp[i] = k[i ^ half];
              }
            }
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float2 cs = *reinterpret_cast<const float2*>(CSt + tt * CST + 2 * rcol[i]);
            const float cc = rsgn[i] != 0.f ? cs.x : 1.f;
            const float ss = rsgn[i] * cs.y;
            q[i] = fmaf(qp[i], ss, q[i] * cc);
            k[i] = fmaf(kp[i], ss, k[i] * cc);
          }
        }
        if (MSPLIT && ROT) {
          f4 lo, hi;
#pragma unroll
          for (int i = 0; i < 4; ++i) { lo[i] = q[i]; hi[i] = q[i + 4]; }
          if constexpr (!SO) {
            st_quad<T>(Qs + row * LQ + n0, lo);
            st_quad<T>(Qs + row * LQ + n0 + 64, hi);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) { lo[i] = k[i]; hi[i] = k[i + 4]; }
          st_quad<T>(Ks + row * LQ + ks_col<!KSW>(row, n0), lo);
          st_quad<T>(Ks + row * LQ + ks_col<!KSW>(row, n0 + 64), hi);
        } else {
          if constexpr (!SO) st_row8<T>(Qs + row * LQ + n0, q);
          st_row8<T>(Ks + row * LQ + ks_col<!KSW>(row, n0), k);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) kt[j][i] = k[i];
      }
      // (FP32) K^T for the carry, each row scaled by its token's scale * end decay (the
      // carry's K~ e^{cum_last - cum}, ops.py:806-816)
      if constexpr (!KTR) {
        const int r0 = (2 * rp) / R, r1 = (2 * rp + 1) / R;
        const float cl = SC[SB_::CL];
        const float e0 = SC[SB_::SCL + r0] * __expf(cl - SC[SB_::CUM + r0]);
        const float e1 = SC[SB_::SCL + r1] * __expf(cl - SC[SB_::CUM + r1]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int n = col_of(i);
          if (FIX || n < N) {
            st_pair<T>(KT + n * LR + swz<ROWS>(2 * rp, n >> KSH), kt[0][i] * e0, kt[1][i] * e1);
          }
        }
      }
    };
    if constexpr (SPLIT || MSPLIT) {
      if (w < 4) {
        stage_qk(std::true_type{});
      } else {
        stage_qk(std::false_type{});
      }
    } else if (qk_on) {
      stage_qk(std::false_type{});
    }
    // value / gate of tokens 2vp, 2vp+1, columns p0 .. p0+3: rank values v mx_r -> VR
    // (row-major; 16-bit also VS, scaled; FP32 VT, transposed and swizzled), rank gates z mz_r
    // -> ZR (row-major)
    if (vz_on) {
      constexpr int VJ = Feed<T, R, FULL>::VJ;
      float v[VJ][4], z[VJ][4];
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[j][i] = raw_get<T>(rv[j], i);
          z[j][i] = raw_get<T>(rz[j], i);
        }
      }
      // (16-bit) rows 2vp, 2vp+1 of VS: the token's scale * end decay (the carry's
      // e^{cum_last - cum} K~ factor, ops.py:806-816, moved onto V)
      float ev0 = 0.f, ev1 = 0.f;
      if constexpr (KTR) {
        const int u0 = (2 * vp) / R, u1 = (2 * vp + 1) / R;
        const float cl = SC[SB_::CL];
        ev0 = SC[SB_::SCL + u0] * __expf(cl - SC[SB_::CUM + u0]);
        ev1 = SC[SB_::SCL + u1] * __expf(cl - SC[SB_::CUM + u1]);
      }
      if (R == 1 && !F32) {
        // the loaded 16-bit words go to LDS unchanged as VR / ZR rows; VS rows scaled
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          f4 sv;
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[i] = v[j][i] * (j ? ev1 : ev0);
          st_quad<T>(VS + (2 * vp + j) * LP + p0, sv);
          if constexpr (SO) continue;
          *reinterpret_cast<u32x2*>(VR + (2 * vp + j) * LP + p0) = (u32x2){rv[j][0], rv[j][1]};
          *reinterpret_cast<u32x2*>(ZR + (2 * vp + j) * LP + p0) = (u32x2){rz[j][0], rz[j][1]};
        }
      } else if (R == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int p = p0 + i;
          if (FIX || p < P) st_pair<T>(VT + p * LR + swz<ROWS>(2 * vp, p >> VSH), v[0][i], v[1][i]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          if constexpr (SO) break;
          f4 vq, zq;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            vq[i] = v[j][i];
            zq[i] = z[j][i];
          }
          st_quad<T>(VR + (2 * vp + j) * LP + p0, vq);
          st_quad<T>(ZR + (2 * vp + j) * LP + p0, zq);
        }
      } else {
        // rows 2vp, 2vp+1: ranks r0, r0 + 1 of token 2vp / R (every lane of the workgroup has a
        // row pair, as for R = 1)
        f4 vq[2];
#pragma unroll
        for (int jr = 0; jr < 2; ++jr) {
          const int row = 2 * vp + jr;
          f4 zq;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            vq[jr][i] = mul_r<T>(v[0][i], mxl[jr][i]);
            zq[i] = mul_r<T>(z[0][i], mzl[jr][i]);
          }
          if constexpr (!SO) {
            st_quad<T>(VR + row * LP + p0, vq[jr]);
            st_quad<T>(ZR + row * LP + p0, zq);
          }
        }
        if constexpr (KTR) {
#pragma unroll
          for (int jr = 0; jr < 2; ++jr) {
            f4 sv;
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[i] = vq[jr][i] * (jr ? ev1 : ev0);
            st_quad<T>(VS + (2 * vp + jr) * LP + p0, sv);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int p = p0 + i;
            if (FIX || p < P) st_pair<T>(VT + p * LR + swz<ROWS>(2 * vp, p >> VSH), vq[0][i], vq[1][i]);
          }
        }
      }
    }
    // the state at the start of this sub-chunk, rounded to the activation dtype -> Sb[p][n]
#pragma unroll
    for (int k = 0; k < kTiles; ++k) {
      const int u = w + kWaves * k;
      if (!SO && (all_tiles || u < n_tiles)) {
        const int ni = u / kPT, pj = u - ni * kPT;
        st_quad<T>(Sb + (16 * pj + l16) * LQ + 16 * ni + 4 * lg, st[k]);
      }
    }
    // the carry's decay of the state, exp(cum_last) S^T: the carry products below accumulate
    // onto it
    {
      const float ecl = SC[SB_::ECL];
      log_decay += SC[SB_::CL];
#pragma unroll
      for (int k = 0; k < kTiles; ++k) {
#pragma unroll
        for (int i = 0; i < 4; ++i) st[k][i] *= ecl;
      }
    }
    __syncthreads();

    // ---- interval 2
    // words of sub-chunk c + 1 into registers; they fly while sub-chunk c computes. FULL issues
    // every load of the loop unconditionally (reads past token L return zero), which keeps the
    // compiler's in-order wait counts exact: no load is waited for before its use. FULL spreads
    // them over the interval in three groups (q / k at its start, value / gate after the
    // scores, side and angle words after the phases) pinned between the compute stages, so the
    // eight waves do not queue all their loads at once.
    auto loads_qk = [&] {
      __builtin_amdgcn_sched_barrier(0);
      fd.words_qk(t0 + TOK, min(TOK, L - t0 - TOK), qk_on, rq, rk);
      __builtin_amdgcn_sched_barrier(0);
    };
    auto loads_vz = [&] {
      __builtin_amdgcn_sched_barrier(0);
      fd.words_vz(t0 + TOK, min(TOK, L - t0 - TOK), vz_on, rv, rz);
      __builtin_amdgcn_sched_barrier(0);
    };
    auto loads_side = [&] {
      __builtin_amdgcn_sched_barrier(0);
      side = fd.side_in(c + 2);
      ang = fd.ang_in(c + 2);
      __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (!FULL && !SHAPE) {
      if (c + 1 < nsub) fd.words(t0 + TOK, min(TOK, L - t0 - TOK), qk_on, vz_on, rq, rk, rv, rz);
      side = fd.side_in(c + 2);
      ang = fd.ang_in(c + 2);
    }

    // (q / k words first: they are waited for first, at the top of the next iteration)
    if constexpr (FULL || SHAPE) loads_qk();

    // outputs for query row tile `it` and P tiles pj = wp, wp + WPR, ...
    const int it = w / WPR, wp = w - it * WPR;
    const int trow = 16 * it + l16;
    const int tq = trow / R;
    // 16-bit: the query rows of this tile, B operand of the scores and A operand of inter
    typename M::v8 qv[F32 ? 1 : NP / 32];
    if constexpr (!F32 && !SO) {
#pragma unroll
      for (int kk = 0; kk < NP / 32; ++kk) {
        qv[kk] = *reinterpret_cast<const typename M::v8*>(Qs + trow * LQ + 32 * kk + 8 * lg);
      }
    }
    // scores Sc^T tiles (rows s, column t), issued before the phase work below
    f4 acc[RT];
#pragma unroll
    for (int sj = 0; sj < RT; ++sj) {
      acc[sj] = zero4();
      if (SO || sj > it) continue;
      if constexpr (!F32) {
#pragma unroll
        for (int kk = 0; kk < NP / 32; ++kk) {
          const typename M::v8 av = *reinterpret_cast<const typename M::v8*>(
              Ks + (16 * sj + l16) * LQ + ks_col<!KSW>(l16, 32 * kk + 8 * lg));
          acc[sj] = M::mma(av, qv[kk], acc[sj]);
        }
      } else {
#pragma unroll 8
        for (int kk = 0; kk < NP; kk += 4) {
          acc[sj] = M::mma(Ks[(16 * sj + l16) * LQ + kk + lg], Qs[trow * LQ + kk + lg], acc[sj]);
        }
      }
    }
    // K~^T V products of the state carry, issued early (they depend only on staged tiles),
    // accumulated onto the decayed state
#pragma unroll
    for (int k = 0; k < kTiles; ++k) {
      const int u = w + kWaves * k;
      if (!all_tiles && u >= n_tiles) continue;
      const int ni = u / kPT, pj = u - ni * kPT;
      const int nrow = 16 * ni + l16, prow = 16 * pj + l16;
      if constexpr (KTR) {
        // A: 8 tokens of column nrow from the row-major Ks, two transposing reads of 4 tokens
        // (in each 16-lane group, lane 4a + b receives element b of the 8-byte vectors of lanes
        // a, a + 4, a + 8, a + 12: lane x addresses token x / 4, columns 4 (x % 4) ..)
        const T* kc = Ks + (l16 >> 2) * LQ + ks_col<!KSW>(l16 >> 2, 16 * ni + 4 * (l16 & 3));
        const T* vc = VS + (l16 >> 2) * LP + 16 * pj + 4 * (l16 & 3);  // B: the same from VS
#pragma unroll
        for (int kk = 0; kk < ROWS; kk += 32) {
          const T* k0 = kc + (kk + 8 * lg) * LQ;
          const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(k0));
          const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(k0 + 4 * LQ));
          const typename M::v8 av = __builtin_bit_cast(
              typename M::v8, (i16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
          const T* v0 = vc + (kk + 8 * lg) * LP;
          const i16x4 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(v0));
          const i16x4 vhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(v0 + 4 * LP));
          const typename M::v8 bv = __builtin_bit_cast(
              typename M::v8, (i16x8){vlo[0], vlo[1], vlo[2], vlo[3], vhi[0], vhi[1], vhi[2], vhi[3]});
          st[k] = M::mma(av, bv, st[k]);
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < ROWS; kk += 4) {
          st[k] = M::mma(KT[nrow * LR + swz<ROWS>(kk + lg, nrow >> KSH)],
                         VT[prow * LR + swz<ROWS>(kk + lg, prow >> VSH)], st[k]);
        }
      }
    }
    if constexpr (FULL || SHAPE) loads_vz();
    // phases of sub-chunk c + 1 (its dt block was computed two iterations ago)
    if (ph_on && c + 1 < nsub) {
      float pa[TPL];
      angles_of(pa);
      phase_stage<PG, TPL, CST, SPLIT, F32>(csb(c + 1), ps, F + Lay::PBASE + ps, F + Lay::POFF + ps,
                                       scb(c + 1) + SB_::DTV, t0 + TOK, L, pg, lane, angles, pa,
                                       fph, fblk, blk_stride);
    }
    if constexpr (FULL || SHAPE) loads_side();
    if constexpr (SO) {
      __syncthreads();
      continue;
    }
    // decayed scores W[t, s] = Sc[t, s] d[t, s] in FP32
    const float cum_t = SC[SB_::CUM + tq];
    const float gam_t = SC[SB_::GAM + tq];
    // the causal masks below compare a copy of tq the compiler cannot see through, so they are
    // evaluated here as vector compares, not hoisted out of the loop into scalar mask registers
    int tq_m = tq;
    __asm__ volatile("" : "+v"(tq_m));
    f4 wsc[RT];
#pragma unroll
    for (int sj = 0; sj < RT; ++sj) {
      wsc[sj] = zero4();
      if (sj > it) continue;
      if (sj < it) {
        // strictly earlier tile: d = exp(cum_t - cend) * (scale_s exp(cend - cum_s)), both <= 1
        const float at = __expf(cum_t - SC[SB_::CEND + sj]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int ts = (16 * sj + 4 * lg + i) / R;
          wsc[sj][i] = acc[sj][i] * (at * SC[SB_::BSC + ts]);
        }
      } else {
        // diagonal tile: every term is read and computed, then selected (no per-lane branches)
        float cs[4], sc[4];
        if constexpr (R == 1) {
          const f4 c4 = *reinterpret_cast<const f4*>(SC + SB_::CUM + 16 * sj + 4 * lg);
          const f4 s4 = *reinterpret_cast<const f4*>(SC + SB_::SCL + 16 * sj + 4 * lg);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            cs[i] = c4[i];
            sc[i] = s4[i];
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int ts = (16 * sj + 4 * lg + i) / R;
            cs[i] = SC[SB_::CUM + ts];
            sc[i] = SC[SB_::SCL + ts];
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int ts = (16 * sj + 4 * lg + i) / R;
          const float lower = sc[i] * __expf(cum_t - cs[i]);
          const float d = tq_m > ts ? lower : (tq_m == ts ? gam_t : 0.f);
          wsc[sj][i] = acc[sj][i] * d;
        }
      }
    }
    // Outputs, computed transposed (Y^T tiles, rows p, columns the row tile's 16 (token, rank)
    // rows): a lane holds 4 consecutive p of one row, stored as one vector.
    const float ecum_t = __expf(cum_t);
    const int rr = trow - tq * R;  // the lane's rank
#pragma unroll
    for (int pq = 0; pq < kPT / WPR; ++pq) {
      const int pj = wp + pq * WPR;
      const int pcol = 16 * pj + l16;  // the A-operand row of V^T / rnd(S)
      const int key = pcol >> VSH;
      f4 yi = zero4(), ye = zero4();
      if constexpr (!F32) {
        // intra: V^T W^T, the K axis permuted as the D-layout of wsc
#pragma unroll
        for (int m = 0; m < (RT + 1) / 2; ++m) {
          if (2 * m > it) continue;
          typename M::v8 av, bv;
          // 4 tokens of column pcol from the row-major VR by a transposing read each
          const T* vr0 = VR + (32 * m + 4 * lg + (l16 >> 2)) * LP + 16 * pj + 4 * (l16 & 3);
          const typename M::v4 b0 = __builtin_bit_cast(
              typename M::v4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                  (__attribute__((address_space(3))) i16x4*)(vr0)));
          const typename M::v4 b1 = __builtin_bit_cast(
              typename M::v4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                  (__attribute__((address_space(3))) i16x4*)(vr0 + 16 * LP)));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            bv[i] = from_f<T>(wsc[2 * m][i]);
            bv[4 + i] = from_f<T>(2 * m + 1 < RT ? wsc[2 * m + 1][i] : 0.f);
            av[i] = b0[i];
            av[4 + i] = b1[i];
          }
          yi = M::mma(av, bv, yi);
        }
        // inter: rnd(S) Q^T
#pragma unroll
        for (int kk = 0; kk < NP / 32; ++kk) {
          const typename M::v8 av =
              *reinterpret_cast<const typename M::v8*>(Sb + pcol * LQ + 32 * kk + 8 * lg);
          ye = M::mma(av, qv[kk], ye);
        }
      } else {
#pragma unroll
        for (int sj = 0; sj < RT; ++sj) {
          if (sj > it) continue;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            yi = M::mma(VT[pcol * LR + swz<ROWS>(16 * sj + 4 * lg + i, key)], wsc[sj][i], yi);
          }
        }
#pragma unroll 8
        for (int kk = 0; kk < NP; kk += 4) {
          ye = M::mma(Sb[pcol * LQ + kk + lg], Qs[trow * LQ + kk + lg], ye);
        }
      }
      // epilogue: row trow (token tq, rank rr), columns pb .. pb+3
      const int pb = 16 * pj + 4 * lg;
      float vv[4], zz[4];
      if constexpr (!F32) {
        const typename M::v4 v4 = *reinterpret_cast<const typename M::v4*>(VR + trow * LP + pb);
        const typename M::v4 z4 = *reinterpret_cast<const typename M::v4*>(ZR + trow * LP + pb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          vv[i] = to_f(v4[i]);
          zz[i] = to_f(z4[i]);
        }
      } else {
        const f4 v4 = *reinterpret_cast<const f4*>(VR + trow * LP + pb);
        const f4 z4 = *reinterpret_cast<const f4*>(ZR + trow * LP + pb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          vv[i] = v4[i];
          zz[i] = z4[i];
        }
      }
      f4 y;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        y[i] = (fmaf(ye[i], ecum_t, yi[i]) + Dh * vv[i]) * silu_fast(zz[i]);
        if (R > 1) y[i] *= F[Lay::MO + rr * kPPad + pb + i];
      }
      if constexpr (R > 1) {
        // MIMO rank sum over the R consecutive lanes of one token (within a 16-lane row): DPP
        // quad permutes for lane ^ 1 and lane ^ 2, a swizzle for lane ^ 4 (no LDS access)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float t = y[i];
          t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                             0, __builtin_bit_cast(int, t), 0xb1, 0xf, 0xf, false));
          if constexpr (R >= 4) {
            t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                               0, __builtin_bit_cast(int, t), 0x4e, 0xf, 0xf, false));
          }
          if constexpr (R >= 8) {
            t += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, t),
                                                                       0x101f));
          }
          y[i] = t;
        }
      }
      if (rr == 0) {
        if constexpr (FIX) {
          // rows of tokens >= L fall outside the buffer extent: the store is dropped
          bstore_quad<T>(y, rs_o,
                         (tq * out_t + o_out + pb * ES) +
                             __builtin_amdgcn_readfirstlane(t0 * out_t));
        } else {
          if (tq < width) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (pb + i < P) out_row[(t0 + tq) * out_t + pb + i] = from_f<T>(y[i]);
            }
          }
        }
      }
    }

    // (the state carry S^T = exp(cum_last) S^T + K~^T V was accumulated above)
    __syncthreads();
  }

  // ---- final k: the biased, rotated k of token L-1, still in Ks from the last sub-chunk
  if (a.final_k.ptr != nullptr && L > 0) {
    const int tl = (L - 1) - (nsub - 1) * TOK;  // its row in the last sub-chunk
    for (int i = tid; i < R * N; i += kThreads) {
      const int r = i / N, n = i - r * N;
      static_cast<T*>(a.final_k.ptr)[b * a.final_k.stride[0] + h * a.final_k.stride[1] +
                                     r * a.final_k.stride[2] + n] =
          Ks[(tl * R + r) * LQ + ks_col<!KSW>(tl * R + r, n)];
    }
  }

  if (a.final_decay.ptr != nullptr && tid == 0) {
    static_cast<float*>(a.final_decay.ptr)[b * a.final_decay.stride[0] +
                                           h * a.final_decay.stride[1]] = log_decay;
  }
  // the last block's increment sum (the earlier blocks' were written as each one ended)
  if (a.block_phase.ptr != nullptr && rotate && angles && L > 0) {
    for (int i = tid; i < S; i += kThreads) {
      static_cast<float*>(a.block_phase.ptr)[b * a.block_phase.stride[0] +
                                             h * a.block_phase.stride[1] +
                                             ((L - 1) >> 6) * a.block_phase.stride[2] +
                                             i * a.block_phase.stride[3]] = F[Lay::PBASE + i];
    }
  }

  // ---- final state
#pragma unroll
  for (int k = 0; k < kTiles; ++k) {
    const int u = w + kWaves * k;
    if (u >= n_tiles) continue;
    const int ni = u / kPT, pj = u - ni * kPT;
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


// ------------------------------------------------------------ 16-wave SISO scan

// scan16_kernel<T, R, SO>: the model's shape in projection form (ranks 1 and 4, N = 128, P = 64,
// 32 angles, one group, 16-bit activations; forwards or backwards) with 1024 threads, so that
// four waves share each SIMD to hide one another's LDS, MFMA and transcendental latency. A
// sub-chunk is 64 rows (token, rank), rank minor: 64 tokens at rank 1, 16 at rank 4, whose
// decay weights, phases and scalars are per token and whose output sums the token's R rows
// (times mimo_out). Per sub-chunk, three intervals between workgroup barriers:
//   A  staging (every wave): row qt's q / k (bias and rotation on prep's normalized rows; waves
//      0-7 the rotated columns, waves 8-15 the others) -> Qs, Ks; row vt's value / gate (times
//      the rounded mimo_x / mimo_z at rank 4) -> VR, ZR and the carry's scaled values -> VS; the
//      state, rounded -> Sb; the side block and angle tile of the next sub-chunk -> LDS;
//   B  waves 0-9 one causal score tile each (Sc^T = K Q^T) and its decay weights W -> WS;
//      every wave the carry products of its two state tiles; the next sub-chunk's global loads
//      are issued here;
//   C  wave w the output tile (row tile w / 4, P tile w % 4): intra V^T W^T from WS, inter
//      rnd(S) Q^T, epilogue, store; waves 0-7, whose row tiles 0 and 1 have the shortest intra
//      products, also the phases of the next sub-chunk (a long dependent chain per wave).
// Same mathematics and rounding points as scan_kernel<T, R, true> (whose header lists them), but
// for q / k, which start from prep's rows rounded after the RMSNorm (the reference's rounding
// point, model.py:48-55).

constexpr int k16Threads = 1024;

// LDS layout, 16-bit elements unless noted. The strides and swizzles make every access pattern
// of the kernel conflict-free under the measured gfx950 LDS behaviour: 16-byte reads of 16 rows
// at one 16-byte chunk (the MFMA operands) with 288-byte rows or an XOR swizzle of 256-byte rows;
// 8-byte accesses (stores, transposing reads) 32 lanes at a time over 64 banks of 4 bytes, so
// the 32 lanes' 8-byte pieces must cover 256 distinct bytes.
//   Qs, Ks  [64 tokens][144]: 288-byte rows
//   Sb      [64 p][128]: 256-byte rows, 16-byte chunk c of row p at c ^ (p % 16) (sb_off)
//   VR, ZR, VS [64 tokens][64]: 128-byte rows, 32-byte pair and chunk half swizzled (v_off)
//   WS      [64 t][80]: 160-byte rows
struct Lay16 {
  static constexpr int ROWS = 64, LQ = kNPad + 16, LS = kNPad, LV = kPPad, LW = kPPad + 16, ES = 2;
  static constexpr int QS = 0;
  static constexpr int KS = QS + ROWS * LQ * ES;
  static constexpr int VR = KS + ROWS * LQ * ES;
  static constexpr int ZR = VR + ROWS * LV * ES;
  static constexpr int VS = ZR + ROWS * LV * ES;
  static constexpr int SB = VS + ROWS * LV * ES;
  static constexpr int WS = SB + kPPad * LS * ES;  // decay weights [t][s'] (s' permuted, below)
  static constexpr int FB = WS + ROWS * LW * ES;
  // floats from FB: two side blocks (scalar blocks), the angle tile, two cos / sin tables, the
  // phase block sum and carry per angle
  static constexpr int SCB = 5 * ROWS + 8, SC0 = 0;
  static constexpr int ANG = SC0 + 2 * SCB;
  static constexpr int CST = 2 * kSMax + 4, CSB = ROWS * CST;
  static constexpr int CS0 = ANG + ROWS * kSMax, PBASE = CS0 + 2 * CSB, POFF = PBASE + kSMax;
  // rank 4: the rounded mimo_x, mimo_z and mimo_out [R][P]
  static constexpr int MX = POFF + kSMax, MZ = MX + 4 * kPPad, MO = MZ + 4 * kPPad;
  static constexpr int BYTES = FB + 4 * (MO + 4 * kPPad);
};
static_assert(Lay16::BYTES <= 160 * 1024, "scan16 LDS layout exceeds 160 KiB");
static_assert(Lay16::FB % 16 == 0 && Lay16::WS % 16 == 0 && Lay16::SB % 16 == 0 &&
              (Lay16::ANG * 4) % 16 == 0 && (Lay16::CS0 * 4) % 16 == 0, "alignment");

// Element offset of column `col` of state row p in Sb (16-byte chunks XOR-swizzled by row).
__device__ __forceinline__ int sb_off(int p, int col) {
  return p * Lay16::LS + 8 * ((col >> 3) ^ (p & 15)) + (col & 7);
}

// Element offset of column `col` of token row r in VR, ZR, VS: the row's 32-byte pair
// (col / 16) XOR (r / 2) % 4 and the chunk within it flipped by (r / 8) % 2. Eight consecutive
// rows then place one pair in eight distinct 32-byte bank groups (the transposing reads), and
// sixteen consecutive rows one chunk in sixteen distinct 16-byte groups (the epilogue reads).
__device__ __forceinline__ int v_off(int r, int col) {
  const int c = col >> 3;
  const int pc = 2 * ((c >> 1) ^ ((r >> 1) & 3)) + ((c & 1) ^ ((r >> 3) & 1));
  return r * Lay16::LV + 8 * pc + (col & 7);
}

// The causal score tiles (row tile it, column tile sj <= it) of waves 0-9: the diagonal tiles,
// whose decay weights take the most arithmetic, on waves 0-3 (one per SIMD).
__device__ __forceinline__ void score_tile16(int w, int& it, int& sj) {
  // w: 0 1 2 3 | 4 5 6 7 8 9  ->  (0,0) (1,1) (2,2) (3,3) | (1,0) (2,0) (2,1) (3,0) (3,1) (3,2)
  const int k = w - 4;
  it = w < 4 ? w : (k < 1 ? 1 : (k < 3 ? 2 : 3));
  sj = w < 4 ? w : (k < 1 ? 0 : (k < 3 ? k - 1 : k - 3));
}

template <typename T, int R, bool SO>
__global__ __launch_bounds__(k16Threads) void scan16_kernel(const m3_scan_args a,
                                                            const ScanGeom g,
                                                            const float* __restrict__ prep) {
  static_assert(R == 1 || R == 4, "scan16_kernel: ranks 1 and 4");
  using M = Mma<T>;
  using Ly = Lay16;
  constexpr int TOK = 64 / R;  // tokens per 64-row sub-chunk (rows (token, rank), rank minor)
  using SB_ = ScBlk<TOK>;
  constexpr int LQ = Ly::LQ, LW = Ly::LW, CST = Ly::CST, ES = 2, S = kSMax;
  // phase: 16 lanes per angle, TPL tokens per lane (waves 0-7)
  constexpr int PG = 16, TPL = TOK / 16;
  const int H = a.heads, L = a.length;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;

  int bid = blockIdx.x;
  if (g.xcd_map) {
    const int per = gridDim.x >> 3;
    bid = (bid & 7) * per + (bid >> 3);
  }
  const int b = bid / H, h = bid - b * H;

  extern __shared__ __attribute__((aligned(16))) char smem[];
  T* Qs = lds_t<T>(smem, Ly::QS);
  T* Ks = lds_t<T>(smem, Ly::KS);
  T* VR = lds_t<T>(smem, Ly::VR);
  T* ZR = lds_t<T>(smem, Ly::ZR);
  T* VS = lds_t<T>(smem, Ly::VS);
  T* Sb = lds_t<T>(smem, Ly::SB);
  T* WS = lds_t<T>(smem, Ly::WS);
  float* F = lds_t<float>(smem, Ly::FB);
  const float Dh = ldx(a.D.ptr, a.D.dtype, h * a.D.stride[0]);

  // ---- lane roles
  // q / k: rows qt and qt + 32 (rank qr), four columns. Rank 1: n0 .. n0+3, waves 0-7 the
  // rotated columns 0-63 (pairs (2j, 2j+1)). Rank 4 (the MIMO rotation pairs column n with
  // n + 64, n < 32): waves 0-7 columns n0, n0+1, n0+64, n0+65 (n0 = 2 (tid % 16)), waves 8-15
  // four of the unrotated columns 32-63 and 96-127.
  const bool rot = w < 8;
  const int qt = (tid & 511) >> 4, qr = qt & (R - 1);
  const int n0 = R == 1 ? 64 * (tid >> 9) + 4 * (tid & 15)
                        : (rot ? 2 * (tid & 15) : ((tid & 15) < 8 ? 32 : 64) + 4 * (tid & 15));
  auto qcol = [&](int i) { return R > 1 && rot ? n0 + (i & 1) + 64 * (i >> 1) : n0 + i; };
  // value / gate: row vt (token vt / R, rank vt % R), columns p0 .. p0+3
  const int vt = tid >> 4, p0 = 4 * (tid & 15);
  // phase (waves 0-7): angle ps, tokens TPL pg .. TPL pg + 3
  const int ps = tid >> 4, pg = tid & 15;
  const bool ph_wave = w < 8;
  // state tiles (ni, pj), k = 0, 1: ni = w / 2, pj = 2 (w % 2) + k; lane holds
  // n = 16 ni + 4 lg + i, p = 16 pj + l16 (S^T in MFMA accumulator layout)
  const int sni = w >> 1, spj0 = 2 * (w & 1);

  for (int s = tid; s < S; s += k16Threads) {
    F[Ly::PBASE + s] = 0.f;
    F[Ly::POFF + s] = a.initial_phase.ptr != nullptr
                          ? static_cast<const float*>(a.initial_phase.ptr)
                                [b * a.initial_phase.stride[0] + h * a.initial_phase.stride[1] +
                                 s * a.initial_phase.stride[2]]
                          : 0.f;
  }

  // rounded biases of the lane's 4 columns, rank qr (the rows come normalized from prep)
  float bq[4], bk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = qcol(i);
    bq[i] = rnd<T>(ldx(a.q_bias.ptr, a.q_bias.dtype,
                       h * a.q_bias.stride[0] + qr * a.q_bias.stride[1] + n));
    bk[i] = rnd<T>(ldx(a.k_bias.ptr, a.k_bias.dtype,
                       h * a.k_bias.stride[0] + qr * a.k_bias.stride[1] + n));
  }
  if constexpr (R > 1) {
    // the rounded mimo_x / mimo_z and mimo_out of this head (ops.py:700-714, 869-877)
    for (int i = tid; i < R * kPPad; i += k16Threads) {
      const int r = i / kPPad, p = i - r * kPPad;
      F[Ly::MX + i] = rnd<T>(ldx(a.mimo_x.ptr, a.mimo_x.dtype,
                                 h * a.mimo_x.stride[0] + r * a.mimo_x.stride[1] + p));
      F[Ly::MZ + i] = rnd<T>(ldx(a.mimo_z.ptr, a.mimo_z.dtype,
                                 h * a.mimo_z.stride[0] + r * a.mimo_z.stride[1] + p));
      F[Ly::MO + i] = ldx(a.mimo_out.ptr, a.mimo_out.dtype,
                          h * a.mimo_out.stride[0] + r * a.mimo_out.stride[1] + p);
    }
  }

  f4 st[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    st[k] = zero4();
    if (a.initial_state.ptr != nullptr) {
      const int p = 16 * (spj0 + k) + l16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = 16 * sni + 4 * lg + i;
        st[k][i] = static_cast<const float*>(a.initial_state.ptr)
            [b * a.initial_state.stride[0] + h * a.initial_state.stride[1] +
             p * a.initial_state.stride[2] + n];
      }
    }
  }
  // Endpoint continuation (ops.py:681-686): S += dt_0 (1 - trap_0) sum_r (v_prev mx_r) k_prev_r^T.
  if (a.initial_k.ptr != nullptr && L > 0) {
    float dt0, adt0;
    dt_adt(true, ldx(a.dt.ptr, a.dt.dtype, b * a.dt.stride[0] + h * a.dt.stride[2]),
           ldx(a.a.ptr, a.a.dtype, b * a.a.stride[0] + h * a.a.stride[2]),
           ldx(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]), dt0, adt0);
    const float tr0 = sigmoidf(ldx(a.trap.ptr, a.trap.dtype,
                                   b * a.trap.stride[0] + h * a.trap.stride[2]));
    const float c0 = dt0 * (1.f - tr0);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int p = 16 * (spj0 + k) + l16;
      const float v0 = to_f(static_cast<const T*>(a.initial_value.ptr)
                                [b * a.initial_value.stride[0] + h * a.initial_value.stride[1] + p]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = 16 * sni + 4 * lg + i;
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

  // ---- global reads: one buffer resource over the batch row of the projection (its extent
  // ends at token L: rows past it read zero, stores past it are dropped) and one over the
  // workspace; per-lane byte offsets at token 0
  const int tok_b = g.tok_b;
  const __amdgpu_buffer_rsrc_t rs_p =
      make_rsrc(g.proj + b * g.proj_b, L * (tok_b < 0 ? -tok_b : tok_b));
  const __amdgpu_buffer_rsrc_t rs_w = make_rsrc(prep, g.ws_bytes);
  // the normalized q / k rows of batch row b: row (token, rank) at 2 N elements, k after q (rows
  // past token L read zero)
  const __amdgpu_buffer_rsrc_t rs_qk =
      make_rsrc(reinterpret_cast<const char*>(prep) + g.ws_qk +
                    static_cast<int64_t>(b) * L * R * 4 * kNPad,
                L * R * 4 * kNPad);
  const int o_qk = qt * 4 * kNPad + n0 * ES;  // row qt (forward order), column n0 of q
  const int o_vz = g.o_v + h * g.vz_h + (vt / R) * tok_b + p0 * ES, d_z = g.o_z - g.o_v;
  const int nsub = g.nsub, scw = g.scw;
  // side words (waves 0-3, one float pair per lane): the scalar block
  const int q2 = 2 * tid;
  const bool side_on = q2 < scw;
  const int side_o =
      side_on ? static_cast<int>(g.ws_sc + static_cast<int64_t>(b * H + h) * nsub * scw + q2) * 4
              : 0;
  const int side_s = scw * 4;
  // angle words (waves 0-7): 4 tokens of one angle each, in the tile order [TOK / 4][S][4]
  const int ang_o = static_cast<int>(g.ws_ang + static_cast<int64_t>(b) * g.L4 * S * 4 + 4 * tid) * 4;
  const int ang_s = (TOK / 4) * S * 16;
  const bool ang_on = tid < TOK * S / 4;

  float* fph = a.final_phase.ptr != nullptr && ph_wave
                   ? static_cast<float*>(a.final_phase.ptr) + b * a.final_phase.stride[0] +
                         h * a.final_phase.stride[1] + ps * a.final_phase.stride[2]
                   : nullptr;
  float* fblk = a.block_phase.ptr != nullptr && ph_wave
                    ? static_cast<float*>(a.block_phase.ptr) + b * a.block_phase.stride[0] +
                          h * a.block_phase.stride[1] + ps * a.block_phase.stride[3]
                    : nullptr;
  const int64_t blk_stride = a.block_phase.stride[2];
  const __amdgpu_buffer_rsrc_t rs_o =
      make_rsrc(const_cast<char*>(g.out_base) + b * g.out_b, L * (g.out_t < 0 ? -g.out_t : g.out_t));
  const int out_t = g.out_t, o_out = h * g.out_h + g.out_o0;

  // q / k words: [token qt, qt + 32][q, k] 4 elements each
  uint32_t rq[2][2], rk[2][2], rv[2], rz[2];
  float2 side = make_float2(0.f, 0.f);
  float4 ang = make_float4(0.f, 0.f, 0.f, 0.f);
  auto load_qk = [&](int t0) {
    // the rows are stored in the call's token order: logical token t at rows t R .. t R + R - 1
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int o = o_qk + (t0 * R + 32 * j) * 4 * kNPad;
      if (R > 1 && rot) {
        // columns n0, n0 + 1 and their rotation partners n0 + 64, n0 + 65
        rq[j][0] = __builtin_amdgcn_raw_buffer_load_b32(rs_qk, o, 0, 0);
        rq[j][1] = __builtin_amdgcn_raw_buffer_load_b32(rs_qk, o + 128, 0, 0);
        rk[j][0] = __builtin_amdgcn_raw_buffer_load_b32(rs_qk, o + 2 * kNPad, 0, 0);
        rk[j][1] = __builtin_amdgcn_raw_buffer_load_b32(rs_qk, o + 2 * kNPad + 128, 0, 0);
      } else {
        bload_words<2>(rq[j], rs_qk, o);
        bload_words<2>(rk[j], rs_qk, o + 2 * kNPad);
      }
    }
  };
  auto load_vz = [&](int t0) {
    bload_words<2>(rv, rs_p, o_vz + t0 * tok_b);
    bload_words<2>(rz, rs_p, o_vz + t0 * tok_b + d_z);
  };
  auto load_side = [&](int c) {
    if (w < 4) {
      const u32x2 v = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_w, side_o + c * side_s, 0, 0));
      side = make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
    }
    if (w < 8) {
      const u32x4 v = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_w, ang_o + c * ang_s, 0, 0));
      ang = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                        __uint_as_float(v[3]));
    }
  };
  float* ANG = F + Ly::ANG;
  // angle tile slot of 4-token group gq and angle s (XOR-keyed by the group's phase lane)
  auto ang_slot = [&](int gq, int s) { return gq * kSMax + (s ^ gq); };
  auto put_side = [&](int c) {
    if (w < 4 && side_on) *reinterpret_cast<float2*>(F + Ly::SC0 + (c & 1) * Ly::SCB + q2) = side;
    if (w < 8 && ang_on) {
      const int gq = tid / S;
      *reinterpret_cast<float4*>(ANG + 4 * ang_slot(gq, tid - gq * S)) = ang;
    }
  };
  auto scb = [&](int c) { return F + Ly::SC0 + (c & 1) * Ly::SCB; };
  auto csb = [&](int c) { return F + Ly::CS0 + (c & 1) * Ly::CSB; };
  auto phases = [&](int c) {
    // phases of sub-chunk c (waves 0-7), from the angle tile and the dt of its side block
    if (ph_wave && c < nsub) {
      float pa[TPL];
      if constexpr (TPL == 4) {
        const float4 v = *reinterpret_cast<const float4*>(ANG + 4 * ang_slot(pg, ps));
        pa[0] = v.x;
        pa[1] = v.y;
        pa[2] = v.z;
        pa[3] = v.w;
      } else {
        pa[0] = ANG[4 * ang_slot(pg >> 2, ps) + (pg & 3)];  // token pg of its 4-token group
      }
      phase_stage<PG, TPL, CST, true, false>(csb(c), ps, F + Ly::PBASE + ps, F + Ly::POFF + ps,
                                             scb(c) + SB_::DTV, c * TOK, L, pg, lane, true, pa,
                                             fph, fblk, blk_stride);
    }
  };

  // prologue: side block and angle tile of sub-chunk 0, its phases; the loads of 0 and 1
  load_side(0);
  load_qk(0);
  load_vz(0);
  put_side(0);
  load_side(1);
  __syncthreads();
  phases(0);
  __syncthreads();

  float log_decay = 0.f;
  for (int c = 0; c < nsub; ++c) {
    const int t0 = c * TOK;
    const float* SC = scb(c);
    const float* CSt = csb(c);

    // ---- A: staging
    if (c + 1 < nsub) put_side(c + 1);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      // row rw (token tt): q = q^ + bias, k = k^ + bias, rotated. Rank 1: pairs (n0, n0+1),
      // (n0+2, n0+3), angles n0 / 2 and n0 / 2 + 1; rank 4: pairs (n0 + e, n0 + 64 + e), angles
      // n0 + e (e < 2). Both angle pairs are adjacent in the cos / sin table row.
      const int rw = qt + 32 * j, tt = rw / R;
      f4 q, k;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        q[i] = raw_get<T>(rq[j], i) + bq[i];
        k[i] = raw_get<T>(rk[j], i) + bk[i];
      }
      if (rot) {
        const f4 cv = *reinterpret_cast<const f4*>(
            CSt + tt * CST + 2 * cs_col<true>(R == 1 ? n0 >> 1 : n0, tt));
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          // the pair's two columns: (2 pp, 2 pp + 1) for rank 1, (pp, pp + 2) for rank 4
          const int u0 = R == 1 ? 2 * pp : pp, u1 = R == 1 ? 2 * pp + 1 : pp + 2;
          const float cc = cv[2 * pp], ss = cv[2 * pp + 1];
          const float q0 = q[u0], q1 = q[u1];
          const float k0 = k[u0], k1 = k[u1];
          q[u0] = fmaf(q0, cc, -(q1 * ss));
          q[u1] = fmaf(q0, ss, q1 * cc);
          k[u0] = fmaf(k0, cc, -(k1 * ss));
          k[u1] = fmaf(k0, ss, k1 * cc);
        }
      }
      if (R > 1 && rot) {
        if constexpr (!SO) {
          st_pair<T>(Qs + rw * LQ + n0, q[0], q[1]);
          st_pair<T>(Qs + rw * LQ + n0 + 64, q[2], q[3]);
        }
        st_pair<T>(Ks + rw * LQ + n0, k[0], k[1]);
        st_pair<T>(Ks + rw * LQ + n0 + 64, k[2], k[3]);
      } else {
        if constexpr (!SO) st_quad<T>(Qs + rw * LQ + n0, q);
        st_quad<T>(Ks + rw * LQ + n0, k);
      }
    }
    {
      // value / gate of row vt (token tv): VR / ZR = v, z (rank 1 as loaded; rank 4 times the
      // rounded mimo_x / mimo_z of the row's rank, rounded), VS = VR * scale * exp(cum_last - cum)
      const int tv = vt / R;
      const float ev = SC[SB_::SCL + tv] * __expf(SC[SB_::CL] - SC[SB_::CUM + tv]);
      f4 sv;
      if constexpr (R == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = raw_get<T>(rv, i) * ev;
        if constexpr (!SO) {
          *reinterpret_cast<u32x2*>(VR + v_off(vt, p0)) = (u32x2){rv[0], rv[1]};
          *reinterpret_cast<u32x2*>(ZR + v_off(vt, p0)) = (u32x2){rz[0], rz[1]};
        }
      } else {
        const int mo = (vt & (R - 1)) * kPPad + p0;
        const f4 mx = *reinterpret_cast<const f4*>(F + Ly::MX + mo);
        f4 vq;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          vq[i] = mul_r<T>(raw_get<T>(rv, i), mx[i]);
          sv[i] = vq[i] * ev;
        }
        if constexpr (!SO) {
          const f4 mz = *reinterpret_cast<const f4*>(F + Ly::MZ + mo);
          f4 zq;
#pragma unroll
          for (int i = 0; i < 4; ++i) zq[i] = mul_r<T>(raw_get<T>(rz, i), mz[i]);
          st_quad<T>(VR + v_off(vt, p0), vq);
          st_quad<T>(ZR + v_off(vt, p0), zq);
        }
      }
      st_quad<T>(VS + v_off(vt, p0), sv);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if constexpr (!SO) st_quad<T>(Sb + sb_off(16 * (spj0 + k) + l16, 16 * sni + 4 * lg), st[k]);
    }
    {
      const float ecl = SC[SB_::ECL];
      log_decay += SC[SB_::CL];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
#pragma unroll
        for (int i = 0; i < 4; ++i) st[k][i] *= ecl;
      }
    }
    __syncthreads();

    // ---- B: score tiles and decay weights, carry products, phases of c + 1; loads of c + 1
    __builtin_amdgcn_sched_barrier(0);
    load_qk(t0 + TOK);
    __builtin_amdgcn_sched_barrier(0);
    if (!SO && w < 10) {
      int it, sj;
      score_tile16(w, it, sj);
      const int tq = 16 * it + l16;
      f4 acc = zero4();
      // (four waves per SIMD hide the operand latency: one k-step's operands in registers at a
      // time keeps the kernel within 128 VGPRs)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const typename M::v8 av = *reinterpret_cast<const typename M::v8*>(
            Ks + (16 * sj + l16) * LQ + 32 * kk + 8 * lg);
        const typename M::v8 bv =
            *reinterpret_cast<const typename M::v8*>(Qs + tq * LQ + 32 * kk + 8 * lg);
        acc = M::mma(av, bv, acc);
        __builtin_amdgcn_sched_barrier(0);
      }
      // decay weights by token: row tq is token tq / R, column rows 16 sj + 4 lg + i are
      // tokens (16 sj + 4 lg + i) / R (rank 4: the one token 4 sj + lg)
      const int tqt = tq / R;
      const float cum_t = SC[SB_::CUM + tqt];
      f4 wv;
      if (sj < it) {
        // d = exp(cum_t - cend) * (scale_s exp(cend - cum_s)), both factors <= 1
        const float at = __expf(cum_t - SC[SB_::CEND + sj]);
        if constexpr (R == 1) {
          const f4 bs = *reinterpret_cast<const f4*>(SC + SB_::BSC + 16 * sj + 4 * lg);
#pragma unroll
          for (int i = 0; i < 4; ++i) wv[i] = acc[i] * (at * bs[i]);
        } else {
          const float bs = SC[SB_::BSC + 4 * sj + lg];
#pragma unroll
          for (int i = 0; i < 4; ++i) wv[i] = acc[i] * (at * bs);
        }
      } else {
        const float gam_t = SC[SB_::GAM + tqt];
        int tq_m = tqt;
        __asm__ volatile("" : "+v"(tq_m));
        if constexpr (R == 1) {
          const f4 c4 = *reinterpret_cast<const f4*>(SC + SB_::CUM + 16 * sj + 4 * lg);
          const f4 s4 = *reinterpret_cast<const f4*>(SC + SB_::SCL + 16 * sj + 4 * lg);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int ts = 16 * sj + 4 * lg + i;
            const float lower = s4[i] * __expf(cum_t - c4[i]);
            const float d = tq_m > ts ? lower : (tq_m == ts ? gam_t : 0.f);
            wv[i] = acc[i] * d;
          }
        } else {
          // same token (every rank pair): gamma; an earlier token: the decayed scale
          const int ts = 4 * sj + lg;
          const float lower = SC[SB_::SCL + ts] * __expf(cum_t - SC[SB_::CUM + ts]);
          const float d = tq_m > ts ? lower : (tq_m == ts ? gam_t : 0.f);
#pragma unroll
          for (int i = 0; i < 4; ++i) wv[i] = acc[i] * d;
        }
      }
      // W[t][s], s = 16 sj + 4 lg + i, at s' = 32 (sj / 2) + 8 lg + 4 (sj % 2) + i: the order of
      // the intra product's K axis (below)
      st_quad<T>(WS + tq * LW + 32 * (sj >> 1) + 8 * lg + 4 * (sj & 1), wv);
    }
    {
      // carry: S^T(ni, pj) += K~^T V~ over the 64 tokens. A: 8 tokens of column n from the
      // row-major Ks by two transposing reads (in each 16-lane group, lane 4a + b receives
      // element b of the 8-byte vectors of lanes a, a + 4, a + 8, a + 12); B: the same from VS.
      // The K axis of k-step kk, lane group lg: tokens kk + 4 lg + j (slots j) and
      // kk + 16 + 4 lg + j (slots 4 + j), so the 32 lanes of each read take 8 consecutive tokens
      const int xr = l16 >> 2, xc = 4 * (l16 & 3);
#pragma unroll
      for (int kk = 0; kk < 64; kk += 32) {  // the 64 rows
        const int r0 = kk + 4 * lg + xr;
        const T* k0 = Ks + r0 * LQ + 16 * sni + xc;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(k0));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(k0 + 16 * LQ));
        const typename M::v8 av = __builtin_bit_cast(
            typename M::v8, (i16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int vc = 16 * (spj0 + k) + xc;
          const i16x4 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(VS + v_off(r0, vc)));
          const i16x4 vhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(VS + v_off(r0 + 16, vc)));
          const typename M::v8 bv = __builtin_bit_cast(
              typename M::v8,
              (i16x8){vlo[0], vlo[1], vlo[2], vlo[3], vhi[0], vhi[1], vhi[2], vhi[3]});
          st[k] = M::mma(av, bv, st[k]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_vz(t0 + TOK);
    __builtin_amdgcn_sched_barrier(0);
    load_side(c + 2);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    // ---- C: output tile (row tile it, P tile pj)
    if constexpr (!SO) {
      const int it = w >> 2, pj = w & 3;
      const int tq = 16 * it + l16;
      f4 yi = zero4(), ye = zero4();
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        if (2 * m > it) continue;
        // intra: V^T W^T over tokens s = 32 m + 4 lg + i and 32 m + 16 + 4 lg + i
        const int vrow = 32 * m + 4 * lg + (l16 >> 2), vcol = 16 * pj + 4 * (l16 & 3);
        const typename M::v4 b0 = __builtin_bit_cast(
            typename M::v4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                (__attribute__((address_space(3))) i16x4*)(VR + v_off(vrow, vcol))));
        const typename M::v4 b1 = __builtin_bit_cast(
            typename M::v4,
            __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(VR + v_off(vrow + 16, vcol))));
        typename M::v8 av, bv = *reinterpret_cast<const typename M::v8*>(WS + tq * LW + 32 * m + 8 * lg);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          av[i] = b0[i];
          av[4 + i] = b1[i];
        }
        if (2 * m + 1 > it) {
          // column tile 2m + 1 lies above it: the operand's upper half (two words) is zero
          // (element-wise 16-bit zeroing took a select and a permute per element)
          u32x4 bw = __builtin_bit_cast(u32x4, bv);
          bw[2] = 0u;
          bw[3] = 0u;
          bv = __builtin_bit_cast(typename M::v8, bw);
        }
        yi = M::mma(av, bv, yi);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        // inter: rnd(S) Q^T
        const typename M::v8 av = *reinterpret_cast<const typename M::v8*>(
            Sb + sb_off(16 * pj + l16, 32 * kk + 8 * lg));
        const typename M::v8 bv =
            *reinterpret_cast<const typename M::v8*>(Qs + tq * LQ + 32 * kk + 8 * lg);
        ye = M::mma(av, bv, ye);
        __builtin_amdgcn_sched_barrier(0);
      }
      // epilogue: row tq (token tq / R), columns pb .. pb+3
      const int pb = 16 * pj + 4 * lg, tqt = tq / R;
      const float ecum_t = __expf(SC[SB_::CUM + tqt]);
      const typename M::v4 v4 = *reinterpret_cast<const typename M::v4*>(VR + v_off(tq, pb));
      const typename M::v4 z4 = *reinterpret_cast<const typename M::v4*>(ZR + v_off(tq, pb));
      f4 y;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        y[i] = (fmaf(ye[i], ecum_t, yi[i]) + Dh * to_f(v4[i])) * silu_fast(to_f(z4[i]));
      }
      if constexpr (R > 1) {
        // times mimo_out of the row's rank, summed over the token's R rows: lanes 4m .. 4m+3
        // of the 16-lane group (DPP quad permutes lane ^ 1 and lane ^ 2)
        const f4 mo = *reinterpret_cast<const f4*>(F + Ly::MO + (tq & (R - 1)) * kPPad + pb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float t = y[i] * mo[i];
          t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                             0, __builtin_bit_cast(int, t), 0xb1, 0xf, 0xf, false));
          t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                             0, __builtin_bit_cast(int, t), 0x4e, 0xf, 0xf, false));
          y[i] = t;
        }
      }
      if (R == 1 || (tq & (R - 1)) == 0) {
        bstore_quad<T>(y, rs_o, (tqt * out_t + o_out + pb * ES) +
                                    __builtin_amdgcn_readfirstlane(t0 * out_t));
      }
    }
    // phases of c + 1: its angle tile and side block came to LDS in A; its cos / sin table is
    // the other buffer than the one A read
    phases(c + 1);
    __syncthreads();
  }

  // ---- final k: the biased, rotated k rows of token L-1, still in Ks from the last sub-chunk
  if (a.final_k.ptr != nullptr && L > 0) {
    const int tl = (L - 1) - (nsub - 1) * TOK;
    for (int i = tid; i < R * kNPad; i += k16Threads) {
      const int r = i / kNPad, n = i - r * kNPad;
      static_cast<T*>(a.final_k.ptr)[b * a.final_k.stride[0] + h * a.final_k.stride[1] +
                                     r * a.final_k.stride[2] + n] = Ks[(tl * R + r) * LQ + n];
    }
  }
  if (a.final_decay.ptr != nullptr && tid == 0) {
    static_cast<float*>(a.final_decay.ptr)[b * a.final_decay.stride[0] +
                                           h * a.final_decay.stride[1]] = log_decay;
  }
  if (a.block_phase.ptr != nullptr && L > 0) {
    for (int i = tid; i < S; i += k16Threads) {
      static_cast<float*>(a.block_phase.ptr)[b * a.block_phase.stride[0] +
                                             h * a.block_phase.stride[1] +
                                             ((L - 1) >> 6) * a.block_phase.stride[2] +
                                             i * a.block_phase.stride[3]] = F[Ly::PBASE + i];
    }
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int p = 16 * (spj0 + k) + l16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = 16 * sni + 4 * lg + i;
      static_cast<float*>(a.final_state.ptr)[b * a.final_state.stride[0] +
                                             h * a.final_state.stride[1] +
                                             p * a.final_state.stride[2] + n] = st[k][i];
    }
  }
}

// ------------------------------------------------------------ segmented scan (composition)

// A sequence split into G equal segments is scanned twice (pass 1: every segment from a zero
// state and zero phase; pass 2: every segment from its true start), both passes viewing the
// [B, L] tensors as [B*G, L/G]. Between them, compose_kernel walks each (b, h)'s segments in
// order. The scan is linear in its initial state and a rotation by phi + psi is the rotation by
// psi followed by phi, so with pass 1's local end state U_g (built from k rotated by local
// phases), log-decay l_g = sum adt and last k k_g:
//   S_{g+1} = e^{l_g} (S_g + c_g sum_r (v_prev mx_r) k_prev_r^T) + U_g Rot(phi_g)^T,
//   k_prev <- Rot(phi_g) k_g,  v_prev <- v at the segment's last token,
// where c_g = dt (1 - trap) at the segment's first token (the endpoint continuation the kernel
// applies to initial_k / initial_value). The phase carry phi is the kernel's own walk over
// 64-token blocks, off <- fmod(off + block sum) (segments start on block boundaries), redone
// from pass 1's block sums: bit for bit the carry the unsplit scan reaches there, the fmod
// representative (sign) included. Pass 2 then starts segment g from (S_g, phi_g, k_prev,
// v_prev) exactly as a prefill continued from a cache, and its last segment's final state,
// phase and k are the call's (gather_kernel).
struct SegGeom {
  int G, Ls, nbs;         // segments per batch row, tokens and 64-token phase blocks per segment
  float* seg_state;       // [B*G][H][P][N] pass-1 end states, then pass 2's
  float* seg_decay;       // [B*G][H]
  float* seg_blk;         // [B*G][H][nbs][S] pass 1's phase block sums (phase mode ANGLES)
  float* seg_phase;       // [B*G][H][S] pass 2's final phases
  void* seg_k;            // [B*G][H][R][N] last k of pass 1, then of pass 2 (activation dtype)
  float* in_state;        // [B*G][H][P][N] pass-2 initial states
  float* in_phase;        // [B*G][H][S]
  void* in_k;             // [B*G][H][R][N]
  void* in_v;             // [B*G][H][P]
};

constexpr int kCompThreads = 256;                         // state-row threads (and gather_kernel's)
constexpr int kCompBlock = 64 + kCompThreads;             // compose_kernel: phase walker + state rows
constexpr int kCompRows = 8;                              // state rows per workgroup
constexpr int kCompPer = kCompRows * kNPad / kCompThreads;  // state elements per thread
constexpr int kWalkBatch = 32;                          // block sums per walker load batch
constexpr int kMaxSegments = 256;                       // bounds compose_kernel's LDS

// Dynamic LDS of compose_kernel (floats): per segment the phase carry at its start [G][S], the
// endpoint coefficient, e^{sum adt} and sum adt [3][G].
static size_t compose_lds_bytes(int G, int S) {
  return sizeof(float) * (static_cast<size_t>(G) * S + static_cast<size_t>(3) * G);
}

// One workgroup per (batch, head, group of kCompRows state rows): the rows are independent in the
// composition (rotations pair columns within a row, the endpoint term is an outer product).
// Wave 0 walks the phase carry through every 64-token block in order; the other four waves
// update the state rows segment by segment behind it. Everything the state update reads except
// the carry (the local end states, last k and last values of pass 1) is loaded segments ahead,
// so the call's critical path is the walk itself. The waves meet through s_ready in LDS, never
// at a barrier: the walker publishes each segment's carry and moves on.
template <typename T, int R>
__global__ __launch_bounds__(kCompBlock) void compose_kernel(const m3_scan_args a,
                                                             const SegGeom sg) {
  const int H = a.heads, N = a.d_state, P = a.head_dim, S = a.num_angles, G = sg.G;
  const int nrg = (P + kCompRows - 1) / kCompRows;  // row groups per (b, h)
  const int bh = blockIdx.x / nrg, rg = blockIdx.x - bh * nrg;
  const int b = bh / H, h = bh - b * H;
  const int p0 = rg * kCompRows, np = min(kCompRows, P - p0);
  const int tid = threadIdx.x;
  const bool angles = a.phase_mode == M3_PHASE_ANGLES;
  const bool walk = angles && S > 0;
  const bool mimo = a.mimo_rotation != 0;
  const bool raw_dt = a.raw_dt != 0;
  const bool lead = rg == 0;  // writes the per-(b, h) outputs: phases, k, decay
  extern __shared__ float dyn[];
  float* s_phig = dyn;             // [G][S] phase carry at each segment's start
  float* s_c0g = s_phig + G * S;   // [G] endpoint coefficient dt (1 - trap)
  float* s_decg = s_c0g + G;       // [G] e^{sum adt}
  float* s_draw = s_decg + G;      // [G] sum adt
  __shared__ int s_ready;          // segments whose starting carry is in s_phig
  auto row = [&](int g) { return (static_cast<int64_t>(b) * G + g) * H + h; };

  // per segment, in parallel: the endpoint coefficient and the decay
  {
    const float dtb = raw_dt ? ldx(a.dt_bias.ptr, a.dt_bias.dtype, h * a.dt_bias.stride[0]) : 0.f;
    for (int g = tid; g < G; g += kCompBlock) {
      const int t0 = g * sg.Ls;
      float dt0, adt0;
      dt_adt(raw_dt, ldx(a.dt.ptr, a.dt.dtype,
                         b * a.dt.stride[0] + t0 * a.dt.stride[1] + h * a.dt.stride[2]),
             ldx(a.a.ptr, a.a.dtype, b * a.a.stride[0] + t0 * a.a.stride[1] + h * a.a.stride[2]),
             dtb, dt0, adt0);
      s_c0g[g] = dt0 * (1.f - sigmoidf(ldx(a.trap.ptr, a.trap.dtype,
                                           b * a.trap.stride[0] + t0 * a.trap.stride[1] +
                                               h * a.trap.stride[2])));
      const float l = sg.seg_decay[row(g)];
      s_draw[g] = l;
      s_decg[g] = expf(l);
    }
  }
  if (tid == 0) s_ready = walk ? 0 : G;
  __syncthreads();

  if (tid < 64) {
    // ---- wave 0: the phase carry, the kernel's own recurrence off <- fmod(off + block sum)
    // over the blocks of segments 0 .. G-2 in order, published at each segment's start. Lanes
    // s < S walk angle s; block sums are loaded a batch ahead of the fmod chain.
    if (!walk || tid >= S) return;
    float off = 0.f;
    if (a.initial_phase.ptr != nullptr) {
      off = static_cast<const float*>(a.initial_phase.ptr)
          [b * a.initial_phase.stride[0] + h * a.initial_phase.stride[1] +
           tid * a.initial_phase.stride[2]];
    }
    auto publish = [&](int g) __attribute__((always_inline)) {
      s_phig[g * S + tid] = off;
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the carry is in LDS before the count
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (tid == 0) __hip_atomic_store(&s_ready, g + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    publish(0);
    const int nbs = sg.nbs, gend = G - 1;
    const int64_t seg_stride = static_cast<int64_t>(H) * nbs * S;  // floats from segment to segment
    const float* blk = sg.seg_blk + row(0) * nbs * S + tid;
    // batches never cross a segment's end; every load is issued (the last one repeated past a
    // short batch's end) so the waits stay exact
    auto load = [&](float (&buf)[kWalkBatch], int g, int k0) __attribute__((always_inline)) {
      const int n = min(kWalkBatch, nbs - k0);
      const float* p = blk + g * seg_stride + static_cast<int64_t>(k0) * S;
#pragma unroll
      for (int u = 0; u < kWalkBatch; ++u) buf[u] = p[min(u, n - 1) * S];
    };
    auto advance = [&](int& g, int& k0) __attribute__((always_inline)) {
      k0 += kWalkBatch;
      if (k0 >= nbs) {
        k0 = 0;
        ++g;
      }
    };
    auto walk_batch = [&](const float (&buf)[kWalkBatch], int g, int k0)
                          __attribute__((always_inline)) {
      const int n = min(kWalkBatch, nbs - k0);
#pragma unroll
      for (int u = 0; u < kWalkBatch; ++u) {
        if (u >= n) break;
        off = m3_fmod_2pi_small(__fadd_rn(off, buf[u]));
      }
      if (k0 + n == nbs) publish(g + 1);  // segment g walked: the carry at segment g + 1's start
    };
    if (gend > 0) {
      float bufA[kWalkBatch], bufB[kWalkBatch];
      int gA = 0, kA = 0;
      load(bufA, gA, kA);
      for (;;) {
        int gB = gA, kB = kA;
        advance(gB, kB);
        const bool moreB = gB < gend;
        load(bufB, moreB ? gB : gA, moreB ? kB : kA);
        walk_batch(bufA, gA, kA);
        if (!moreB) break;
        int gC = gB, kC = kB;
        advance(gC, kC);
        const bool moreC = gC < gend;
        load(bufA, moreC ? gC : gB, moreC ? kC : kB);
        walk_batch(bufB, gB, kB);
        if (!moreC) break;
        gA = gC;
        kA = kC;
      }
    }
    return;
  }

  // ---- waves 1-4: this workgroup's state rows, segment by segment
  const int tb = tid - 64;
  const int lgN = 31 - __builtin_clz(N);  // d_state is a power of 2 dividing kCompThreads
  const int RN = np << lgN;               // this workgroup's state elements
  const int n = tb & (N - 1);             // the thread's column: element e = tb + kCompThreads i
  // rotation partner of column n (-1: not rotated), whether n is the pair's first element, and
  // the pair's angle: SISO pairs (2j, 2j+1), j < S; MIMO pairs (j, j + 2S), j < S
  const int S2 = 2 * S;
  bool lo;
  int j;
  int part;
  if (!mimo) {
    lo = (n & 1) == 0;
    j = n >> 1;
    part = (angles && n < S2) ? (n ^ 1) : -1;
  } else {
    lo = n < S2;
    j = lo ? n : n - S2;
    part = (angles && j < S) ? (lo ? n + S2 : j) : -1;
  }
  const int np_n = part >= 0 ? part : n;
  auto rot = [&](float x, float xp, float c, float sn) {
    return lo ? x * c - xp * sn : xp * sn + x * c;
  };
  T* in_k = static_cast<T*>(sg.in_k);
  T* in_v = static_cast<T*>(sg.in_v);
  const T* seg_k = static_cast<const T*>(sg.seg_k);
  const T* value = static_cast<const T*>(a.value.ptr);
  int pl[kCompPer];
#pragma unroll
  for (int i = 0; i < kCompPer; ++i) pl[i] = min(tb + kCompThreads * i, RN - 1) >> lgN;

  // the start: the caller's state, k and value (zero without them)
  float st[kCompPer], vp[kCompPer], kp[R], mxr[R][kCompPer];
#pragma unroll
  for (int i = 0; i < kCompPer; ++i) {
    const int e = tb + kCompThreads * i;
    st[i] = (e < RN && a.initial_state.ptr != nullptr)
                ? static_cast<const float*>(a.initial_state.ptr)
                      [b * a.initial_state.stride[0] + h * a.initial_state.stride[1] +
                       (p0 + pl[i]) * a.initial_state.stride[2] + n]
                : 0.f;
    vp[i] = a.initial_k.ptr != nullptr
                ? to_f(static_cast<const T*>(a.initial_value.ptr)
                           [b * a.initial_value.stride[0] + h * a.initial_value.stride[1] +
                            p0 + pl[i]])
                : 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      mxr[r][i] = R > 1 ? rnd<T>(ldx(a.mimo_x.ptr, a.mimo_x.dtype,
                                     h * a.mimo_x.stride[0] + r * a.mimo_x.stride[1] + p0 + pl[i]))
                        : 1.f;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    kp[r] = a.initial_k.ptr != nullptr
                ? to_f(static_cast<const T*>(a.initial_k.ptr)
                           [b * a.initial_k.stride[0] + h * a.initial_k.stride[1] +
                            r * a.initial_k.stride[2] + n])
                : 0.f;
  }

  // a ring of D segments' inputs: local end state (the element and its rotation partner), last
  // k (column n and its partner, every rank) and the value of the last token (the thread's rows)
  constexpr int D = R <= 4 ? 4 : 2;
  float ru[D][kCompPer], rup[D][kCompPer], rk[D][R], rkp[D][R], rv[D][kCompPer];
  auto fetch = [&](int d, int g) __attribute__((always_inline)) {
    const int gc = min(g, G - 1);  // past the end: a repeat of the last segment, unused
    const int64_t sh = row(gc);
    const float* U = sg.seg_state + (sh * P + p0) * N;
#pragma unroll
    for (int i = 0; i < kCompPer; ++i) {
      ru[d][i] = U[(pl[i] << lgN) + n];
      rup[d][i] = U[(pl[i] << lgN) + np_n];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      rk[d][r] = to_f(seg_k[sh * R * N + r * N + n]);
      rkp[d][r] = to_f(seg_k[sh * R * N + r * N + np_n]);
    }
    const int tl = gc * sg.Ls + sg.Ls - 1;
#pragma unroll
    for (int i = 0; i < kCompPer; ++i) {
      rv[d][i] = to_f(value[b * a.value.stride[0] + tl * a.value.stride[1] +
                            h * a.value.stride[2] + p0 + pl[i]]);
    }
  };
#pragma unroll
  for (int d = 0; d < D; ++d) fetch(d, d);

  for (int g0 = 0; g0 < G; g0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int g = g0 + d;
      if (g >= G) break;
      const int64_t sh = row(g);
      float u[kCompPer], up[kCompPer], kx[R], kxp[R], vl[kCompPer];
#pragma unroll
      for (int i = 0; i < kCompPer; ++i) {
        u[i] = ru[d][i];
        up[i] = rup[d][i];
        vl[i] = rv[d][i];
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        kx[r] = rk[d][r];
        kxp[r] = rkp[d][r];
      }
      fetch(d, g + D);

      // (1) segment g's start for pass 2
#pragma unroll
      for (int i = 0; i < kCompPer; ++i) {
        const int e = tb + kCompThreads * i;
        if (e < RN) sg.in_state[(sh * P + p0) * N + e] = st[i];
      }
      if (lead && tb < N) {
#pragma unroll
        for (int r = 0; r < R; ++r) in_k[sh * R * N + r * N + n] = from_f<T>(kp[r]);
      }
      if (n == 0) {
#pragma unroll
        for (int i = 0; i < kCompPer; ++i) {
          if (tb + kCompThreads * i < RN) in_v[sh * P + p0 + pl[i]] = from_f<T>(vp[i]);
        }
      }
      // the carry at segment g's start, once the walker has published it. The walker is a wave
      // of this workgroup (resident with it) and publishes every segment without waiting on
      // anything, so the wait always ends; the spin cap (seconds) only keeps a defect from
      // becoming a hang. LDS operations of one wave complete in order and the walker drains its
      // carry stores before the count, so a count above g means the carry is readable.
      float cs = 1.f, sn = 0.f;
      if (walk) {
        for (int spin = 0;
             __hip_atomic_load(&s_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <= g &&
             spin < (1 << 24);
             ++spin) {
          __builtin_amdgcn_s_sleep(2);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (part >= 0) __sincosf(s_phig[g * S + j], &sn, &cs);
        if (lead && tb < S) sg.in_phase[sh * S + tb] = s_phig[g * S + tb];
      }

      // (2) the state at the segment's end: e^l (S + c0 sum_r (v_prev mx_r) k_prev_r^T) + Rot U
      const float c0 = s_c0g[g], dec = s_decg[g];
#pragma unroll
      for (int i = 0; i < kCompPer; ++i) {
        if (tb + kCompThreads * i >= RN) continue;
        float endpoint = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) endpoint += (R > 1 ? mul_r<T>(vp[i], mxr[r][i]) : vp[i]) * kp[r];
        const float uu = part >= 0 ? rot(u[i], up[i], cs, sn) : u[i];
        st[i] = dec * (st[i] + c0 * endpoint) + uu;
      }
      // (3) the next segment's endpoint: this segment's last k, rotated by its carry, and value
#pragma unroll
      for (int r = 0; r < R; ++r) {
        kp[r] = part >= 0 ? rnd<T>(rot(kx[r], kxp[r], cs, sn)) : rnd<T>(kx[r]);
      }
#pragma unroll
      for (int i = 0; i < kCompPer; ++i) vp[i] = vl[i];
    }
  }

  // the call's decay (its final state, phase and k come from pass 2: gather_kernel)
  if (lead && tb == 0 && a.final_decay.ptr != nullptr) {
    float decay_sum = 0.f;
    for (int g = 0; g < G; ++g) decay_sum += s_draw[g];
    static_cast<float*>(a.final_decay.ptr)[b * a.final_decay.stride[0] +
                                           h * a.final_decay.stride[1]] = decay_sum;
  }
}

// The call's final state, phase and k: pass 2's of each batch row's last segment.
template <typename T, int R>
__global__ __launch_bounds__(kCompThreads) void gather_kernel(const m3_scan_args a,
                                                              const SegGeom sg) {
  const int H = a.heads, N = a.d_state, P = a.head_dim, S = a.num_angles;
  const int b = blockIdx.x / H, h = blockIdx.x - b * H;
  const int64_t sh = (static_cast<int64_t>(b) * sg.G + sg.G - 1) * H + h;
  // the state: every element loaded before any is stored (the compiler cannot tell the two
  // buffers apart, so a load-store loop would take one round trip per element per thread)
  {
    constexpr int kPer = kPPad * kNPad / kCompThreads;
    const int lgN = 31 - __builtin_clz(N), PN = P * N;
    const float* src = sg.seg_state + sh * PN;
    float v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int e = threadIdx.x + kCompThreads * u;
      v[u] = e < PN ? src[e] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int e = threadIdx.x + kCompThreads * u;
      if (e < PN) {
        static_cast<float*>(a.final_state.ptr)[b * a.final_state.stride[0] +
                                               h * a.final_state.stride[1] +
                                               (e >> lgN) * a.final_state.stride[2] +
                                               (e & (N - 1))] = v[u];
      }
    }
  }
  if (a.final_phase.ptr != nullptr) {
    for (int i = threadIdx.x; i < S; i += kCompThreads) {
      static_cast<float*>(a.final_phase.ptr)[b * a.final_phase.stride[0] +
                                             h * a.final_phase.stride[1] +
                                             i * a.final_phase.stride[2]] = sg.seg_phase[sh * S + i];
    }
  }
  if (a.final_k.ptr != nullptr) {
    for (int i = threadIdx.x; i < R * N; i += kCompThreads) {
      const int r = i / N, n = i - r * N;
      static_cast<T*>(a.final_k.ptr)[b * a.final_k.stride[0] + h * a.final_k.stride[1] +
                                     r * a.final_k.stride[2] + n] =
          static_cast<const T*>(sg.seg_k)[sh * R * N + i];
    }
  }
  // Segments start on 64-token block boundaries, so block j of segment g is block g * nbs + j
  // of the sequence, and its increment sum does not depend on the carry: pass 1's sums are the
  // call's.
  if (a.block_phase.ptr != nullptr) {
    // 16 elements per thread loaded, then stored (as the state above)
    constexpr int kPer = 16;
    const int nb = sg.G * sg.nbs;
    for (int e0 = threadIdx.x; e0 < nb * S; e0 += kPer * kCompThreads) {
      float v[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int e = e0 + kCompThreads * u;
        if (e < nb * S) {
          const int blk = e / S, i = e - blk * S, g = blk / sg.nbs, j = blk - g * sg.nbs;
          const int64_t src = ((static_cast<int64_t>(b) * sg.G + g) * H + h) * sg.nbs + j;
          v[u] = sg.seg_blk[src * S + i];
        }
      }
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int e = e0 + kCompThreads * u;
        if (e < nb * S) {
          const int blk = e / S, i = e - blk * S;
          static_cast<float*>(a.block_phase.ptr)[b * a.block_phase.stride[0] +
                                                 h * a.block_phase.stride[1] +
                                                 blk * a.block_phase.stride[2] +
                                                 i * a.block_phase.stride[3]] = v[u];
        }
      }
    }
  }
}

// ------------------------------------------------------------------ host side

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A call scan16_kernel may serve (the projection form is checked later, at launch): the model's
// SISO shape in a 16-bit activation dtype with RMSNorm, head biases, raw dt and angle phases.
static bool scan16_candidate(const m3_scan_args& a) {
  return (a.act_dtype == M3_BF16 || a.act_dtype == M3_F16) &&
         (a.rank == 1 || a.rank == 4) && a.groups == 1 &&
         a.d_state == kNPad && a.head_dim == kPPad && a.num_angles == kSMax &&
         a.q_norm_w.ptr != nullptr && a.k_norm_w.ptr != nullptr && a.q_bias.ptr != nullptr &&
         a.k_bias.ptr != nullptr && a.raw_dt != 0 && a.phase_mode == M3_PHASE_ANGLES &&
         (a.mimo_rotation != 0) == (a.rank > 1);
}

// Prep workspace regions (floats, each 16-byte aligned) and the sub-chunk geometry; returns the
// workspace size in bytes.
static size_t ws_layout(const m3_scan_args& a, ScanGeom& g) {
  const int rows = a.act_dtype == M3_F32 ? Mma<float>::ROWS : Mma<__bf16>::ROWS;
  const int rank = a.rank > 0 ? a.rank : 1;
  g.tok = rows / rank > 0 ? rows / rank : 1;
  const int64_t len = a.length > 0 ? a.length : 0;
  g.nsub = static_cast<int>((len + g.tok - 1) / g.tok);
  g.scw = 5 * g.tok + 8;  // ScBlk<tok>::SIZE
  g.L4 = static_cast<int>((len + 3) / 4);
  const bool norm = a.q_norm_w.ptr != nullptr;
  const bool angles = a.phase_mode == M3_PHASE_ANGLES;
  const int64_t batch = a.batch > 0 ? a.batch : 0;
  int64_t off = 0;
  auto take = [&](int64_t n) {
    const int64_t o = off;
    off += (n + 3) / 4 * 4;
    return o;
  };
  g.ws_norm = norm ? take(batch * len * a.groups * a.rank * 2) : -1;
  g.ws_ang = angles ? take(batch * g.L4 * a.num_angles * 4) : -1;
  g.ws_sc = take(batch * a.heads * g.nsub * g.scw);
  const int64_t bytes = off * static_cast<int64_t>(sizeof(float));
  // the projection form's 32-bit offsets run up to two sub-chunk strides past the end
  g.ws_bytes = bytes < (int64_t{1} << 30) ? static_cast<int>(bytes) : -1;
  g.ws_qk = -1;
  g.qk_bytes = -1;
  const int64_t qk = batch * len * (a.rank > 0 ? a.rank : 1) * 2 * a.d_state * 2;
  if (scan16_candidate(a) && qk < (int64_t{1} << 30)) {
    // 256-byte aligned, addressed in 32 bits (the rows' offsets run up to two sub-chunks past
    // the end); larger calls take scan_kernel, which reads the raw rows
    g.ws_qk = (bytes + 255) / 256 * 256;
    g.qk_bytes = static_cast<int>(qk);
    return static_cast<size_t>(g.ws_qk + qk);
  }
  return static_cast<size_t>(bytes);
}

template <typename T>
static ScanGeom make_geom(const m3_scan_args& a) {
  ScanGeom g{};
  const int es = sizeof(T);
  const int total = a.batch * a.heads;
  g.xcd_map = (total % 8 == 0) ? 1 : 0;
  // vector loads need every row start aligned: base pointers and all outer strides
  auto vec_ok = [&](const m3_tensor& t, int dims, int need) {
    if ((reinterpret_cast<uintptr_t>(t.ptr) % need) != 0) return false;
    for (int i = 0; i < dims - 1; ++i) {
      if ((t.stride[i] * es) % need != 0) return false;
    }
    return true;
  };
  g.vec_qk = (a.d_state % 8 == 0) && vec_ok(a.q, 5, 16) && vec_ok(a.k, 5, 16);
  auto nw_ok = [](const m3_tensor& t) {
    return t.ptr != nullptr && t.stride[0] == 1 && reinterpret_cast<uintptr_t>(t.ptr) % 8 == 0;
  };
  g.vec_nw = (a.d_state % 8 == 0) && nw_ok(a.q_norm_w) && nw_ok(a.k_norm_w);
  const int vneed = es * 4;  // 4 elements per v / z load
  g.vec_vz = (a.head_dim % 4 == 0) && vec_ok(a.value, 4, vneed) && vec_ok(a.gate, 4, vneed);
  ws_layout(a, g);
  return g;
}

// Projection form: q, k, value, gate, dt, a, trap all of the activation dtype and slices of one
// projection row (same batch and token strides, every slice's per-token extent inside one token
// row), out token-major, and every offset the kernel forms below 2^31 bytes. Fills the byte
// geometry of `g`.
static bool projection_form(const m3_scan_args& a, ScanGeom& g, int es) {
  const m3_tensor* ts[7] = {&a.q, &a.k, &a.value, &a.gate, &a.dt, &a.a, &a.trap};
  for (const m3_tensor* t : ts) {
    if (t->dtype != a.act_dtype || t->stride[0] != a.q.stride[0] ||
        t->stride[1] != a.q.stride[1]) {
      return false;
    }
  }
  for (int i = 2; i < 5; ++i) {
    if (a.k.stride[i] != a.q.stride[i]) return false;
  }
  for (int i = 2; i < 4; ++i) {
    if (a.gate.stride[i] != a.value.stride[i]) return false;
  }
  if (a.a.stride[2] != a.dt.stride[2] || a.trap.stride[2] != a.dt.stride[2]) return false;
  const int64_t lim = INT32_MAX;
  const bool rev = a.q.stride[1] < 0;  // every per-token tensor runs the same way (validated)
  const int64_t tok = (rev ? -a.q.stride[1] : a.q.stride[1]) * es;
  const int64_t ext_q = ((a.groups - 1) * a.q.stride[2] + (a.rank - 1) * a.q.stride[3] +
                         a.d_state) * es;
  const int64_t ext_v = ((a.heads - 1) * a.value.stride[2] + a.head_dim) * es;
  const int64_t ext_s = ((a.heads - 1) * a.dt.stride[2] + 1) * es;
  const int64_t ext[7] = {ext_q, ext_q, ext_v, ext_v, ext_s, ext_s, ext_s};
  const char* base = static_cast<const char*>(a.q.ptr);
  for (const m3_tensor* t : ts) base = std::min(base, static_cast<const char*>(t->ptr));
  int64_t off[7];
  for (int i = 0; i < 7; ++i) {
    off[i] = static_cast<const char*>(ts[i]->ptr) - base;
    if (off[i] + ext[i] > tok) return false;
  }
  const int64_t out_tok = (rev ? -a.out.stride[1] : a.out.stride[1]) * es;
  if (((a.heads - 1) * a.out.stride[2] + a.head_dim) * es > out_tok) return false;
  const int64_t len = a.length;
  if (len * tok >= lim || len * out_tok >= lim || len * a.groups * a.rank * 8 >= lim ||
      static_cast<int64_t>(g.L4) * a.num_angles * 16 >= lim ||
      static_cast<int64_t>(g.nsub) * g.scw * 4 >= lim) {
    return false;
  }
  // backwards: the slices' pointers address logical token 0, the physical row L - 1; the buffer
  // starts at physical row 0 and logical token t sits (L - 1 - t) rows above it
  const int64_t shift = rev ? (len - 1) * tok : 0;
  g.proj = base - shift;
  g.proj_b = a.q.stride[0] * es;
  g.tok_b = static_cast<int>(rev ? -tok : tok);
  g.o_q = static_cast<int>(off[0] + shift);
  g.o_k = static_cast<int>(off[1] + shift);
  g.o_v = static_cast<int>(off[2] + shift);
  g.o_z = static_cast<int>(off[3] + shift);
  g.o_dt = static_cast<int>(off[4] + shift);
  g.o_a = static_cast<int>(off[5] + shift);
  g.o_tr = static_cast<int>(off[6] + shift);
  g.qk_g = static_cast<int>(a.q.stride[2] * es);
  g.qk_r = static_cast<int>(a.q.stride[3] * es);
  g.vz_h = static_cast<int>(a.value.stride[2] * es);
  g.sc_h = static_cast<int>(a.dt.stride[2] * es);
  g.out_b = a.out.stride[0] * es;
  g.out_t = static_cast<int>(rev ? -out_tok : out_tok);
  g.out_h = static_cast<int>(a.out.stride[2] * es);
  g.out_o0 = static_cast<int>(rev ? (len - 1) * out_tok : 0);
  g.out_base = static_cast<const char*>(a.out.ptr) - g.out_o0;
  return true;
}

// The model's own shape (N = 128, P = 64, S = 32, norm, bias, raw dt, angle phases, the rank's
// rotation) in projection form: the specialization with every shape and mode a compile-time
// constant and guard-free buffer addressing.
static bool full_shape(const m3_scan_args& a, ScanGeom& g, int R) {
  return a.length > 0 && a.groups == 1 && g.ws_bytes > 0 && a.d_state == kNPad &&
         a.head_dim == kPPad &&
         a.num_angles == kSMax &&
         a.q_norm_w.ptr != nullptr && a.q_bias.ptr != nullptr && a.raw_dt != 0 &&
         a.phase_mode == M3_PHASE_ANGLES && (a.mimo_rotation != 0) == (R > 1) && g.vec_qk &&
         g.vec_vz && projection_form(a, g, a.act_dtype == M3_F32 ? 4 : 2);
}

// The model's shape with the generic inputs (scan_kernel's SHAPE form): N = 128, P = 64, 32
// angles when rotating, one group, vector-aligned q / k and value / gate rows, a workspace
// below 2^30 bytes. Its reads and the output go through one buffer resource per tensor and
// (batch, head) at 32-bit byte offsets, so every token stride is positive, each token's row
// (ranks, or heads for the output) ends below the next token's, and L + 256 rows (the loads
// run up to two sub-chunks and a token group ahead) stay below 2^31 bytes. Sets the output
// geometry.
static bool model_shape(const m3_scan_args& a, ScanGeom& g, int es) {
  // (rank 1 rotates the pairs (2j, 2j+1) only)
  if (!(a.d_state == kNPad && a.head_dim == kPPad && a.groups == 1 && g.vec_qk && g.vec_vz &&
        (a.phase_mode == M3_PHASE_NONE || a.num_angles == kSMax) && g.ws_bytes > 0 &&
        (a.rank > 1 || a.mimo_rotation == 0) &&
        g.ws_bytes < (1 << 30))) {
    return false;
  }
  const int64_t rows = static_cast<int64_t>(a.length) + 256;
  // a token's row of `span` elements below the next token's, L + 256 rows in 32 bits
  auto fits = [&](const m3_tensor& t, int64_t span, int64_t esz) {
    return t.stride[1] > 0 && span <= t.stride[1] && rows * t.stride[1] * esz < INT32_MAX;
  };
  for (const m3_tensor* t : {&a.q, &a.k}) {
    if (t->stride[3] < 0 || !fits(*t, (a.rank - 1) * t->stride[3] + a.d_state, es)) return false;
  }
  // the output is stored 4 elements at a time
  const int64_t o4 = 4 * es;
  if (reinterpret_cast<uintptr_t>(a.out.ptr) % o4 != 0 || (a.out.stride[0] * es) % o4 != 0 ||
      (a.out.stride[1] * es) % o4 != 0 || (a.out.stride[2] * es) % o4 != 0) {
    return false;
  }
  if (!fits(a.value, a.head_dim, es) || !fits(a.gate, a.head_dim, es) ||
      !fits(a.out, (a.heads - 1) * a.out.stride[2] + a.head_dim, es) || a.out.stride[2] < 0) {
    return false;
  }
  if (a.phase_mode == M3_PHASE_GIVEN &&
      (a.phase.stride[3] < 0 || !fits(a.phase, (a.num_angles - 1) * a.phase.stride[3] + 1, 4))) {
    return false;
  }
  g.out_base = static_cast<const char*>(a.out.ptr);
  g.out_b = a.out.stride[0] * es;
  g.out_t = static_cast<int>(a.out.stride[1] * es);
  g.out_h = static_cast<int>(a.out.stride[2] * es);
  g.out_o0 = 0;
  return true;
}

template <typename T, int R, bool FULL, bool SO = false, bool SHAPE = false>
static int launch_kernel(const m3_scan_args& a, const ScanGeom& g, const float* prep, dim3 grid,
                         dim3 block, hipStream_t stream) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_kernel<T, R, FULL, SO, SHAPE>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       Layout<T>::BYTES);
    if (e != hipSuccess) {
      return fail(M3_ELAUNCH, "m3_scan_fwd: hipFuncSetAttribute: %s", hipGetErrorString(e));
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((scan_kernel<T, R, FULL, SO, SHAPE>), grid, block, Layout<T>::BYTES, stream,
                     a, g, prep);
  return check_launch("m3_scan_fwd");
}

template <typename T, int R, bool SO>
static int launch_kernel16(const m3_scan_args& a, const ScanGeom& g, const float* prep,
                           dim3 grid, hipStream_t stream) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan16_kernel<T, R, SO>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, Lay16::BYTES);
    if (e != hipSuccess) {
      return fail(M3_ELAUNCH, "m3_scan_fwd: hipFuncSetAttribute: %s", hipGetErrorString(e));
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((scan16_kernel<T, R, SO>), grid, dim3(k16Threads), Lay16::BYTES, stream, a, g,
                     prep);
  return check_launch("m3_scan_fwd");
}

// One pass: the prep kernel (unless `run_prep` is false: its workspace already holds this
// geometry's results) and the scan kernel.
// `state_only`: the caller needs only the end state, decay, last k and phase block sums (the
// outputs are not written where the state-only kernel form applies: the model's shape, 16-bit).
template <typename T, int R>
static int launch_pass(const m3_scan_args& a, hipStream_t stream, bool run_prep,
                       bool state_only = false) {
  ScanGeom g = make_geom<T>(a);
  static_assert(Layout<T>::BYTES <= 160 * 1024, "LDS layout exceeds 160 KiB");
  const float* prep = nullptr;
  const size_t need = ws_layout(a, g);
  if (need > 0) {
    if (a.workspace == nullptr || a.workspace_bytes < need || !aligned16(a.workspace)) {
      return fail(M3_EWORKSPACE, "m3_scan_fwd: needs a 16-byte aligned workspace of %zu bytes",
                  need);
    }
    prep = static_cast<const float*>(a.workspace);
    const int64_t tokens = static_cast<int64_t>(a.batch) * a.length;
    const int64_t rows = g.ws_norm >= 0 ? tokens * 2 * a.groups * a.rank : 0;
    const int64_t ang = g.ws_ang >= 0 ? static_cast<int64_t>(a.batch) * g.L4 * a.num_angles * 4 : 0;
    const int64_t blocks = static_cast<int64_t>(a.batch) * g.nsub;  // scalar-block workgroups
    if (rows >= INT32_MAX || ang >= INT32_MAX || blocks >= INT32_MAX || tokens >= INT32_MAX) {
      return fail(M3_EUNSUPPORTED, "m3_scan_fwd: too many tokens for one launch");
    }
    // the 16-wave kernel (below) reads prep's normalized rows, not the factors: their 4-byte
    // stores, one per row, would only add partial-line writes
    const bool k16 = sizeof(T) == 2 && (R == 1 || R == 4) && g.ws_qk >= 0 && g.qk_bytes > 0 &&
                     full_shape(a, g, R);
    g.norm_factors = k16 ? 0 : 1;
    constexpr int kNormRows = norm_rows<T, R>();
    const int64_t nb_norm = (rows + 16 * kNormRows - 1) / (16 * kNormRows);
    const int64_t nb_ang = (ang / 4 + 256 * kAngQuads - 1) / (256 * kAngQuads), nb_sc = blocks;
    if (run_prep && nb_norm + nb_ang + nb_sc > 0) {
      const dim3 pgrid(static_cast<unsigned>(nb_norm + nb_ang + nb_sc)), pblock(256);
      hipLaunchKernelGGL((prep_kernel<T, R>), pgrid, pblock, 0, stream, a, g,
                         static_cast<float*>(a.workspace), static_cast<int>(nb_norm),
                         static_cast<int>(nb_ang));
      int rc = check_launch("m3_scan_fwd (prep)");
      if (rc != M3_OK) return rc;
    }
  }
  const dim3 grid(static_cast<unsigned>(a.batch) * a.heads), block(kThreads);
  if (full_shape(a, g, R) && prep != nullptr) {
    if constexpr (sizeof(T) == 2 && (R == 1 || R == 4)) {
      // the model's shape at ranks 1 and 4: the 16-wave kernel, when prep wrote the normalized
      // rows (below 2^30 bytes of them)
      if (g.ws_qk >= 0 && g.qk_bytes > 0) {
        if (state_only) return launch_kernel16<T, R, true>(a, g, prep, grid, stream);
        return launch_kernel16<T, R, false>(a, g, prep, grid, stream);
      }
    }
    if constexpr (sizeof(T) == 2) {
      if (state_only) return launch_kernel<T, R, true, true>(a, g, prep, grid, block, stream);
    }
    return launch_kernel<T, R, true>(a, g, prep, grid, block, stream);
  }
  if (prep != nullptr && model_shape(a, g, static_cast<int>(sizeof(T)))) {
    return launch_kernel<T, R, false, false, true>(a, g, prep, grid, block, stream);
  }
  return launch_kernel<T, R, false>(a, g, prep, grid, block, stream);
}

// Sub-chunk length of a call's geometry.
static int sub_chunk_tokens(const m3_scan_args& a) {
  ScanGeom g{};
  ws_layout(a, g);
  return g.tok;
}

// Whether the [B, L] tensors can be viewed as [B*G, L/G]: each batch row of every per-token
// tensor is its L tokens at the token stride.
static bool segmentable(const m3_scan_args& a) {
  // one batch row: its stride never matters (also for a call running backwards)
  const bool one = a.batch == 1;
  const m3_tensor* ts[] = {&a.q, &a.k, &a.value, &a.gate, &a.dt, &a.a, &a.trap, &a.out};
  for (const m3_tensor* t : ts) {
    if (!one && t->stride[0] != static_cast<int64_t>(a.length) * t->stride[1]) return false;
  }
  if (!one && a.phase_mode != M3_PHASE_NONE &&
      a.phase.stride[0] != static_cast<int64_t>(a.length) * a.phase.stride[1]) {
    return false;
  }
  return a.head_dim <= kPPad && a.d_state <= kNPad;
}

// Segments a call's sequence is split into: 1 for none, -1 for an explicit request that cannot
// be met. Automatic (segments == 0): the G of least estimated time among 1 and the powers of 2
// from 4 up that cut L into equal segments of at least 8 sub-chunks (whole 64-token phase
// blocks with angle phases). With one workgroup per (b, h, segment), G segments take
// ceil(B H G c / 256) rounds over the 256 CUs of 1 / G of the unsplit workgroup's time (c calls
// of this shape sharing the GPU, 1 alone), times 1.37 for a split, whose state-only first pass
// and composition cost 0.37 of its second pass (config 5 long); ties go to the smaller G. At
// config 5 long (24 (b, h) pairs) that is G = 32 alone (3 full rounds; 622 us per call against
// 689 at G = 8) and G = 16 for its two concurrent directions (1,070 against 1,100 us).
static bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

static double split_cost(int64_t bhc, int G) {
  const double rounds = static_cast<double>((bhc * G + 255) / 256);
  return G == 1 ? rounds : 1.37 * rounds / G;
}

// The shapes the chunked MFMA kernel tiles: d_state a power of 2 up to 128, head_dim up to 64,
// up to 32 angles, ranks 1, 2, 4 and 8. Others take the recurrent scan (rscan.hip).
static bool tiled_shape(const m3_scan_args& a) {
  return pow2(a.d_state) && a.d_state >= 4 && a.d_state <= kNPad && a.head_dim <= kPPad &&
         a.num_angles <= kSMax && (a.rank == 1 || a.rank == 2 || a.rank == 4 || a.rank == 8);
}

static int segments_for(const m3_scan_args& a, int concurrent = 1) {
  if (!tiled_shape(a)) return a.segments > 1 ? -1 : 1;
  if (a.segments == 1 || a.length <= 0 || a.batch <= 0) return 1;
  if (a.segments < 0) return -1;
  if (!segmentable(a)) return a.segments > 1 ? -1 : 1;
  const int64_t bh = static_cast<int64_t>(a.batch) * a.heads;
  // segments start on the 64-token phase blocks (counted from the call's start)
  const int align = a.phase_mode == M3_PHASE_ANGLES ? 64 : 1;
  if (a.segments > 1) {
    const bool ok = a.segments <= kMaxSegments &&
                    a.length % (static_cast<int64_t>(a.segments) * align) == 0 &&
                    bh * a.segments <= INT32_MAX;
    return ok ? a.segments : -1;
  }
  const int tok = sub_chunk_tokens(a);
  const int64_t bhc = bh * (concurrent > 1 ? concurrent : 1);
  int best = 1;
  double best_cost = split_cost(bhc, 1);
  for (int G = 4; G <= kMaxSegments && bh * G <= INT32_MAX; G *= 2) {
    if (a.length % (static_cast<int64_t>(G) * align) != 0 || a.length / G < 8 * tok) break;
    const double c = split_cost(bhc, G);
    if (c < best_cost * (1.0 - 1e-9)) {
      best = G;
      best_cost = c;
    }
  }
  return best;
}

static m3_tensor contiguous(void* p, int dtype, std::initializer_list<int64_t> dims) {
  m3_tensor t{};
  t.ptr = p;
  t.dtype = dtype;
  int64_t st = 1;
  const int nd = static_cast<int>(dims.size());
  for (int i = nd - 1; i >= 0; --i) {
    t.stride[i] = st;
    st *= dims.begin()[i];
  }
  return t;
}

// Pass-1 argument block (pointers into the workspace filled in at launch) and the byte offsets
// of the segment buffers, after the prep region.
struct SegPlan {
  m3_scan_args a1;
  size_t prep_bytes, total_bytes;
  size_t o_state, o_decay, o_blk, o_phase, o_k, o_in_state, o_in_phase, o_in_k, o_in_v;
};

static SegPlan plan_segments(const m3_scan_args& a, int G) {
  SegPlan sp{};
  m3_scan_args& a1 = sp.a1;
  a1 = a;
  const int Ls = a.length / G;
  a1.batch = a.batch * G;
  a1.length = Ls;
  a1.segments = 1;
  for (m3_tensor* t : {&a1.q, &a1.k, &a1.value, &a1.gate, &a1.dt, &a1.a, &a1.trap, &a1.out}) {
    t->stride[0] = t->stride[1] * Ls;
  }
  if (a.phase_mode != M3_PHASE_NONE) a1.phase.stride[0] = a1.phase.stride[1] * Ls;
  a1.initial_state = m3_tensor{};
  a1.initial_phase = m3_tensor{};
  a1.initial_k = m3_tensor{};
  a1.initial_value = m3_tensor{};
  ScanGeom g1{};
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  sp.prep_bytes = up(ws_layout(a1, g1));
  const size_t es = a.act_dtype == M3_F32 ? 4 : 2;
  const size_t rows = static_cast<size_t>(a1.batch) * a.heads;
  size_t off = sp.prep_bytes;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += up(bytes);
    return o;
  };
  const size_t PN = static_cast<size_t>(a.head_dim) * a.d_state;
  sp.o_state = take(rows * PN * 4);
  sp.o_decay = take(rows * 4);
  sp.o_blk = take(rows * ((a1.length + 63) / 64) * a.num_angles * 4);
  sp.o_phase = take(rows * a.num_angles * 4);
  sp.o_k = take(rows * a.rank * a.d_state * es);
  sp.o_in_state = take(rows * PN * 4);
  sp.o_in_phase = take(rows * a.num_angles * 4);
  sp.o_in_k = take(rows * a.rank * a.d_state * es);
  sp.o_in_v = take(rows * a.head_dim * es);
  sp.total_bytes = off;
  return sp;
}

// The segmented scan: pass 1 (prep + scan of every segment from zero), the composition, pass 2
// (scan of every segment from its true start; prep's results are the same and are reused).
template <typename T, int R>
static int launch_segmented(const m3_scan_args& a, int G, hipStream_t stream) {
  SegPlan sp = plan_segments(a, G);
  if (a.workspace == nullptr || a.workspace_bytes < sp.total_bytes || !aligned16(a.workspace)) {
    return fail(M3_EWORKSPACE, "m3_scan_fwd: needs a 16-byte aligned workspace of %zu bytes",
                sp.total_bytes);
  }
  char* ws = static_cast<char*>(a.workspace);
  const int64_t BG = sp.a1.batch, H = a.heads, P = a.head_dim, N = a.d_state, S = a.num_angles;
  const bool angles = a.phase_mode == M3_PHASE_ANGLES;
  SegGeom sg{};
  sg.G = G;
  sg.Ls = sp.a1.length;
  sg.nbs = (sg.Ls + 63) / 64;
  sg.seg_state = reinterpret_cast<float*>(ws + sp.o_state);
  sg.seg_decay = reinterpret_cast<float*>(ws + sp.o_decay);
  sg.seg_blk = reinterpret_cast<float*>(ws + sp.o_blk);
  sg.seg_phase = reinterpret_cast<float*>(ws + sp.o_phase);
  sg.seg_k = ws + sp.o_k;
  sg.in_state = reinterpret_cast<float*>(ws + sp.o_in_state);
  sg.in_phase = reinterpret_cast<float*>(ws + sp.o_in_phase);
  sg.in_k = ws + sp.o_in_k;
  sg.in_v = ws + sp.o_in_v;

  m3_scan_args a1 = sp.a1;
  a1.workspace = ws;
  a1.workspace_bytes = sp.prep_bytes;
  a1.final_state = contiguous(sg.seg_state, M3_F32, {BG, H, P, N});
  a1.final_decay = contiguous(sg.seg_decay, M3_F32, {BG, H});
  a1.final_phase = m3_tensor{};
  a1.block_phase = angles ? contiguous(sg.seg_blk, M3_F32, {BG, H, sg.nbs, S}) : m3_tensor{};
  a1.final_k = contiguous(sg.seg_k, a.act_dtype, {BG, H, R, N});
  int rc = launch_pass<T, R>(a1, stream, true, /*state_only=*/true);
  if (rc != M3_OK) return rc;

  // at most kMaxSegments x kSMax + 3 kMaxSegments floats: within the default 64 KiB
  const size_t clds = compose_lds_bytes(G, S);
  static_assert(sizeof(float) * (kMaxSegments * kSMax + 3 * kMaxSegments) <= 65536,
                "compose_kernel's LDS fits the default limit");
  const unsigned row_groups = static_cast<unsigned>((P + kCompRows - 1) / kCompRows);
  hipLaunchKernelGGL((compose_kernel<T, R>),
                     dim3(static_cast<unsigned>(a.batch) * a.heads * row_groups),
                     dim3(kCompBlock), clds, stream, a, sg);
  rc = check_launch("m3_scan_fwd (compose)");
  if (rc != M3_OK) return rc;

  m3_scan_args a2 = a1;
  a2.initial_state = contiguous(sg.in_state, M3_F32, {BG, H, P, N});
  a2.initial_phase = angles ? contiguous(sg.in_phase, M3_F32, {BG, H, S}) : m3_tensor{};
  a2.initial_k = contiguous(sg.in_k, a.act_dtype, {BG, H, R, N});
  a2.initial_value = contiguous(sg.in_v, a.act_dtype, {BG, H, P});
  a2.final_state = a1.final_state;
  a2.final_phase = angles ? contiguous(sg.seg_phase, M3_F32, {BG, H, S}) : m3_tensor{};
  a2.final_k = a1.final_k;
  a2.final_decay = m3_tensor{};
  a2.block_phase = m3_tensor{};
  rc = launch_pass<T, R>(a2, stream, false);
  if (rc != M3_OK) return rc;
  hipLaunchKernelGGL((gather_kernel<T, R>), dim3(static_cast<unsigned>(a.batch) * a.heads),
                     dim3(kCompThreads), 0, stream, a, sg);
  return check_launch("m3_scan_fwd (gather)");
}

template <typename T, int R>
static int launch_scan_r(const m3_scan_args& a, hipStream_t stream) {
  const int G = segments_for(a);
  if (G < 0) {
    return fail(M3_EUNSUPPORTED,
                "m3_scan_fwd: %d segments need 1 < segments <= 256 dividing L into whole "
                "64-token blocks (angle phases), and token-major batch rows",
                a.segments);
  }
  if (G > 1) return launch_segmented<T, R>(a, G, stream);
  return launch_pass<T, R>(a, stream, true);
}

template <typename T>
static int launch_scan(const m3_scan_args& a, hipStream_t stream) {
  switch (a.rank) {
    case 1: return launch_scan_r<T, 1>(a, stream);
    case 2: return launch_scan_r<T, 2>(a, stream);
    case 4: return launch_scan_r<T, 4>(a, stream);
    case 8: return launch_scan_r<T, 8>(a, stream);
    default: return fail(M3_EUNSUPPORTED, "m3_scan_fwd: rank %d not in {1, 2, 4, 8}", a.rank);
  }
}

// A per-token tensor may run backwards (stride[1] < 0: token t at ptr + t * stride[1]; the
// reverse direction of a bidirectional layer reads the forward projection this way); the
// other checks see the forward stride.
static int check_token_tensor(const m3_tensor& t, const char* name, int dims, int64_t inner,
                              bool required, int dtype) {
  m3_tensor f = t;
  if (f.stride[1] < 0) f.stride[1] = -f.stride[1];
  return check_tensor(f, name, dims, inner, required, dtype);
}

static int validate_scan(const m3_scan_args& a) {
  if (a.batch < 0 || a.length < 0 || a.heads <= 0 || a.groups <= 0 || a.rank <= 0 ||
      a.d_state <= 0 || a.head_dim <= 0 || a.num_angles < 0) {
    return fail(M3_EINVAL, "m3_scan_fwd: invalid dimensions");
  }
  if (a.heads % a.groups != 0) return fail(M3_EINVAL, "m3_scan_fwd: heads %% groups != 0");
  if (!valid_dtype(a.act_dtype)) return fail(M3_EINVAL, "m3_scan_fwd: invalid act_dtype");
  if (a.d_state < 4) return fail(M3_EUNSUPPORTED, "m3_scan_fwd: d_state %d < 4", a.d_state);
  if (!tiled_shape(a) && !rscan_fits(a)) {
    return fail(M3_EUNSUPPORTED,
                "m3_scan_fwd: rank %d, d_state %d, head_dim %d, %d angles: the recurrent scan's "
                "per-token q / k / value vectors exceed 160 KiB of LDS",
                a.rank, a.d_state, a.head_dim, a.num_angles);
  }
  if (!tiled_shape(a) && a.segments > 1) {
    return fail(M3_EUNSUPPORTED, "m3_scan_fwd: segments > 1 need a shape the MFMA kernel tiles");
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
  if ((rc = check_token_tensor(a.q, "q", 5, N, true, act)) ||
      (rc = check_token_tensor(a.k, "k", 5, N, true, act)) ||
      (rc = check_tensor(a.q_norm_w, "q_norm_w", 1, N, false, -1)) ||
      (rc = check_tensor(a.k_norm_w, "k_norm_w", 1, N, a.q_norm_w.ptr != nullptr, -1)) ||
      (rc = check_tensor(a.q_bias, "q_bias", 3, N, false, -1)) ||
      (rc = check_tensor(a.k_bias, "k_bias", 3, N, a.q_bias.ptr != nullptr, -1)) ||
      (rc = check_token_tensor(a.value, "value", 4, P, true, act)) ||
      (rc = check_token_tensor(a.gate, "gate", 4, P, true, act)) ||
      (rc = check_token_tensor(a.dt, "dt", 3, 1, true, -1)) ||
      (rc = check_token_tensor(a.a, "a", 3, 1, true, -1)) ||
      (rc = check_tensor(a.dt_bias, "dt_bias", 1, 1, a.raw_dt != 0, -1)) ||
      (rc = check_token_tensor(a.trap, "trap", 3, 1, true, -1)) ||
      (rc = check_token_tensor(a.phase, "phase", angles ? 3 : 4, 1,
                               a.phase_mode != M3_PHASE_NONE,
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
      (rc = check_token_tensor(a.out, "out", 4, P, true, act)) ||
      (rc = check_tensor(a.final_state, "final_state", 4, N, true, M3_F32)) ||
      (rc = check_tensor(a.final_phase, "final_phase", 3, 1, false, M3_F32)) ||
      (rc = check_tensor(a.final_decay, "final_decay", 2, 1, false, M3_F32)) ||
      (rc = check_tensor(a.block_phase, "block_phase", 4, 1, false, M3_F32)) ||
      (rc = check_tensor(a.final_k, "final_k", 4, N, false, act))) {
    return rc;
  }
  if ((a.q_norm_w.ptr == nullptr) != (a.k_norm_w.ptr == nullptr) ||
      (a.q_bias.ptr == nullptr) != (a.k_bias.ptr == nullptr)) {
    return fail(M3_EINVAL, "m3_scan_fwd: q/k norm weights and biases come in pairs");
  }
  // per-token offsets within one batch row are 32-bit in the kernel
  const int64_t lim = INT32_MAX;
  const m3_tensor* per_token[] = {&a.q, &a.k, &a.value, &a.gate, &a.dt, &a.a, &a.trap, &a.out};
  for (const m3_tensor* t : per_token) {
    if (static_cast<int64_t>(a.length) * (t->stride[1] < 0 ? -t->stride[1] : t->stride[1]) >=
        lim) {
      return fail(M3_EUNSUPPORTED, "m3_scan_fwd: a batch row exceeds 2^31 elements");
    }
  }
  if (a.phase_mode != M3_PHASE_NONE &&
      static_cast<int64_t>(a.length) * (a.phase.stride[1] < 0 ? -a.phase.stride[1]
                                                               : a.phase.stride[1]) >= lim) {
    return fail(M3_EUNSUPPORTED, "m3_scan_fwd: a batch row of phase exceeds 2^31 elements");
  }
  if (a.length > 1) {
    const bool back = a.q.stride[1] < 0;
    const m3_tensor* ts[] = {&a.k, &a.value, &a.gate, &a.dt, &a.a, &a.trap, &a.out};
    bool same = true;
    for (const m3_tensor* t : ts) same = same && ((t->stride[1] < 0) == back);
    if (a.phase_mode != M3_PHASE_NONE) same = same && ((a.phase.stride[1] < 0) == back);
    if (!same) {
      return fail(M3_EINVAL, "m3_scan_fwd: per-token tensors must all run the same way");
    }
  }
  if ((a.final_phase.ptr != nullptr || a.block_phase.ptr != nullptr) && !angles) {
    return fail(M3_EINVAL, "m3_scan_fwd: final_phase / block_phase need phase_mode ANGLES");
  }
  return M3_OK;
}

}  // namespace m3

extern "C" int m3_scan_workspace_size(const m3_scan_args* args, size_t* bytes) {
  m3::clear_error();
  if (args == nullptr || bytes == nullptr) {
    return m3::fail(M3_EINVAL, "m3_scan_workspace_size: NULL argument");
  }
  m3::ScanGeom g{};
  if (!m3::tiled_shape(*args)) {  // the recurrent scan needs no workspace
    *bytes = 0;
    return M3_OK;
  }
  const int G = m3::segments_for(*args);
  *bytes = G > 1 ? m3::plan_segments(*args, G).total_bytes : m3::ws_layout(*args, g);
  return M3_OK;
}

extern "C" int m3_scan_segments(const m3_scan_args* args, int concurrent_calls,
                                int* segments) {
  m3::clear_error();
  if (args == nullptr || segments == nullptr) {
    return m3::fail(M3_EINVAL, "m3_scan_segments: NULL argument");
  }
  if (concurrent_calls < 1) {
    return m3::fail(M3_EINVAL, "m3_scan_segments: concurrent_calls must be at least 1");
  }
  const int G = m3::segments_for(*args, concurrent_calls);
  if (G < 0) {
    return m3::fail(M3_EUNSUPPORTED, "m3_scan_segments: the requested %d segments cannot be met",
                    args->segments);
  }
  *segments = G;
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
  if (!tiled_shape(a)) return launch_recurrent_scan(a, stream);
  switch (a.act_dtype) {
    case M3_F32: return launch_scan<float>(a, stream);
    case M3_BF16: return launch_scan<__bf16>(a, stream);
    default: return launch_scan<_Float16>(a, stream);
  }
}
