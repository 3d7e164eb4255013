/*
 * mamba3_hip.h -- C ABI of libmamba3_hip.so, the MI355X (gfx950) Mamba-3 mixer hot path.
 *
 * Plain C: device pointers, element strides and sizes; no C++ or torch types cross this
 * boundary and no exception escapes it. Every entry point:
 *   - returns M3_OK (0) or a non-zero status; m3_last_error() then describes the failure
 *     (thread-local string, valid until the next call on the same thread);
 *   - allocates nothing, never synchronises the device and never reads device memory on the
 *     host, so every call is safe inside hipGraph stream capture;
 *   - enqueues its kernels on the stream it is given (torch's current stream in the Python
 *     host), on the device that is current for the calling thread.
 *
 * Tensors are passed as m3_tensor: a device pointer, a dtype and element strides, outermost
 * axis first. Shapes are given once, by the dimension fields of the argument struct, and the
 * axis order of every tensor is documented next to it. A NULL pointer marks an optional
 * tensor as absent. The innermost axis of q, k, value, gate, out, the state and every
 * parameter tensor must have stride 1.
 *
 * The reference (jreoka/mamba3) exposes this path through two Python plugin hooks that return
 * None to fall back, and three Triton launchers; the entry points below replace them:
 *   m3_scan_fwd     <- mamba3/ops.py:253-367  _fused_chunk_scan  (and its driver ops.py:370-505,
 *                      launchers chunk_main _triton.py:416-497 / chunk_state _triton.py:500-561);
 *                      also the portable mamba3_scan ops.py:544-822 and, with the raw-projection
 *                      inputs, the prologue of _Mamba3Mixer.forward model.py:165-256, 282-309.
 *   m3_chunk_state  <- mamba3/_triton.py:500-561  chunk_state (the per-chunk state update).
 *   m3_step         <- mamba3/ops.py:87-190  fused_step (launcher _triton.py:950-1151) and the
 *                      portable mamba3_step ops.py:825-879 with the step prologue of
 *                      _Mamba3Mixer.step model.py:431-469.
 * m3_linear has no reference hook: it takes the decode step's projection GEMMs (see below).
 */
#ifndef MAMBA3_HIP_H
#define MAMBA3_HIP_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M3_ABI_VERSION 4

/* Element types. */
enum { M3_F32 = 0, M3_BF16 = 1, M3_F16 = 2 };

/* Status codes. */
enum {
  M3_OK = 0,
  M3_EINVAL = 1,       /* malformed arguments (NULL required pointer, bad stride, bad dims) */
  M3_EUNSUPPORTED = 2, /* well-formed but outside what the kernels implement */
  M3_ELAUNCH = 3,      /* the HIP runtime refused a launch */
  M3_EWORKSPACE = 4    /* workspace missing or too small */
};

/* Phase source for the rotation of q and k. */
enum {
  M3_PHASE_NONE = 0,   /* q and k are used as given (already rotated, or no rotation) */
  M3_PHASE_GIVEN = 1,  /* scan: phase [B, L, H, S] FP32 is given */
  M3_PHASE_ANGLES = 2  /* angles [B, L, S] (scan) or [B, S] (step): the kernel accumulates the
                          bounded phase itself, model.py:215-256 (scan) / model.py:460-466 (step) */
};

typedef struct {
  void* ptr;          /* device pointer; NULL = absent */
  int32_t dtype;      /* M3_F32 / M3_BF16 / M3_F16 */
  int32_t reserved;
  int64_t stride[5];  /* element strides, outermost axis first; unused trailing entries 0 */
} m3_tensor;

/*
 * Chunked SSD over whole sequences (one call per layer and direction).
 *
 * Dimension names: B batch, L length, H heads, G q/k groups (H % G == 0), R MIMO rank,
 * N d_state, P head_dim, S num_angles.
 *
 * Two input forms share this struct:
 *  - hook form (ops.mamba3_scan / _fused_chunk_scan): q, k are RMS-normed, dt/a hold dt and
 *    adt in FP32, the phase is given or absent;
 *  - projection form (the model): q, k are raw slices of the in_proj output and q_norm_w /
 *    k_norm_w are set (RMSNorm over N, eps norm_eps), dt/a hold the raw dd_dt / dd_A logits with
 *    raw_dt = 1 (dt = softplus(dd_dt + dt_bias), adt = -max(heavy_tail(dd_A), 1e-4) * dt), and
 *    phase holds the raw angles (M3_PHASE_ANGLES) continued from initial_phase.
 */
typedef struct {
  int32_t batch, length, heads, groups, rank, d_state, head_dim, num_angles;
  int32_t chunk;          /* the caller's chunk size; advisory, the kernel tiles by itself */
  int32_t act_dtype;      /* dtype of q, k, value, gate, out, initial_k, initial_value, final_k */
  int32_t mimo_rotation;  /* 0: SISO adjacent pairs (2i, 2i+1); 1: MIMO quarters (i, 2S + i) */
  int32_t raw_dt;         /* 0: dt / a are FP32 dt / adt; 1: raw logits (see above) */
  int32_t phase_mode;     /* M3_PHASE_* */
  int32_t segments;       /* 0: the library picks; 1: one pass per (b, h); G > 1: G segments */
  float norm_eps;
  m3_tensor q, k;                   /* [B, L, G, R, N] */
  m3_tensor q_norm_w, k_norm_w;     /* [N] optional (C_norm.weight / B_norm.weight) */
  m3_tensor q_bias, k_bias;         /* [H, R, N] optional, both or neither (C_bias / B_bias) */
  m3_tensor value, gate;            /* [B, L, H, P] */
  m3_tensor dt, a;                  /* [B, L, H] */
  m3_tensor dt_bias;                /* [H] (raw_dt = 1) */
  m3_tensor trap;                   /* [B, L, H] trapezoid logits */
  m3_tensor phase;                  /* [B, L, H, S] FP32 (GIVEN) or angles [B, L, S] (ANGLES) */
  m3_tensor initial_phase;          /* [B, H, S] FP32 optional (ANGLES) */
  m3_tensor D;                      /* [H] */
  m3_tensor mimo_x, mimo_z, mimo_out; /* [H, R, P], required iff R > 1 */
  m3_tensor initial_state;          /* [B, H, P, N] FP32 optional */
  m3_tensor initial_k;              /* [B, H, R, N] optional, with initial_value: endpoint */
  m3_tensor initial_value;          /* [B, H, P] */
  m3_tensor out;                    /* [B, L, H, P] */
  m3_tensor final_state;            /* [B, H, P, N] FP32 */
  m3_tensor final_phase;            /* [B, H, S] FP32 optional (ANGLES): phase of token L-1 */
  m3_tensor final_k;                /* [B, H, R, N] optional: biased, rotated k of token L-1 */
  m3_tensor final_decay;            /* [B, H] FP32 optional: sum of adt over the sequence */
  m3_tensor block_phase;            /* [B, H, ceil(L / 64), S] FP32 optional (ANGLES): the sum of
                                       each 64-token block's bounded phase increments */
  void* workspace;                  /* device scratch, m3_scan_workspace_size() bytes */
  size_t workspace_bytes;
} m3_scan_args;

/* Bytes of device workspace m3_scan_fwd needs for these arguments (0 is possible). */
int m3_scan_workspace_size(const m3_scan_args* args, size_t* bytes);
/*
 * The segment count m3_scan_fwd uses for these arguments when `concurrent_calls` calls of this
 * shape run on the GPU at once (1: alone); with args->segments == 0 the library picks it, else
 * the explicit request is checked. A caller running such calls together (the two directions of
 * a bidirectional layer) passes the result as args->segments before sizing the workspace.
 * No counterpart in the reference, whose portable scan has no segments (ops.py:544-822).
 */
int m3_scan_segments(const m3_scan_args* args, int concurrent_calls, int* segments);
int m3_scan_fwd(const m3_scan_args* args, hipStream_t stream);

/*
 * m3_scan_fwd without a caller workspace. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under hipGraph stream capture, tight serving loops,
 * harnesses that forbid hipMalloc). The call uses the library's own device scratch, one static
 * array of M3_SCRATCH_BYTES per GPU, held until the process ends; args->workspace and
 * args->workspace_bytes are ignored. It allocates, frees and synchronises nothing. A call that
 * needs more than M3_SCRATCH_BYTES (m3_scan_workspace_size) fails with M3_EWORKSPACE. Every call
 * on one GPU uses that GPU's one scratch, which keeps the last call's contents: calls that overlap
 * in time on one GPU (on different streams) race, so the caller must order them.
 */
#define M3_SCRATCH_BYTES (64u << 20)
int m3_scan_fwd_noalloc(const m3_scan_args* args, hipStream_t stream);

/*
 * One chunk's state update, _triton.py:294-413:
 *   state_out = exp(cum_last) * state_in + sum_rows value_r^T (k * scale * exp(cum_last - cum))
 * over the W tokens of a chunk, rows flattened (token, rank). cum is the within-chunk cumulative
 * sum of adt and cum_last = cum[W-1]. k * scale and its product with the end decay are rounded to
 * the activation dtype, as ops.py:743 and ops.py:806-807 do.
 */
typedef struct {
  int32_t batch, width, heads, rank, d_state, head_dim;
  int32_t act_dtype;
  int32_t reserved;
  m3_tensor k;          /* [B, H, W, R, N] activation dtype (biased, rotated) */
  m3_tensor value;      /* [B, H, W, R, P] activation dtype (rank values) */
  m3_tensor cumulative; /* [B, H, W] FP32 */
  m3_tensor scale;      /* [B, H, W] FP32 */
  m3_tensor state_in;   /* [B, H, P, N] FP32 */
  m3_tensor state_out;  /* [B, H, P, N] FP32; may equal state_in */
} m3_chunk_state_args;

int m3_chunk_state(const m3_chunk_state_args* args, hipStream_t stream);

/*
 * One decode token for every (batch, head): phase advance, rotation, trapezoid update of the
 * FP32 state, readout, D skip, SiLU gate and MIMO rank sum.
 *   hook form (ops.fused_step): q, k head-expanded and biased [B, H, R, N], unrotated,
 *     phase_mode ANGLES with angles [B, S]; or phase_mode NONE with rotated q, k (mamba3_step).
 *   projection form (the model): raw q, k [B, G, R, N] with norm weights and biases, raw
 *     dt / a logits, angles [B, S].
 * The cache outputs may alias the cache inputs (in-place update): each workgroup reads its
 * (batch, head) slice of phase_in, state_in, prev_k and prev_value before writing it.
 */
typedef struct {
  int32_t batch, heads, groups, rank, d_state, head_dim, num_angles;
  int32_t act_dtype, mimo_rotation, raw_dt, phase_mode;
  float norm_eps;
  m3_tensor q, k;                   /* [B, G, R, N] */
  m3_tensor q_norm_w, k_norm_w;     /* [N] optional */
  m3_tensor q_bias, k_bias;         /* [H, R, N] optional */
  m3_tensor value, gate;            /* [B, H, P] */
  m3_tensor dt, a, dt_bias, trap;   /* dt, a, trap [B, H]; dt_bias [H] */
  m3_tensor angles;                 /* [B, S] (ANGLES) */
  m3_tensor D;                      /* [H] */
  m3_tensor mimo_x, mimo_z, mimo_out; /* [H, R, P], required iff R > 1 */
  m3_tensor phase_in;               /* [B, H, S] FP32 */
  m3_tensor state_in;               /* [B, H, P, N] FP32 */
  m3_tensor prev_k;                 /* [B, H, R, N] activation dtype */
  m3_tensor prev_value;             /* [B, H, P] activation dtype */
  m3_tensor out;                    /* [B, H, P] */
  m3_tensor phase_out;              /* [B, H, S] FP32 */
  m3_tensor state_out;              /* [B, H, P, N] FP32 */
  m3_tensor k_out;                  /* [B, H, R, N]: the rotated k of this token */
  m3_tensor value_out;              /* [B, H, P] optional: copy of value (next prev_value) */
} m3_step_args;

int m3_step(const m3_step_args* args, hipStream_t stream);

/*
 * A linear layer of the decode path, out[M, N] = x'[M, K] * weight[N, K]^T (+ residual[M, N]),
 * for few rows (M <= 256, one row per batch element): 16-bit x, weight, residual and out of one
 * dtype, FP32 accumulation, one rounding. x' is x, or with norm_weight the RMS-normalised
 * x * rsqrt(mean_k x^2 + norm_eps) * norm_weight (M <= 32, or M <= 64 with K a multiple of
 * 256). It has no counterpart among the
 * reference's plugin hooks: it replaces the block's RMSNorm, the in_proj / out_proj nn.Linear
 * calls and the residual add of a decode step (mamba3/model.py:441-458, 514-520), where a
 * general GEMM leaves most of the GPU idle.
 * K is a multiple of 32; x and weight rows are 16-byte aligned. The split of K over workgroups
 * keeps FP32 partial sums in the caller's workspace (m3_linear_workspace_size, 0 when unsplit).
 */
typedef struct {
  int64_t m, n, k;
  int32_t dtype;        /* M3_BF16 or M3_F16 */
  float norm_eps;
  m3_tensor x;          /* [M, K] */
  m3_tensor weight;     /* [N, K] */
  m3_tensor norm_weight;/* [K] optional, 16-byte aligned */
  m3_tensor residual;   /* [M, N] optional */
  m3_tensor out;        /* [M, N]; may not overlap x or weight, may equal residual */
  void* workspace;
  size_t workspace_bytes;
} m3_linear_args;

int m3_linear_workspace_size(const m3_linear_args* args, size_t* bytes);
int m3_linear(const m3_linear_args* args, hipStream_t stream);

/*
 * The residual stream between mixers, one pass: s = x (+ add, summed in FP32 and rounded to x's
 * dtype), optionally sum_out = s, and out = (s * rsqrt(mean(s^2) + eps)) * weight (the weight
 * rounded to x's dtype, out rounded to out's dtype). It has no counterpart among the reference's
 * plugin hooks: it replaces the block's residual add (mamba3/model.py:511-512), the RMSNorm that
 * follows it (the next block's norm, model.py:48-55, 499-510, or norm_f, 591, 607) and, under
 * autocast, the cast of the normed rows to the projection's dtype.
 * dim is 256, 512, 768, 1024 or 2048; x, add and out of one 16-bit dtype, or an FP32 x with any
 * add and out dtype; sum_out has x's dtype and may equal x; out overlaps nothing. Rows start
 * 4-element aligned, innermost stride 1.
 */
typedef struct {
  int64_t rows, dim;
  float eps;
  int32_t reserved;
  m3_tensor x;          /* [rows, dim] */
  m3_tensor add;        /* [rows, dim] optional */
  m3_tensor weight;     /* [dim] */
  m3_tensor sum_out;    /* [rows, dim] optional (needs add): x + add in x's dtype */
  m3_tensor out;        /* [rows, dim] */
} m3_rms_norm_args;

int m3_rms_norm(const m3_rms_norm_args* args, hipStream_t stream);

const char* m3_last_error(void);
int m3_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA3_HIP_H */
