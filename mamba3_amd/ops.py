"""Mamba-3 hot-path operators, executed by the HIP library (``include/mamba3_hip.h``).

Mirrors the operator interface of the reference ``mamba3/ops.py`` (jreoka/mamba3): the
same function names, argument meanings and ``ValueError`` validation messages. The
difference is the dispatch contract: the reference's hooks (``fused_step``,
``_fused_chunk_scan``) return ``None`` to fall back to a portable PyTorch path. This
package has no fallback. Every call runs the HIP kernels on a ROCm device or raises:
``RuntimeError`` for CPU tensors, for autograd use, and for a missing library;
``HipError`` for a failing call.

Module flags ``_HIP_LAST_DISPATCH`` / ``_HIP_LAST_SCAN_DISPATCH`` record that the last
step / scan ran on the HIP path (the reference's ``_TRITON_LAST_DISPATCH`` /
``_TRITON_LAST_SCAN_DISPATCH``, ``ops.py:14,18``).
"""

from __future__ import annotations

import torch

from . import _hip

_HIP_LAST_DISPATCH = False
_HIP_LAST_SCAN_DISPATCH = False
NORM_EPS = 1e-5
# Sequence segments of a scan call: 0 lets the library split long sequences of few (batch,
# head) pairs over more workgroups (two passes and a composition of the segment states); 1 never
# splits; G > 1 asks for G equal segments.
SCAN_SEGMENTS = 0


def heavy_tail_activation(x: torch.Tensor) -> torch.Tensor:
    """``1 + x`` for ``x >= 0``, ``1 / (1 - x)`` otherwise (reference ``ops.py:28-32``).

    Kept under the reference's name for callers that import it; no path of this package
    calls it: the kernels apply the activation to the raw ``dd_A`` logits themselves.
    """
    return torch.where(x >= 0, 1.0 + x, torch.reciprocal(1.0 - x.clamp_max(0)))


def _require_device(*tensors: torch.Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "mamba3_amd runs the Mamba-3 hot path on ROCm devices only "
                f"(got a tensor on {t.device}); there is no CPU path")
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError("all tensors must be on the same device")
    if device is None:
        raise RuntimeError("no device tensor given")
    return device


def _require_inference(*tensors: torch.Tensor | None) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise RuntimeError(
            "mamba3_amd implements the inference hot path (forward, prefill, step) and has no "
            "backward; run it under torch.no_grad() or torch.inference_mode()")


def _inner(t: torch.Tensor | None) -> torch.Tensor | None:
    """A view whose innermost axis has stride 1 (copy only when it does not)."""
    if t is None or t.dim() == 0 or t.shape[-1] <= 1 or t.stride(-1) == 1:
        return t
    return t.contiguous()


def _state32(t: torch.Tensor) -> torch.Tensor:
    t = t if t.dtype == torch.float32 else t.float()
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 4 for s in t.stride()[:-1]):
        t = t.contiguous()
    return t


def _param(t: torch.Tensor | None) -> torch.Tensor | None:
    """Small parameter tensors: contiguous, any of f32 / bf16 / f16."""
    if t is None:
        return None
    t = t.detach()
    if t.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        t = t.float()
    return t.contiguous()


# --------------------------------------------------------------------------- scan


def _validate_scan(q, k, value, gate, adt, dt, trap_logits, D, mimo_x, mimo_z, mimo_out,
                   chunk_size, initial_state, initial_k, initial_value, phase, q_bias, k_bias):
    """Argument checks of the reference ``mamba3_scan`` (``ops.py:574-631``)."""
    if q.shape != k.shape or q.ndim != 5:
        raise ValueError("q and k must have matching [B, L, G, R, N] shapes")
    batch, length, qk_heads, rank, d_state = q.shape
    if value.ndim != 4 or gate.shape != value.shape:
        raise ValueError("value and gate must have matching [B, L, H, P] shapes")
    if value.shape[:2] != (batch, length):
        raise ValueError("value dimensions must match q and k")
    heads = value.shape[2]
    if heads % qk_heads != 0:
        raise ValueError("value heads must be divisible by Q/K groups")
    if adt.shape != (batch, length, heads):
        raise ValueError("adt must have shape [B, L, H]")
    if dt.shape != adt.shape or trap_logits.shape != adt.shape:
        raise ValueError("dt and trap_logits must match adt")
    if D.shape != (heads,):
        raise ValueError("D must have shape [H]")
    if (q_bias is None) != (k_bias is None):
        raise ValueError("q_bias and k_bias must be provided together")
    if q_bias is not None:
        expected_bias = (heads, rank, d_state)
        if q_bias.shape != expected_bias or k_bias.shape != expected_bias:
            raise ValueError(f"Q/K biases must have shape {expected_bias}")
    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    if phase is not None and (phase.ndim != 4 or phase.shape[:3] != (batch, length, heads)):
        raise ValueError("phase must have shape [B, L, H, S]")
    head_dim = value.shape[-1]
    expected_state = (batch, heads, head_dim, d_state)
    if initial_state is not None and initial_state.shape != expected_state:
        raise ValueError(f"initial_state must have shape {expected_state}")
    projections = (mimo_x, mimo_z, mimo_out)
    if rank == 1:
        if any(p is not None for p in projections):
            raise ValueError("SISO inputs must not provide MIMO projections")
    else:
        expected_projection = (heads, rank, head_dim)
        if any(p is None or p.shape != expected_projection for p in projections):
            raise ValueError(f"MIMO projections must have shape {expected_projection}")
    if initial_k is not None or initial_value is not None:
        expected_k = (batch, heads, rank, d_state)
        expected_value = (batch, heads, head_dim)
        if initial_k is None or initial_k.shape != expected_k:
            raise ValueError(f"initial_k must have shape {expected_k}")
        if initial_value is None or initial_value.shape != expected_value:
            raise ValueError(f"initial_value must have shape {expected_value}")


def mamba3_scan(q, k, value, gate, adt, dt, trap_logits, D, *, mimo_x=None, mimo_z=None,
                mimo_out=None, chunk_size=64, initial_state=None, initial_k=None,
                initial_value=None, phase=None, mimo_rotation=False, q_bias=None, k_bias=None):
    """Chunked Mamba-3 SSD with an FP32 state (reference ``ops.py:544-822``).

    ``q/k [B,L,G,R,N]`` (RMS-normed, unbiased, unrotated), ``value/gate [B,L,H,P]``,
    ``adt/dt [B,L,H]`` FP32, ``trap_logits [B,L,H]``, optional ``phase [B,L,H,S]`` FP32.
    Returns ``(output [B,L,H,P], state [B,H,P,N] FP32)``. One HIP launch for the whole
    sequence; ``chunk_size`` is validated and passed on as advisory.
    """
    global _HIP_LAST_SCAN_DISPATCH
    _HIP_LAST_SCAN_DISPATCH = False
    _validate_scan(q, k, value, gate, adt, dt, trap_logits, D, mimo_x, mimo_z, mimo_out,
                   chunk_size, initial_state, initial_k, initial_value, phase, q_bias, k_bias)
    device = _require_device(q, k, value, gate, adt, dt, trap_logits, D, initial_state,
                             initial_k, initial_value, phase, q_bias, k_bias, mimo_x)
    _require_inference(q, k, value, gate, adt, dt, trap_logits, D, mimo_x, mimo_z, mimo_out,
                       initial_state, initial_k, initial_value, phase, q_bias, k_bias)
    batch, length, groups, rank, d_state = q.shape
    heads, head_dim = value.shape[2], value.shape[3]
    if not (q.dtype == k.dtype == value.dtype == gate.dtype):
        raise ValueError("q, k, value and gate must share one dtype")
    state_in = None if initial_state is None else _state32(initial_state)
    final_state = torch.empty(batch, heads, head_dim, d_state, device=device,
                              dtype=torch.float32)
    if length == 0 or batch == 0:
        if state_in is None:
            final_state.zero_()
        else:
            final_state.copy_(state_in)
        return value.clone(), final_state
    out = torch.empty(batch, length, heads, head_dim, device=device, dtype=value.dtype)
    num_angles = 0 if phase is None else phase.shape[-1]
    args = _hip.ScanArgs(
        batch=batch, length=length, heads=heads, groups=groups, rank=rank, d_state=d_state,
        head_dim=head_dim, num_angles=num_angles, chunk=chunk_size,
        act_dtype=_hip.dtype_code(q.dtype), mimo_rotation=int(bool(mimo_rotation)), raw_dt=0,
        phase_mode=_hip.PHASE_NONE if phase is None else _hip.PHASE_GIVEN, norm_eps=NORM_EPS,
        segments=SCAN_SEGMENTS)
    keep = [_inner(q), _inner(k), _inner(value), _inner(gate), adt.float(), dt.float(),
            trap_logits, None if phase is None else phase.float(), _param(D), _param(mimo_x),
            _param(mimo_z), _param(mimo_out), _param(q_bias), _param(k_bias), state_in,
            _inner(initial_k), _inner(initial_value)]
    (args.q, args.k, args.value, args.gate, args.a, args.dt, args.trap, args.phase, args.D,
     args.mimo_x, args.mimo_z, args.mimo_out, args.q_bias, args.k_bias, args.initial_state,
     args.initial_k, args.initial_value) = (_hip.tensor(t) for t in keep)
    args.out = _hip.tensor(out)
    args.final_state = _hip.tensor(final_state)
    with torch.cuda.device(device):
        keep.append(_hip.scan_workspace(args, device))
        _hip.call("m3_scan_fwd", args, device)
    _HIP_LAST_SCAN_DISPATCH = True
    return out, final_state


def chunk_state(k, value, cumulative, scale, state, output, *, width: int, rank: int) -> None:
    """One chunk's state update (reference ``_triton.py:500-561``), written into ``output``.

    ``k [B,H,W,R,N]`` biased and rotated, ``value [B,H,W,R,P]`` rank values,
    ``cumulative/scale [B,H,W]`` FP32, ``state/output [B,H,P,N]`` FP32 (may be the same).
    """
    device = _require_device(k, value, cumulative, scale, state, output)
    batch, heads, head_dim, d_state = state.shape
    if k.shape[2] < width or value.shape[2] < width:
        raise ValueError("width exceeds the chunk tensors")
    if output.dtype != torch.float32 or state.dtype != torch.float32:
        raise ValueError("state and output must be float32")
    args = _hip.ChunkStateArgs(batch=batch, width=width, heads=heads, rank=rank,
                               d_state=d_state, head_dim=head_dim,
                               act_dtype=_hip.dtype_code(k.dtype))
    keep = [_inner(k), _inner(value), cumulative.float(), scale.float(), _inner(state)]
    args.k, args.value, args.cumulative, args.scale, args.state_in = (
        _hip.tensor(t) for t in keep)
    if output.stride(-1) != 1:
        raise ValueError("output must have a unit innermost stride")
    args.state_out = _hip.tensor(output)
    with torch.cuda.device(device):
        _hip.call("m3_chunk_state", args, device)


# --------------------------------------------------------------------------- step


def _step_call(q, k, value, gate, adt, dt, trap_logits, angle_rate, D, cache, *, mimo_x,
               mimo_z, mimo_out, phase_mode, raw=None, out_cache=None):
    phase, state, prev_k, prev_v = cache
    device = _require_device(q, k, value, gate, state, prev_k, prev_v, D)
    batch, groups, rank, d_state = q.shape
    heads, head_dim = value.shape[1], value.shape[2]
    num_angles = phase.shape[-1]
    out = torch.empty(batch, heads, head_dim, device=device, dtype=value.dtype)
    if out_cache is None:
        phase_out = torch.empty(batch, heads, num_angles, device=device, dtype=torch.float32)
        state_out = torch.empty(batch, heads, head_dim, d_state, device=device,
                                dtype=torch.float32)
        k_out = torch.empty(batch, heads, rank, d_state, device=device, dtype=q.dtype)
        value_out = None
    else:
        phase_out, state_out, k_out, value_out = out_cache
    if batch == 0:
        return out, (phase_out, state_out, k_out, value if value_out is None else value_out)
    args = _hip.StepArgs(batch=batch, heads=heads, groups=groups, rank=rank, d_state=d_state,
                         head_dim=head_dim, num_angles=num_angles,
                         act_dtype=_hip.dtype_code(q.dtype), mimo_rotation=int(rank > 1),
                         raw_dt=int(raw is not None), phase_mode=phase_mode, norm_eps=NORM_EPS)
    keep = [_inner(q), _inner(k), _inner(value), _inner(gate), dt, adt, trap_logits,
            angle_rate, _param(D), _param(mimo_x), _param(mimo_z), _param(mimo_out),
            phase, _state32(state), _inner(prev_k), _inner(prev_v)]
    (args.q, args.k, args.value, args.gate, args.dt, args.a, args.trap, args.angles, args.D,
     args.mimo_x, args.mimo_z, args.mimo_out, args.phase_in, args.state_in, args.prev_k,
     args.prev_value) = (_hip.tensor(t) for t in keep)
    if raw is not None:
        q_norm_w, k_norm_w, q_bias, k_bias, dt_bias = (_param(t) for t in raw)
        keep += [q_norm_w, k_norm_w, q_bias, k_bias, dt_bias]
        args.q_norm_w, args.k_norm_w = _hip.tensor(q_norm_w), _hip.tensor(k_norm_w)
        args.q_bias, args.k_bias = _hip.tensor(q_bias), _hip.tensor(k_bias)
        args.dt_bias = _hip.tensor(dt_bias)
    args.out = _hip.tensor(out)
    args.phase_out = _hip.tensor(phase_out)
    args.state_out = _hip.tensor(state_out)
    args.k_out = _hip.tensor(k_out)
    args.value_out = _hip.tensor(value_out)
    with torch.cuda.device(device):
        _hip.call("m3_step", args, device)
    return out, (phase_out, state_out, k_out, value if value_out is None else value_out)


def _validate_step_shapes(q, k, value, gate, adt, dt, trap_logits, D, cache, mimo_x, mimo_z,
                          mimo_out, angle_rate=None):
    """Shape checks of the reference fused step launcher (``_triton.py:968-1044``)."""
    phase, state, previous_k, previous_value = cache
    if q.ndim != 4 or q.shape != k.shape:
        raise ValueError("q and k must have the same [B, H, R, N] shape")
    batch, heads, rank, d_state = q.shape
    head_dim = value.shape[-1]
    num_angles = phase.shape[-1]
    expected = {
        "value": (batch, heads, head_dim), "gate": (batch, heads, head_dim),
        "adt": (batch, heads), "dt": (batch, heads), "trap_logits": (batch, heads),
        "D": (heads,), "phase": (batch, heads, num_angles),
        "state": (batch, heads, head_dim, d_state),
        "previous_k": (batch, heads, rank, d_state),
        "previous_value": (batch, heads, head_dim),
    }
    given = {"value": value, "gate": gate, "adt": adt, "dt": dt, "trap_logits": trap_logits,
             "D": D, "phase": phase, "state": state, "previous_k": previous_k,
             "previous_value": previous_value}
    if angle_rate is not None:
        expected["angle_rate"] = (batch, num_angles)
        given["angle_rate"] = angle_rate
    for name, shape in expected.items():
        if tuple(given[name].shape) != shape:
            raise ValueError(f"invalid {name} shape: expected {shape}, "
                             f"got {tuple(given[name].shape)}")
    if not (q.dtype == k.dtype == value.dtype == gate.dtype):
        raise ValueError("q, k, value, and gate must have the same dtype")
    if previous_k.dtype != q.dtype or previous_value.dtype != value.dtype:
        raise ValueError("K/value cache dtypes must match current activations")
    if phase.dtype != torch.float32 or state.dtype != torch.float32:
        raise ValueError("phase and state must be float32")
    if rank > 1:
        for name, proj in (("mimo_x", mimo_x), ("mimo_z", mimo_z), ("mimo_out", mimo_out)):
            if proj is None or proj.shape != (heads, rank, head_dim):
                raise ValueError(f"invalid {name} shape: expected {(heads, rank, head_dim)}")
    elif mimo_x is not None:
        raise ValueError("MIMO projections require rank > 1")


def fused_step(q, k, value, gate, adt, dt, trap_logits, angle_rate, D, cache, *, mimo_x=None,
               mimo_z=None, mimo_out=None):
    """One decode token with the phase advance and rotation fused (``ops.py:87-190``).

    Inputs are head-expanded, biased and unrotated: ``q/k [B,H,R,N]``, ``value/gate
    [B,H,P]``, ``adt/dt/trap_logits [B,H]``, ``angle_rate [B,S]``; ``cache = (phase
    [B,H,S] FP32, state [B,H,P,N] FP32, prev_k [B,H,R,N], prev_value [B,H,P])``.
    Returns ``(output [B,H,P], (phase', state', k_rot, value))``.
    """
    global _HIP_LAST_DISPATCH
    _HIP_LAST_DISPATCH = False
    _validate_step_shapes(q, k, value, gate, adt, dt, trap_logits, D, cache, mimo_x, mimo_z,
                          mimo_out, angle_rate)
    _require_inference(q, k, value, gate, adt, dt, trap_logits, angle_rate, D, *cache)
    result = _step_call(q, k, value, gate, adt, dt, trap_logits, angle_rate, D, cache,
                        mimo_x=mimo_x, mimo_z=mimo_z, mimo_out=mimo_out,
                        phase_mode=_hip.PHASE_ANGLES)
    _HIP_LAST_DISPATCH = True
    return result


def mamba3_step(q, k, value, gate, adt, dt, trap_logits, D, cache, *, mimo_x=None,
                mimo_z=None, mimo_out=None):
    """One exact recurrent update with rotated ``q/k [B,H,R,N]`` (``ops.py:825-879``).

    The cache phase is passed through unchanged.
    """
    global _HIP_LAST_DISPATCH
    _HIP_LAST_DISPATCH = False
    _validate_step_shapes(q, k, value, gate, adt, dt, trap_logits, D, cache, mimo_x, mimo_z,
                          mimo_out)
    _require_inference(q, k, value, gate, adt, dt, trap_logits, D, *cache)
    out, nxt = _step_call(q, k, value, gate, adt, dt, trap_logits, None, D, cache,
                          mimo_x=mimo_x, mimo_z=mimo_z, mimo_out=mimo_out,
                          phase_mode=_hip.PHASE_NONE)
    _HIP_LAST_DISPATCH = True
    return out, nxt


# --------------------------------------------------------------------------- projection form


def split_projection(proj: torch.Tensor, mixer) -> dict[str, torch.Tensor]:
    """Views into the ``in_proj`` output in the reference split order (``model.py:147-163``):
    ``[z, x, B, C, dd_dt, dd_A, trap, angles]``."""
    d_inner, n, r = mixer.d_inner, mixer.d_state, mixer.mimo_rank
    h, p, s = mixer.nheads, mixer.headdim, mixer.num_angles
    sizes = (d_inner, d_inner, n * r, n * r, h, h, h, s)
    z, x, b, c, ddt, da, trap, ang = torch.split(proj, sizes, dim=-1)
    lead = proj.shape[:-1]
    return dict(
        z=z.unflatten(-1, (h, p)), x=x.unflatten(-1, (h, p)),
        k=b.unflatten(-1, (1, r, n)), q=c.unflatten(-1, (1, r, n)),
        dt=ddt, a=da, trap=trap, angles=ang, lead=lead)


def _backwards(desc: _hip.Tensor, length: int) -> None:
    """Make a per-token descriptor run backwards: token t at the old token L - 1 - t."""
    if desc.ptr is None or length <= 1:
        return
    size = 4 if desc.dtype == _hip.F32 else 2
    desc.ptr += (length - 1) * desc.stride[1] * size
    desc.stride[1] = -desc.stride[1]


class ScanCall:
    """One ``m3_scan_fwd`` launch over the raw ``in_proj`` output ``[B, L, proj]``, prepared once.

    Holds the argument block, the outputs, the workspace and references to every tensor the
    block points at; ``launch()`` enqueues the call on the device's current stream and may be
    repeated (each launch rewrites the outputs). Fuses the reference mixer's ``_project`` (B/C
    RMSNorm, dt, adt; ``model.py:165``), ``_phase`` (``model.py:215``), bias, rotation and the
    chunked SSD (reference ``model.py:282-309``).

    ``reverse=True`` scans the sequence from its last token to its first, reading ``proj`` and
    writing ``out`` through backwards token strides: ``out`` then holds, in forward order,
    what scanning ``flip(proj)`` and flipping the result back gives (the reverse direction of
    a bidirectional layer, reference ``model.py:330-362``, without either flip or a second
    projection).

    ``concurrent``: how many calls of this shape run at once (2 for the two directions of a
    bidirectional layer). A long sequence of few (batch, head) pairs is split into segments
    sized for the calls' combined grid, unless ``SCAN_SEGMENTS`` fixes the split.
    """

    def __init__(self, proj: torch.Tensor, mixer, *, cache=None, want_cache: bool = False,
                 chunk_size: int = 256, reverse: bool = False, concurrent: int = 1):
        self.device = _require_device(proj)
        v = split_projection(proj, mixer)
        batch, length = proj.shape[0], proj.shape[1]
        h, p, n, r = mixer.nheads, mixer.headdim, mixer.d_state, mixer.mimo_rank
        s = mixer.num_angles
        act = proj.dtype
        if cache is not None:
            init_phase, init_state, init_k, init_v = cache
            if init_k.dtype != act or init_v.dtype != act:
                raise ValueError("K/value cache dtypes must match the activations")
        else:
            init_phase = init_state = init_k = init_v = None
        dev = self.device
        self.out = torch.empty(batch, length, h, p, device=dev, dtype=act)
        self.final_state = torch.empty(batch, h, p, n, device=dev, dtype=torch.float32)
        self.final_phase = (torch.empty(batch, h, s, device=dev, dtype=torch.float32)
                            if want_cache else None)
        self.final_k = torch.empty(batch, h, r, n, device=dev, dtype=act) if want_cache else None
        args = _hip.ScanArgs(
            batch=batch, length=length, heads=h, groups=1, rank=r, d_state=n, head_dim=p,
            num_angles=s, chunk=chunk_size, act_dtype=_hip.dtype_code(act),
            mimo_rotation=int(r > 1), raw_dt=1, phase_mode=_hip.PHASE_ANGLES,
            norm_eps=NORM_EPS, segments=SCAN_SEGMENTS)
        params = [_param(t) for t in (mixer.C_norm.weight, mixer.B_norm.weight, mixer.C_bias,
                                      mixer.B_bias, mixer.dt_bias, mixer.D, mixer.mimo_x,
                                      mixer.mimo_z, mixer.mimo_out)]
        keep = [v["q"], v["k"], v["x"], v["z"], v["dt"], v["a"], v["trap"], v["angles"],
                init_phase, None if init_state is None else _state32(init_state),
                _inner(init_k), _inner(init_v), *params]
        (args.q, args.k, args.value, args.gate, args.dt, args.a, args.trap, args.phase,
         args.initial_phase, args.initial_state, args.initial_k, args.initial_value,
         args.q_norm_w, args.k_norm_w, args.q_bias, args.k_bias, args.dt_bias, args.D,
         args.mimo_x, args.mimo_z, args.mimo_out) = (_hip.tensor(t) for t in keep)
        args.out = _hip.tensor(self.out)
        args.final_state = _hip.tensor(self.final_state)
        args.final_phase = _hip.tensor(self.final_phase)
        args.final_k = _hip.tensor(self.final_k)
        if reverse:
            if cache is not None or want_cache:
                raise ValueError("a reverse scan has no cache")
            for desc in (args.q, args.k, args.value, args.gate, args.dt, args.a, args.trap,
                         args.phase, args.out):
                _backwards(desc, length)
        if concurrent > 1 and args.segments == 0:
            # `concurrent` calls of this shape share the GPU (the two directions of a
            # bidirectional layer): the library's segment choice for their combined grid
            args.segments = _hip.scan_segments(args, concurrent)
        with torch.cuda.device(dev):
            keep.append(_hip.scan_workspace(args, dev))
        self.args = args
        self._keep = keep

    def launch(self) -> None:
        global _HIP_LAST_SCAN_DISPATCH
        _HIP_LAST_SCAN_DISPATCH = False
        with torch.cuda.device(self.device):
            _hip.call("m3_scan_fwd", self.args, self.device)
        _HIP_LAST_SCAN_DISPATCH = True


def scan_projection(proj: torch.Tensor, mixer, *, cache=None, want_cache: bool = False,
                    chunk_size: int = 256, reverse: bool = False, concurrent: int = 1):
    """The whole mixer scan from the raw ``in_proj`` output ``[B, L, proj]``.

    Fuses the reference mixer's ``_project`` (B/C RMSNorm, dt, adt; ``model.py:165``),
    ``_phase``, bias, rotation and the chunked SSD (reference ``model.py:282-309``). Returns ``(mixed [B,L,H,P], state, final_phase,
    final_k)``; the last two are ``None`` unless ``want_cache``. ``reverse``, ``concurrent``: see
    ``ScanCall``.
    """
    call = ScanCall(proj, mixer, cache=cache, want_cache=want_cache, chunk_size=chunk_size,
                    reverse=reverse, concurrent=concurrent)
    call.launch()
    return call.out, call.final_state, call.final_phase, call.final_k


def step_projection(proj: torch.Tensor, mixer, cache, *, inplace: bool = False):
    """One decode token from the raw ``in_proj`` output ``[B, 1, proj]``.

    Fuses the reference mixer's ``_project`` and ``_expand_qk`` (``model.py:165``, ``201``),
    the phase advance, the rotation and the step (reference ``model.py:431-484``). With ``inplace`` the cache tensors are updated in
    place (the hipGraph decoder's static cache) and returned.
    """
    global _HIP_LAST_DISPATCH
    _HIP_LAST_DISPATCH = False
    v = split_projection(proj[:, 0], mixer)  # q, k: [B, G=1, R, N]; x, z: [B, H, P]
    q, k = v["q"], v["k"]
    out_cache = cache if inplace else None
    out, nxt = _step_call(
        q, k, v["x"], v["z"], v["a"], v["dt"], v["trap"], v["angles"], mixer.D, cache,
        mimo_x=mixer.mimo_x, mimo_z=mixer.mimo_z, mimo_out=mixer.mimo_out,
        phase_mode=_hip.PHASE_ANGLES,
        raw=(mixer.C_norm.weight, mixer.B_norm.weight, mixer.C_bias, mixer.B_bias,
             mixer.dt_bias),
        out_cache=out_cache)
    _HIP_LAST_DISPATCH = True
    return out, nxt


# --------------------------------------------------------------------------- decode GEMMs

LINEAR_MAX_ROWS = 256
# The fused RMSNorm takes up to 32 rows, or up to 64 when K is a multiple of 256.
LINEAR_NORM_MAX_ROWS = 64
# Decode steps run in_proj (with the block's RMSNorm fused) on ``linear`` up to
# DECODE_LINEAR_ROWS rows, and out_proj (with the residual add fused) up to
# DECODE_LINEAR_OUT_ROWS. Measured on the decode shapes with cold weights: above these, hipBLASLt
# (plus the separate norm or add) is faster.
DECODE_LINEAR_ROWS = 64
DECODE_LINEAR_OUT_ROWS = 64


def linear_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether ``linear(x, weight)`` takes these operands: 2-D, on one ROCm device, both
    bfloat16 or both float16, at most ``LINEAR_MAX_ROWS`` rows, K a multiple of 32 with
    16-byte aligned rows, no autograd, and no autocast that would compute in another dtype."""
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        return False
    if x.device.type != "cuda" or weight.device != x.device:
        return False
    if x.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != x.dtype:
        return False
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") != x.dtype:
        return False
    if torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad):
        return False
    m, k = x.shape
    if not 0 < m <= LINEAR_MAX_ROWS or k % 32 != 0 or weight.shape[0] == 0:
        return False
    for t in (x, weight):
        if t.stride(1) != 1 or t.stride(0) % 8 != 0 or t.data_ptr() % 16 != 0:
            return False
    return True


def linear_norm_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether ``linear(x, weight, norm_weight=...)`` takes these operands: ``linear_supported``
    and at most 32 rows, or at most ``LINEAR_NORM_MAX_ROWS`` with K a multiple of 256."""
    if not linear_supported(x, weight):
        return False
    m, k = x.shape
    return m <= 32 or (m <= LINEAR_NORM_MAX_ROWS and k % 256 == 0)


def linear(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor | None = None, *,
           out: torch.Tensor | None = None, norm_weight: torch.Tensor | None = None,
           norm_eps: float = NORM_EPS) -> torch.Tensor:
    """``x @ weight.T (+ residual)`` for the few rows of a decode step (``m3_linear``).

    ``x`` is ``[M, K]`` (``M <= 256``), ``weight`` the ``[N, K]`` weight of an ``nn.Linear``
    without bias, both bfloat16 or both float16 (``linear_supported``); ``residual`` and
    ``out`` are ``[M, N]`` of that dtype. Products accumulate in FP32; the residual is added
    to the FP32 sum, which is rounded once. With ``norm_weight`` (``[K]``; ``M <= 32``, or
    ``M <= 64`` with K a multiple of 256) ``x`` is first RMS-normalised, as
    ``F.rms_norm(x, (K,), norm_weight, norm_eps)``. This replaces
    the decode step's RMSNorm, ``in_proj`` / ``out_proj`` calls and the block's residual add
    (reference ``model.py:441-458, 514-520``).
    """
    device = _require_device(x, weight, residual, out, norm_weight)
    _require_inference(x, weight, residual, norm_weight)
    if not linear_supported(x, weight):
        raise ValueError(
            f"linear: unsupported operands x {tuple(x.shape)} {x.dtype} strides {x.stride()}, "
            f"weight {tuple(weight.shape)} {weight.dtype} strides {weight.stride()}")
    m, n = x.shape[0], weight.shape[0]
    for name, t in (("residual", residual), ("out", out)):
        if t is not None and (tuple(t.shape) != (m, n) or t.dtype != x.dtype):
            raise ValueError(f"linear: {name} must be [{m}, {n}] {x.dtype}, got "
                             f"{tuple(t.shape)} {t.dtype}")
    if norm_weight is not None:
        if not linear_norm_supported(x, weight):
            raise ValueError(f"linear: norm_weight needs at most 32 rows, or at most "
                             f"{LINEAR_NORM_MAX_ROWS} with K a multiple of 256")
        norm_weight = norm_weight.detach().to(x.dtype).contiguous()
        if norm_weight.shape != (x.shape[1],):
            raise ValueError(f"linear: norm_weight must be [{x.shape[1]}]")
        if norm_weight.data_ptr() % 16:
            norm_weight = norm_weight.clone()
    residual = _inner(residual)
    if out is None:
        out = torch.empty(m, n, dtype=x.dtype, device=device)
    elif out.stride(1) != 1:
        raise ValueError("linear: out needs a unit inner stride")
    args = _hip.LinearArgs()
    args.m, args.n, args.k = m, n, x.shape[1]
    args.dtype = _hip.dtype_code(x.dtype)
    args.x = _hip.tensor(x)
    args.weight = _hip.tensor(weight.detach())
    args.norm_weight = _hip.tensor(norm_weight)
    args.norm_eps = float(norm_eps)
    args.residual = _hip.tensor(residual)
    args.out = _hip.tensor(out)
    ws = _hip.scan_workspace(args, device, "m3_linear_workspace_size")
    _hip.call("m3_linear", args, device)
    del ws
    return out


# --------------------------------------------------------------------------- residual stream

RMS_NORM_DIMS = (256, 512, 768, 1024, 2048)
_FLOAT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _rows_ok(t: torch.Tensor) -> bool:
    return t.is_contiguous() and t.data_ptr() % (4 * t.element_size()) == 0


def rms_norm_supported(x: torch.Tensor, weight: torch.Tensor, add: torch.Tensor | None = None,
                       out_dtype: torch.dtype | None = None) -> bool:
    """Whether ``rms_norm`` takes these operands: contiguous rows on one ROCm device, the last
    axis in ``RMS_NORM_DIMS``, an FP32 ``x`` with any ``add`` / ``out_dtype`` or a 16-bit ``x``
    with both of its own dtype, and no autograd."""
    out_dtype = out_dtype or x.dtype
    if x.device.type != "cuda" or x.dim() < 1 or x.shape[-1] not in RMS_NORM_DIMS:
        return False
    if x.dtype not in _FLOAT_DTYPES or out_dtype not in _FLOAT_DTYPES:
        return False
    if weight.device != x.device or tuple(weight.shape) != (x.shape[-1],):
        return False
    if weight.dtype not in _FLOAT_DTYPES or not _rows_ok(x):
        return False
    if add is not None:
        if add.device != x.device or add.shape != x.shape or not _rows_ok(add):
            return False
        if add.dtype not in _FLOAT_DTYPES or (x.dtype != torch.float32 and add.dtype != x.dtype):
            return False
    if x.dtype != torch.float32 and out_dtype != x.dtype:
        return False
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, weight, add)):
        return False
    return True


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = NORM_EPS, *,
             add: torch.Tensor | None = None, keep_sum: bool = False,
             out_dtype: torch.dtype | None = None):
    """One pass of the residual stream (``m3_rms_norm``): ``s = x + add`` (or ``x``), then
    ``F.rms_norm(s, (d,), weight.to(s.dtype), eps)`` written as ``out_dtype`` (default
    ``x.dtype``). Returns ``(out, s)`` with ``s`` only when ``keep_sum`` (``add`` given).

    ``s`` is the reference's ``hidden_states + mixed`` (``model.py:511-512``; an FP32 ``x``
    takes an ``add`` of any dtype), ``out`` its next RMSNorm (``model.py:48-55``) already in
    the dtype the next projection computes in, so the add, the norm and autocast's cast are one
    pass over the rows instead of three.
    """
    out_dtype = out_dtype or x.dtype
    device = _require_device(x, weight, add)
    _require_inference(x, weight, add)
    if not rms_norm_supported(x, weight, add, out_dtype):
        raise ValueError(f"rms_norm: unsupported operands x {tuple(x.shape)} {x.dtype}, add "
                         f"{None if add is None else (tuple(add.shape), add.dtype)}, out "
                         f"{out_dtype}")
    if keep_sum and add is None:
        raise ValueError("rms_norm: keep_sum needs add")
    d = x.shape[-1]
    rows = x.numel() // d
    w = weight.detach()
    if w.data_ptr() % (4 * w.element_size()) or not w.is_contiguous():
        w = w.contiguous().clone()
    out = torch.empty(x.shape, dtype=out_dtype, device=device)
    s = torch.empty_like(x) if keep_sum else None
    if rows == 0:
        return out, s
    args = _hip.RmsNormArgs()
    args.rows, args.dim, args.eps = rows, d, float(eps)
    args.x = _hip.tensor(x.view(rows, d))
    args.add = _hip.tensor(None if add is None else add.view(rows, d))
    args.weight = _hip.tensor(w)
    args.sum_out = _hip.tensor(None if s is None else s.view(rows, d))
    args.out = _hip.tensor(out.view(rows, d))
    _hip.call("m3_rms_norm", args, device)
    return out, s


__all__ = ["heavy_tail_activation", "mamba3_scan", "mamba3_step", "fused_step", "chunk_state",
           "ScanCall", "scan_projection", "step_projection", "split_projection", "linear",
           "linear_supported", "rms_norm", "rms_norm_supported"]
