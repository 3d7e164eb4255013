"""CPU oracle: restatement of the reference's portable PyTorch Mamba-3 path.

TEST INFRASTRUCTURE ONLY. Imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; never by the product package
``mamba3_amd``.

Every function restates one piece of jreoka/mamba3 (file:line cited in its
docstring) as a pure function over tensors and a parameter dictionary whose
keys are the reference's ``state_dict`` names. The low-precision rounding
points of the reference are kept: bias and rotation in the activation dtype,
``scale`` cast to the activation dtype before ``k * scale``, the decayed scores
cast before the value GEMM, the FP32 state cast to the activation dtype for the
inter-chunk and readout GEMMs, ``end_decay`` cast before ``k * end_decay``.
GEMMs take their operands as given and accumulate in FP32.

Pinning (how each function is checked; see ``tests/test_oracle.py``):

* ``heavy_tail`` -- closed form and derivative (reference
  ``tests/test_scan.py:145-152``).
* ``rotate`` -- known answers (``tests/test_scan.py:155-168``), the rotation
  matrix closed form, norm preservation, golden vectors (f32 and bf16).
* ``phase_scan`` -- sequential fmod recurrence
  (``tests/test_model.py:225-250``), constant-increment closed form
  (``tests/test_model.py:252-273``), golden vectors.
* ``ssd_scan`` -- independent float64 per-token recurrence
  (``oracle/recurrence.py``), chunk-size invariance, continuation, empty
  input, Mamba-2 / linear-attention special cases, golden vectors (f32, bf16).
* ``step_update`` -- one step of the float64 recurrence, golden vectors.
* ``init_params`` / ``project`` / ``mixer_*`` / ``model_*`` -- golden vectors
  generated from the reference (parameter checksums, forward, prefill + cache,
  decode steps, bidirectional forward, bf16 autocast).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch.nn import functional as F

TWO_PI = 2.0 * math.pi
PHASE_BLOCK = 64  # model.py:25
A_FLOOR = 1e-4  # model.py:22
EXPANSION = 2  # model.py:19
CANONICAL_HEAD_DIM = 64  # model.py:20
ROPE_FRACTION = 0.5  # model.py:21
NORM_EPS = 1e-5  # model.py:43


@dataclass(frozen=True)
class Dims:
    """Derived mixer sizes (model.py:74-108)."""

    d_model: int
    d_state: int
    mimo_rank: int

    @property
    def d_inner(self) -> int:
        return EXPANSION * self.d_model

    @property
    def headdim(self) -> int:
        return math.gcd(self.d_inner, CANONICAL_HEAD_DIM)

    @property
    def nheads(self) -> int:
        return self.d_inner // self.headdim

    @property
    def num_angles(self) -> int:
        return int(self.d_state * ROPE_FRACTION) // 2

    @property
    def split_sizes(self) -> tuple[int, ...]:
        nr = self.d_state * self.mimo_rank
        h = self.nheads
        return (self.d_inner, self.d_inner, nr, nr, h, h, h, self.num_angles)

    @property
    def proj_size(self) -> int:
        return sum(self.split_sizes)

    @property
    def inference_chunk(self) -> int:
        """model.py:26-37 (inference branch)."""
        return 256 if self.mimo_rank == 1 else max(16, 128 // self.mimo_rank)


# ---------------------------------------------------------------------------
# parameters


def _kaiming_linear(out_features: int, in_features: int) -> torch.Tensor:
    w = torch.empty(out_features, in_features)
    torch.nn.init.kaiming_uniform_(w, a=math.sqrt(5))
    return w


def init_params(d_model: int, d_state: int = 128, depth: int = 4, mimo_rank: int = 1,
                causal: bool = True) -> dict[str, torch.Tensor]:
    """Parameters in the reference's creation order (model.py:103-145, 559-568).

    Consumes the global torch RNG exactly as the reference constructor does:
    per layer ``in_proj`` (kaiming uniform), ``torch.rand(H)`` for ``dt_bias``,
    then ``out_proj``; the remaining tensors are constants. ``out_proj`` is
    divided by ``sqrt(depth)``.
    """
    dims = Dims(d_model, d_state, mimo_rank)
    h, r, n, p = dims.nheads, mimo_rank, d_state, dims.headdim
    params: dict[str, torch.Tensor] = {}
    for i in range(depth):
        pre = f"layers.{i}.mixer."
        params[f"layers.{i}.norm.weight"] = torch.ones(d_model)
        params[pre + "in_proj.weight"] = _kaiming_linear(dims.proj_size, d_model)
        params[pre + "B_norm.weight"] = torch.ones(n)
        params[pre + "C_norm.weight"] = torch.ones(n)
        params[pre + "B_bias"] = torch.ones(h, r, n)
        params[pre + "C_bias"] = torch.ones(h, r, n)
        u = torch.rand(h)
        dt = torch.exp(u * (math.log(0.1) - math.log(0.001)) + math.log(0.001)).clamp_min(1e-4)
        params[pre + "dt_bias"] = dt + torch.log(-torch.expm1(-dt))
        params[pre + "D"] = torch.ones(h)
        if mimo_rank > 1:
            params[pre + "mimo_x"] = torch.full((h, r, p), 1.0 / r)
            params[pre + "mimo_z"] = torch.ones(h, r, p)
            params[pre + "mimo_out"] = torch.full((h, r, p), 1.0 / r)
        params[pre + "out_proj.weight"] = _kaiming_linear(d_model, dims.d_inner)
        if not causal:
            params[pre + "direction_logit"] = torch.zeros(d_model)
    params["norm_f.weight"] = torch.ones(d_model)
    for i in range(depth):
        params[f"layers.{i}.mixer.out_proj.weight"] /= math.sqrt(depth)
    return params


# ---------------------------------------------------------------------------
# elementwise pieces


def heavy_tail(x: torch.Tensor) -> torch.Tensor:
    """ops.py:28-32: ``1 + x`` for ``x >= 0``, ``1 / (1 - x)`` otherwise."""
    return torch.where(x >= 0, 1.0 + x, 1.0 / (1.0 - x.clamp_max(0)))


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = NORM_EPS) -> torch.Tensor:
    """model.py:42-55: RMSNorm over the last axis, result in the input dtype."""
    return F.rms_norm(x, (x.shape[-1],), weight.to(dtype=x.dtype), eps).to(dtype=x.dtype)


def rotate(q: torch.Tensor, k: torch.Tensor, phase: torch.Tensor, *, mimo: bool):
    """ops.py:35-84: real-coordinate rotation of Q/K by ``phase [B,L,H,S]``.

    SISO rotates adjacent pairs ``(2i, 2i+1)`` for ``i < S``; MIMO rotates the
    first state quarter against the third. cos/sin are FP32 then cast to the
    activation dtype; products and sums are in the activation dtype.
    """
    s = phase.shape[-1]
    c = torch.cos(phase.unsqueeze(3)).to(q.dtype)
    sn = torch.sin(phase.unsqueeze(3)).to(q.dtype)

    def one(t: torch.Tensor) -> torch.Tensor:
        if mimo:
            a, b2, b, d2, tail = (t[..., :s], t[..., s:2 * s], t[..., 2 * s:3 * s],
                                  t[..., 3 * s:4 * s], t[..., 4 * s:])
            ra = a * c - b * sn
            rb = a * sn + b * c
            return torch.cat((ra, b2, rb, d2, tail), dim=-1)
        pairs = t[..., :2 * s].unflatten(-1, (s, 2))
        a, b = pairs[..., 0], pairs[..., 1]
        ra = a * c - b * sn
        rb = a * sn + b * c
        return torch.cat((torch.stack((ra, rb), dim=-1).flatten(-2), t[..., 2 * s:]), dim=-1)

    return one(q), one(k)


def phase_increment(angles: torch.Tensor, dt: torch.Tensor) -> torch.Tensor:
    """model.py:225-230 / 460-465: ``fmod(pi * tanh(angle) * dt, 2 pi)``.

    ``angles [..., S]`` and ``dt [..., H]`` broadcast to ``[..., H, S]``.
    """
    return torch.fmod(math.pi * torch.tanh(angles.float()).unsqueeze(-2) * dt.unsqueeze(-1),
                      TWO_PI)


def phase_scan(angles: torch.Tensor, dt: torch.Tensor,
               initial_phase: torch.Tensor | None = None) -> torch.Tensor:
    """model.py:215-256: bounded phase accumulation.

    The increments are summed in 64-token blocks counted from the start of the
    call; each block adds an fmod-reduced carry, and the carry itself is
    fmod-reduced block to block. Returns ``[B, L, H, S]`` FP32.
    """
    inc = phase_increment(angles, dt)
    batch, length, heads, count = inc.shape
    carry = (torch.zeros(batch, heads, count, dtype=inc.dtype, device=inc.device)
             if initial_phase is None else initial_phase)
    out = torch.empty_like(inc)
    for s0 in range(0, length, PHASE_BLOCK):
        local = torch.cumsum(inc[:, s0:s0 + PHASE_BLOCK], dim=1)
        out[:, s0:s0 + PHASE_BLOCK] = torch.fmod(local + carry.unsqueeze(1), TWO_PI)
        carry = torch.fmod(carry + local[:, -1], TWO_PI)
    return out


def _rank_values(value: torch.Tensor, projection: torch.Tensor | None) -> torch.Tensor:
    """ops.py:193-199: ``value [..., H, P] -> [..., H, R, P]`` (times mimo_x/z)."""
    if projection is None:
        return value.unsqueeze(-2)
    return value.unsqueeze(-2) * projection.to(value.dtype)


def _bmm_f32(left: torch.Tensor, right: torch.Tensor) -> torch.Tensor:
    """ops.py:508-533 with ``accumulate_float``: operands as given, FP32 result."""
    lead = left.shape[:-2]
    with torch.autocast(left.device.type, enabled=False):
        out = torch.bmm(left.reshape(-1, *left.shape[-2:]).float(),
                        right.reshape(-1, *right.shape[-2:]).float())
    return out.reshape(*lead, left.shape[-2], right.shape[-1])


def _expand_heads(t: torch.Tensor, heads: int) -> torch.Tensor:
    """ops.py:700-709: groups ``[B, L, G, R, N] -> [B, L, H, R, N]``."""
    groups = t.shape[2]
    if groups == heads:
        return t
    if groups == 1:
        return t.expand(-1, -1, heads, -1, -1)
    return t.repeat_interleave(heads // groups, dim=2)


# ---------------------------------------------------------------------------
# the chunked SSD and the decode step


def ssd_scan(q, k, value, gate, adt, dt, trap_logits, D, *, mimo_x=None, mimo_z=None,
             mimo_out=None, chunk_size=64, initial_state=None, initial_k=None,
             initial_value=None, phase=None, mimo_rotation=False, q_bias=None,
             k_bias=None):
    """ops.py:544-822: chunked Mamba-3 SSD with an FP32 state carry.

    ``q/k [B,L,G,R,N]``, ``value/gate [B,L,H,P]``, ``adt/dt/trap_logits
    [B,L,H]``. Returns ``(output [B,L,H,P], state [B,H,P,N] FP32)``.
    """
    batch, length, _, rank, d_state = q.shape
    heads, head_dim = value.shape[2], value.shape[3]
    act = q.dtype
    if initial_state is None:
        state = torch.zeros(batch, heads, head_dim, d_state, dtype=torch.float32,
                            device=value.device)
    else:
        state = initial_state.float()
    if length == 0:
        return value.clone(), state

    # exp-trapezoidal discretization (ops.py:659-671)
    trap = torch.sigmoid(trap_logits.float())
    gamma = dt * trap
    right = torch.zeros_like(dt)
    right[:, :-1] = dt[:, 1:] * (1.0 - trap[:, 1:])
    scale = gamma + right
    diag = gamma / scale
    scale_act = scale.to(k.dtype)

    # endpoint continuation (ops.py:681-686)
    if initial_k is not None:
        prev_v = _rank_values(initial_value, mimo_x)  # [B,H,R,P]
        outer = _bmm_f32(prev_v.transpose(-1, -2), initial_k)
        state = state + (dt[:, 0] * (1.0 - trap[:, 0]))[..., None, None] * outer

    # expand, bias, rotate once (ops.py:700-714)
    qf = _expand_heads(q, heads)
    kf = _expand_heads(k, heads)
    if q_bias is not None:
        qf = qf + q_bias.to(act)
        kf = kf + k_bias.to(k.dtype)
    if phase is not None:
        qf, kf = rotate(qf, kf, phase, mimo=mimo_rotation)
    v_rank = _rank_values(value, mimo_x)  # [B,L,H,R,P]
    z_rank = _rank_values(gate, mimo_z)
    d_f = D.float()[None, :, None, None, None]

    outputs = []
    for c0 in range(0, length, chunk_size):
        sl = slice(c0, min(c0 + chunk_size, length))
        width = sl.stop - sl.start
        qc = qf[:, sl].permute(0, 2, 1, 3, 4)  # [B,H,W,R,N]
        kc = kf[:, sl].permute(0, 2, 1, 3, 4)
        vc = v_rank[:, sl].permute(0, 2, 1, 3, 4)  # [B,H,W,R,P]
        zc = z_rank[:, sl].permute(0, 2, 1, 3, 4)
        cum = torch.cumsum(adt[:, sl].float().permute(0, 2, 1), dim=-1)  # [B,H,W]
        ks = kc * scale_act[:, sl].permute(0, 2, 1)[..., None, None]
        q2 = qc.flatten(2, 3)
        k2 = ks.flatten(2, 3)
        v2 = vc.flatten(2, 3)

        inter = _bmm_f32(state.to(act), q2.transpose(-1, -2)).transpose(-1, -2)
        inter = inter.reshape(batch, heads, width, rank, head_dim) * torch.exp(cum)[..., None, None]

        scores = _bmm_f32(q2, k2.transpose(-1, -2)).reshape(batch, heads, width, rank, width, rank)
        lower = torch.ones(width, width, dtype=torch.bool, device=q.device).tril()
        decay = torch.exp((cum[..., :, None] - cum[..., None, :]).masked_fill(~lower, -torch.inf))
        eye = torch.eye(width, dtype=torch.bool, device=q.device)
        decay = torch.where(eye, diag[:, sl].permute(0, 2, 1)[..., :, None], decay)
        weighted = (scores * decay[:, :, :, None, :, None]).reshape(
            batch, heads, width * rank, width * rank).to(v2.dtype)
        intra = _bmm_f32(weighted, v2).reshape(batch, heads, width, rank, head_dim)

        y = inter + intra + d_f * vc.float()
        y = y * F.silu(zc.float())
        if mimo_out is not None:
            y = (y * mimo_out.float()[None, :, None]).sum(dim=3)
        else:
            y = y.squeeze(3)
        outputs.append(y.permute(0, 2, 1, 3).to(value.dtype))

        # state carry (ops.py:804-816)
        end_decay = torch.exp(cum[..., -1:] - cum)
        sk = ks * end_decay[..., None, None].to(ks.dtype)
        update = _bmm_f32(v2.transpose(-1, -2), sk.flatten(2, 3))
        state = torch.exp(cum[..., -1])[..., None, None] * state + update
    return torch.cat(outputs, dim=1).to(value.dtype), state


def step_update(q, k, value, gate, adt, dt, trap_logits, D, cache, *, mimo_x=None,
                mimo_z=None, mimo_out=None):
    """ops.py:825-879: one exact recurrent update with rotated ``q/k [B,H,R,N]``.

    ``cache = (phase, state, prev_k, prev_value)``; phase is passed through.
    """
    phase, state, prev_k, prev_v = cache
    v_r = _rank_values(value, mimo_x)  # [B,H,R,P]
    z_r = _rank_values(gate, mimo_z)
    pv_r = _rank_values(prev_v, mimo_x)
    trap = torch.sigmoid(trap_logits.float())
    alpha = torch.exp(adt.float())
    beta = (1.0 - trap) * dt * alpha
    gamma = trap * dt
    nxt = (alpha[..., None, None] * state.float()
           + beta[..., None, None] * _bmm_f32(pv_r.transpose(-1, -2), prev_k)
           + gamma[..., None, None] * _bmm_f32(v_r.transpose(-1, -2), k))
    y = _bmm_f32(q, nxt.to(q.dtype).transpose(-1, -2))  # [B,H,R,P]
    y = y + D.float()[None, :, None, None] * v_r.float()
    y = y * F.silu(z_r.float())
    if mimo_out is not None:
        y = (y * mimo_out.float()[None]).sum(dim=2)
    else:
        y = y.squeeze(2)
    return y.to(value.dtype), (phase, nxt, k, value)


# ---------------------------------------------------------------------------
# mixer and model


def project(params, pre: str, h: torch.Tensor, dims: Dims):
    """model.py:165-199: in_proj, then ``split_projection``."""
    return split_projection(params, pre, F.linear(h, params[pre + "in_proj.weight"]), dims)


def split_projection(params, pre: str, proj: torch.Tensor, dims: Dims):
    """model.py:147-199 after in_proj: split, B/C RMSNorm, dt, adt of ``proj [B, L, proj]``."""
    batch, length, _ = proj.shape
    z, x, b, c, ddt, da, trap, ang = torch.split(proj, dims.split_sizes, dim=-1)
    h_, p_, r_, n_ = dims.nheads, dims.headdim, dims.mimo_rank, dims.d_state
    z = z.reshape(batch, length, h_, p_)
    x = x.reshape(batch, length, h_, p_)
    b = rms_norm(b.reshape(batch, length, r_, 1, n_), params[pre + "B_norm.weight"])
    c = rms_norm(c.reshape(batch, length, r_, 1, n_), params[pre + "C_norm.weight"])
    k = b.permute(0, 1, 3, 2, 4)
    q = c.permute(0, 1, 3, 2, 4)
    dt = F.softplus(ddt.float() + params[pre + "dt_bias"].float())
    decay = (-heavy_tail(da.float())).clamp(max=-A_FLOOR)
    return q, k, x, z, decay * dt, dt, trap, ang


def expand_bias(params, pre: str, q, k, heads: int):
    """model.py:201-213: broadcast groups to heads and add the head biases."""
    q = _expand_heads(q, heads) + params[pre + "C_bias"].to(q.dtype)
    k = _expand_heads(k, heads) + params[pre + "B_bias"].to(k.dtype)
    return q, k


def _mimo(params, pre):
    return (params.get(pre + "mimo_x"), params.get(pre + "mimo_z"), params.get(pre + "mimo_out"))


def mixer_scan(params, pre: str, proj: torch.Tensor, dims: Dims, cache=None, *,
               chunk: int | None = None):
    """model.py:282-327: the mixer's scan from its in_proj output ``proj [B, L, proj]``.

    Returns ``(mixed [B, L, H, P], cache)`` where ``cache`` is the layer cache the
    sequence leaves (``(phase, state, k_rot, value)`` of the last token, model.py:315-327).
    """
    chunk = chunk or dims.inference_chunk
    mx, mz, mo = _mimo(params, pre)
    mimo = dims.mimo_rank > 1
    q, k, x, z, adt, dt, trap, ang = split_projection(params, pre, proj, dims)
    phase = phase_scan(ang, dt, cache[0] if cache is not None else None)
    mixed, state = ssd_scan(
        q, k, x, z, adt, dt, trap, params[pre + "D"], mimo_x=mx, mimo_z=mz, mimo_out=mo,
        chunk_size=chunk, initial_state=cache[1] if cache is not None else None,
        initial_k=cache[2] if cache is not None else None,
        initial_value=cache[3] if cache is not None else None, phase=phase,
        mimo_rotation=mimo, q_bias=params[pre + "C_bias"], k_bias=params[pre + "B_bias"])
    fq, fk = expand_bias(params, pre, q[:, -1:], k[:, -1:], dims.nheads)
    _, fk = rotate(fq, fk, phase[:, -1:], mimo=mimo)
    return mixed, (phase[:, -1].clone(), state, fk[:, 0].clone(), x[:, -1].clone())


def mixer_forward(params, pre: str, h: torch.Tensor, dims: Dims, *, causal: bool = True,
                  cache=None, return_cache: bool = False, chunk: int | None = None):
    """model.py:270-362: one mixer over a full sequence (optionally with cache)."""
    w_in = params[pre + "in_proj.weight"]
    mixed, next_cache = mixer_scan(params, pre, F.linear(h, w_in), dims, cache, chunk=chunk)
    w_out = params[pre + "out_proj.weight"]
    out = F.linear(mixed.flatten(-2), w_out)
    if causal:
        return (out, next_cache) if return_cache else out
    mixed_r, _ = mixer_scan(params, pre, F.linear(torch.flip(h, dims=(1,)), w_in), dims,
                            chunk=chunk)
    back = F.linear(torch.flip(mixed_r, dims=(1,)).flatten(-2), w_out)
    blend = torch.sigmoid(params[pre + "direction_logit"]).to(dtype=out.dtype)
    return out * blend + back * (1.0 - blend)


def zero_cache(dims: Dims, batch: int, act: torch.dtype, device=None):
    """model.py:364-402: a zero layer cache ``(phase, state, prev_k, prev_v)``."""
    return (
        torch.zeros(batch, dims.nheads, dims.num_angles, device=device),
        torch.zeros(batch, dims.nheads, dims.headdim, dims.d_state, device=device),
        torch.zeros(batch, dims.nheads, dims.mimo_rank, dims.d_state, device=device, dtype=act),
        torch.zeros(batch, dims.nheads, dims.headdim, device=device, dtype=act),
    )


def mixer_step(params, pre: str, h: torch.Tensor, dims: Dims, cache):
    """model.py:422-484 (portable branch): one decode token ``h [B,1,d]``."""
    q, k, x, z, adt, dt, trap, ang = project(params, pre, h, dims)
    q, k = expand_bias(params, pre, q, k, dims.nheads)
    if cache is None:
        cache = zero_cache(dims, h.shape[0], x.dtype, h.device)
    inc = phase_increment(ang[:, 0], dt[:, 0])
    phase = torch.fmod(cache[0] + inc, TWO_PI)
    q, k = rotate(q, k, phase.unsqueeze(1), mimo=dims.mimo_rank > 1)
    mx, mz, mo = _mimo(params, pre)
    mixed, nxt = step_update(q[:, 0], k[:, 0], x[:, 0], z[:, 0], adt[:, 0], dt[:, 0], trap[:, 0],
                             params[pre + "D"], (phase, cache[1], cache[2], cache[3]),
                             mimo_x=mx, mimo_z=mz, mimo_out=mo)
    return F.linear(mixed.flatten(-2), params[pre + "out_proj.weight"]).unsqueeze(1), nxt


def _depth(params) -> int:
    return sum(1 for name in params if name.endswith(".mixer.in_proj.weight"))


def model_forward(params, x: torch.Tensor, dims: Dims, *, causal: bool = True,
                  chunk: int | None = None) -> torch.Tensor:
    """model.py:585-591: pre-norm residual stack then ``norm_f``."""
    if x.shape[0] == 0 or x.shape[1] == 0:
        return x.clone()
    for i in range(_depth(params)):
        h = rms_norm(x, params[f"layers.{i}.norm.weight"])
        x = x + mixer_forward(params, f"layers.{i}.mixer.", h, dims, causal=causal, chunk=chunk)
    return rms_norm(x, params["norm_f.weight"])


def model_prefill(params, x: torch.Tensor, dims: Dims, *, chunk: int | None = None):
    """model.py:593-607: forward that also returns the per-layer decode cache."""
    caches = []
    for i in range(_depth(params)):
        h = rms_norm(x, params[f"layers.{i}.norm.weight"])
        out, cache = mixer_forward(params, f"layers.{i}.mixer.", h, dims, return_cache=True,
                                   chunk=chunk)
        x = x + out
        caches.append(cache)
    return rms_norm(x, params["norm_f.weight"]), caches


def model_step(params, x: torch.Tensor, dims: Dims, caches=None):
    """model.py:609-630: one token through every layer."""
    depth = _depth(params)
    caches = list(caches) if caches is not None else [None] * depth
    new = []
    for i in range(depth):
        h = rms_norm(x, params[f"layers.{i}.norm.weight"])
        out, cache = mixer_step(params, f"layers.{i}.mixer.", h, dims, caches[i])
        x = x + out
        new.append(cache)
    return rms_norm(x, params["norm_f.weight"]), new
