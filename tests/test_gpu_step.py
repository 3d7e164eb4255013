"""Decode step on the GPU (``m3_step``) against the CPU oracle.

Hook form (the reference's ``fused_step`` / ``mamba3_step`` interface): head-expanded,
biased q/k; the kernel owns the phase advance and the rotation. Tolerances follow the
build's parity bar: FP32 outputs and state within 1e-4 (abs and rel), 16-bit outputs
within 2e-2.
"""

from __future__ import annotations

import math

import pytest
import torch

from mamba3_amd import ops
from oracle import portable as op

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _inputs(rank, dtype, *, batch=3, heads=4, head_dim=64, d_state=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    s = d_state // 4 if rank > 1 else d_state // 4
    q = torch.randn(batch, heads, rank, d_state, generator=g) + 1.0
    k = torch.randn(batch, heads, rank, d_state, generator=g) + 1.0
    value = torch.randn(batch, heads, head_dim, generator=g)
    gate = torch.randn(batch, heads, head_dim, generator=g)
    dt = torch.rand(batch, heads, generator=g) * 0.1 + 0.001
    adt = -torch.rand(batch, heads, generator=g) * 0.3 * dt * 10
    trap = torch.randn(batch, heads, generator=g)
    angle_rate = torch.randn(batch, s, generator=g) * 2
    D = torch.randn(heads, generator=g)
    phase = (torch.rand(batch, heads, s, generator=g) * 2 - 1) * 2 * math.pi
    state = torch.randn(batch, heads, head_dim, d_state, generator=g)
    prev_k = torch.randn(batch, heads, rank, d_state, generator=g)
    prev_v = torch.randn(batch, heads, head_dim, generator=g)
    mimo = [None, None, None]
    if rank > 1:
        mimo = [torch.randn(heads, rank, head_dim, generator=g) / rank,
                torch.randn(heads, rank, head_dim, generator=g),
                torch.randn(heads, rank, head_dim, generator=g) / rank]
    act = [t.to(dtype) for t in (q, k, value, gate, trap, angle_rate, prev_k, prev_v)]
    q, k, value, gate, trap, angle_rate, prev_k, prev_v = act
    return dict(q=q, k=k, value=value, gate=gate, adt=adt, dt=dt, trap_logits=trap,
                angle_rate=angle_rate, D=D, cache=(phase, state, prev_k, prev_v),
                mimo_x=mimo[0], mimo_z=mimo[1], mimo_out=mimo[2])


def _oracle_fused(inp):
    phase, state, prev_k, prev_v = inp["cache"]
    ph = torch.fmod(phase + op.phase_increment(inp["angle_rate"], inp["dt"]), op.TWO_PI)
    rank = inp["q"].shape[2]
    qr, kr = op.rotate(inp["q"][:, None], inp["k"][:, None], ph[:, None], mimo=rank > 1)
    y, nxt = op.step_update(qr[:, 0], kr[:, 0], inp["value"], inp["gate"], inp["adt"],
                            inp["dt"], inp["trap_logits"], inp["D"], (ph, state, prev_k, prev_v),
                            mimo_x=inp["mimo_x"], mimo_z=inp["mimo_z"],
                            mimo_out=inp["mimo_out"])
    return y, (ph, nxt[1], kr[:, 0], inp["value"])


def _dev(inp):
    out = {}
    for name, t in inp.items():
        if name == "cache":
            out[name] = tuple(x.to(DEV) for x in t)
        else:
            out[name] = None if t is None else t.to(DEV)
    return out


def _tol(dtype):
    return dict(rtol=1e-4, atol=1e-4) if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rank", [1, 2, 4, 8])
@pytest.mark.parametrize("dims", [(64, 128), (32, 16)])
def test_fused_step_matches_oracle(dtype, rank, dims):
    head_dim, d_state = dims
    inp = _inputs(rank, dtype, head_dim=head_dim, d_state=d_state, seed=rank)
    y_ref, (ph_ref, s_ref, k_ref, _) = _oracle_fused(inp)
    with torch.inference_mode():
        y, (ph, s, k, v) = ops.fused_step(**_dev(inp))
    assert ops._HIP_LAST_DISPATCH
    torch.cuda.synchronize()
    print(f"step {dtype} R={rank} P={head_dim} N={d_state}: "
          f"y {(y.float().cpu() - y_ref.float()).abs().max():.2e} "
          f"S {(s.cpu() - s_ref).abs().max():.2e}", flush=True)
    torch.testing.assert_close(y.float().cpu(), y_ref.float(), **_tol(dtype))
    torch.testing.assert_close(ph.cpu(), ph_ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(k.float().cpu(), k_ref.float(), **_tol(dtype))
    torch.testing.assert_close(s.cpu(), s_ref, rtol=1e-4, atol=1e-4 if dtype == torch.float32
                               else 2e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rank", [1, 2, 4])
def test_fused_step_many_heads_matches_oracle(dtype, rank):
    """1088 (batch, head) pairs: the launch shape of large decode batches (256 threads per
    pair: 8 state rows per thread for rank 1 and FP32 rank 2; for 16-bit ranks 2 and 4 the
    update and readout on MFMA; the LDS-staged kernel for FP32 rank 4), at the model's head
    shape, both out of place and with the outputs aliasing the cache."""
    inp = _inputs(rank, dtype, batch=17, heads=64, seed=20 + rank)
    y_ref, (ph_ref, s_ref, k_ref, _) = _oracle_fused(inp)
    d = _dev(inp)
    with torch.inference_mode():
        y, (ph, s, k, v) = ops.fused_step(**d)
    torch.cuda.synchronize()
    print(f"step B=17 H=64 {dtype} R={rank}: "
          f"y {(y.float().cpu() - y_ref.float()).abs().max():.2e} "
          f"S {(s.cpu() - s_ref).abs().max():.2e}", flush=True)
    torch.testing.assert_close(y.float().cpu(), y_ref.float(), **_tol(dtype))
    torch.testing.assert_close(ph.cpu(), ph_ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(k.float().cpu(), k_ref.float(), **_tol(dtype))
    s_tol = 1e-4 if dtype == torch.float32 else 2e-3
    torch.testing.assert_close(s.cpu(), s_ref, rtol=1e-4, atol=s_tol)
    cache = tuple(t.clone() for t in d["cache"])
    with torch.inference_mode():
        y2, nxt = ops._step_call(d["q"], d["k"], d["value"], d["gate"], d["adt"], d["dt"],
                                 d["trap_logits"], d["angle_rate"], d["D"], cache,
                                 mimo_x=d["mimo_x"], mimo_z=d["mimo_z"],
                                 mimo_out=d["mimo_out"], phase_mode=2, out_cache=cache)
    assert all(a.data_ptr() == b.data_ptr() for a, b in zip(nxt, cache))
    torch.testing.assert_close(y2, y)
    torch.testing.assert_close(cache[1], s)
    torch.testing.assert_close(cache[0], ph)
    torch.testing.assert_close(cache[2], k)
    torch.testing.assert_close(cache[3].cpu(), inp["value"])


@pytest.mark.parametrize("rank", [1, 4])
def test_mamba3_step_uses_rotated_inputs_and_passes_phase(rank):
    inp = _inputs(rank, torch.float32, seed=11)
    inp.pop("angle_rate")
    y_ref, nxt_ref = op.step_update(**inp)
    with torch.inference_mode():
        y, nxt = ops.mamba3_step(**_dev(inp))
    torch.testing.assert_close(y.cpu(), y_ref, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(nxt[1].cpu(), nxt_ref[1], rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(nxt[0].cpu(), inp["cache"][0])
    torch.testing.assert_close(nxt[2].cpu(), inp["k"])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_step_in_place_cache_update(dtype):
    """Outputs may alias the cache (the hipGraph decoder path)."""
    inp = _inputs(4, dtype, seed=5)
    y_ref, (ph_ref, s_ref, k_ref, _) = _oracle_fused(inp)
    d = _dev(inp)
    cache = tuple(t.clone() for t in d["cache"])
    with torch.inference_mode():
        y, nxt = ops._step_call(d["q"], d["k"], d["value"], d["gate"], d["adt"], d["dt"],
                                d["trap_logits"], d["angle_rate"], d["D"], cache,
                                mimo_x=d["mimo_x"], mimo_z=d["mimo_z"], mimo_out=d["mimo_out"],
                                phase_mode=2, out_cache=cache)
    assert all(a.data_ptr() == b.data_ptr() for a, b in zip(nxt, cache))
    torch.testing.assert_close(y.float().cpu(), y_ref.float(), **_tol(dtype))
    torch.testing.assert_close(cache[1].cpu(), s_ref, rtol=1e-4,
                               atol=1e-4 if dtype == torch.float32 else 2e-3)
    torch.testing.assert_close(cache[0].cpu(), ph_ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(cache[3].cpu(), inp["value"])


def _chain_512(dtype, rank, *, fused: bool):
    """Run 512 decode steps on the kernel and the oracle; return state / output errors.

    Each side carries its own cache. With ``fused`` the kernel advances the phase and
    rotates q/k itself (``fused_step``); otherwise both sides get the oracle's rotated q/k
    for every step (``mamba3_step``) and the kernel's cache k is that rotated k.
    """
    batch, heads, head_dim, d_state = 2, 4, 64, 128
    base = _inputs(rank, dtype, batch=batch, heads=heads, head_dim=head_dim, d_state=d_state,
                   seed=99)
    zero_cache = (torch.zeros(batch, heads, d_state // 4),
                  torch.zeros(batch, heads, head_dim, d_state),
                  torch.zeros(batch, heads, rank, d_state, dtype=dtype),
                  torch.zeros(batch, heads, head_dim, dtype=dtype))
    ref_cache = zero_cache
    dev_cache = tuple(t.to(DEV) for t in zero_cache)
    g = torch.Generator().manual_seed(123)
    worst_y = worst_rel = 0.0
    max_y = 0.0
    for _ in range(512):
        step = dict(base)
        for name in ("q", "k", "value", "gate", "angle_rate"):
            step[name] = (torch.randn(base[name].shape, generator=g) +
                          (1.0 if name in ("q", "k") else 0.0)).to(dtype)
        step["dt"] = torch.rand(batch, heads, generator=g) * 0.1 + 0.001
        step["adt"] = -torch.rand(batch, heads, generator=g) * step["dt"] * 2
        step["trap_logits"] = torch.randn(batch, heads, generator=g).to(dtype)
        step["cache"] = ref_cache
        if fused:
            y_ref, ref_cache = _oracle_fused(step)
            step_d = _dev(step)
            step_d["cache"] = dev_cache
            with torch.inference_mode():
                y, dev_cache = ops.fused_step(**step_d)
        else:
            ph = torch.fmod(ref_cache[0] + op.phase_increment(step["angle_rate"], step["dt"]),
                            op.TWO_PI)
            qr, kr = op.rotate(step["q"][:, None], step["k"][:, None], ph[:, None],
                               mimo=rank > 1)
            step["q"], step["k"] = qr[:, 0], kr[:, 0]
            step.pop("angle_rate")
            step["cache"] = (ph, *ref_cache[1:])
            y_ref, ref_cache = op.step_update(**step)
            step_d = _dev(step)
            step_d["cache"] = (step_d["cache"][0], *dev_cache[1:])
            with torch.inference_mode():
                y, dev_cache = ops.mamba3_step(**step_d)
        ref_cache = tuple(t.clone() for t in ref_cache)
        dy = (y.float().cpu() - y_ref.float()).abs()
        worst_y = max(worst_y, dy.max().item())
        # relative to the output's magnitude (floor 1): a 16-bit output rounds to 2^-8 relative
        worst_rel = max(worst_rel, (dy / y_ref.float().abs().clamp_min(1.0)).max().item())
        max_y = max(max_y, y_ref.float().abs().max().item())
    err = (dev_cache[1].cpu() - ref_cache[1]).abs().max().item()
    scale = ref_cache[1].abs().max().item()
    print(f"512 steps {dtype} R={rank} fused={fused}: state max abs {err:.3e}, "
          f"rel {err / scale:.3e}, |S|max {scale:.2f}, outputs max abs {worst_y:.3e} "
          f"(|y|max {max_y:.1f}, rel {worst_rel:.3e})", flush=True)
    return err, scale, worst_y, worst_rel


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rank", [1, 4])
def test_state_after_512_steps(dtype, rank):
    """the FP32 state after 512 decode steps within 1e-4 (max abs).

    Teacher-forced: both sides get identical rotated q/k for every step, so the check
    isolates the recurrence (state update, readout, gate) over 512 steps. 16-bit outputs are
    checked relative to their magnitude (2e-2): the FP32 readout sums in another order than
    the CPU's, so an output can round to the neighbouring 16-bit value.
    """
    err, _, worst_y, worst_rel = _chain_512(dtype, rank, fused=False)
    assert err <= 1e-4
    if dtype == torch.float32:
        assert worst_y <= 1e-4
    else:
        assert worst_rel <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rank", [1, 4])
def test_fused_state_after_512_steps(dtype, rank):
    """512 steps with the phase advanced and q/k rotated by the kernel itself.

    FP32: state within 1e-4. 16-bit: the phase is carried across steps, so 1-ulp FP32
    differences between the GPU's and the CPU's tanh / cos / sin accumulate; when such a
    difference crosses a bf16 rounding boundary of the rotated k, that element differs by
    one bf16 ulp and moves the state by about gamma * v * ulp(k) ~ 5e-4. The 16-bit bar is
    therefore relative: max |dS| / max |S| <= 1e-3.
    """
    err, scale, _, worst_rel = _chain_512(dtype, rank, fused=True)
    if dtype == torch.float32:
        assert err <= 1e-4
    else:
        assert err / scale <= 1e-3
        assert worst_rel <= 2e-2
