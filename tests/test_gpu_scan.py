"""Chunked scan on the GPU (``m3_scan_fwd``, ``m3_chunk_state``) against the CPU oracle.

The oracle runs the reference's portable algorithm in the same activation dtype on the
CPU. FP32: within 1e-4 (abs and rel) at any chunk size. 16-bit: the chunk size decides
where the reference rounds (the FP32 state is cast to the activation dtype for the inter
term at chunk starts, the end decay is rounded relative to the chunk end). So two checks:

* against the oracle run at the kernel's own sub-chunk (64 // R tokens), where the chunk
  boundaries coincide;
* against the oracle at the reference's inference chunk (256 for R = 1, 32 for R > 1,
  model.py:26-37).

In both, the 16-bit bar is 2e-2 relative to the output scale (max |dy| / max |y|) and 1e-2
in norm (||dy|| / ||y||); the FP32 state within 2e-2 of its scale. The kernel evaluates the
per-token products (bias, rotation, k * scale) in FP32 and rounds once where they become
MFMA operands, while the reference rounds after each of them, so 16-bit outputs differ from
the oracle by a few units in the last place of their own magnitude. With these unnormalised
inputs (|y| up to ~170, where one bf16 unit is 0.5 to 1) some elements sit outside an
elementwise 2e-2 of the oracle's bf16 result, as they sit outside 2e-2 of the FP32 result in
the oracle's own bf16 run. So each 16-bit case also runs the oracle in FP32 on the same inputs
and applies ``conftest.bf16_parity``: the kernel is at least as close to FP32 as the
reference's 16-bit path (norm, max and elementwise count), and >= 98% of elements meet the
elementwise bar against the oracle's 16-bit result.
"""

from __future__ import annotations

import math

import pytest
import torch

from conftest import bf16_parity
from mamba3_amd import ops
from oracle import portable as op

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _inputs(rank, dtype, *, batch=2, length=133, heads=3, head_dim=64, d_state=128,
            groups=1, seed=0, phase=True, bias=True, initial=True):
    g = torch.Generator().manual_seed(seed)
    s = d_state // 4
    q = torch.randn(batch, length, groups, rank, d_state, generator=g)
    k = torch.randn(batch, length, groups, rank, d_state, generator=g)
    value = torch.randn(batch, length, heads, head_dim, generator=g)
    gate = torch.randn(batch, length, heads, head_dim, generator=g)
    dt = torch.rand(batch, length, heads, generator=g) * 0.1 + 0.001
    adt = -torch.rand(batch, length, heads, generator=g) * dt * 3
    trap = torch.randn(batch, length, heads, generator=g)
    D = torch.randn(heads, generator=g)
    inp = dict(q=q.to(dtype), k=k.to(dtype), value=value.to(dtype), gate=gate.to(dtype),
               adt=adt, dt=dt, trap_logits=trap.to(dtype), D=D)
    if rank > 1:
        inp["mimo_x"] = torch.randn(heads, rank, head_dim, generator=g) / rank
        inp["mimo_z"] = torch.randn(heads, rank, head_dim, generator=g)
        inp["mimo_out"] = torch.randn(heads, rank, head_dim, generator=g) / rank
    if phase:
        inp["phase"] = (torch.rand(batch, length, heads, s, generator=g) * 2 - 1) * 2 * math.pi
        inp["mimo_rotation"] = rank > 1
    if bias:
        inp["q_bias"] = 1 + 0.1 * torch.randn(heads, rank, d_state, generator=g)
        inp["k_bias"] = 1 + 0.1 * torch.randn(heads, rank, d_state, generator=g)
    if initial:
        inp["initial_state"] = torch.randn(batch, heads, head_dim, d_state, generator=g) * 0.3
        inp["initial_k"] = torch.randn(batch, heads, rank, d_state, generator=g).to(dtype)
        inp["initial_value"] = torch.randn(batch, heads, head_dim, generator=g).to(dtype)
    return inp


def _kernel_chunk(dtype, rank):
    return (32 if dtype == torch.float32 else 64) // rank


def _reference_chunk(rank):
    return 256 if rank == 1 else max(16, 128 // rank)


def _run_both(inp, chunk=64):
    y_ref, s_ref = op.ssd_scan(**inp, chunk_size=chunk)
    dev = {n: (t.to(DEV) if isinstance(t, torch.Tensor) else t) for n, t in inp.items()}
    with torch.inference_mode():
        y, s = ops.mamba3_scan(**dev, chunk_size=chunk)
    assert ops._HIP_LAST_SCAN_DISPATCH
    torch.cuda.synchronize()
    return y.cpu(), s.cpu(), y_ref, s_ref


def _report(tag, y, s, y_ref, s_ref):
    ey = (y.float() - y_ref.float()).abs().max().item()
    es = (s - s_ref).abs().max().item()
    en = ((y.float() - y_ref.float()).norm() / y_ref.float().norm()).item()
    d = (y.float() - y_ref.float()).abs()
    out = d > 2e-2 + 2e-2 * y_ref.float().abs()
    worst = (d / (2e-2 + 2e-2 * y_ref.float().abs())).max().item()
    print(f"{tag}: y max abs {ey:.2e} (|y|max {y_ref.float().abs().max():.2f}), "
          f"||dy||/||y|| {en:.2e}, S max abs {es:.2e} (|S|max {s_ref.abs().max():.2f}); "
          f"elementwise 2e-2/2e-2: {int(out.sum())} of {d.numel()} outside, worst ratio "
          f"{worst:.2f}", flush=True)


def _fp32_oracle(inp, chunk):
    """The oracle in FP32 on the same (16-bit-valued) inputs: the 16-bit paths' accuracy
    reference."""
    f = {n: (t.float() if isinstance(t, torch.Tensor) and t.is_floating_point() else t)
         for n, t in inp.items()}
    return op.ssd_scan(**f, chunk_size=chunk)


def _check(dtype, y, s, y_ref, s_ref, inp=None, chunk=None, min_inside=0.985):
    if dtype == torch.float32:
        torch.testing.assert_close(y, y_ref, rtol=1e-4, atol=1e-4)
        torch.testing.assert_close(s, s_ref, rtol=1e-4, atol=1e-4)
    else:
        dy = y.float() - y_ref.float()
        assert dy.abs().max() <= 2e-2 * y_ref.float().abs().max()
        assert dy.norm() <= 1e-2 * y_ref.float().norm()
        assert (s - s_ref).abs().max() <= 2e-2 * s_ref.abs().max()
        if inp is not None:
            y32, s32 = _fp32_oracle(inp, chunk)
            bf16_parity(f"scan {dtype} R={inp['q'].shape[3]} output", y, y_ref, y32,
                        min_inside=min_inside)
            bf16_parity(f"scan {dtype} R={inp['q'].shape[3]} state", s, s_ref, s32,
                        elementwise=False)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rank", [1, 2, 4, 8])
def test_scan_matches_oracle(dtype, rank):
    inp = _inputs(rank, dtype, seed=rank)
    y, s, y_ref, s_ref = _run_both(inp, chunk=_kernel_chunk(dtype, rank))
    _report(f"scan {dtype} R={rank} aligned chunks", y, s, y_ref, s_ref)
    _check(dtype, y, s, y_ref, s_ref, inp, _kernel_chunk(dtype, rank))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rank", [1, 2, 4, 8])
def test_scan_matches_oracle_at_reference_chunk(dtype, rank):
    inp = _inputs(rank, dtype, seed=rank, length=300)
    y, s, y_ref, s_ref = _run_both(inp, chunk=_reference_chunk(rank))
    _report(f"scan {dtype} R={rank} reference chunk", y, s, y_ref, s_ref)
    _check(dtype, y, s, y_ref, s_ref, inp, _reference_chunk(rank))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rank", [1, 4])
@pytest.mark.parametrize("flags", [(False, False, False), (True, False, False),
                                   (False, True, True)])
def test_scan_optional_inputs(dtype, rank, flags):
    phase, bias, initial = flags
    inp = _inputs(rank, dtype, seed=7, phase=phase, bias=bias, initial=initial, length=70)
    y, s, y_ref, s_ref = _run_both(inp, chunk=_kernel_chunk(dtype, rank))
    _check(dtype, y, s, y_ref, s_ref, inp, _kernel_chunk(dtype, rank))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rank", [1, 4])
@pytest.mark.parametrize("dims", [(4, 8), (32, 16), (16, 32)])
def test_scan_small_padded_dims(dtype, rank, dims):
    """P and N below the MFMA tile sizes (zero-padded operands)."""
    head_dim, d_state = dims
    inp = _inputs(rank, dtype, seed=3, head_dim=head_dim, d_state=d_state, length=37)
    y, s, y_ref, s_ref = _run_both(inp, chunk=_kernel_chunk(dtype, rank))
    _check(dtype, y, s, y_ref, s_ref, inp, _kernel_chunk(dtype, rank))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("length", [1, 2, 63, 64, 65, 300])
def test_scan_ragged_lengths(length, dtype):
    inp = _inputs(1, dtype, seed=length, length=length)
    y, s, y_ref, s_ref = _run_both(inp, chunk=_kernel_chunk(dtype, 1))
    _check(dtype, y, s, y_ref, s_ref, inp, _kernel_chunk(dtype, 1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rank", [1, 4])
def test_scan_strided_views(dtype, rank):
    """q / k, value / gate and the phases as column slices of wider rows (token strides longer
    than the rows they hold, each at its own offset; NaN around them): the same results as the
    contiguous inputs, against the oracle."""
    length = 200
    inp = _inputs(rank, dtype, seed=21 + rank, length=length)
    dev = {n: (t.to(DEV) if isinstance(t, torch.Tensor) else t) for n, t in inp.items()}

    def widen(t, extra):
        wide = torch.full((*t.shape[:-1], t.shape[-1] + extra), float("nan"), dtype=t.dtype,
                          device=DEV)
        wide[..., extra // 2:extra // 2 + t.shape[-1]] = t
        return wide[..., extra // 2:extra // 2 + t.shape[-1]]

    for name in ("q", "k"):
        dev[name] = widen(dev[name], 16)
    for name in ("value", "gate"):
        dev[name] = widen(dev[name], 64)
    dev["phase"] = widen(dev["phase"], 8)
    assert dev["value"].stride(1) > dev["value"].shape[2] * dev["value"].shape[3]
    y_ref, s_ref = op.ssd_scan(**inp, chunk_size=_kernel_chunk(dtype, rank))
    with torch.inference_mode():
        y, s = ops.mamba3_scan(**dev, chunk_size=_kernel_chunk(dtype, rank))
    assert ops._HIP_LAST_SCAN_DISPATCH
    _check(dtype, y.cpu(), s.cpu(), y_ref, s_ref, inp, _kernel_chunk(dtype, rank))


def test_scan_head_groups():
    """q/k with one group per head (G = H), as ops.mamba3_scan allows."""
    inp = _inputs(1, torch.float32, seed=9, groups=3)
    y, s, y_ref, s_ref = _run_both(inp)
    _check(torch.float32, y, s, y_ref, s_ref)


def test_scan_empty_sequence_preserves_state():
    """Reference tests/test_scan.py:261-282."""
    q = torch.empty(2, 0, 1, 1, 8, device=DEV)
    v = torch.empty(2, 0, 3, 4, device=DEV)
    st = torch.randn(2, 3, 4, 8, device=DEV)
    with torch.inference_mode():
        out, fs = ops.mamba3_scan(q, q, v, v, torch.empty(2, 0, 3, device=DEV),
                                  torch.empty(2, 0, 3, device=DEV),
                                  torch.empty(2, 0, 3, device=DEV), torch.ones(3, device=DEV),
                                  initial_state=st, initial_k=torch.randn(2, 3, 1, 8, device=DEV),
                                  initial_value=torch.randn(2, 3, 4, device=DEV))
    assert out.shape == v.shape
    torch.testing.assert_close(fs, st)


@pytest.mark.parametrize("rank", [1, 4])
def test_scan_continuation(rank):
    """Reference tests/test_scan.py:228-258, on the HIP path."""
    inp = _inputs(rank, torch.float32, seed=21, length=150, phase=False, bias=False,
                  initial=False)
    dev = {n: (t.to(DEV) if isinstance(t, torch.Tensor) else t) for n, t in inp.items()}
    seq = ("q", "k", "value", "gate", "adt", "dt", "trap_logits")
    split = 77
    with torch.inference_mode():
        full, full_state = ops.mamba3_scan(**dev)
        first = {n: (t[:, :split] if n in seq else t) for n, t in dev.items()}
        y1, s1 = ops.mamba3_scan(**first)
        second = {n: (t[:, split:] if n in seq else t) for n, t in dev.items()}
        y2, s2 = ops.mamba3_scan(**second, initial_state=s1, initial_k=dev["k"][:, split - 1, 0:1]
                                 .expand(-1, 3, -1, -1), initial_value=dev["value"][:, split - 1])
    torch.testing.assert_close(torch.cat((y1, y2), 1), full, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(s2, full_state, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rank", [1, 4])
def test_chunk_state_matches_oracle(dtype, rank):
    """The standalone per-chunk state update (reference _triton.py:500-561); 16-bit operands at
    this shape take the MFMA form (6 (b, h) pairs: 128-row passes over 37 x rank rows, the last
    one ragged)."""
    g = torch.Generator().manual_seed(4)
    batch, heads, width, p, n = 2, 3, 37, 64, 128
    k = torch.randn(batch, heads, width, rank, n, generator=g).to(dtype)
    v = torch.randn(batch, heads, width, rank, p, generator=g).to(dtype)
    adt = -torch.rand(batch, heads, width, generator=g) * 0.05
    cum = torch.cumsum(adt, -1)
    scale = torch.rand(batch, heads, width, generator=g) * 0.1
    state = torch.randn(batch, heads, p, n, generator=g)
    ks = k * scale.to(dtype)[..., None, None]
    ke = ks * torch.exp(cum[..., -1:] - cum).to(dtype)[..., None, None]
    upd = torch.bmm(v.flatten(2, 3).float().transpose(-1, -2).flatten(0, 1),
                    ke.flatten(2, 3).float().flatten(0, 1)).unflatten(0, (batch, heads))
    want = torch.exp(cum[..., -1])[..., None, None] * state + upd
    out = torch.empty(batch, heads, p, n, device=DEV)
    with torch.inference_mode():
        ops.chunk_state(k.to(DEV), v.to(DEV), cum.to(DEV), scale.to(DEV), state.to(DEV), out,
                        width=width, rank=rank)
    torch.testing.assert_close(out.cpu(), want, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("shape", [(3, 7, 50, 2, torch.bfloat16), (32, 32, 75, 2, torch.float16)])
def test_chunk_state_in_place(shape):
    """state_out aliasing state_in: each lane rewrites only the state elements it read.
    21 (b, h) pairs take the MFMA form's 128-row passes (100 rows), 1024 pairs its 64-row passes
    (150 rows: 3 passes, the last one ragged)."""
    batch, heads, width, rank, dtype = shape
    g = torch.Generator().manual_seed(11)
    p, n = 64, 128
    k = torch.randn(batch, heads, width, rank, n, generator=g).to(dtype)
    v = torch.randn(batch, heads, width, rank, p, generator=g).to(dtype)
    cum = torch.cumsum(-torch.rand(batch, heads, width, generator=g) * 0.05, -1)
    scale = torch.rand(batch, heads, width, generator=g) * 0.1
    state = torch.randn(batch, heads, p, n, generator=g)
    ks = k * scale.to(dtype)[..., None, None]
    ke = ks * torch.exp(cum[..., -1:] - cum).to(dtype)[..., None, None]
    upd = torch.bmm(v.flatten(2, 3).float().transpose(-1, -2).flatten(0, 1),
                    ke.flatten(2, 3).float().flatten(0, 1)).unflatten(0, (batch, heads))
    want = torch.exp(cum[..., -1])[..., None, None] * state + upd
    st = state.to(DEV)
    out = torch.empty_like(st)
    with torch.inference_mode():
        ops.chunk_state(k.to(DEV), v.to(DEV), cum.to(DEV), scale.to(DEV), st, out,
                        width=width, rank=rank)
        ops.chunk_state(k.to(DEV), v.to(DEV), cum.to(DEV), scale.to(DEV), st, st,
                        width=width, rank=rank)
    # 1e-3: the reference rounds exp(cl - cum) to 16 bits from the CPU's expf, the kernel from
    # the device's; where the two straddle a rounding boundary, one token's whole contribution
    # moves by a 16-bit ulp (about 6e-5 x |v|), which 76,800 tokens hit a few times. A missing or
    # misplaced pass moves most elements by 1e-1 or more.
    torch.testing.assert_close(out.cpu(), want, rtol=1e-3, atol=1e-3)
    assert torch.equal(st, out)  # in place and out of place agree bit for bit


# Shapes outside the MFMA kernel's tiles (d_state not a power of 2 or above 128, head_dim above
# 64, ranks 3, 5, 6, 7): the recurrent scan. FP32 within 1e-4 of the oracle's chunked scan (the
# same recurrence, summed in another order); 16-bit at the 16-bit parity bar.
RECURRENT = [
    # (rank, d_state, head_dim, heads, length)
    (1, 256, 64, 2, 150),
    (1, 96, 32, 3, 130),
    (1, 20, 24, 2, 70),
    (1, 64, 128, 2, 90),
    (4, 256, 64, 2, 70),
    (3, 16, 16, 3, 80),
    (8, 256, 32, 1, 40),
    (1, 1024, 64, 2, 70),   # 256 KiB state: updated in final_state
    (16, 128, 64, 2, 50),   # rank 16: two readout groups
    (12, 64, 32, 1, 40),    # rank 12: a partial second group
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", RECURRENT)
def test_recurrent_scan_matches_oracle(shape, dtype):
    rank, d_state, head_dim, heads, length = shape
    inp = _inputs(rank, dtype, seed=rank + d_state, heads=heads, head_dim=head_dim,
                  d_state=d_state, length=length)
    chunk = 32
    dev = {n: (t.to(DEV) if isinstance(t, torch.Tensor) else t) for n, t in inp.items()}
    with torch.inference_mode():
        y, s = ops.mamba3_scan(**dev, chunk_size=chunk)
    assert ops._HIP_LAST_SCAN_DISPATCH
    torch.cuda.synchronize()
    y_ref, s_ref = op.ssd_scan(**inp, chunk_size=chunk)
    _report(f"recurrent scan {dtype} {shape}", y.cpu(), s.cpu(), y_ref, s_ref)
    # d_state 1024: each output sums 1024 rounded state entries, and two 16-bit paths that are
    # equally accurate against FP32 (the accuracy checks) agree on fewer elements (97.1%)
    _check(dtype, y.cpu(), s.cpu(), y_ref, s_ref, inp, chunk,
           min_inside=0.96 if d_state >= 1024 else 0.985)
