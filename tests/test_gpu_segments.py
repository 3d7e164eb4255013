"""The segmented scan: a long sequence of few (batch, head) pairs split into G segments.

``m3_scan_fwd`` scans every segment from a zero state and phase, composes the segment states in
order (decay, endpoint term, rotation by the segment's phase offset), then rescans every segment
from its true start. Checked against the oracle and against the unsplit scan on the same inputs:
FP32 within 1e-4 (abs and rel); 16-bit outputs within 2e-2 of the output scale. The split forms
FP32 sums in another order, so split and unsplit agree to FP32 rounding, not bitwise.
"""

from __future__ import annotations

import pytest
import torch

from conftest import bf16_parity
from mamba3_amd import Mamba3, ops
from oracle import portable as op
from test_gpu_scan import _inputs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
F32 = dict(rtol=1e-4, atol=1e-4)


@pytest.fixture
def segments(monkeypatch):
    def set_segments(g: int) -> None:
        monkeypatch.setattr(ops, "SCAN_SEGMENTS", g)
    return set_segments


def _scan(inp, chunk):
    dev = {n: (t.to(DEV) if isinstance(t, torch.Tensor) else t) for n, t in inp.items()}
    with torch.inference_mode():
        y, s = ops.mamba3_scan(**dev, chunk_size=chunk)
    assert ops._HIP_LAST_SCAN_DISPATCH
    return y.cpu(), s.cpu()


def _scale_close(got, want, tol=2e-2):
    scale = want.abs().max().item()
    err = (got.float() - want.float()).abs().max().item()
    assert err <= tol * scale, f"max |d| {err:.3e} > {tol} x scale {scale:.3e}"


@pytest.mark.parametrize("rank", [1, 4])
@pytest.mark.parametrize("phase,initial", [(True, True), (False, False), (True, False)])
@pytest.mark.parametrize("segs", [2, 4, 8])
def test_fp32_split_matches_unsplit_and_oracle(rank, phase, initial, segs, segments):
    inp = _inputs(rank, torch.float32, batch=2, length=1024, heads=2, seed=40 + segs,
                  phase=phase, initial=initial)
    chunk = 32 // rank
    segments(1)
    y1, s1 = _scan(inp, chunk)
    segments(segs)
    y2, s2 = _scan(inp, chunk)
    torch.testing.assert_close(y2, y1, **F32)
    torch.testing.assert_close(s2, s1, **F32)
    y_ref, s_ref = op.ssd_scan(**inp, chunk_size=chunk)
    torch.testing.assert_close(y2, y_ref, **F32)
    torch.testing.assert_close(s2, s_ref, **F32)


@pytest.mark.parametrize("rank,segs,length,head_dim,d_state", [
    (1, 32, 4096, 64, 128),  # 32 segments: the prefetch ring wraps eight times
    (2, 2, 8192, 36, 64),    # a 4-row last row group, d_state 64
    (8, 4, 4096, 64, 128),   # rank 8: the composition's shallower prefetch ring
])
def test_fp32_split_composition_shapes(rank, segs, length, head_dim, d_state, segments):
    """The composition's state rows at the segment counts, row groups and ranks the tests above
    leave out: split against unsplit, FP32, with given phases (no carry to walk) and an initial
    state."""
    inp = _inputs(rank, torch.float32, batch=1, length=length, heads=2, head_dim=head_dim,
                  d_state=d_state, seed=80 + rank, phase=True, initial=True)
    chunk = 32 // rank
    segments(1)
    y1, s1 = _scan(inp, chunk)
    segments(segs)
    y2, s2 = _scan(inp, chunk)
    torch.testing.assert_close(y2, y1, **F32)
    torch.testing.assert_close(s2, s1, **F32)


@pytest.mark.parametrize("rank", [1, 4])
def test_bf16_split_matches_unsplit(rank, segments):
    inp = _inputs(rank, torch.bfloat16, batch=1, length=2048, heads=3, seed=50 + rank)
    chunk = 64 // rank
    segments(1)
    y1, s1 = _scan(inp, chunk)
    segments(8)
    y2, s2 = _scan(inp, chunk)
    _scale_close(y2, y1)
    _scale_close(s2, s1)
    y_ref, s_ref = op.ssd_scan(**inp, chunk_size=chunk)
    _scale_close(y2, y_ref)
    y32, s32 = op.ssd_scan(**{n: (t.float() if isinstance(t, torch.Tensor) else t)
                              for n, t in inp.items()}, chunk_size=chunk)
    # measured 99.151% (R = 1) and 99.856% (R = 4) within 2e-2 of the 16-bit oracle
    bf16_parity(f"split bf16 R={rank} output", y2, y_ref, y32,
                min_inside=0.99 if rank == 1 else 0.997)
    bf16_parity(f"split bf16 R={rank} state", s2, s_ref, s32, elementwise=False)


def test_explicit_segments_must_divide_the_length(segments):
    inp = _inputs(1, torch.float32, batch=1, length=1000, heads=2, seed=3)
    segments(3)
    with pytest.raises(ops._hip.HipError, match="segments"):
        _scan(inp, 32)


def _model(rank, seed):
    torch.manual_seed(seed)
    model = Mamba3(128, d_state=128, depth=1, mimo_rank=rank).eval()
    params = {k: v.detach().clone() for k, v in model.state_dict().items()}
    return model.to(DEV), params, op.Dims(128, 128, rank)


def _workspace_bytes(model, x):
    mixer = model.layers[0].mixer
    with torch.inference_mode():
        proj = mixer.in_proj(model.layers[0].norm(x))
        call = ops.ScanCall(proj, mixer)
    ws = call._keep[-1]
    return 0 if ws is None else ws.numel()


@pytest.mark.parametrize("rank", [1, 4])
@pytest.mark.parametrize("bf16", [False, True])
def test_model_auto_split_matches_oracle(rank, bf16, segments):
    """B = 1 with 4 heads leaves most CUs idle: the library splits the 4096 tokens on its own
    (the workspace grows by the segment buffers), and forward and prefill still match."""
    model, params, dims = _model(rank, seed=60 + rank)
    torch.manual_seed(61)
    x = torch.randn(1, 4096, 128)
    xd = x.to(DEV)
    segments(1)
    unsplit = _workspace_bytes(model, xd)
    segments(0)
    assert _workspace_bytes(model, xd) > unsplit
    ctx_cpu = torch.autocast("cpu", dtype=torch.bfloat16, enabled=bf16)
    ctx_gpu = torch.autocast("cuda", dtype=torch.bfloat16, enabled=bf16)
    with torch.inference_mode(), ctx_cpu:
        want = op.model_forward(params, x, dims)
        _, want_cache = op.model_prefill(params, x, dims)
    with torch.inference_mode(), ctx_gpu:
        got = model(xd)
        _, cache = model.prefill(xd)
    if bf16:
        _scale_close(got.cpu(), want)
        for g, w in zip(cache[0], want_cache[0]):
            _scale_close(g.cpu(), w)
    else:
        torch.testing.assert_close(got.cpu(), want, **F32)
        for g, w in zip(cache[0], want_cache[0]):
            torch.testing.assert_close(g.cpu().float(), w.float(), **F32)


@pytest.mark.parametrize("d_model,d_state,rank,segs,length", [
    (128, 128, 1, 32, 4096),  # 31 segments of 2 phase blocks: one short walker batch each
    (18, 64, 2, 2, 8192),     # 64 blocks per segment (two walker batches); 4-row heads
    (64, 128, 8, 4, 4096),    # rank 8
    (32, 128, 1, 256, 16384), # the most segments, one phase block each
    (64, 64, 4, 3, 1536),     # a segment count that is no power of 2; rank 4, d_state 64
])
def test_model_split_walks_the_phase_carry(d_model, d_state, rank, segs, length, segments):
    """The model's projection form (angle increments: the composition walks the phase carry
    block by block) split into segments equals the unsplit prefill, FP32: output and every
    cache tensor, the phase cache bit for bit."""
    torch.manual_seed(90 + rank)
    model = Mamba3(d_model, d_state=d_state, depth=1, mimo_rank=rank).eval().to(DEV)
    x = torch.randn(1, length, d_model, device=DEV)
    with torch.inference_mode():
        segments(1)
        want, want_cache = model.prefill(x)
        segments(segs)
        got, cache = model.prefill(x)
    torch.testing.assert_close(got, want, **F32)
    mixer = model.layers[0].mixer
    phase_shape = (1, mixer.nheads, mixer.num_angles)
    phases = 0
    for g, w in zip(cache[0], want_cache[0]):
        if tuple(w.shape) == phase_shape:
            assert torch.equal(g, w), "the split's phase carry differs from the unsplit scan's"
            phases += 1
        else:
            torch.testing.assert_close(g, w, **F32)
    assert phases == 1


def test_split_scan_continues_from_a_cache(segments):
    """A split mixer scan continued from the cache of a split scan of the first half equals one
    unsplit scan of the whole sequence (outputs and every cache tensor)."""
    model, _, _ = _model(1, seed=70)
    torch.manual_seed(71)
    x = torch.randn(1, 4096, 128, device=DEV)
    with torch.inference_mode():
        mixer = model.layers[0].mixer
        h = model.layers[0].norm(x)
        segments(1)
        full, full_cache = mixer(h, return_cache=True)
        segments(0)
        first, cache = mixer(h[:, :2048], return_cache=True)
        second, cache2 = mixer(h[:, 2048:], cache=cache, return_cache=True)
    torch.testing.assert_close(torch.cat((first, second), 1), full, **F32)
    for a, b in zip(cache2, full_cache):
        torch.testing.assert_close(a, b, **F32)


def test_split_scan_writes_the_callers_block_phase(segments):
    """``block_phase`` (each 64-token block's phase-increment sum) of a call split into
    segments equals the unsplit call's: every segment's sums reach the caller's buffer."""
    model, _, _ = _model(1, seed=72)
    torch.manual_seed(73)
    x = torch.randn(1, 4096, 128, device=DEV)
    mixer = model.layers[0].mixer
    blocks = {}
    with torch.inference_mode():
        proj = mixer.in_proj(model.layers[0].norm(x))
        for g in (1, 8):
            segments(g)
            call = ops.ScanCall(proj, mixer)
            buf = torch.full((1, mixer.nheads, 64, mixer.num_angles), float("nan"), device=DEV)
            call.args.block_phase = ops._hip.tensor(buf)
            call.launch()
            torch.cuda.synchronize()
            blocks[g] = buf.cpu()
    assert torch.isfinite(blocks[1]).all()
    torch.testing.assert_close(blocks[8], blocks[1], rtol=0, atol=0)
