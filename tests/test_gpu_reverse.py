"""The reverse scan (backwards token strides), which the bidirectional layer uses.

``ScanCall(proj, mixer, reverse=True)`` reads the projection from its last token to its first
and writes its output back in forward order. It runs the same arithmetic in the same order as
scanning a flipped copy of the projection and flipping the output back, so the two agree bit
for bit, whether or not the library splits the sequence into segments.
"""

from __future__ import annotations

import pytest
import torch

from mamba3_amd import Mamba3, ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _mixer(rank, d_model=128, seed=0):
    torch.manual_seed(seed)
    model = Mamba3(d_model, d_state=128, depth=1, mimo_rank=rank, causal=False).eval().to(DEV)
    return model.layers[0].mixer


@pytest.mark.parametrize("rank", [1, 4])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,length", [(2, 333), (1, 4096)])
def test_reverse_scan_equals_the_flipped_scan(rank, dtype, batch, length):
    """(1, 4096) is long enough for the library to split the sequence (B = 1, 4 heads)."""
    mixer = _mixer(rank, seed=rank)
    g = torch.Generator(device="cpu").manual_seed(length + rank)
    proj = torch.randn(batch, length, mixer.in_proj.weight.shape[0], generator=g).to(dtype)
    proj = proj.to(DEV)
    with torch.inference_mode():
        back = ops.ScanCall(proj, mixer, reverse=True)
        back.launch()
        flipped = ops.ScanCall(torch.flip(proj, dims=(1,)).contiguous(), mixer)
        flipped.launch()
    torch.cuda.synchronize()
    assert torch.equal(back.out, torch.flip(flipped.out, dims=(1,)))
    assert torch.equal(back.final_state, flipped.final_state)


def test_reverse_scan_has_no_cache():
    mixer = _mixer(1)
    proj = torch.randn(1, 64, mixer.in_proj.weight.shape[0], device=DEV)
    with torch.inference_mode(), pytest.raises(ValueError, match="no cache"):
        ops.ScanCall(proj, mixer, reverse=True, want_cache=True)


def test_bidirectional_layer_uses_one_projection(monkeypatch):
    """The bidirectional forward projects once (the reverse direction reads it backwards)."""
    mixer = _mixer(1)
    calls = []
    real = mixer.in_proj.forward
    monkeypatch.setattr(mixer.in_proj, "forward", lambda x: calls.append(1) or real(x))
    with torch.inference_mode():
        mixer(torch.randn(2, 100, 128, device=DEV))
    assert len(calls) == 1


def test_bidirectional_model_with_split_concurrent_directions_matches_oracle():
    """B = 1, L = 4096, 4 heads: both directions are split into segments and run on two
    streams at once; the FP32 forward matches the oracle within 1e-4, and repeated forwards
    agree bit for bit (no stream-ordering or buffer-reuse race)."""
    from oracle import portable as op

    torch.manual_seed(21)
    model = Mamba3(128, d_state=128, depth=2, mimo_rank=1, causal=False).eval()
    params = {k: v.detach().clone() for k, v in model.state_dict().items()}
    model = model.to(DEV)
    torch.manual_seed(22)
    x = torch.randn(1, 4096, 128)
    with torch.inference_mode():
        want = op.model_forward(params, x, op.Dims(128, 128, 1), causal=False)
        xd = x.to(DEV)
        outs = [model(xd) for _ in range(3)]
    torch.cuda.synchronize()
    torch.testing.assert_close(outs[0].cpu(), want, rtol=1e-4, atol=1e-4)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
