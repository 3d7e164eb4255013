"""m3_rms_norm (the residual stream between mixers) and the model's fused layer loop.

The sum is the reference's ``hidden_states + mixed`` (``model.py:511-512``) and must match
torch's add bit for bit; the normed rows are ``F.rms_norm`` with the weight in the rows' dtype
(``model.py:48-55``), written in the dtype the next projection computes in. The sum of squares
is reduced in another order than torch's, so FP32 outputs agree to 1e-5 relative and 16-bit
outputs to one rounding step of their dtype.
"""

from __future__ import annotations

import pytest
import torch
from torch.nn import functional as F

from mamba3_amd import Mamba3, ops
from oracle import portable as op

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _reference(x, add, weight, eps, out_dtype):
    s = x if add is None else x + add
    out = F.rms_norm(s.float(), (s.shape[-1],), weight.to(s.dtype).float(), eps)
    return out.to(out_dtype), s


def _close(got, want):
    if got.dtype == torch.float32:
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)
    else:
        # one rounding step of the 16-bit dtype (the FP32 values before rounding differ in the
        # last bits)
        step = 2.0 ** -7 if got.dtype == torch.bfloat16 else 2.0 ** -10
        torch.testing.assert_close(got.float(), want.float(), rtol=step, atol=step)


CASES = [
    # x dtype, add dtype (None: no add), out dtype
    (torch.float32, None, torch.bfloat16),
    (torch.float32, torch.bfloat16, torch.bfloat16),
    (torch.float32, torch.bfloat16, torch.float32),
    (torch.float32, torch.float32, torch.float32),
    (torch.float32, torch.float16, torch.float16),
    (torch.bfloat16, torch.bfloat16, torch.bfloat16),
    (torch.float16, None, torch.float16),
]


@pytest.mark.parametrize("dim", [256, 768, 1024, 2048])
@pytest.mark.parametrize("x_dtype,add_dtype,out_dtype", CASES)
def test_rms_norm_matches_torch(dim, x_dtype, add_dtype, out_dtype):
    g = torch.Generator().manual_seed(dim)
    rows = 37  # not a multiple of the rows a workgroup takes
    x = (torch.randn(rows, dim, generator=g) * 3).to(x_dtype).to(DEV)
    add = None if add_dtype is None else torch.randn(rows, dim, generator=g).to(add_dtype).to(DEV)
    weight = (1 + 0.1 * torch.randn(dim, generator=g)).to(DEV)
    with torch.inference_mode():
        out, s = ops.rms_norm(x, weight, 1e-5, add=add, keep_sum=add is not None,
                              out_dtype=out_dtype)
    want, s_want = _reference(x, add, weight, 1e-5, out_dtype)
    assert out.dtype == out_dtype
    _close(out, want)
    if add is not None:
        assert s.dtype == x.dtype and torch.equal(s, s_want)


def test_rms_norm_rows_of_a_3d_tensor_and_large_values():
    """[B, L, d] rows, values far from unit scale (the norm is scale-free)."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(3, 129, 1024, generator=g) * 1e3).to(DEV)
    add = (torch.randn(3, 129, 1024, generator=g) * 1e3).to(torch.bfloat16).to(DEV)
    weight = torch.randn(1024, generator=g).to(DEV)
    with torch.inference_mode():
        out, s = ops.rms_norm(x, weight, add=add, keep_sum=True, out_dtype=torch.float32)
    want, s_want = _reference(x, add, weight, 1e-5, torch.float32)
    assert out.shape == x.shape and torch.equal(s, s_want)
    _close(out, want)


def test_rms_norm_rejects_unsupported_operands():
    x = torch.randn(4, 384, device=DEV)
    w = torch.ones(384, device=DEV)
    assert not ops.rms_norm_supported(x, w)
    with torch.inference_mode(), pytest.raises(ValueError, match="unsupported"):
        ops.rms_norm(x, w)
    x = torch.randn(4, 256, device=DEV, dtype=torch.bfloat16)
    assert not ops.rms_norm_supported(x, torch.ones(256, device=DEV), out_dtype=torch.float32)


def _count_norm_calls(monkeypatch):
    calls = []
    real = ops.rms_norm

    def counted(*a, **k):
        calls.append(1)
        return real(*a, **k)

    monkeypatch.setattr(ops, "rms_norm", counted)
    return calls


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("causal", [True, False])
def test_model_fused_layer_loop_matches_the_unfused_one(monkeypatch, bf16, causal):
    """depth 3, d_model 256: one m3_rms_norm per layer plus norm_f, against the same model with
    the residual stream in torch (FP32 within 1e-5, bf16 autocast within the 16-bit bar)."""
    torch.manual_seed(11)
    model = Mamba3(256, d_state=128, depth=3, mimo_rank=1, causal=causal).eval().to(DEV)
    x = torch.randn(2, 200, 256, device=DEV)
    ctx = torch.autocast("cuda", dtype=torch.bfloat16, enabled=bf16)
    calls = _count_norm_calls(monkeypatch)
    with torch.inference_mode(), ctx:
        fused = model(x)
    assert len(calls) == 4
    monkeypatch.setattr(ops, "rms_norm_supported", lambda *a, **k: False)
    with torch.inference_mode(), ctx:
        plain = model(x)
    assert fused.dtype == plain.dtype == torch.float32
    if bf16:
        scale = plain.abs().max().item()
        assert (fused - plain).abs().max().item() <= 2e-2 * scale
    else:
        torch.testing.assert_close(fused, plain, rtol=1e-5, atol=1e-5)


def test_model_prefill_with_the_fused_loop_matches_the_oracle():
    """Config 1's shape (d_model 256, depth 6) in FP32: prefill output and every cache tensor
    against the oracle within 1e-4."""
    torch.manual_seed(0)
    model = Mamba3(256, d_state=128, depth=6, mimo_rank=1).eval()
    params = {k: v.detach().clone() for k, v in model.state_dict().items()}
    model = model.to(DEV)
    torch.manual_seed(1)
    x = torch.randn(2, 300, 256)
    with torch.inference_mode():
        want, want_cache = op.model_prefill(params, x, op.Dims(256, 128, 1))
        got, cache = model.prefill(x.to(DEV))
    torch.testing.assert_close(got.cpu(), want, rtol=1e-4, atol=1e-4)
    for layer, want_layer in zip(cache, want_cache):
        for g, w in zip(layer, want_layer):
            torch.testing.assert_close(g.cpu().float(), w.float(), rtol=1e-4, atol=1e-4)
