"""``m3_linear`` (the decode step's projection GEMMs) against a torch FP32 reference.

The HIP kernel multiplies 16-bit operands exactly in FP32, accumulates in FP32 and rounds
once. The reference takes the same 16-bit values, converts them to FP32 and multiplies with
torch.matmul (FP32 on the CPU). Bound per element: one rounding of the output (2^-8 relative
for bf16, 2^-11 for f16) plus FP32 accumulation-order error, bounded here by
2^-16 * sum_k |x_mk| |w_nk| (about 2^-24 * K per term, with K <= 8192).
"""

from __future__ import annotations

import pytest
import torch

from mamba3_amd import Mamba3, ops
from oracle import portable as op

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}


def _check(got: torch.Tensor, x, w, residual=None):
    xf, wf = x.float().cpu(), w.float().cpu()
    want = xf @ wf.T
    if residual is not None:
        want = want + residual.float().cpu()
    bound = ULP[x.dtype] * want.abs() + 2.0 ** -16 * (xf.abs() @ wf.abs().T) + 1e-30
    err = (got.float().cpu() - want).abs()
    worst = (err / bound).max().item()
    assert worst <= 1.0, f"max error / bound = {worst:.3f}"


SHAPES = [
    (1, 8672, 2048),    # decode B = 1 in_proj (the gemv kernel, two rows per wave)
    (2, 2048, 4096),    # decode B = 2 out_proj (gemv, one row per wave, 8 chunks per lane)
    (3, 1001, 512),     # gemv: one chunk per lane, N not a multiple of the 4 rows a workgroup owns
    (4, 7, 1536),       # gemv: fewer rows than one workgroup, K / 512 odd
    (4, 8195, 1024),    # gemv: two rows per wave, the last wave half past N
    (5, 2048, 2048),    # five rows: the wide kernel, one 16-row tile, four waves
    (7, 2048, 4096),    # out_proj, ragged rows (wide, eight waves)
    (16, 1000, 2048),   # N not a multiple of the wide kernel's 16 rows
    (9, 37, 512),       # wide, one wave, fewer weight rows than a workgroup
    (5, 8672, 2048),    # decode B = 5 in_proj: the stream kernel, 32-row tile, 48 weight rows
    (17, 8672, 2048),   # stream, 32-row tile, 17 rows
    (32, 2048, 4096),   # decode B = 32 out_proj: stream, 32-row tile, 16 weight rows
    (24, 3000, 1536),   # stream, 16 weight rows, N ragged
    (20, 4100, 1280),   # stream, 32 weight rows (N / 16 just past the 256 CUs)
    (33, 8672, 2048),   # stream, 64-row tile, ragged rows
    (64, 8672, 2048),   # decode B = 64 in_proj (64-row tile, 48 weight rows)
    (64, 2048, 4096),   # decode B = 64 out_proj (two 32-row blocks, 16 weight rows)
    (40, 5000, 768),    # stream, 64-row tile, 32 weight rows, ragged N
    (48, 12289, 256),   # stream, one stage of K, more workgroups than CUs, one row past N / 16
    (5, 100, 800),      # K not a multiple of 256: the rows kernel
    (200, 4144, 1024),  # the 128-row tile, ragged rows and columns
    (256, 8672, 2048),  # decode B = 256 in_proj (config 4)
    (256, 2048, 4096),  # decode B = 256 out_proj (K split)
    (3, 24, 32),        # one K step, fewer columns than a wave unit
    (40, 96, 96),       # the tile kernel with K % 64 == 32: a half last stage
    (100, 200, 160),    # the same with the 128-row tile and ragged rows / columns
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", SHAPES)
def test_linear_matches_fp32_reference(shape, dtype):
    m, n, k = shape
    g = torch.Generator(device="cpu").manual_seed(m * 7 + n + k)
    x = torch.randn(m, k, generator=g).to(dtype).to(DEV)
    w = (torch.randn(n, k, generator=g) / k ** 0.5).to(dtype).to(DEV)
    res = torch.randn(m, n, generator=g).to(dtype).to(DEV)
    with torch.inference_mode():
        _check(ops.linear(x, w), x, w)
        _check(ops.linear(x, w, res), x, w, res)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 8672, 2048), (2, 8672, 2048), (3, 1001, 4096),
                                   (4, 13, 512), (5, 2048, 4096), (16, 1000, 2048),
                                   (32, 4144, 1024), (17, 8672, 2048), (30, 77, 4096),
                                   (12, 500, 1536), (5, 8672, 2048), (64, 8672, 2048),
                                   (48, 300, 4096), (40, 5000, 768), (20, 100, 800)])
def test_linear_fused_rms_norm_matches_fp32_reference(shape, dtype):
    """norm_weight: x is RMS-normalised first. The kernel rounds x * norm_weight (not the
    normalised value) to the operand dtype, one rounding per element either way, so the bound
    gains one operand rounding: ULP * sum_k |xn_mk| |w_nk|."""
    m, n, k = shape
    g = torch.Generator(device="cpu").manual_seed(m + n + k + 1)
    x = (3 * torch.randn(m, k, generator=g)).to(dtype)
    w = (torch.randn(n, k, generator=g) / k ** 0.5).to(dtype)
    nw = (1 + 0.5 * torch.randn(k, generator=g)).to(dtype)
    res = torch.randn(m, n, generator=g).to(dtype)
    eps = 1e-5
    xf, wf = x.float(), w.float()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * nw.float()
    want = xn @ wf.T + res.float()
    bound = ULP[dtype] * (want.abs() + xn.abs() @ wf.abs().T) + 2.0 ** -16 * (
        xn.abs() @ wf.abs().T) + 1e-30
    with torch.inference_mode():
        got = ops.linear(x.to(DEV), w.to(DEV), res.to(DEV), norm_weight=nw.to(DEV),
                         norm_eps=eps)
    worst = ((got.float().cpu() - want).abs() / bound).max().item()
    assert worst <= 1.0, f"max error / bound = {worst:.3f}"


def test_linear_strided_views_and_in_place_residual():
    g = torch.Generator(device="cpu").manual_seed(3)
    big_x = torch.randn(40, 2048 + 64, generator=g).to(torch.bfloat16).to(DEV)
    big_w = (torch.randn(600, 2048 + 32, generator=g) / 45).to(torch.bfloat16).to(DEV)
    x, w = big_x[3:, :2048], big_w[:, 32:]  # row strides 2112 / 2080, 16-byte aligned
    assert x.stride(0) == 2112 and w.stride(0) == 2080
    res = torch.randn(37, 600, generator=g).to(torch.bfloat16).to(DEV)
    keep = res.clone()
    with torch.inference_mode():
        out = ops.linear(x, w, res, out=res)  # out aliases the residual
    assert out.data_ptr() == res.data_ptr()
    _check(out, x, w, keep)


def test_linear_gemv_strided_rows_and_in_place_residual():
    """The gemv kernel (M <= 4) with strided x / weight rows and out aliasing the residual."""
    g = torch.Generator(device="cpu").manual_seed(5)
    big_x = torch.randn(9, 2048 + 64, generator=g).to(torch.bfloat16).to(DEV)
    big_w = (torch.randn(1030, 2048 + 32, generator=g) / 45).to(torch.bfloat16).to(DEV)
    x, w = big_x[1:8:2, :2048], big_w[:, 32:]  # 4 rows of stride 4224, weight stride 2080
    assert x.stride(0) == 4224 and w.stride(0) == 2080
    res = torch.randn(4, 1030, generator=g).to(torch.bfloat16).to(DEV)
    keep = res.clone()
    with torch.inference_mode():
        out = ops.linear(x, w, res, out=res)
    assert out.data_ptr() == res.data_ptr()
    _check(out, x, w, keep)


@pytest.mark.parametrize("rows", [6, 20, 40])
def test_linear_wide_and_stream_strided_rows_and_in_place_residual(rows):
    """The wide kernel (6 rows) and the stream kernel (20 and 40 rows) with strided x /
    weight rows and out aliasing the residual, with and without the fused RMSNorm."""
    g = torch.Generator(device="cpu").manual_seed(7 + rows)
    big_x = torch.randn(2 * rows + 1, 4096 + 64, generator=g).to(torch.bfloat16).to(DEV)
    big_w = (torch.randn(700, 4096 + 32, generator=g) / 64).to(torch.bfloat16).to(DEV)
    x, w = big_x[1::2, :4096], big_w[:, 32:]  # rows of stride 8320, weight stride 4128
    assert x.shape[0] == rows and x.stride(0) == 8320 and w.stride(0) == 4128
    res = torch.randn(rows, 700, generator=g).to(torch.bfloat16).to(DEV)
    keep = res.clone()
    with torch.inference_mode():
        out = ops.linear(x, w, res, out=res)
    assert out.data_ptr() == res.data_ptr()
    _check(out, x, w, keep)
    nw = (1 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16).to(DEV)
    with torch.inference_mode():
        got = ops.linear(x, w, norm_weight=nw, norm_eps=1e-5)
    # the bound of test_linear_fused_rms_norm_matches_fp32_reference
    xf, wf = x.float().cpu(), w.float().cpu()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5) * nw.float().cpu()
    want = xn @ wf.T
    bound = ULP[torch.bfloat16] * (want.abs() + xn.abs() @ wf.abs().T) + 2.0 ** -16 * (
        xn.abs() @ wf.abs().T) + 1e-30
    worst = ((got.float().cpu() - want).abs() / bound).max().item()
    assert worst <= 1.0, f"max error / bound = {worst:.3f}"


def test_linear_repeated_calls_are_deterministic():
    g = torch.Generator(device="cpu").manual_seed(4)
    x = torch.randn(5, 4096, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(2048, 4096, generator=g) / 64).to(torch.bfloat16).to(DEV)
    with torch.inference_mode():
        first = ops.linear(x, w)
        for _ in range(3):
            assert torch.equal(ops.linear(x, w), first)


def test_linear_rejects_what_it_does_not_take():
    x = torch.randn(4, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(32, 64, device=DEV, dtype=torch.bfloat16)
    assert ops.linear_supported(x, w)
    assert not ops.linear_supported(x.float(), w.float())
    assert not ops.linear_supported(torch.randn(257, 64, device=DEV, dtype=torch.bfloat16), w)
    assert not ops.linear_supported(x[:, :48], w[:, :48])  # K % 32
    assert not ops.linear_supported(x[:, 1:33], w[:, :32])  # misaligned rows
    with pytest.raises(ValueError, match="unsupported operands"):
        ops.linear(x.half(), w)
    with pytest.raises(ValueError, match="residual"):
        ops.linear(x, w, torch.zeros(4, 31, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="at most 32 rows"):
        big = torch.randn(33, 64, device=DEV, dtype=torch.bfloat16)
        ops.linear(big, w, norm_weight=torch.ones(64, device=DEV, dtype=torch.bfloat16))


@pytest.mark.parametrize("rank", [1, 4])
@pytest.mark.parametrize("batch,per_layer", [(3, 2), (40, 1)])
def test_bf16_weight_decode_matches_oracle(rank, batch, per_layer, monkeypatch):
    """A bf16-weight model's decode steps run their projections on ops.linear (counted: both
    at 3 rows, RMSNorm fused into in_proj and the residual into out_proj; out_proj only at 40
    rows) and match the oracle model fed the same bf16-rounded weights and inputs in FP32."""
    torch.manual_seed(21 + rank)
    model = Mamba3(128, d_state=128, depth=2, mimo_rank=rank).eval().to(torch.bfloat16)
    model = model.to(DEV)
    dims = op.Dims(128, 128, rank)
    x = torch.randn(batch, 12, 128).to(torch.bfloat16)
    calls = []
    real = ops.linear

    def counting(*args, **kwargs):
        calls.append(args[0].shape)
        return real(*args, **kwargs)

    monkeypatch.setattr(ops, "linear", counting)
    with torch.no_grad():  # the block norms carry real weights, not ones
        for layer in model.layers:
            layer.norm.weight.mul_(torch.linspace(0.5, 1.5, 128, dtype=torch.bfloat16,
                                                  device=DEV))
    params = {k: v.detach().float().cpu().clone() for k, v in model.state_dict().items()}
    with torch.inference_mode():
        _, want_cache = op.model_prefill(params, x[:, :4].float(), dims)
        want = []
        for t in range(4, 12):
            o, want_cache = op.model_step(params, x[:, t:t + 1].float(), dims, want_cache)
            want.append(o)
        want = torch.cat(want, 1)
        _, cache = model.prefill(x[:, :4].to(DEV))
        got = []
        for t in range(4, 12):
            o, cache = model.step(x[:, t:t + 1].to(DEV), cache)
            got.append(o)
        got = torch.cat(got, 1)
    assert len(calls) == 8 * 2 * per_layer  # 8 tokens x 2 layers x projections on linear
    # every intermediate of the bf16 model is rounded to bf16, the oracle's stay FP32: the 16-bit
    # bar of the scan tests, 2e-2 of the output scale elementwise and 1e-2 in norm
    d = got.float().cpu() - want
    assert d.abs().max().item() <= 2e-2 * want.abs().max().item()
    assert d.norm().item() <= 1e-2 * want.norm().item()


def test_decode_with_a_half_last_stage_matches_oracle():
    """``Mamba3(48)`` with bf16 weights at batch 40: out_proj has K = 96 (a multiple of 32,
    not of 64) and 40 rows, so it takes the tile kernel with a 32-wide last stage."""
    torch.manual_seed(90)
    model = Mamba3(48, d_state=16, depth=2, mimo_rank=1).eval()
    params = {k: v.detach().clone().to(torch.bfloat16) for k, v in model.state_dict().items()}
    model = model.to(DEV, torch.bfloat16)
    dims = op.Dims(48, 16, 1)
    x = torch.randn(40, 4, 48).to(torch.bfloat16)
    cache, want_cache = None, None
    with torch.inference_mode():
        for t in range(4):
            got, cache = model.step(x[:, t:t + 1].to(DEV), cache)
            want, want_cache = op.model_step(params, x[:, t:t + 1], dims, want_cache)
            torch.testing.assert_close(got.float().cpu(), want.float(), rtol=2e-2, atol=2e-2)
