"""``Mamba3`` on the GPU against the CPU oracle model (same seeded weights and inputs).

FP32 within 1e-4 (abs and rel); bf16 autocast within 2e-2. The dispatch flags prove that
the HIP kernels, not some other path, produced the results.
"""

from __future__ import annotations

import pytest
import torch

from conftest import bf16_parity
from mamba3_amd import Mamba3, ops
from oracle import portable as op

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
F32 = dict(rtol=1e-4, atol=1e-4)
BF16 = dict(rtol=2e-2, atol=2e-2)


def _model(d_model, d_state, depth, rank, seed, causal=True):
    torch.manual_seed(seed)
    model = Mamba3(d_model, d_state=d_state, depth=depth, mimo_rank=rank, causal=causal).eval()
    params = {k: v.detach().clone() for k, v in model.state_dict().items()}
    return model.to(DEV), params, op.Dims(d_model, d_state, rank)


def _oracle_ctx(bf16: bool):
    return torch.autocast("cpu", dtype=torch.bfloat16) if bf16 else torch.autocast(
        "cpu", enabled=False)


def _gpu_ctx(bf16: bool):
    return torch.autocast("cuda", dtype=torch.bfloat16) if bf16 else torch.autocast(
        "cuda", enabled=False)


CASES = [(64, 16, 2, 1), (64, 16, 2, 4), (128, 128, 2, 1), (128, 128, 1, 4), (32, 8, 2, 1),
         (64, 16, 2, 8), (128, 128, 1, 8)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("case", CASES)
def test_forward_prefill_steps_match_oracle(case, bf16):
    d_model, d_state, depth, rank = case
    model, params, dims = _model(d_model, d_state, depth, rank, seed=10 + rank)
    torch.manual_seed(1)
    x = torch.randn(2, 75, d_model)
    split = 66
    tol = BF16 if bf16 else F32
    with torch.inference_mode(), _oracle_ctx(bf16):
        want = op.model_forward(params, x, dims)
        want_prefix, want_cache = op.model_prefill(params, x[:, :split], dims)
        want_steps = []
        for t in range(split, x.shape[1]):
            o, want_cache = op.model_step(params, x[:, t:t + 1], dims, want_cache)
            want_steps.append(o)
        want_steps = torch.cat(want_steps, 1)
    xd = x.to(DEV)
    with torch.inference_mode(), _gpu_ctx(bf16):
        got = model(xd)
        assert ops._HIP_LAST_SCAN_DISPATCH
        prefix, cache = model.prefill(xd[:, :split])
        steps = []
        for t in range(split, x.shape[1]):
            o, cache = model.step(xd[:, t:t + 1], cache)
            assert ops._HIP_LAST_DISPATCH
            steps.append(o)
        steps = torch.cat(steps, 1)
    torch.cuda.synchronize()
    print(f"model {case} bf16={bf16}: forward {(got.float().cpu() - want.float()).abs().max():.2e}"
          f" steps {(steps.float().cpu() - want_steps.float()).abs().max():.2e}", flush=True)
    torch.testing.assert_close(got.float().cpu(), want.float(), **tol)
    torch.testing.assert_close(prefix.float().cpu(), want_prefix.float(), **tol)
    torch.testing.assert_close(steps.float().cpu(), want_steps.float(), **tol)
    for layer, want_layer in zip(cache, want_cache):
        for a, b in zip(layer, want_layer):
            torch.testing.assert_close(a.float().cpu(), b.float(), **tol)


@pytest.mark.parametrize("length", [1, 15, 16, 17, 63, 64, 65, 130, 700])
@pytest.mark.parametrize("rank", [1, 4])
def test_model_shape_lengths_match_oracle(length, rank):
    """The model's shape (N 128, P 64, 32 angles: the full-shape kernels; the 16-wave scan's
    64-row sub-chunks are 64 tokens at rank 1 and 16 at rank 4) in bf16 autocast over 1 to 44
    sub-chunks, ragged and exact: forward output, prefill output and cache."""
    model, params, dims = _model(128, 128, 1, rank, seed=30 + rank)
    torch.manual_seed(31)
    x = torch.randn(2, length, 128)
    with torch.inference_mode(), _oracle_ctx(True):
        want = op.model_forward(params, x, dims)
        _, want_cache = op.model_prefill(params, x, dims)
    with torch.inference_mode(), _gpu_ctx(True):
        got = model(x.to(DEV))
        assert ops._HIP_LAST_SCAN_DISPATCH
        prefix, cache = model.prefill(x.to(DEV))
    torch.cuda.synchronize()
    print(f"model shape R={rank} L={length}: forward "
          f"{(got.float().cpu() - want.float()).abs().max():.2e}", flush=True)
    torch.testing.assert_close(got.float().cpu(), want.float(), **BF16)
    torch.testing.assert_close(prefix.float().cpu(), want.float(), **BF16)
    for a, b in zip(cache[0], want_cache[0]):
        torch.testing.assert_close(a.float().cpu(), b.float(), **BF16)


@pytest.mark.parametrize("rank", [1, 4])
def test_cached_steps_match_full_forward(rank):
    """Reference tests/test_model.py:164-184 (step-by-step from an empty cache)."""
    model, _, _ = _model(16, 8, 2, rank, seed=2)
    torch.manual_seed(2)
    x = torch.randn(2, 11, 16, device=DEV)
    cache = None
    outs = []
    with torch.inference_mode():
        want = model(x)
        for t in range(x.shape[1]):
            o, cache = model.step(x[:, t:t + 1], cache)
            outs.append(o)
    torch.testing.assert_close(torch.cat(outs, 1), want, rtol=2e-5 * 5, atol=2e-6 * 50)


@pytest.mark.parametrize("rank", [1, 4])
def test_prefill_cache_continues_without_rescanning(rank):
    """Reference tests/test_model.py:187-202."""
    model, _, _ = _model(16, 8, 2, rank, seed=3)
    torch.manual_seed(3)
    x = torch.randn(2, 15, 16, device=DEV)
    with torch.inference_mode():
        want = model(x)
        prefix, cache = model.prefill(x[:, :9])
        outs = [prefix]
        for t in range(9, 15):
            o, cache = model.step(x[:, t:t + 1], cache)
            outs.append(o)
    torch.testing.assert_close(torch.cat(outs, 1), want, **F32)


def test_prefill_continues_from_a_cache():
    """Scan continuation through the model: prefill(a) then forward(b, cache)."""
    model, _, _ = _model(64, 128, 1, 1, seed=4)
    torch.manual_seed(4)
    x = torch.randn(2, 200, 64, device=DEV)
    with torch.inference_mode():
        mixer = model.layers[0].mixer
        h = model.layers[0].norm(x)
        full, full_cache = mixer(h, return_cache=True)
        first, cache = mixer(h[:, :130], return_cache=True)
        second, cache2 = mixer(h[:, 130:], cache=cache, return_cache=True)
    torch.testing.assert_close(torch.cat((first, second), 1), full, **F32)
    for a, b in zip(cache2, full_cache):
        torch.testing.assert_close(a, b, **F32)


def test_prefill_cache_does_not_retain_prefix_storage():
    """Reference tests/test_model.py:205-210."""
    model, _, _ = _model(32, 16, 1, 1, seed=5)
    with torch.inference_mode():
        _, cache = model.prefill(torch.randn(2, 257, 32, device=DEV))
    for t in (cache[0][0], cache[0][2], cache[0][3]):
        assert t.untyped_storage().nbytes() == t.numel() * t.element_size()


def test_graph_decoder_matches_forward_and_resets():
    """Reference tests/test_model.py:338-379 (hipGraph capture), plus the oracle: the replayed
    outputs and every cache tensor against ``oracle.model_step``'s chain."""
    model, params, dims = _model(64, 128, 1, 1, seed=5)
    torch.manual_seed(5)
    x_cpu = torch.randn(2, 5, 64)
    x = x_cpu.to(DEV)
    ref_cache = None
    ref_outs = []
    with torch.inference_mode():
        for t in range(5):
            o, ref_cache = model.step(x[:, t:t + 1], ref_cache)
            ref_outs.append(o)
        oracle_cache = None
        oracle_outs = []
        for t in range(5):
            o, oracle_cache = op.model_step(params, x_cpu[:, t:t + 1], dims, oracle_cache)
            oracle_outs.append(o)
    decoder = model.cuda_graph(batch_size=2)
    with torch.inference_mode():
        want = model(x)
        got = torch.cat([decoder(x[:, t:t + 1]).clone() for t in range(5)], 1)
    torch.testing.assert_close(got, want, rtol=2e-4, atol=2e-5 * 5)
    torch.testing.assert_close(got, torch.cat(ref_outs, 1), rtol=2e-4, atol=2e-5)
    torch.testing.assert_close(got.cpu(), torch.cat(oracle_outs, 1), **F32)
    for g_layer, r_layer, o_layer in zip(decoder.cache, ref_cache, oracle_cache):
        for a, b, c in zip(g_layer, r_layer, o_layer):
            torch.testing.assert_close(a, b, rtol=2e-4, atol=2e-5)
            torch.testing.assert_close(a.cpu(), c, **F32)
    decoder.reset()
    with torch.inference_mode():
        again = decoder(x[:, :1]).clone()
    torch.testing.assert_close(again, want[:, :1], rtol=2e-4, atol=2e-5 * 5)
    with torch.no_grad():
        model.layers[0].mixer.D.add_(0.1)
    with pytest.raises(RuntimeError, match="recreate"):
        decoder.validate()
    with pytest.raises(ValueError, match="gradient"):
        decoder(x[:, :1].clone().requires_grad_())
    # storage moved under the same Parameter object and version: `p.data = ...`, `Module.to`
    fresh = model.cuda_graph(batch_size=2)
    fresh.validate()
    weight = model.layers[0].mixer.in_proj.weight
    weight.data = weight.data.clone()
    with pytest.raises(RuntimeError, match="recreate"):
        fresh(x[:, :1], validate=True)
    fresh = model.cuda_graph(batch_size=2)
    model.to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="recreate"):
        fresh.validate()


@pytest.mark.parametrize("batch", [3, 40, 70])
@pytest.mark.parametrize("rank", [1, 4])
def test_graph_decoder_bf16_weights_against_oracle(rank, batch):
    """bf16 weights, FP32 state: a prefill loaded into the graph decoder (``load_cache``), then
    40 replays with eager work in between. Against the eager HIP steps: outputs within 1e-2,
    states within 1e-4. Against the oracle: the bf16 parity bar (``conftest.bf16_parity``) on the
    outputs, with the oracle's chain in bf16 and in FP32 (same bf16-valued weights), and the
    FP32 states at least as close to the FP32 chain as the oracle's bf16 chain is. Batch 3 runs
    the block's norm and residual inside ``m3_linear`` (gemv), batch 40 its out_proj on the
    stream kernel in two row blocks, batch 70 the general-GEMM loop with each residual add fused
    into the next RMSNorm."""
    model, params, dims = _model(128, 128, 2, rank, seed=6)
    model = model.to(torch.bfloat16)
    torch.manual_seed(6)
    x_cpu = torch.randn(batch, 70, 128).to(torch.bfloat16)
    x = x_cpu.to(DEV)
    split = 30
    decoder = model.cuda_graph(batch_size=batch)
    with torch.inference_mode():
        _, cache = model.prefill(x[:, :split])
    decoder.load_cache(cache)
    eager_cache = [tuple(t.clone() for t in layer) for layer in cache]
    got, eager = [], []
    with torch.inference_mode():
        for t in range(split, x.shape[1]):
            got.append(decoder(x[:, t:t + 1]).clone())
            e, eager_cache = model.step(x[:, t:t + 1], eager_cache)
            eager.append(e)
    torch.cuda.synchronize()
    got, eager = torch.cat(got, 1), torch.cat(eager, 1)
    torch.testing.assert_close(got.float(), eager.float(), rtol=1e-2, atol=1e-2)
    for g_layer, e_layer in zip(decoder.cache, eager_cache):
        torch.testing.assert_close(g_layer[1], e_layer[1], rtol=1e-4, atol=1e-4)
    chains = {}
    for dtype in (torch.bfloat16, torch.float32):
        p_run = {k: v.to(torch.bfloat16).to(dtype) for k, v in params.items()}
        with torch.inference_mode():
            _, c = op.model_prefill(p_run, x_cpu[:, :split].to(dtype), dims)
            outs = []
            for t in range(split, x.shape[1]):
                o, c = op.model_step(p_run, x_cpu[:, t:t + 1].to(dtype), dims, c)
                outs.append(o)
        chains[dtype] = (torch.cat(outs, 1), c)
    (w16, c16), (w32, c32) = chains[torch.bfloat16], chains[torch.float32]
    bf16_parity(f"graph bf16 R={rank} outputs", got, w16, w32,
                min_inside=0.999)  # measured 99.993% and more
    bf16_parity(f"graph bf16 R={rank} states", torch.stack([c[1] for c in decoder.cache]),
                torch.stack([c[1] for c in c16]), torch.stack([c[1] for c in c32]),
                elementwise=False, max_slack=1.5)


@pytest.mark.parametrize("rank", [1, 4])
def test_bidirectional_matches_oracle(rank):
    model, params, dims = _model(64, 128, 2, rank, seed=12, causal=False)
    torch.manual_seed(12)
    x = torch.randn(2, 90, 64)
    with torch.inference_mode():
        want = op.model_forward(params, x, dims, causal=False)
        got = model(x.to(DEV)).cpu()
    torch.testing.assert_close(got, want, **F32)


def test_bidirectional_is_non_causal():
    """Reference tests/test_model.py:119-137."""
    model, _, _ = _model(16, 8, 1, 1, seed=11, causal=False)
    first = torch.randn(1, 12, 16, device=DEV)
    second = first.clone()
    second[:, 5:] = torch.randn_like(second[:, 5:])
    with torch.inference_mode():
        a, b = model(first), model(second)
    assert torch.isfinite(a).all()
    assert not torch.allclose(a[:, 0], b[:, 0], rtol=1e-5, atol=1e-6)


def test_causal_prefix_is_unchanged():
    """Reference tests/test_model.py:107-116."""
    model, _, _ = _model(16, 8, 2, 1, seed=0)
    first = torch.randn(1, 12, 16, device=DEV)
    second = first.clone()
    second[:, 7:] = torch.randn_like(second[:, 7:])
    with torch.inference_mode():
        a, b = model(first), model(second)
    torch.testing.assert_close(a[:, :7], b[:, :7], rtol=0, atol=1e-7)


def test_config1_parity():
    """BASELINE config 1 on the GPU in FP32: forward, prefill(960) + 64 steps, vs the oracle."""
    model, params, dims = _model(256, 128, 6, 1, seed=0)
    torch.manual_seed(0)
    Mamba3(256, d_state=128, depth=6, mimo_rank=1)  # consume the RNG as the config does
    x = torch.randn(2, 1024, 256)
    with torch.inference_mode():
        want = op.model_forward(params, x, dims)
        xd = x.to(DEV)
        got = model(xd)
        prefix, cache = model.prefill(xd[:, :960])
        steps = []
        for i in range(64):
            o, cache = model.step(xd[:, 960 + i:961 + i], cache)
            steps.append(o)
        steps = torch.cat(steps, 1).cpu()
    torch.testing.assert_close(got.cpu(), want, **F32)
    torch.testing.assert_close(prefix.cpu(), want[:, :960], **F32)
    torch.testing.assert_close(steps, want[:, 960:], **F32)


# Models whose shapes the MFMA scan does not tile (the recurrent scan), and whose decode step
# runs on the step kernels (d_state 256) or as a one-token recurrent scan (d_state not a power
# of 2, rank 3; d_state 1024, whose 256 KiB state is updated in final_state instead of LDS;
# rank 16, read out in two groups of 8): forward, prefill and steps against the oracle.
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("case", [(64, 256, 1, 1), (48, 96, 2, 1), (32, 8, 2, 3), (64, 64, 1, 6),
                                  (64, 1024, 1, 1), (64, 128, 1, 16)])
def test_recurrent_shapes_match_oracle(case, bf16):
    d_model, d_state, depth, rank = case
    model, params, dims = _model(d_model, d_state, depth, rank, seed=30 + rank)
    torch.manual_seed(31)
    x = torch.randn(2, 75, d_model)
    split = 66
    with torch.inference_mode(), _oracle_ctx(bf16):
        want = op.model_forward(params, x, dims)
        want_prefix, want_cache = op.model_prefill(params, x[:, :split], dims)
        want_steps = []
        for t in range(split, x.shape[1]):
            o, want_cache = op.model_step(params, x[:, t:t + 1], dims, want_cache)
            want_steps.append(o)
        want_steps = torch.cat(want_steps, 1)
    xd = x.to(DEV)
    with torch.inference_mode(), _gpu_ctx(bf16):
        got = model(xd)
        assert ops._HIP_LAST_SCAN_DISPATCH
        prefix, cache = model.prefill(xd[:, :split])
        steps = []
        for t in range(split, x.shape[1]):
            o, cache = model.step(xd[:, t:t + 1], cache)
            assert ops._HIP_LAST_DISPATCH
            steps.append(o)
        steps = torch.cat(steps, 1)
    torch.cuda.synchronize()
    tol = BF16 if bf16 else F32
    print(f"recurrent model {case} bf16={bf16}: forward "
          f"{(got.float().cpu() - want.float()).abs().max():.2e} steps "
          f"{(steps.float().cpu() - want_steps.float()).abs().max():.2e}", flush=True)
    torch.testing.assert_close(got.float().cpu(), want.float(), **tol)
    torch.testing.assert_close(prefix.float().cpu(), want_prefix.float(), **tol)
    torch.testing.assert_close(steps.float().cpu(), want_steps.float(), **tol)
    for layer, want_layer in zip(cache, want_cache):
        for a, b in zip(layer, want_layer):
            torch.testing.assert_close(a.float().cpu(), b.float(), **tol)
