"""The plugin hooks on the GPU: they run the HIP library (same results as ``mamba3_amd.ops``,
checked against the oracle) and fall back with one warning for a shape the library refuses."""

from __future__ import annotations

import warnings

import pytest
import torch

from mamba3_amd import hooks, ops
from oracle import portable as op
from test_gpu_scan import _inputs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    for name in hooks.DISABLE_ENV:
        monkeypatch.delenv(name, raising=False)
    hooks.reset_failures()
    yield
    hooks.reset_failures()


def _hook_args(inp):
    full = dict(mimo_x=None, mimo_z=None, mimo_out=None, initial_state=None, initial_k=None,
                initial_value=None, phase=None, mimo_rotation=False, q_bias=None, k_bias=None)
    full.update(inp)
    return full


@pytest.mark.parametrize("rank", [1, 4])
def test_scan_hook_runs_the_library(rank):
    inp = _inputs(rank, torch.bfloat16, seed=80 + rank, length=100)
    dev = {n: (t.to(DEV) if isinstance(t, torch.Tensor) else t) for n, t in inp.items()}
    with torch.inference_mode():
        got = hooks.fused_chunk_scan(**_hook_args(dev), chunk_size=64 // rank)
    assert got is not None and hooks._HIP_LAST_SCAN_DISPATCH
    y_ref, s_ref = op.ssd_scan(**inp, chunk_size=64 // rank)
    dy = (got[0].float().cpu() - y_ref.float()).abs().max()
    assert dy <= 2e-2 * y_ref.float().abs().max()
    torch.testing.assert_close(got[1].cpu(), s_ref, rtol=2e-2, atol=2e-2)


def test_scan_hook_falls_back_once_for_a_refused_shape():
    # rank 64 at d_state 128: its per-token q / k / value rows exceed what either scan kernel
    # holds (the recurrent scan's 160 KiB of LDS): one warning, then the cached key
    inp = _inputs(1, torch.bfloat16, seed=3, length=20, phase=False, bias=False, initial=False)
    dev = {n: (t.to(DEV) if isinstance(t, torch.Tensor) else t) for n, t in inp.items()}
    q = dev["q"].expand(-1, -1, -1, 64, -1).contiguous()
    heads, p = dev["value"].shape[2], dev["value"].shape[3]
    mimo = torch.ones(heads, 64, p, device=DEV)
    args = _hook_args(dict(dev, q=q, k=q.clone(), mimo_x=mimo, mimo_z=mimo, mimo_out=mimo))
    with torch.inference_mode():
        with pytest.warns(RuntimeWarning, match="unavailable"):
            assert hooks.fused_chunk_scan(**args, chunk_size=16) is None
        with warnings.catch_warnings():
            warnings.simplefilter("error")
            assert hooks.fused_chunk_scan(**args, chunk_size=16) is None
    assert not hooks._HIP_LAST_SCAN_DISPATCH


def test_step_hook_runs_the_library_and_the_switch_turns_it_off(monkeypatch):
    g = torch.Generator().manual_seed(9)
    b, h, n, p, s = 3, 4, 128, 64, 32
    args = dict(q=torch.randn(b, h, 1, n, generator=g), k=torch.randn(b, h, 1, n, generator=g),
                value=torch.randn(b, h, p, generator=g), gate=torch.randn(b, h, p, generator=g),
                adt=-torch.rand(b, h, generator=g) * 0.1, dt=torch.rand(b, h, generator=g) * 0.1,
                trap_logits=torch.randn(b, h, generator=g), angle_rate=torch.randn(b, s, generator=g),
                D=torch.ones(h))
    cache = (torch.zeros(b, h, s), torch.randn(b, h, p, n, generator=g) * 0.1,
             torch.randn(b, h, 1, n, generator=g), torch.randn(b, h, p, generator=g))
    dev = {k: v.to(DEV) for k, v in args.items()}
    dcache = tuple(t.to(DEV) for t in cache)
    with torch.inference_mode():
        got = hooks.fused_step(**dev, cache=dcache)
        assert got is not None and hooks._HIP_LAST_DISPATCH
        want = ops.fused_step(**dev, cache=dcache)
        torch.testing.assert_close(got[0], want[0], rtol=0, atol=0)
        monkeypatch.setenv("MAMBA3_DISABLE_HIP", "1")
        assert hooks.fused_step(**dev, cache=dcache) is None
        assert not hooks._HIP_LAST_DISPATCH
