"""The plugin hooks' dispatch contract (``mamba3_amd.hooks``) without a GPU.

The reference's hooks (``mamba3/ops.py:87-190, 253-367``) return ``None`` to hand a call back to
the portable path: off the GPU, with autograd recording, behind ``MAMBA3_DISABLE_TRITON``, and,
after one ``RuntimeWarning``, for every later call with a key that failed. The same contract is
checked here: the GPU gates with CPU tensors, the switches, and the warn-once negative cache with
the library call replaced by one that fails (no device is touched).
"""

from __future__ import annotations

import warnings

import pytest
import torch

from mamba3_amd import hooks, ops


def _step_inputs(rank=1, n=16, p=8, h=2, b=2, s=4):
    q = torch.randn(b, h, rank, n)
    cache = (torch.zeros(b, h, s), torch.zeros(b, h, p, n), torch.zeros(b, h, rank, n),
             torch.zeros(b, h, p))
    return dict(q=q, k=q.clone(), value=torch.randn(b, h, p), gate=torch.randn(b, h, p),
                adt=-torch.rand(b, h), dt=torch.rand(b, h), trap_logits=torch.randn(b, h),
                angle_rate=torch.randn(b, s), D=torch.ones(h), cache=cache)


def _scan_inputs(b=1, length=5, h=2, n=16, p=8):
    q = torch.randn(b, length, 1, 1, n)
    return dict(q=q, k=q.clone(), value=torch.randn(b, length, h, p),
                gate=torch.randn(b, length, h, p), adt=-torch.rand(b, length, h),
                dt=torch.rand(b, length, h), trap_logits=torch.randn(b, length, h),
                D=torch.ones(h), mimo_x=None, mimo_z=None, mimo_out=None, chunk_size=64,
                initial_state=None, initial_k=None, initial_value=None, phase=None,
                mimo_rotation=False, q_bias=None, k_bias=None)


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    for name in hooks.DISABLE_ENV:
        monkeypatch.delenv(name, raising=False)
    hooks.reset_failures()
    yield
    hooks.reset_failures()


def test_cpu_tensors_and_autograd_return_none_without_a_warning():
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        with torch.inference_mode():
            assert hooks.fused_step(**_step_inputs()) is None
            assert hooks.fused_chunk_scan(**_scan_inputs()) is None
        assert torch.is_grad_enabled()
        assert hooks.fused_step(**_step_inputs()) is None  # autograd recording: the caller's path
    assert not hooks._HIP_LAST_DISPATCH and not hooks._HIP_LAST_SCAN_DISPATCH


@pytest.mark.parametrize("name", hooks.DISABLE_ENV)
def test_switches_disable_the_hooks(name, monkeypatch):
    monkeypatch.setattr(hooks, "_on_rocm", lambda *t: True)
    called = []
    monkeypatch.setattr(ops, "fused_step", lambda *a, **k: called.append(1) or "ran")
    with torch.inference_mode():
        assert hooks.fused_step(**_step_inputs()) == "ran"
        monkeypatch.setenv(name, "1")
        assert hooks.disabled()
        assert hooks.fused_step(**_step_inputs()) is None
    assert called == [1]


def test_failure_warns_once_per_key_and_is_remembered(monkeypatch):
    monkeypatch.setattr(hooks, "_on_rocm", lambda *t: True)
    calls = []

    def failing(*args, **kwargs):
        calls.append(1)
        raise ops._hip.HipError("m3_scan_fwd", 2, "shape not served")

    monkeypatch.setattr(ops, "mamba3_scan", failing)
    with torch.inference_mode():
        with pytest.warns(RuntimeWarning, match="chunked scan is unavailable"):
            assert hooks.fused_chunk_scan(**_scan_inputs()) is None
        with warnings.catch_warnings():
            warnings.simplefilter("error")
            assert hooks.fused_chunk_scan(**_scan_inputs()) is None  # cached: no call, no warning
        assert calls == [1]
        # another key (another d_state) is tried again
        with pytest.warns(RuntimeWarning):
            assert hooks.fused_chunk_scan(**_scan_inputs(n=32)) is None
        assert calls == [1, 1]
    assert not hooks._HIP_LAST_SCAN_DISPATCH


def test_scan_gates_follow_the_reference(monkeypatch):
    monkeypatch.setattr(hooks, "_on_rocm", lambda *t: True)
    monkeypatch.setattr(ops, "mamba3_scan", lambda *a, **k: ("y", "s"))
    with torch.inference_mode():
        assert hooks.fused_chunk_scan(**_scan_inputs()) == ("y", "s")
        assert hooks._HIP_LAST_SCAN_DISPATCH
        inp = _scan_inputs()
        inp["adt"] = inp["adt"].double()  # adt must be FP32
        assert hooks.fused_chunk_scan(**inp) is None
        inp = _scan_inputs()
        inp["value"] = inp["value"].half()  # one activation dtype
        assert hooks.fused_chunk_scan(**inp) is None


def test_bind_installs_the_hooks_and_sets_the_reference_flags(monkeypatch):
    """``hooks.bind`` replaces the reference's hook bindings (``ops._fused_chunk_scan``,
    ``ops.fused_step`` and the name ``model.fused_step`` imported at ``model.py:11``) and mirrors
    every dispatch into the reference's ``_TRITON_LAST_DISPATCH`` / ``_TRITON_LAST_SCAN_DISPATCH``,
    which its tests assert (``tests/test_scan.py:423``, ``tests/test_model.py:465``). Stub modules
    stand for ``mamba3.ops`` and ``mamba3.model``."""
    import types
    ref_ops = types.ModuleType("stub_ops")
    ref_ops._TRITON_LAST_DISPATCH = False
    ref_ops._TRITON_LAST_SCAN_DISPATCH = False
    ref_model = types.ModuleType("stub_model")
    monkeypatch.setattr(hooks, "_FLAG_TARGETS", [])
    hooks.bind(ref_ops, ref_model)
    hooks.bind(ref_ops, ref_model)  # binding twice keeps one flag target
    assert hooks._FLAG_TARGETS == [ref_ops]
    assert ref_ops._fused_chunk_scan is hooks.fused_chunk_scan
    assert ref_ops.fused_step is hooks.fused_step and ref_model.fused_step is hooks.fused_step

    monkeypatch.setattr(hooks, "_on_rocm", lambda *t: True)
    monkeypatch.setattr(ops, "mamba3_scan", lambda *a, **k: ("y", "s"))
    monkeypatch.setattr(ops, "fused_step", lambda *a, **k: ("o", "c"))
    with torch.inference_mode():
        assert ref_ops._fused_chunk_scan(**_scan_inputs()) == ("y", "s")
        assert ref_ops._TRITON_LAST_SCAN_DISPATCH and not ref_ops._TRITON_LAST_DISPATCH
        assert ref_model.fused_step(**_step_inputs()) == ("o", "c")
        assert ref_ops._TRITON_LAST_DISPATCH
        monkeypatch.setenv("MAMBA3_DISABLE_TRITON", "1")
        assert ref_ops._fused_chunk_scan(**_scan_inputs()) is None
        assert ref_model.fused_step(**_step_inputs()) is None
    assert not ref_ops._TRITON_LAST_SCAN_DISPATCH and not ref_ops._TRITON_LAST_DISPATCH
