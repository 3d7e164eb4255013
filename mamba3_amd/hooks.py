"""The reference's two plugin points, served by the HIP library.

jreoka/mamba3 sends its hot path through two hooks in ``mamba3/ops.py`` that return ``None``
to hand a call back to its portable PyTorch path: ``fused_step`` (``ops.py:87-190``) and
``_fused_chunk_scan`` (``ops.py:253-367``). This module holds drop-in bodies for both, with the
reference's dispatch contract:

* ``None`` (the caller runs its own path) when the call is outside what the library serves:
  autograd recording, tensors off a ROCm device, an activation dtype other than float32 /
  bfloat16 / float16, a scan whose ``adt`` is not FP32, the switch ``MAMBA3_DISABLE_HIP=1``
  (or the reference's own ``MAMBA3_DISABLE_TRITON=1``, so its A/B tests keep working), or a
  call key that failed before;
* when the library refuses or fails a call: one ``RuntimeWarning`` per call key, the key is
  remembered (the negative cache: later calls with it return ``None`` without trying), and
  ``None``;
* ``_HIP_LAST_DISPATCH`` / ``_HIP_LAST_SCAN_DISPATCH`` tell whether the last call ran on the
  GPU (the reference's ``_TRITON_LAST_DISPATCH`` / ``_TRITON_LAST_SCAN_DISPATCH``,
  ``ops.py:14, 18``). ``bind`` installs both hooks into the reference's modules and makes every
  call also set those two flags there, so the reference's dispatch assertions
  (``tests/test_scan.py:423``, ``tests/test_model.py:465``) hold with the hooks bound.

The call keys are the reference's: device, the dtypes of every tensor argument and the shape
parameters (``ops.py:110-126``, ``ops.py:288-302``). Everything else (validation and its
``ValueError`` messages, the launches) is ``mamba3_amd.ops``; this module only decides
whether to try, and turns a failure into the fallback. Unlike ``mamba3_amd.ops``, which raises,
these hooks never raise for a call the library cannot serve: that is their contract.
"""

from __future__ import annotations

import os
import warnings

import torch

from . import ops

DISABLE_ENV = ("MAMBA3_DISABLE_HIP", "MAMBA3_DISABLE_TRITON")
_ACT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)

_STEP_FAILURES: set[tuple[object, ...]] = set()
_SCAN_FAILURES: set[tuple[object, ...]] = set()
_HIP_LAST_DISPATCH = False
_HIP_LAST_SCAN_DISPATCH = False
# modules whose `_TRITON_LAST_DISPATCH` / `_TRITON_LAST_SCAN_DISPATCH` mirror the flags above
_FLAG_TARGETS: list[object] = []


def _set_step_flag(value: bool) -> None:
    global _HIP_LAST_DISPATCH
    _HIP_LAST_DISPATCH = value
    for module in _FLAG_TARGETS:
        module._TRITON_LAST_DISPATCH = value


def _set_scan_flag(value: bool) -> None:
    global _HIP_LAST_SCAN_DISPATCH
    _HIP_LAST_SCAN_DISPATCH = value
    for module in _FLAG_TARGETS:
        module._TRITON_LAST_SCAN_DISPATCH = value


def bind(ops_module, model_module=None) -> None:
    """Serve the reference's two hooks from this module.

    ``ops_module`` is the reference's ``mamba3.ops``: its ``_fused_chunk_scan`` (called by name
    from ``mamba3_scan``, ``ops.py:635``) and ``fused_step`` become the bodies here, and every
    call sets its ``_TRITON_LAST_DISPATCH`` / ``_TRITON_LAST_SCAN_DISPATCH`` as the reference's
    own bodies do (``ops.py:109, 181, 285, 358``). ``model_module`` is ``mamba3.model``, which
    imports ``fused_step`` by name (``model.py:11``, called at ``441``), so its binding is
    replaced too.
    """
    ops_module._fused_chunk_scan = fused_chunk_scan
    ops_module.fused_step = fused_step
    if model_module is not None:
        model_module.fused_step = fused_step
    if not any(m is ops_module for m in _FLAG_TARGETS):
        _FLAG_TARGETS.append(ops_module)


def disabled() -> bool:
    """Whether an environment switch turns the library's hot path off."""
    return any(os.getenv(name, "0") == "1" for name in DISABLE_ENV)


def _on_rocm(*tensors: torch.Tensor | None) -> bool:
    return all(t is None or t.device.type == "cuda" for t in tensors) and torch.version.hip is not None


def _try(call, key, failures: set, what: str):
    """Run ``call``; on any exception warn once for ``key``, remember it, return ``None``."""
    try:
        return call()
    except Exception as error:  # the fallback contract: the caller's own path takes over
        if key not in failures:
            failures.add(key)
            warnings.warn(f"{what} is unavailable on the HIP path; using PyTorch ({error})",
                          RuntimeWarning, stacklevel=3)
        return None


def fused_step(q, k, value, gate, adt, dt, trap_logits, angle_rate, D, cache, *, mimo_x=None,
               mimo_z=None, mimo_out=None):
    """One decode token on the GPU, or ``None`` (reference ``ops.fused_step``, ``ops.py:87-190``).

    Arguments and result are the reference's: head-expanded, biased, unrotated ``q / k
    [B, H, R, N]``, ``value / gate [B, H, P]``, ``adt / dt / trap_logits [B, H]``, ``angle_rate
    [B, S]``, ``cache = (phase, state, prev_k, prev_value)``; returns ``(output [B, H, P],
    (phase', state', k_rot, value))``.
    """
    _set_step_flag(False)
    key = (q.device, q.dtype, k.dtype, value.dtype, gate.dtype, adt.dtype, dt.dtype,
           trap_logits.dtype, angle_rate.dtype, D.dtype, tuple(t.dtype for t in cache),
           q.shape[-1], value.shape[-1], q.shape[2], cache[0].shape[-1])
    if (torch.is_grad_enabled() or disabled() or key in _STEP_FAILURES
            or q.dtype not in _ACT_DTYPES or not _on_rocm(q, k, value, gate, adt, dt, *cache)):
        return None
    result = _try(lambda: ops.fused_step(q, k, value, gate, adt, dt, trap_logits, angle_rate, D,
                                         cache, mimo_x=mimo_x, mimo_z=mimo_z,
                                         mimo_out=mimo_out),
                  key, _STEP_FAILURES, "fused Mamba-3 decoding")
    _set_step_flag(result is not None)
    return result


def fused_chunk_scan(q, k, value, gate, adt, dt, trap_logits, D, *, mimo_x, mimo_z, mimo_out,
                     chunk_size, initial_state, initial_k, initial_value, phase, mimo_rotation,
                     q_bias, k_bias):
    """The chunked SSD on the GPU, or ``None`` (reference ``ops._fused_chunk_scan``,
    ``ops.py:253-367``): ``(output [B, L, H, P], state [B, H, P, N] FP32)``."""
    _set_scan_flag(False)
    key = (q.device, q.dtype, k.dtype, value.dtype, gate.dtype, adt.dtype, dt.dtype,
           trap_logits.dtype, D.dtype, q.shape[-1], value.shape[-1], q.shape[3], chunk_size)
    if (torch.is_grad_enabled() or disabled() or key in _SCAN_FAILURES
            or q.dtype not in _ACT_DTYPES or adt.dtype != torch.float32
            or not (k.dtype == value.dtype == gate.dtype == q.dtype)
            or not _on_rocm(q, k, value, gate, adt, dt, trap_logits, D, phase, initial_state)):
        return None
    result = _try(lambda: ops.mamba3_scan(
        q, k, value, gate, adt, dt, trap_logits, D, mimo_x=mimo_x, mimo_z=mimo_z,
        mimo_out=mimo_out, chunk_size=chunk_size, initial_state=initial_state,
        initial_k=initial_k, initial_value=initial_value, phase=phase,
        mimo_rotation=mimo_rotation, q_bias=q_bias, k_bias=k_bias),
        key, _SCAN_FAILURES, "fused Mamba-3 chunked scan")
    _set_scan_flag(result is not None)
    return result


def reset_failures() -> None:
    """Forget the negative cache (the keys that failed before)."""
    _STEP_FAILURES.clear()
    _SCAN_FAILURES.clear()


__all__ = ["fused_step", "fused_chunk_scan", "bind", "disabled", "reset_failures", "DISABLE_ENV"]
