"""``m3_scan_fwd_noalloc`` (the scan with the library's own per-GPU scratch, no workspace
argument) against ``m3_scan_fwd`` with a workspace, through the C ABI.

Same kernels on the same inputs, so the results must be identical bit for bit: two calls in a
row, the second smaller (the scratch keeps the first call's contents, which the second must not
depend on), in the model's projection form (bf16) and in FP32 rank 4, unsplit and split into
segments. The calls allocate no device memory.
"""

from __future__ import annotations

import ctypes
import gc

import pytest
import torch

from mamba3_amd import Mamba3, _hip, ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
_SET_UP: list[bool] = []  # whether this process made the library's first no-alloc call


def _noalloc(call: ops.ScanCall) -> None:
    args = type(call.args).from_buffer_copy(call.args)
    args.workspace = None
    args.workspace_bytes = 0
    _hip.call("m3_scan_fwd_noalloc", args, call.device)


def _outputs(call: ops.ScanCall):
    return [t.clone() for t in (call.out, call.final_state, call.final_phase, call.final_k)]


@pytest.mark.parametrize("case", [
    # (d_model, rank, dtype, [(batch, length), ...]): the second call is smaller
    (1024, 1, torch.bfloat16, [(4, 4096), (2, 700)]),
    (256, 4, torch.float32, [(3, 1000), (1, 130)]),
    (128, 1, torch.bfloat16, [(1, 4096), (1, 1024)]),  # split into segments
])
def test_noalloc_scan_equals_the_workspace_scan(case):
    d_model, rank, dtype, calls = case
    torch.manual_seed(d_model + rank)
    mixer = Mamba3(d_model, d_state=128, depth=1, mimo_rank=rank).eval().layers[0].mixer
    mixer = mixer.to(DEV)
    for batch, length in calls:
        x = torch.randn(batch, length, d_model, device=DEV)
        with torch.inference_mode():
            proj = mixer.in_proj(x).to(dtype)
            call = ops.ScanCall(proj, mixer, want_cache=True)
            call.launch()
            want = _outputs(call)
            if not _SET_UP:
                # the library's set-up on this device: its first call looks up the scratch
                # array, and the runtime maps the array (M3_SCRATCH_BYTES) then, once per
                # process; the calls measured below must allocate nothing at all
                _noalloc(call)
                torch.cuda.synchronize()
                _SET_UP.append(True)
            for t in (call.out, call.final_state, call.final_phase, call.final_k):
                t.fill_(float("nan"))
            torch.cuda.synchronize()
            # garbage of earlier tests collected now, not during the call: the count below then
            # moves only if the call allocates
            gc.collect()
            gc.disable()
            try:
                before = torch.cuda.memory_allocated(DEV)
                free_before = torch.cuda.mem_get_info(DEV)[0]
                _noalloc(call)
                torch.cuda.synchronize()
                after = torch.cuda.memory_allocated(DEV)
                free_after = torch.cuda.mem_get_info(DEV)[0]
            finally:
                gc.enable()
            # torch's allocator count, and the driver's free memory, which also sees a
            # hipMalloc made outside torch
            assert after == before
            assert free_after == free_before
            got = _outputs(call)
        print(f"noalloc d={d_model} R={rank} {dtype} B={batch} L={length}: workspace "
              f"{0 if call._keep[-1] is None else call._keep[-1].numel()} bytes", flush=True)
        for g, w in zip(got, want):
            assert torch.equal(g, w)
