"""The C ABI without a GPU: exports, struct layout against the header, host-side checks."""

from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess

import pytest
import torch  # noqa: F401  (load order: torch before the HIP library)

from conftest import ROOT
from mamba3_amd import _hip

HEADER = os.path.join(ROOT, "include", "mamba3_hip.h")


def _declared_functions() -> list[str]:
    text = open(HEADER).read()
    return re.findall(r"^(?:int|const char\*)\s+(m3_\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_hip.LIB_PATH):
        pytest.skip("libmamba3_hip.so is not built (run __graft_entry__.build())")
    return _hip.load()


def test_header_declares_the_expected_entry_points():
    assert sorted(_declared_functions()) == sorted(_hip.ENTRY_POINTS)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.m3_abi_version() == _hip.ABI_VERSION
    assert lib.m3_last_error() == b""


def _c_layout() -> dict[str, tuple[int, dict[str, int]]]:
    """sizeof / offsetof of every struct field, from the header compiled with gcc."""
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    structs = {"m3_tensor": _hip.Tensor, "m3_scan_args": _hip.ScanArgs,
               "m3_step_args": _hip.StepArgs, "m3_chunk_state_args": _hip.ChunkStateArgs,
               "m3_linear_args": _hip.LinearArgs, "m3_rms_norm_args": _hip.RmsNormArgs}
    lines = ['#include "mamba3_hip.h"', "#include <stdio.h>", "#include <stddef.h>",
             "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["return 0;", "}"]
    tmp = os.path.join(os.environ.get("TMPDIR", "/tmp"), f"m3_layout_{os.getpid()}")
    with open(tmp + ".c", "w") as f:
        f.write("\n".join(lines))
    inc = ["-I/opt/rocm/include", f"-I{os.path.join(ROOT, 'include')}"]
    subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", *inc, tmp + ".c", "-o", tmp], check=True)
    out = subprocess.run([tmp], check=True, capture_output=True, text=True).stdout
    os.remove(tmp)
    os.remove(tmp + ".c")
    layout: dict[str, tuple[int, dict[str, int]]] = {}
    for line in out.splitlines():
        cname, field, value = line.split()
        size, fields = layout.get(cname, (0, {}))
        if field == "sizeof":
            size = int(value)
        else:
            fields[field] = int(value)
        layout[cname] = (size, fields)
    return layout


def test_ctypes_structs_match_the_header_layout():
    layout = _c_layout()
    for cname, py in (("m3_tensor", _hip.Tensor), ("m3_scan_args", _hip.ScanArgs),
                      ("m3_step_args", _hip.StepArgs),
                      ("m3_chunk_state_args", _hip.ChunkStateArgs),
                      ("m3_linear_args", _hip.LinearArgs),
                      ("m3_rms_norm_args", _hip.RmsNormArgs)):
        size, fields = layout[cname]
        assert ctypes.sizeof(py) == size, cname
        for field, _ in py._fields_:
            assert getattr(py, field).offset == fields[field], (cname, field)


def test_null_arguments_are_rejected_without_touching_the_device(lib):
    for name in ("m3_scan_fwd", "m3_step", "m3_chunk_state", "m3_linear", "m3_rms_norm"):
        rc = getattr(lib, name)(None, None)
        assert rc == 1, name
        assert b"NULL" in lib.m3_last_error()


def test_scan_validation_on_the_host(lib):
    args = _hip.ScanArgs(batch=1, length=4, heads=2, groups=1, rank=1, d_state=2,
                         head_dim=8, num_angles=1)
    rc = lib.m3_scan_fwd(ctypes.byref(args), None)
    assert rc == 2 and b"d_state 2 < 4" in lib.m3_last_error()
    args.d_state = 12  # not a power of 2: the recurrent scan, which checks the same tensors
    rc = lib.m3_scan_fwd(ctypes.byref(args), None)
    assert rc == 1 and b"q: required tensor is NULL" in lib.m3_last_error()
    args.d_state = 16
    rc = lib.m3_scan_fwd(ctypes.byref(args), None)
    assert rc == 1 and b"q: required tensor is NULL" in lib.m3_last_error()
    args.heads, args.groups = 3, 2
    assert lib.m3_scan_fwd(ctypes.byref(args), None) == 1
    assert b"heads % groups" in lib.m3_last_error()


def test_step_validation_on_the_host(lib):
    args = _hip.StepArgs(batch=1, heads=2, groups=1, rank=3, d_state=16, head_dim=8,
                         num_angles=4, phase_mode=_hip.PHASE_ANGLES, mimo_rotation=1)
    # rank 3 runs as a one-token recurrent scan; the angle count check comes first for MIMO
    args.num_angles = 3
    assert lib.m3_step(ctypes.byref(args), None) == 2
    assert b"num_angles" in lib.m3_last_error()
    args.num_angles = 4
    assert lib.m3_step(ctypes.byref(args), None) == 1
    assert b"required tensor is NULL" in lib.m3_last_error()


def test_tensor_descriptor_records_pointer_dtype_and_strides():
    t = torch.zeros(2, 3, 4, dtype=torch.bfloat16)[:, 1:, ::2]
    d = _hip.tensor(t)
    assert d.ptr == t.data_ptr()
    assert d.dtype == _hip.BF16
    assert list(d.stride)[:3] == list(t.stride())
    assert list(d.stride)[3:] == [0, 0]
    assert _hip.tensor(None).ptr is None


def _linear_args(m: int, n: int, k: int) -> _hip.LinearArgs:
    """Argument block with fake, aligned device pointers: only host checks run on it."""
    args = _hip.LinearArgs(m=m, n=n, k=k, dtype=_hip.BF16)
    for name, (rows, cols, ptr) in {"x": (m, k, 0x10000), "weight": (n, k, 0x20000),
                                    "out": (m, n, 0x30000)}.items():
        t = getattr(args, name)
        t.ptr, t.dtype = ptr, _hip.BF16
        t.stride[0], t.stride[1] = cols, 1
    return args


def test_linear_validation_and_workspace_on_the_host(lib):
    size = ctypes.c_size_t(0)
    # one row against 512 x 4064 (K not a multiple of 512: the rows kernel): 32 column
    # workgroups, K split in two -> two FP32 partials
    args = _linear_args(1, 512, 4064)
    assert lib.m3_linear_workspace_size(ctypes.byref(args), ctypes.byref(size)) == 0
    assert size.value == 2 * 1 * 512 * 4
    # ... unless the RMSNorm is fused in, which keeps K whole in one workgroup
    args.norm_weight.ptr, args.norm_weight.dtype, args.norm_eps = 0x40000, _hip.BF16, 1e-5
    args.norm_weight.stride[0] = 1
    assert lib.m3_linear_workspace_size(ctypes.byref(args), ctypes.byref(size)) == 0
    assert size.value == 0
    # the decode shapes run unsplit: the gemv kernel up to 4 rows and the wide kernel up to 32
    # (K a multiple of 512 up to 4096), 2 x 136 tiles of 256 rows
    for m, n, k in ((1, 8672, 2048), (4, 512, 4096), (16, 2048, 4096), (256, 8672, 2048)):
        args = _linear_args(m, n, k)
        assert lib.m3_linear_workspace_size(ctypes.byref(args), ctypes.byref(size)) == 0
        assert size.value == 0
    # a split call without its workspace is refused before any launch
    args = _linear_args(1, 512, 4064)
    assert lib.m3_linear(ctypes.byref(args), None) == 4
    assert b"workspace" in lib.m3_last_error()
    # the fused norm: up to 64 rows with K a multiple of 256, else up to 32
    for m, k, code in ((64, 2048, 0), (65, 2048, 2), (33, 2080, 2), (32, 2080, 0)):
        args = _linear_args(m, 64, k)
        args.norm_weight.ptr, args.norm_weight.dtype = 0x40000, _hip.BF16
        args.norm_weight.stride[0] = 1
        assert lib.m3_linear_workspace_size(ctypes.byref(args), ctypes.byref(size)) == code, (m, k)
        if code:
            assert b"M <= 32" in lib.m3_last_error()
    for field, value, code, text in (("m", 257, 2, b"M = 257"), ("k", 2040, 2, b"K % 32"),
                                     ("dtype", _hip.F32, 2, b"dtype")):
        args = _linear_args(4, 64, 2048)
        setattr(args, field, value)
        assert lib.m3_linear_workspace_size(ctypes.byref(args), ctypes.byref(size)) == code
        assert text in lib.m3_last_error(), field
    args = _linear_args(4, 64, 2048)
    args.x.ptr = 0x10008  # 8-byte aligned rows
    assert lib.m3_linear_workspace_size(ctypes.byref(args), ctypes.byref(size)) == 2
    assert b"16-byte aligned" in lib.m3_last_error()
    args = _linear_args(4, 64, 2048)
    args.out.stride[0] = 32  # rows of out overlap
    assert lib.m3_linear_workspace_size(ctypes.byref(args), ctypes.byref(size)) == 1
    args = _linear_args(4, 64, 2048)
    args.weight.ptr = None
    assert lib.m3_linear_workspace_size(ctypes.byref(args), ctypes.byref(size)) == 1
    assert b"weight: required tensor is NULL" in lib.m3_last_error()


def _hook_scan_args(batch: int, length: int, heads: int, segments: int) -> _hip.ScanArgs:
    """A hook-form scan (no phase) over contiguous tensors at fake, aligned device pointers:
    host-side checks and the workspace query only."""
    n, p = 64, 64
    args = _hip.ScanArgs(batch=batch, length=length, heads=heads, groups=1, rank=1, d_state=n,
                         head_dim=p, num_angles=0, chunk=64, act_dtype=_hip.BF16,
                         phase_mode=_hip.PHASE_NONE, segments=segments)
    shapes = {"q": (length, 1, 1, n), "k": (length, 1, 1, n), "value": (length, heads, p),
              "gate": (length, heads, p), "dt": (length, heads), "a": (length, heads),
              "trap": (length, heads), "out": (length, heads, p), "final_state": (heads, p, n),
              "D": ()}
    ptr = 0x100000
    for name, dims in shapes.items():
        t = getattr(args, name)
        t.ptr, t.dtype = ptr, (_hip.F32 if name in ("final_state", "D") else _hip.BF16)
        ptr += 1 << 28
        full = (batch, *dims) if name != "D" else (heads,)
        stride = 1
        for i in range(len(full) - 1, -1, -1):
            t.stride[i] = stride
            stride *= full[i]
    return args


def test_scan_split_decision_on_the_host(lib):
    size = ctypes.c_size_t(0)

    def ws(batch, length, heads, segments):
        args = _hook_scan_args(batch, length, heads, segments)
        assert lib.m3_scan_workspace_size(ctypes.byref(args), ctypes.byref(size)) == 0
        return size.value

    # 4 (batch, head) pairs over 4096 tokens: split (the workspace gains the segment buffers)
    assert ws(1, 4096, 4, 0) > ws(1, 4096, 4, 1)
    assert ws(1, 4096, 4, 8) > ws(1, 4096, 4, 1)
    # 256 pairs fill the GPU; 512 tokens are too short to split: one pass each
    assert ws(8, 4096, 32, 0) == ws(8, 4096, 32, 1)
    assert ws(1, 512, 4, 0) == ws(1, 512, 4, 1)
    # an explicit split that does not divide the sequence is refused before any launch
    args = _hook_scan_args(1, 4096, 4, 3)
    assert lib.m3_scan_fwd(ctypes.byref(args), None) == 2
    assert b"segments" in lib.m3_last_error()


def test_scan_segment_choice_on_the_host(lib):
    """The automatic split minimises the estimated rounds of workgroups over the 256 CUs: 24
    (b, h) pairs over 65,536 tokens alone take 32 segments (768 workgroups, three full rounds),
    two such calls together 16 each; 256 pairs fill the GPU unsplit; an explicit request is
    checked, not replaced."""
    g = ctypes.c_int(0)

    def segs(batch, length, heads, segments=0, concurrent=1):
        args = _hook_scan_args(batch, length, heads, segments)
        assert lib.m3_scan_segments(ctypes.byref(args), concurrent, ctypes.byref(g)) == 0
        return g.value

    assert segs(1, 65536, 24) == 32
    assert segs(1, 65536, 24, concurrent=2) == 16
    assert segs(8, 4096, 32) == 1
    assert segs(1, 4096, 4) == 8
    assert segs(1, 512, 4) == 1
    assert segs(1, 65536, 24, segments=8, concurrent=2) == 8
    args = _hook_scan_args(1, 4096, 4, 3)
    assert lib.m3_scan_segments(ctypes.byref(args), 1, ctypes.byref(g)) == 2
    assert b"segments" in lib.m3_last_error()
    assert lib.m3_scan_segments(ctypes.byref(args), 0, ctypes.byref(g)) == 1


def test_scan_backwards_token_strides_on_the_host(lib):
    """Per-token tensors may run backwards (the reverse scan), but all of them together."""
    args = _hook_scan_args(1, 128, 2, 1)
    args.value.stride[1] = -args.value.stride[1]
    assert lib.m3_scan_fwd(ctypes.byref(args), None) == 1
    assert b"run the same way" in lib.m3_last_error()


def _norm_args(rows: int, dim: int, x_dtype=_hip.F32, out_dtype=_hip.BF16) -> _hip.RmsNormArgs:
    """m3_rms_norm arguments with fake, aligned device pointers: only host checks run on them."""
    args = _hip.RmsNormArgs(rows=rows, dim=dim, eps=1e-5)
    for name, ptr, dt in (("x", 0x100000, x_dtype), ("weight", 0x200000, _hip.F32),
                          ("out", 0x300000, out_dtype)):
        t = getattr(args, name)
        t.ptr, t.dtype = ptr, dt
        t.stride[0], t.stride[1] = (dim, 1) if name != "weight" else (1, 0)
    return args


def test_rms_norm_validation_on_the_host(lib):
    args = _norm_args(0, 1024)
    assert lib.m3_rms_norm(ctypes.byref(args), None) == 0  # no rows: nothing to launch
    args = _norm_args(8, 384)
    assert lib.m3_rms_norm(ctypes.byref(args), None) == 2
    assert b"multiple of 256" in lib.m3_last_error()
    args = _norm_args(8, 1024)
    args.sum_out.ptr, args.sum_out.dtype = 0x400000, _hip.F32
    args.sum_out.stride[0], args.sum_out.stride[1] = 1024, 1
    assert lib.m3_rms_norm(ctypes.byref(args), None) == 1
    assert b"sum_out needs add" in lib.m3_last_error()
    args = _norm_args(8, 1024)
    args.out.ptr = 0x100000 + 4 * 1024  # inside x's rows
    assert lib.m3_rms_norm(ctypes.byref(args), None) == 1
    assert b"overlaps" in lib.m3_last_error()
    args = _norm_args(8, 1024, x_dtype=_hip.BF16, out_dtype=_hip.F32)
    assert lib.m3_rms_norm(ctypes.byref(args), None) == 2
    assert b"own dtype" in lib.m3_last_error()
    args = _norm_args(8, 1024)
    args.x.stride[0] = 1026  # rows not 4-element aligned
    assert lib.m3_rms_norm(ctypes.byref(args), None) == 2
    assert b"aligned" in lib.m3_last_error()


def test_noalloc_scan_rejects_calls_beyond_its_scratch(lib):
    """m3_scan_fwd_noalloc refuses a call whose workspace would exceed M3_SCRATCH_BYTES before
    touching the device (the size check needs only the dimensions and which inputs are set)."""
    args = _hip.ScanArgs(batch=64, length=65536, heads=32, groups=1, rank=1, d_state=128,
                         head_dim=64, num_angles=32, chunk=256, act_dtype=_hip.BF16,
                         mimo_rotation=0, raw_dt=1, phase_mode=_hip.PHASE_ANGLES, norm_eps=1e-5,
                         segments=1)
    args.q_norm_w.ptr = args.k_norm_w.ptr = 256  # set, never dereferenced by the size query
    need = ctypes.c_size_t(0)
    assert lib.m3_scan_workspace_size(ctypes.byref(args), ctypes.byref(need)) == 0
    assert need.value > _hip.SCRATCH_BYTES
    rc = lib.m3_scan_fwd_noalloc(ctypes.byref(args), None)
    assert rc == 4  # M3_EWORKSPACE
    assert b"scratch" in lib.m3_last_error()
    assert lib.m3_scan_fwd_noalloc(None, None) == 1


def test_recurrent_shapes_need_no_workspace(lib):
    """Shapes the MFMA scan does not tile take the recurrent scan, which needs no workspace and
    cannot be split into segments; d_state below 4 is refused."""
    def args(**kw):
        base = dict(batch=2, length=100, heads=2, groups=1, rank=1, d_state=96, head_dim=32,
                    num_angles=24, chunk=64, act_dtype=_hip.BF16, mimo_rotation=0, raw_dt=0,
                    phase_mode=_hip.PHASE_GIVEN, norm_eps=1e-5, segments=0)
        base.update(kw)
        return _hip.ScanArgs(**base)
    need = ctypes.c_size_t(123)
    assert lib.m3_scan_workspace_size(ctypes.byref(args()), ctypes.byref(need)) == 0
    assert need.value == 0
    assert lib.m3_scan_workspace_size(ctypes.byref(args(d_state=128, num_angles=32, head_dim=64)),
                                      ctypes.byref(need)) == 0
    assert need.value > 0
    assert lib.m3_scan_fwd(ctypes.byref(args(segments=4)), None) == 2
    assert b"segments" in lib.m3_last_error()
    assert lib.m3_scan_fwd(ctypes.byref(args(d_state=2, num_angles=0)), None) == 2
    # any rank: rank 9 passes the shape checks (and stops at the missing tensors); a per-token
    # footprint beyond 160 KiB of LDS (7 x 64 x 96 floats of q / k rows alone) is refused
    assert lib.m3_scan_fwd(ctypes.byref(args(rank=9, mimo_rotation=1)), None) == 1
    assert b"required tensor is NULL" in lib.m3_last_error()
    assert lib.m3_scan_fwd(ctypes.byref(args(rank=64, mimo_rotation=1)), None) == 2
    assert b"160 KiB" in lib.m3_last_error()

