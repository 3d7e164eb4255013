"""ctypes binding of ``libmamba3_hip.so`` (declared in ``include/mamba3_hip.h``).

The library is loaded lazily, after ``torch`` (so it binds to the HIP runtime torch
already mapped). There is no fallback: a missing library, an ABI mismatch or a failing
call raises.
"""

from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmamba3_hip.so")
ABI_VERSION = 4

F32, BF16, F16 = 0, 1, 2
PHASE_NONE, PHASE_GIVEN, PHASE_ANGLES = 0, 1, 2
_DTYPE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported", 3: "launch failed",
          4: "workspace"}


class HipError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, name: str, code: int, message: str) -> None:
        super().__init__(f"{name}: {STATUS.get(code, code)}: {message}")
        self.code = code


class Tensor(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("dtype", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("stride", ctypes.c_int64 * 5)]


_T = Tensor


class ScanArgs(ctypes.Structure):
    _fields_ = [
        *[(n, ctypes.c_int32) for n in ("batch", "length", "heads", "groups", "rank", "d_state",
                                        "head_dim", "num_angles", "chunk", "act_dtype",
                                        "mimo_rotation", "raw_dt", "phase_mode", "segments")],
        ("norm_eps", ctypes.c_float),
        *[(n, _T) for n in ("q", "k", "q_norm_w", "k_norm_w", "q_bias", "k_bias", "value",
                            "gate", "dt", "a", "dt_bias", "trap", "phase", "initial_phase",
                            "D", "mimo_x", "mimo_z", "mimo_out", "initial_state", "initial_k",
                            "initial_value", "out", "final_state", "final_phase", "final_k",
                            "final_decay", "block_phase")],
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class ChunkStateArgs(ctypes.Structure):
    _fields_ = [
        *[(n, ctypes.c_int32) for n in ("batch", "width", "heads", "rank", "d_state",
                                        "head_dim", "act_dtype", "reserved")],
        *[(n, _T) for n in ("k", "value", "cumulative", "scale", "state_in", "state_out")],
    ]


class StepArgs(ctypes.Structure):
    _fields_ = [
        *[(n, ctypes.c_int32) for n in ("batch", "heads", "groups", "rank", "d_state",
                                        "head_dim", "num_angles", "act_dtype", "mimo_rotation",
                                        "raw_dt", "phase_mode")],
        ("norm_eps", ctypes.c_float),
        *[(n, _T) for n in ("q", "k", "q_norm_w", "k_norm_w", "q_bias", "k_bias", "value",
                            "gate", "dt", "a", "dt_bias", "trap", "angles", "D", "mimo_x",
                            "mimo_z", "mimo_out", "phase_in", "state_in", "prev_k",
                            "prev_value", "out", "phase_out", "state_out", "k_out",
                            "value_out")],
    ]


class LinearArgs(ctypes.Structure):
    _fields_ = [
        *[(n, ctypes.c_int64) for n in ("m", "n", "k")],
        ("dtype", ctypes.c_int32), ("norm_eps", ctypes.c_float),
        *[(n, _T) for n in ("x", "weight", "norm_weight", "residual", "out")],
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


class RmsNormArgs(ctypes.Structure):
    _fields_ = [
        *[(n, ctypes.c_int64) for n in ("rows", "dim")],
        ("eps", ctypes.c_float), ("reserved", ctypes.c_int32),
        *[(n, _T) for n in ("x", "add", "weight", "sum_out", "out")],
    ]


ENTRY_POINTS = ("m3_scan_fwd", "m3_scan_workspace_size", "m3_scan_segments", "m3_scan_fwd_noalloc",
                "m3_chunk_state", "m3_step", "m3_linear", "m3_linear_workspace_size",
                "m3_rms_norm", "m3_last_error", "m3_abi_version")
SCRATCH_BYTES = 64 << 20  # M3_SCRATCH_BYTES: the no-alloc scan's per-GPU scratch

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library once; raise if it is missing or its ABI differs."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m mamba3_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    for name in ("m3_scan_fwd", "m3_scan_fwd_noalloc", "m3_chunk_state", "m3_step", "m3_linear",
                 "m3_rms_norm"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    for name in ("m3_scan_workspace_size", "m3_linear_workspace_size"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
    lib.m3_scan_segments.restype = ctypes.c_int
    lib.m3_scan_segments.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
    lib.m3_last_error.restype = ctypes.c_char_p
    lib.m3_last_error.argtypes = []
    lib.m3_abi_version.restype = ctypes.c_int
    lib.m3_abi_version.argtypes = []
    version = lib.m3_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH}: ABI version {version}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def tensor(t: torch.Tensor | None) -> Tensor:
    """Describe a tensor (device pointer, dtype, element strides) for the C ABI."""
    out = Tensor()
    if t is None:
        return out
    if t.dim() > 5:
        raise ValueError("tensors passed to the HIP library have at most 5 dims")
    out.ptr = t.data_ptr() if t.numel() > 0 else None
    out.dtype = _DTYPE[t.dtype]
    for i, s in enumerate(t.stride()):
        out.stride[i] = s
    return out


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16")


def scan_workspace(args: ctypes.Structure, device: torch.device,
                   query: str = "m3_scan_workspace_size") -> torch.Tensor | None:
    """Allocate (through torch's caching allocator) the workspace an entry point needs, as
    its ``query`` function reports it, and record it in ``args``; the caller keeps the
    returned tensor alive across the call."""
    lib = load()
    nbytes = ctypes.c_size_t(0)
    rc = getattr(lib, query)(ctypes.byref(args), ctypes.byref(nbytes))
    if rc != 0:
        raise HipError(query, rc, lib.m3_last_error().decode(errors="replace"))
    if nbytes.value == 0:
        return None
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=device)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = nbytes.value
    return ws


def scan_segments(args: ctypes.Structure, concurrent: int) -> int:
    """The segment count the library picks for a scan call when ``concurrent`` calls of its
    shape share the GPU (``m3_scan_segments``)."""
    lib = load()
    g = ctypes.c_int(0)
    rc = lib.m3_scan_segments(ctypes.byref(args), concurrent, ctypes.byref(g))
    if rc != 0:
        raise HipError("m3_scan_segments", rc, lib.m3_last_error().decode(errors="replace"))
    return g.value


def call(name: str, args: ctypes.Structure, device: torch.device) -> None:
    """Invoke an entry point on ``device``'s current torch stream; raise on failure."""
    lib = load()
    stream = torch.cuda.current_stream(device).cuda_stream
    rc = getattr(lib, name)(ctypes.byref(args), ctypes.c_void_p(stream))
    if rc != 0:
        raise HipError(name, rc, lib.m3_last_error().decode(errors="replace"))
