"""Write the golden input/output vectors that pin the oracle to the reference.

Run in the build container only (the reference tree is not present on the GPU
box):

    PYTHONPATH=/root/reference python tests/golden/make_golden.py

It imports the reference package ``mamba3`` (jreoka/mamba3) from
``/root/reference`` and records, as small ``.npz`` files next to this script,
the outputs of the reference's *portable* CPU path for the compositions that no
closed form or invariant pins on its own:

* parameter creation order under ``torch.manual_seed`` (``model.py:109-145``,
  ``model.py:565-568``) -- stored as per-parameter checksums;
* the projection split, B/C RMSNorm, the pre-norm residual stack and
  ``norm_f`` (``model.py:147-199``, ``model.py:499-512``, ``model.py:585-591``);
* the prefill cache contents (``model.py:315-327``) and the decode step
  (``model.py:422-484``);
* the bidirectional blend (``model.py:330-362``);
* the bf16 rounding points of ``ops.mamba3_scan`` / ``ops.mamba3_step``
  (``ops.py:659-822``, ``ops.py:825-879``) on CPU bfloat16 tensors.

Every array is stored as float32 (bf16 values are exactly representable).
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = os.environ.get("MAMBA3_REFERENCE", "/root/reference")


def _import_reference():
    if REFERENCE not in sys.path:
        sys.path.insert(0, REFERENCE)
    import mamba3  # noqa: PLC0415
    import mamba3.ops as ops  # noqa: PLC0415

    return mamba3, ops


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).cpu().numpy()


def _param_checksums(model: torch.nn.Module) -> dict[str, np.ndarray]:
    out = {}
    names = []
    for name, p in model.named_parameters():
        v = p.detach().double()
        names.append(name)
        out[f"param/{name}"] = np.array(
            [v.sum().item(), v.square().sum().item(), *v.flatten()[:4].tolist()]
            + [0.0] * max(0, 4 - v.numel()),
            dtype=np.float64,
        )
        out[f"shape/{name}"] = np.array(tuple(p.shape), dtype=np.int64)
    out["param_order"] = np.array(names)
    return out


def _cache_arrays(prefix: str, cache) -> dict[str, np.ndarray]:
    out = {}
    for i, layer in enumerate(cache):
        for j, name in enumerate(("phase", "state", "k", "v")):
            out[f"{prefix}/{i}/{name}"] = _np(layer[j])
    return out


def make_model_case(mamba3, *, d_model, d_state, depth, rank, seed, batch, length,
                    split, autocast_bf16=False):
    torch.manual_seed(seed)
    model = mamba3.Mamba3(d_model, d_state=d_state, depth=depth, mimo_rank=rank).eval()
    x = torch.randn(batch, length, d_model)
    arrays = {"x": _np(x), **_param_checksums(model)}
    ctx = (
        torch.autocast("cpu", dtype=torch.bfloat16)
        if autocast_bf16
        else torch.autocast("cpu", enabled=False)
    )
    with torch.inference_mode(), ctx:
        arrays["forward"] = _np(model(x))
        prefix, cache = model.prefill(x[:, :split])
        arrays["prefill"] = _np(prefix)
        arrays.update(_cache_arrays("prefill_cache", cache))
        steps = []
        for index in range(split, length):
            out, cache = model.step(x[:, index : index + 1], cache)
            steps.append(out)
        arrays["steps"] = _np(torch.cat(steps, dim=1))
        arrays.update(_cache_arrays("final_cache", cache))
    return arrays


def make_config1(mamba3):
    """BASELINE config 1 (CPU reference run), stored as a summary."""
    torch.manual_seed(0)
    model = mamba3.Mamba3(256, d_state=128, depth=6, mimo_rank=1).eval()
    x = torch.randn(2, 1024, 256)
    arrays = {**_param_checksums(model)}
    with torch.inference_mode():
        full = model(x)
        prefix, cache = model.prefill(x[:, :960])
        steps = []
        for i in range(64):
            out, cache = model.step(x[:, 960 + i : 961 + i], cache)
            steps.append(out)
        steps = torch.cat(steps, dim=1)
    arrays["x_norms"] = _np(x.norm(dim=-1))
    arrays["forward_head"] = _np(full[:, :8])
    arrays["forward_tail"] = _np(full[:, -64:, :64])
    arrays["forward_norms"] = _np(full.norm(dim=-1))
    arrays["prefill_norms"] = _np(prefix.norm(dim=-1))
    arrays["steps"] = _np(steps[:, :, :64])
    arrays["steps_norms"] = _np(steps.norm(dim=-1))
    for i, layer in enumerate(cache):
        phase, state, k, v = layer
        arrays[f"final_cache/{i}/phase"] = _np(phase)
        arrays[f"final_cache/{i}/state_norms"] = _np(state.norm(dim=(-1, -2)))
        arrays[f"final_cache/{i}/state_slice"] = _np(state[:, :, :4, :16])
        arrays[f"final_cache/{i}/k"] = _np(k)
        arrays[f"final_cache/{i}/v"] = _np(v)
    return arrays


def make_bidir(mamba3, rank: int):
    torch.manual_seed(40 + rank)
    model = mamba3.Mamba3(16, d_state=8, depth=2, mimo_rank=rank, causal=False).eval()
    x = torch.randn(2, 12, 16)
    arrays = {"x": _np(x), **_param_checksums(model)}
    with torch.inference_mode():
        arrays["forward"] = _np(model(x))
    return arrays


def _hook_inputs(rank: int, dtype: torch.dtype, seed: int):
    g = torch.Generator().manual_seed(seed)
    batch, length, heads, head_dim, d_state = 2, 13, 3, 8, 16
    angles = d_state // 4 if rank > 1 else 3
    q = torch.randn(batch, length, 1, rank, d_state, generator=g)
    k = torch.randn(batch, length, 1, rank, d_state, generator=g)
    value = torch.randn(batch, length, heads, head_dim, generator=g)
    gate = torch.randn(batch, length, heads, head_dim, generator=g)
    adt = -torch.rand(batch, length, heads, generator=g) * 0.3
    dt = torch.rand(batch, length, heads, generator=g) * 0.1 + 0.001
    trap = torch.randn(batch, length, heads, generator=g)
    D = torch.randn(heads, generator=g)
    phase = (torch.rand(batch, length, heads, angles, generator=g) * 2 - 1) * 2 * math.pi
    q_bias = 1.0 + 0.1 * torch.randn(heads, rank, d_state, generator=g)
    k_bias = 1.0 + 0.1 * torch.randn(heads, rank, d_state, generator=g)
    init_state = torch.randn(batch, heads, head_dim, d_state, generator=g) * 0.5
    init_k = torch.randn(batch, heads, rank, d_state, generator=g)
    init_v = torch.randn(batch, heads, head_dim, generator=g)
    if rank > 1:
        mimo_x = torch.randn(heads, rank, head_dim, generator=g) / rank
        mimo_z = torch.randn(heads, rank, head_dim, generator=g)
        mimo_out = torch.randn(heads, rank, head_dim, generator=g) / rank
    else:
        mimo_x = mimo_z = mimo_out = None
    act = dict(q=q, k=k, value=value, gate=gate, trap=trap, init_k=init_k, init_v=init_v)
    act = {name: t.to(dtype) for name, t in act.items()}
    return dict(act, adt=adt, dt=dt, D=D, phase=phase, q_bias=q_bias, k_bias=k_bias,
                init_state=init_state, mimo_x=mimo_x, mimo_z=mimo_z, mimo_out=mimo_out)


def make_hook_scan(ops, rank: int, dtype: torch.dtype, chunk: int):
    inp = _hook_inputs(rank, dtype, seed=7 + rank)
    with torch.inference_mode():
        out, state = ops.mamba3_scan(
            inp["q"], inp["k"], inp["value"], inp["gate"], inp["adt"], inp["dt"],
            inp["trap"], inp["D"], mimo_x=inp["mimo_x"], mimo_z=inp["mimo_z"],
            mimo_out=inp["mimo_out"], chunk_size=chunk,
            initial_state=inp["init_state"], initial_k=inp["init_k"],
            initial_value=inp["init_v"], phase=inp["phase"], mimo_rotation=rank > 1,
            q_bias=inp["q_bias"], k_bias=inp["k_bias"],
        )
    arrays = {f"in/{n}": _np(t) for n, t in inp.items() if t is not None}
    arrays["chunk"] = np.array(chunk)
    arrays["out"] = _np(out)
    arrays["state"] = _np(state)
    return arrays


def make_hook_step(ops, rank: int, dtype: torch.dtype):
    inp = _hook_inputs(rank, dtype, seed=17 + rank)
    t = 5
    q = inp["q"][:, t].expand(-1, inp["value"].shape[2], -1, -1).contiguous()
    k = inp["k"][:, t].expand(-1, inp["value"].shape[2], -1, -1).contiguous()
    cache = (inp["phase"][:, 0], inp["init_state"], inp["init_k"], inp["init_v"])
    with torch.inference_mode():
        out, nxt = ops.mamba3_step(
            q, k, inp["value"][:, t], inp["gate"][:, t], inp["adt"][:, t], inp["dt"][:, t],
            inp["trap"][:, t], inp["D"], cache, mimo_x=inp["mimo_x"],
            mimo_z=inp["mimo_z"], mimo_out=inp["mimo_out"],
        )
    arrays = {
        "in/q": _np(q), "in/k": _np(k), "in/value": _np(inp["value"][:, t]),
        "in/gate": _np(inp["gate"][:, t]), "in/adt": _np(inp["adt"][:, t]),
        "in/dt": _np(inp["dt"][:, t]), "in/trap": _np(inp["trap"][:, t]),
        "in/D": _np(inp["D"]), "in/phase": _np(cache[0]), "in/state": _np(cache[1]),
        "in/prev_k": _np(cache[2]), "in/prev_v": _np(cache[3]),
    }
    for name in ("mimo_x", "mimo_z", "mimo_out"):
        if inp[name] is not None:
            arrays[f"in/{name}"] = _np(inp[name])
    arrays["out"] = _np(out)
    arrays["state"] = _np(nxt[1])
    return arrays


def make_phase(mamba3):
    torch.manual_seed(23)
    mixer = mamba3.Mamba3(16, d_state=16, depth=1).layers[0].mixer
    g = torch.Generator().manual_seed(29)
    length = 200
    angles = torch.randn(2, length, mixer.num_angles, generator=g) * 2.0
    dt = torch.rand(2, length, mixer.nheads, generator=g) * 3.0
    initial = (torch.rand(2, mixer.nheads, mixer.num_angles, generator=g) * 2 - 1) * 6.0
    with torch.inference_mode():
        phase0 = mixer._phase(angles, dt, None)
        phase1 = mixer._phase(angles, dt, initial)
    return {"angles": _np(angles), "dt": _np(dt), "initial": _np(initial),
            "phase_none": _np(phase0), "phase_init": _np(phase1)}


def make_rotate(ops):
    g = torch.Generator().manual_seed(31)
    arrays = {}
    for mimo, width in ((False, 3), (True, 4)):
        q = torch.randn(2, 5, 3, 2, 16, generator=g)
        k = torch.randn(2, 5, 3, 2, 16, generator=g)
        phase = (torch.rand(2, 5, 3, width, generator=g) * 2 - 1) * 2 * math.pi
        tag = "mimo" if mimo else "siso"
        arrays[f"{tag}/q"] = _np(q)
        arrays[f"{tag}/k"] = _np(k)
        arrays[f"{tag}/phase"] = _np(phase)
        for dname, dtype in (("f32", torch.float32), ("bf16", torch.bfloat16)):
            rq, rk = ops.rotate_qk(q.to(dtype), k.to(dtype), phase, mimo=mimo)
            arrays[f"{tag}/{dname}/q"] = _np(rq)
            arrays[f"{tag}/{dname}/k"] = _np(rk)
    return arrays


def main() -> None:
    mamba3, ops = _import_reference()
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    os.environ.pop("MAMBA3_CHUNK_SIZE", None)
    files = {}
    for rank in (1, 4):
        files[f"model_r{rank}_f32.npz"] = make_model_case(
            mamba3, d_model=64, d_state=16, depth=2, rank=rank, seed=100 + rank,
            batch=2, length=37, split=9)
        files[f"model_r{rank}_bf16.npz"] = make_model_case(
            mamba3, d_model=64, d_state=16, depth=2, rank=rank, seed=100 + rank,
            batch=2, length=37, split=9, autocast_bf16=True)
        files[f"bidir_r{rank}.npz"] = make_bidir(mamba3, rank)
        for dname, dtype in (("f32", torch.float32), ("bf16", torch.bfloat16)):
            files[f"scan_r{rank}_{dname}.npz"] = make_hook_scan(ops, rank, dtype, chunk=5)
            files[f"step_r{rank}_{dname}.npz"] = make_hook_step(ops, rank, dtype)
    files["phase.npz"] = make_phase(mamba3)
    files["rotate.npz"] = make_rotate(ops)
    files["config1.npz"] = make_config1(mamba3)
    for name, arrays in files.items():
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **arrays)
        print(f"wrote {name}: {os.path.getsize(path) / 1024:.1f} KiB")


if __name__ == "__main__":
    main()
