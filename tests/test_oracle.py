"""Pin the CPU oracle (``oracle/``) before trusting it as the parity checker.

Each check is chosen so that a plausible slip in the oracle (a dropped term, a
swapped sign or index, a transposed operand, a missed rounding point) fails at
least one of them: closed forms, an independent float64 recurrence, invariants,
and golden vectors written from the reference by ``tests/golden/make_golden.py``.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import golden
from oracle import portable as op
from oracle.recurrence import recurrent_scan


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.asarray(a)).to(dtype)


# --------------------------------------------------------------------------- closed forms


def test_heavy_tail_closed_form_and_gradient():
    """Reference tests/test_scan.py:145-152."""
    x = torch.tensor([-3.0, -0.5, 0.0, 0.5, 3.0], requires_grad=True)
    want = torch.where(x >= 0, 1.0 + x, 1.0 / (1.0 - x))
    got = op.heavy_tail(x)
    torch.testing.assert_close(got, want)
    got.sum().backward()
    torch.testing.assert_close(x.grad, torch.where(x >= 0, torch.ones_like(x), want.square()))


def test_rotation_known_answers():
    """Reference tests/test_scan.py:155-168."""
    q = torch.tensor([[[[[1.0, 0.0, 2.0, 0.0, 5.0, 6.0, 7.0, 8.0]]]]])
    phase = torch.tensor([[[[math.pi / 2, 0.0]]]])
    got, _ = op.rotate(q, q, phase, mimo=False)
    want = torch.tensor([[[[[0.0, 1.0, 2.0, 0.0, 5.0, 6.0, 7.0, 8.0]]]]])
    torch.testing.assert_close(got, want, atol=1e-6, rtol=0)
    q = torch.tensor([[[[[1.0, 2.0, 3.0, 4.0, 0.0, 5.0, 6.0, 7.0]]]]])
    got, _ = op.rotate(q, q, phase, mimo=True)
    want = torch.tensor([[[[[0.0, 2.0, 3.0, 4.0, 1.0, 5.0, 6.0, 7.0]]]]])
    torch.testing.assert_close(got, want, atol=1e-6, rtol=0)


@pytest.mark.parametrize("mimo", [False, True])
def test_rotation_matrix_closed_form_and_norm(mimo):
    g = torch.Generator().manual_seed(3)
    n, s = 16, 4
    q = torch.randn(2, 3, 2, 1, n, generator=g, dtype=torch.float64)
    phase = torch.rand(2, 3, 2, s, generator=g, dtype=torch.float64) * 12 - 6
    got, _ = op.rotate(q, q, phase, mimo=mimo)
    want = q.clone()
    for i in range(s):
        a, b = (i, 2 * s + i) if mimo else (2 * i, 2 * i + 1)
        c, sn = torch.cos(phase[..., i]), torch.sin(phase[..., i])
        want[..., 0, a] = c * q[..., 0, a] - sn * q[..., 0, b]
        want[..., 0, b] = sn * q[..., 0, a] + c * q[..., 0, b]
    torch.testing.assert_close(got, want)
    torch.testing.assert_close(got.norm(dim=-1), q.norm(dim=-1))


def test_rotation_golden_f32_and_bf16():
    data = golden("rotate.npz")
    for tag, mimo in (("siso", False), ("mimo", True)):
        phase = _t(data[f"{tag}/phase"])
        for dname, dtype in (("f32", torch.float32), ("bf16", torch.bfloat16)):
            q = _t(data[f"{tag}/q"]).to(dtype)
            k = _t(data[f"{tag}/k"]).to(dtype)
            rq, rk = op.rotate(q, k, phase, mimo=mimo)
            torch.testing.assert_close(rq.float(), _t(data[f"{tag}/{dname}/q"]), rtol=0, atol=0)
            torch.testing.assert_close(rk.float(), _t(data[f"{tag}/{dname}/k"]), rtol=0, atol=0)


# --------------------------------------------------------------------------- phase


def test_phase_matches_sequential_fmod_recurrence():
    """Reference tests/test_model.py:225-250 (bounded per-block accumulation)."""
    length, heads, count = 2048, 2, 2
    angles = torch.full((1, length, count), 3.0)
    dt = torch.full((1, length, heads), 100.0)
    phase = op.phase_scan(angles, dt)
    inc = torch.fmod(math.pi * torch.tanh(angles[:, 0]).unsqueeze(1) * dt[:, 0].unsqueeze(-1),
                     2 * math.pi)
    state = torch.zeros_like(phase[:, 0])
    want = []
    for _ in range(length):
        state = torch.fmod(state + inc, 2 * math.pi)
        want.append(state)
    want = torch.stack(want, dim=1)
    circ = torch.remainder(phase - want + math.pi, 2 * math.pi) - math.pi
    assert circ.abs().max() < 2e-3
    assert phase.abs().max() < 2 * math.pi


def test_phase_constant_negative_increment_closed_form():
    """Reference tests/test_model.py:252-273, on the CPU."""
    length, heads, count = 131_072, 1, 2
    raw = math.atanh(-1e-4 / math.pi)
    angles = torch.full((1, length, count), raw)
    dt = torch.ones(1, length, heads)
    phase = op.phase_scan(angles, dt)
    pos = torch.arange(1, length + 1, dtype=torch.float64)
    want = torch.remainder(pos * (math.pi * math.tanh(raw)), 2 * math.pi).float()
    circ = torch.remainder(phase - want[None, :, None, None] + math.pi, 2 * math.pi) - math.pi
    assert circ.abs().max() < 2e-3


def test_phase_golden():
    data = golden("phase.npz")
    angles, dt, init = _t(data["angles"]), _t(data["dt"]), _t(data["initial"])
    torch.testing.assert_close(op.phase_scan(angles, dt), _t(data["phase_none"]), rtol=0, atol=0)
    torch.testing.assert_close(op.phase_scan(angles, dt, init), _t(data["phase_init"]),
                               rtol=0, atol=0)


# --------------------------------------------------------------------------- scan vs recurrence


def _scan_inputs(rank, *, seed, batch=2, length=7, heads=3, head_dim=4, d_state=8,
                 extras=False):
    """Shapes and ranges of the reference helper tests/test_scan.py:101-124."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, length, heads, rank, d_state, generator=g)
    k = torch.randn(batch, length, heads, rank, d_state, generator=g)
    v = torch.randn(batch, length, heads, head_dim, generator=g)
    z = torch.randn(batch, length, heads, head_dim, generator=g)
    adt = -torch.rand(batch, length, heads, generator=g) * 0.2
    dt = torch.rand(batch, length, heads, generator=g) * 0.1 + 0.001
    lam = torch.randn(batch, length, heads, generator=g)
    D = torch.randn(heads, generator=g)
    mx = mz = mo = None
    if rank > 1:
        mx = torch.randn(heads, rank, head_dim, generator=g) / rank
        mz = torch.randn(heads, rank, head_dim, generator=g)
        mo = torch.randn(heads, rank, head_dim, generator=g) / rank
    inp = dict(q=q, k=k, value=v, gate=z, adt=adt, dt=dt, trap_logits=lam, D=D, mimo_x=mx,
               mimo_z=mz, mimo_out=mo)
    if extras:
        inp["initial_state"] = torch.randn(batch, heads, head_dim, d_state, generator=g)
        inp["initial_k"] = torch.randn(batch, heads, rank, d_state, generator=g)
        inp["initial_value"] = torch.randn(batch, heads, head_dim, generator=g)
    return inp


def _oracle_scan(inp, chunk, **kw):
    a = dict(inp)
    return op.ssd_scan(a.pop("q"), a.pop("k"), a.pop("value"), a.pop("gate"), a.pop("adt"),
                       a.pop("dt"), a.pop("trap_logits"), a.pop("D"), chunk_size=chunk, **a, **kw)


def _recurrence(inp, q=None, k=None):
    return recurrent_scan(
        (inp["q"] if q is None else q).numpy(), (inp["k"] if k is None else k).numpy(),
        inp["value"].numpy(), inp["gate"].numpy(), inp["adt"].numpy(), inp["dt"].numpy(),
        inp["trap_logits"].numpy(), inp["D"].numpy(),
        mimo_x=None if inp["mimo_x"] is None else inp["mimo_x"].numpy(),
        mimo_z=None if inp["mimo_z"] is None else inp["mimo_z"].numpy(),
        mimo_out=None if inp["mimo_out"] is None else inp["mimo_out"].numpy(),
        state0=None if "initial_state" not in inp else inp["initial_state"].numpy(),
        k0=None if "initial_k" not in inp else inp["initial_k"].numpy(),
        v0=None if "initial_value" not in inp else inp["initial_value"].numpy())


@pytest.mark.parametrize("rank,chunk", [(1, 3), (4, 2), (4, 5), (1, 1), (2, 7), (1, 64)])
@pytest.mark.parametrize("extras", [False, True])
def test_chunked_scan_matches_float64_recurrence(rank, chunk, extras):
    """Reference tests/test_scan.py:171-192 (plus an initial state / endpoint)."""
    inp = _scan_inputs(rank, seed=42 + rank, extras=extras)
    y, s = _oracle_scan(inp, chunk)
    y_ref, s_ref = _recurrence(inp)
    np.testing.assert_allclose(y.numpy(), y_ref, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(s.numpy(), s_ref, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("rank", [1, 4])
def test_chunked_scan_with_bias_and_phase_matches_recurrence(rank):
    """Bias and rotation are per-token: applying them outside must agree."""
    inp = _scan_inputs(rank, seed=5, length=11, d_state=16)
    g = torch.Generator().manual_seed(9)
    s = 4 if rank > 1 else 3
    phase = torch.rand(2, 11, 3, s, generator=g) * 12 - 6
    qb = 1 + 0.1 * torch.randn(3, rank, 16, generator=g)
    kb = 1 + 0.1 * torch.randn(3, rank, 16, generator=g)
    y, st = _oracle_scan(inp, 4, phase=phase, mimo_rotation=rank > 1, q_bias=qb, k_bias=kb)
    rq, rk = op.rotate(inp["q"] + qb, inp["k"] + kb, phase, mimo=rank > 1)
    y_ref, s_ref = _recurrence(inp, rq, rk)
    np.testing.assert_allclose(y.numpy(), y_ref, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(st.numpy(), s_ref, rtol=2e-5, atol=2e-6)


def test_recurrence_reduces_to_decayed_linear_attention():
    """trap -> +inf gives beta = 0, gamma = dt: a Mamba-2 style decayed attention.

    y_t = silu(z_t) * (sum_{s<=t} exp(sum_{u=s+1..t} adt_u) dt_s (q_t . k_s) v_s + D v_t)
    """
    inp = _scan_inputs(1, seed=77, length=9)
    inp["trap_logits"] = torch.full_like(inp["trap_logits"], 60.0)
    y_ref, _ = _recurrence(inp)
    q = inp["q"].double()[:, :, :, 0]
    k = inp["k"].double()[:, :, :, 0]
    v, z = inp["value"].double(), inp["gate"].double()
    adt, dt, D = inp["adt"].double(), inp["dt"].double(), inp["D"].double()
    cum = torch.cumsum(adt, dim=1)
    want = torch.zeros_like(v)
    for t in range(v.shape[1]):
        for s_ in range(t + 1):
            w = torch.exp(cum[:, t] - cum[:, s_]) * dt[:, s_] * (q[:, t] * k[:, s_]).sum(-1)
            want[:, t] += w[..., None] * v[:, s_]
    want = (want + D[None, None, :, None] * v) * torch.nn.functional.silu(z)
    np.testing.assert_allclose(y_ref, want.numpy(), rtol=1e-10, atol=1e-12)
    y, _ = _oracle_scan(inp, 4)
    np.testing.assert_allclose(y.numpy(), want.numpy(), rtol=2e-5, atol=2e-6)


def test_recurrence_reduces_to_trapezoidal_linear_attention():
    """adt = 0 (alpha = 1): the state is a plain trapezoidal running sum.

    S_t = sum_{s<=t} (gamma_s + beta_{s+1}) U_s with beta_{t+1} excluded at s = t.
    """
    inp = _scan_inputs(1, seed=78, length=8)
    inp["adt"] = torch.zeros_like(inp["adt"])
    _, s_ref = _recurrence(inp)
    dt = inp["dt"].double()
    trap = torch.sigmoid(inp["trap_logits"].double())
    gamma, beta = trap * dt, (1 - trap) * dt
    k = inp["k"].double()[:, :, :, 0]
    v = inp["value"].double()
    length = v.shape[1]
    want = torch.zeros(2, 3, 4, 8, dtype=torch.float64)
    for s_ in range(length):
        w = gamma[:, s_] + (beta[:, s_ + 1] if s_ + 1 < length else 0.0)
        want += w[..., None, None] * v[:, s_][..., :, None] * k[:, s_][..., None, :]
    np.testing.assert_allclose(s_ref, want.numpy(), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("rank", [1, 4])
def test_scan_chunk_size_invariance(rank):
    inp = _scan_inputs(rank, seed=3, length=23, extras=True)
    y1, s1 = _oracle_scan(inp, 1)
    for chunk in (2, 5, 8, 23, 64):
        y, s = _oracle_scan(inp, chunk)
        torch.testing.assert_close(y, y1, rtol=2e-5, atol=2e-6)
        torch.testing.assert_close(s, s1, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("rank", [1, 4])
def test_scan_continuation(rank):
    """Reference tests/test_scan.py:228-258."""
    inp = _scan_inputs(rank, seed=42 + rank)
    full, full_state = _oracle_scan(inp, 3)
    split = 4
    seq = ("q", "k", "value", "gate", "adt", "dt", "trap_logits")
    first = {n: (t[:, :split] if n in seq else t) for n, t in inp.items()}
    second = {n: (t[:, split:] if n in seq else t) for n, t in inp.items()}
    y1, s1 = _oracle_scan(first, 3)
    second.update(initial_state=s1, initial_k=inp["k"][:, split - 1],
                  initial_value=inp["value"][:, split - 1])
    y2, s2 = _oracle_scan(second, 3)
    torch.testing.assert_close(torch.cat((y1, y2), dim=1), full, rtol=2e-5, atol=2e-6)
    torch.testing.assert_close(s2, full_state, rtol=2e-5, atol=2e-6)


def test_empty_scan_preserves_state():
    """Reference tests/test_scan.py:261-282."""
    q = torch.empty(2, 0, 3, 1, 8)
    v = torch.empty(2, 0, 3, 4)
    st = torch.randn(2, 3, 4, 8)
    out, fs = op.ssd_scan(q, q, v, v, torch.empty(2, 0, 3), torch.empty(2, 0, 3),
                          torch.empty(2, 0, 3), torch.ones(3), initial_state=st,
                          initial_k=torch.randn(2, 3, 1, 8), initial_value=torch.randn(2, 3, 4))
    assert out.shape == v.shape
    torch.testing.assert_close(fs, st)


@pytest.mark.parametrize("rank", [1, 4])
def test_step_matches_one_recurrence_step(rank):
    inp = _scan_inputs(rank, seed=91, length=1, extras=True)
    y_ref, s_ref = _recurrence(inp)
    cache = (None, inp["initial_state"], inp["initial_k"], inp["initial_value"])
    y, nxt = op.step_update(inp["q"][:, 0], inp["k"][:, 0], inp["value"][:, 0],
                            inp["gate"][:, 0], inp["adt"][:, 0], inp["dt"][:, 0],
                            inp["trap_logits"][:, 0], inp["D"], cache, mimo_x=inp["mimo_x"],
                            mimo_z=inp["mimo_z"], mimo_out=inp["mimo_out"])
    np.testing.assert_allclose(y.numpy(), y_ref[:, 0], rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(nxt[1].numpy(), s_ref, rtol=2e-5, atol=2e-6)


# --------------------------------------------------------------------------- golden: hook level


def _hook_from_golden(data, dtype):
    def get(name, dt=torch.float32):
        key = f"in/{name}"
        return _t(data[key]).to(dt) if key in data else None

    return dict(q=get("q", dtype), k=get("k", dtype), value=get("value", dtype),
                gate=get("gate", dtype), adt=get("adt"), dt=get("dt"),
                trap_logits=get("trap", dtype), D=get("D"), mimo_x=get("mimo_x"),
                mimo_z=get("mimo_z"), mimo_out=get("mimo_out"),
                initial_state=get("init_state"), initial_k=get("init_k", dtype),
                initial_value=get("init_v", dtype)), get("phase"), get("q_bias"), get("k_bias")


@pytest.mark.parametrize("rank", [1, 4])
@pytest.mark.parametrize("dname,dtype", [("f32", torch.float32), ("bf16", torch.bfloat16)])
def test_scan_golden(rank, dname, dtype):
    data = golden(f"scan_r{rank}_{dname}.npz")
    inp, phase, qb, kb = _hook_from_golden(data, dtype)
    y, s = _oracle_scan(inp, int(data["chunk"]), phase=phase, mimo_rotation=rank > 1,
                        q_bias=qb, k_bias=kb)
    tol = dict(rtol=1e-6, atol=1e-6) if dtype == torch.float32 else dict(rtol=0, atol=0)
    torch.testing.assert_close(y.float(), _t(data["out"]), **tol)
    torch.testing.assert_close(s, _t(data["state"]), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("rank", [1, 4])
@pytest.mark.parametrize("dname,dtype", [("f32", torch.float32), ("bf16", torch.bfloat16)])
def test_step_golden(rank, dname, dtype):
    data = golden(f"step_r{rank}_{dname}.npz")
    g = lambda n, dt=torch.float32: _t(data[f"in/{n}"]).to(dt) if f"in/{n}" in data else None  # noqa: E731
    cache = (g("phase"), g("state"), g("prev_k", dtype), g("prev_v", dtype))
    y, nxt = op.step_update(g("q", dtype), g("k", dtype), g("value", dtype), g("gate", dtype),
                            g("adt"), g("dt"), g("trap", dtype), g("D"), cache,
                            mimo_x=g("mimo_x"), mimo_z=g("mimo_z"), mimo_out=g("mimo_out"))
    tol = dict(rtol=1e-6, atol=1e-6) if dtype == torch.float32 else dict(rtol=0, atol=0)
    torch.testing.assert_close(y.float(), _t(data["out"]), **tol)
    torch.testing.assert_close(nxt[1], _t(data["state"]), rtol=1e-6, atol=1e-6)


# --------------------------------------------------------------------------- golden: model level


def _check_params(data, params):
    order = [str(n) for n in data["param_order"]]
    assert sorted(order) == sorted(params)
    for name in order:
        v = params[name].double()
        want = data[f"param/{name}"]
        assert tuple(v.shape) == tuple(data[f"shape/{name}"])
        got = np.array([v.sum().item(), v.square().sum().item(), *v.flatten()[:4].tolist()]
                       + [0.0] * max(0, 4 - v.numel()))
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12, err_msg=name)


def _cache_check(data, prefix, caches, **tol):
    for i, layer in enumerate(caches):
        for j, name in enumerate(("phase", "state", "k", "v")):
            torch.testing.assert_close(layer[j].float(), _t(data[f"{prefix}/{i}/{name}"]), **tol)


@pytest.mark.parametrize("rank", [1, 4])
@pytest.mark.parametrize("mode", ["f32", "bf16"])
def test_model_golden(rank, mode):
    data = golden(f"model_r{rank}_{mode}.npz")
    torch.manual_seed(100 + rank)
    params = op.init_params(64, d_state=16, depth=2, mimo_rank=rank)
    _check_params(data, params)
    dims = op.Dims(64, 16, rank)
    x = _t(data["x"])
    tol = dict(rtol=1e-5, atol=1e-5) if mode == "f32" else dict(rtol=1e-2, atol=1e-2)
    ctx = (torch.autocast("cpu", dtype=torch.bfloat16) if mode == "bf16"
           else torch.autocast("cpu", enabled=False))
    with torch.inference_mode(), ctx:
        torch.testing.assert_close(op.model_forward(params, x, dims), _t(data["forward"]), **tol)
        prefix, caches = op.model_prefill(params, x[:, :9], dims)
        torch.testing.assert_close(prefix, _t(data["prefill"]), **tol)
        _cache_check(data, "prefill_cache", caches, **tol)
        outs = []
        for t in range(9, x.shape[1]):
            o, caches = op.model_step(params, x[:, t:t + 1], dims, caches)
            outs.append(o)
        torch.testing.assert_close(torch.cat(outs, 1), _t(data["steps"]), **tol)
        _cache_check(data, "final_cache", caches, **tol)


@pytest.mark.parametrize("rank", [1, 4])
def test_bidirectional_golden(rank):
    data = golden(f"bidir_r{rank}.npz")
    torch.manual_seed(40 + rank)
    params = op.init_params(16, d_state=8, depth=2, mimo_rank=rank, causal=False)
    _check_params(data, params)
    with torch.inference_mode():
        y = op.model_forward(params, _t(data["x"]), op.Dims(16, 8, rank), causal=False)
    torch.testing.assert_close(y, _t(data["forward"]), rtol=1e-5, atol=1e-5)


def test_config1_golden():
    """Mamba3(256, 128, 6, 1), seed 0, x [2, 1024, 256]."""
    data = golden("config1.npz")
    torch.manual_seed(0)
    params = op.init_params(256, d_state=128, depth=6, mimo_rank=1)
    _check_params(data, params)
    x = torch.randn(2, 1024, 256)
    np.testing.assert_allclose(x.norm(dim=-1).numpy(), data["x_norms"], rtol=1e-6)
    dims = op.Dims(256, 128, 1)
    tol = dict(rtol=1e-4, atol=1e-4)
    with torch.inference_mode():
        full = op.model_forward(params, x, dims)
        torch.testing.assert_close(full[:, :8], _t(data["forward_head"]), **tol)
        torch.testing.assert_close(full[:, -64:, :64], _t(data["forward_tail"]), **tol)
        torch.testing.assert_close(full.norm(dim=-1), _t(data["forward_norms"]), **tol)
        prefix, caches = op.model_prefill(params, x[:, :960], dims)
        steps = []
        for i in range(64):
            o, caches = op.model_step(params, x[:, 960 + i:961 + i], dims, caches)
            steps.append(o)
        steps = torch.cat(steps, 1)
    torch.testing.assert_close(steps[:, :, :64], _t(data["steps"]), **tol)
    torch.testing.assert_close(steps, full[:, 960:], **tol)
    for i, (phase, state, k, v) in enumerate(caches):
        torch.testing.assert_close(phase, _t(data[f"final_cache/{i}/phase"]), **tol)
        torch.testing.assert_close(state.norm(dim=(-1, -2)),
                                   _t(data[f"final_cache/{i}/state_norms"]), **tol)
        torch.testing.assert_close(state[:, :, :4, :16],
                                   _t(data[f"final_cache/{i}/state_slice"]), **tol)
