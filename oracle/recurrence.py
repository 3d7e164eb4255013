"""Float64 per-token Mamba-3 recurrence in numpy (test infrastructure only).

Independent of ``oracle.portable``: no chunking, no torch, no low-precision
casts. It restates the recurrence from the reference README
(``README.md:117-124``) and the per-token loop of the reference's test helper
``tests/test_scan.py:21-98``::

    alpha = exp(adt);  beta = (1 - sigmoid(lam)) * dt * alpha;  gamma = sigmoid(lam) * dt
    S_t   = alpha * S_{t-1} + beta * U_{t-1} + gamma * U_t,   U_t = sum_r (v_t * mx_r) outer k_{t,r}
    y_t   = sum_r mo_r * (S_t q_{t,r} + D * v_t * mx_r) * silu(z_t * mz_r)

``q``/``k`` are per head and already biased and rotated: ``[B, L, H, R, N]``.
The pinning checks for this module are the closed forms in
``tests/test_oracle.py`` (Mamba-2 special case, linear attention).
"""

from __future__ import annotations

import numpy as np


def _silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


def _sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


def recurrent_scan(q, k, v, z, adt, dt, trap_logits, D, *, mimo_x=None, mimo_z=None,
                   mimo_out=None, state0=None, k0=None, v0=None):
    """Return ``(y [B,L,H,P], state [B,H,P,N])`` in float64."""
    q, k, v, z = (np.asarray(a, dtype=np.float64) for a in (q, k, v, z))
    adt, dt, lam, D = (np.asarray(a, dtype=np.float64) for a in (adt, dt, trap_logits, D))
    batch, length, heads, rank, n = q.shape
    p = v.shape[-1]
    mx = np.ones((heads, rank, p)) if mimo_x is None else np.asarray(mimo_x, np.float64)
    mz = np.ones((heads, rank, p)) if mimo_z is None else np.asarray(mimo_z, np.float64)
    mo = np.ones((heads, rank, p)) if mimo_out is None else np.asarray(mimo_out, np.float64)
    state = np.zeros((batch, heads, p, n)) if state0 is None else np.asarray(state0, np.float64).copy()
    prev_k = np.zeros((batch, heads, rank, n)) if k0 is None else np.asarray(k0, np.float64)
    prev_v = np.zeros((batch, heads, p)) if v0 is None else np.asarray(v0, np.float64)
    y = np.zeros((batch, length, heads, p))
    for t in range(length):
        trap = _sigmoid(lam[:, t])
        alpha = np.exp(adt[:, t])
        beta = (1.0 - trap) * dt[:, t] * alpha
        gamma = trap * dt[:, t]
        u_prev = np.einsum("bhp,hrp,bhrn->bhpn", prev_v, mx, prev_k)
        u_cur = np.einsum("bhp,hrp,bhrn->bhpn", v[:, t], mx, k[:, t])
        state = alpha[..., None, None] * state + beta[..., None, None] * u_prev \
            + gamma[..., None, None] * u_cur
        read = np.einsum("bhpn,bhrn->bhrp", state, q[:, t])
        read = read + D[None, :, None, None] * v[:, t][:, :, None, :] * mx[None]
        read = read * _silu(z[:, t][:, :, None, :] * mz[None])
        y[:, t] = (read * mo[None]).sum(axis=2)
        prev_k, prev_v = k[:, t], v[:, t]
    return y, state
