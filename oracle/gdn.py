"""CPU restatement of mlx-runner's packed gated-delta (GDN) recurrence.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s checker, and only as the checker.  The HIP product path
never imports this module.

The recurrence is the one ``src/gdn_packed.metal`` runs for
``gdnKernelRun`` (src/model.zig:284-319) and ``gdnStepOwned`` runs op by op
(src/model.zig:1006-1045).  For each batch b and value head hv (key head
hk = hv / (Hv / Hk), src/gdn_packed.metal ``hk_idx``), with the state
S[Dv, Dk] and per step t:

    S      = S * g[t]                         (decay, scalar per head)
    kv[r]  = sum_d S[r, d] * k[t, d]
    dlt[r] = (v[t, r] - kv[r]) * beta[t]
    S      = S + dlt[r] * k[t, d]             (rank-1 update)
    y[t,r] = sum_d S[r, d] * q[t, d]

Shapes: q, k [B, T, Hk, Dk]; v [B, T, Hv, Dv]; g, beta [B, T, Hv];
state [B, Hv, Dv, Dk]; y [B, T, Hv, Dv].
"""
from __future__ import annotations

import numpy as np


def _heads(x: np.ndarray, Hv: int) -> np.ndarray:
    """[B, T, Hk, D] -> [B, T, Hv, D]: value head hv reads key head hv / (Hv / Hk)."""
    Hk = x.shape[2]
    assert Hv % Hk == 0, (Hv, Hk)
    return np.repeat(x, Hv // Hk, axis=2)


def gdn_recurrence(q, k, v, g, beta, state, *, acc: str = "f64"):
    """Returns (y [B, T, Hv, Dv], state_out [B, Hv, Dv, Dk]).

    acc="f64": every operation in float64 (the reference value).
    acc="f32": float32, each dot product accumulated sequentially over d in the
    order of the reference's CPU check (src/model.zig:1650-1673).
    """
    dt = np.float64 if acc == "f64" else np.float32
    B, T, Hk, Dk = q.shape
    Hv = v.shape[2]
    qh = _heads(np.asarray(q, dt), Hv)  # [B, T, Hv, Dk]
    kh = _heads(np.asarray(k, dt), Hv)
    v = np.asarray(v, dt)
    g = np.asarray(g, dt)
    beta = np.asarray(beta, dt)
    S = np.array(state, dtype=dt, copy=True)  # [B, Hv, Dv, Dk]
    y = np.zeros(v.shape, dtype=dt)
    for t in range(T):
        kt, qt = kh[:, t], qh[:, t]  # [B, Hv, Dk]
        S *= g[:, t][:, :, None, None]
        if acc == "f64":
            kv = np.einsum("bhrd,bhd->bhr", S, kt)
        else:
            kv = np.zeros(S.shape[:3], dt)
            for d in range(Dk):
                kv = kv + S[..., d] * kt[:, :, None, d]
        dlt = (v[:, t] - kv) * beta[:, t][:, :, None]  # [B, Hv, Dv]
        S += dlt[..., None] * kt[:, :, None, :]
        if acc == "f64":
            y[:, t] = np.einsum("bhrd,bhd->bhr", S, qt)
        else:
            o = np.zeros(S.shape[:3], dt)
            for d in range(Dk):
                o = o + S[..., d] * qt[:, :, None, d]
            y[:, t] = o
    return y, S


def gdn_recurrence_loops(q, k, v, g, beta, state):
    """The same recurrence as scalar Python loops in float64 (tiny shapes only):
    the brute-force check of the vectorised form."""
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    S = [[[[float(state[b][h][r][d]) for d in range(Dk)] for r in range(Dv)] for h in range(Hv)] for b in range(B)]
    y = np.zeros((B, T, Hv, Dv))
    for b in range(B):
        for t in range(T):
            for h in range(Hv):
                hk = h // (Hv // Hk)
                gt, bt = float(g[b][t][h]), float(beta[b][t][h])
                for r in range(Dv):
                    row = S[b][h][r]
                    kv = 0.0
                    for d in range(Dk):
                        row[d] *= gt
                        kv += row[d] * float(k[b][t][hk][d])
                    dl = (float(v[b][t][h][r]) - kv) * bt
                    o = 0.0
                    for d in range(Dk):
                        row[d] += float(k[b][t][hk][d]) * dl
                        o += row[d] * float(q[b][t][hk][d])
                    y[b, t, h, r] = o
    return y, np.array(S)


def reference_pattern_case():
    """Inputs of the reference's kernel test (src/model.zig:1615-1642): Hv=2, Hk=1,
    Dk=128, Dv=8, T=3, B=1, deterministic patterns; its bars are max |dy| < 0.05
    and max |dS| < 1e-3 against its f32 CPU recurrence."""
    hv, hk, dk, dv, t = 2, 1, 128, 8, 3
    f = np.float32  # the reference computes the patterns in f32 (f32 operands, f32 products)
    i = np.arange(t * hk * dk)
    q = (((i % 13) - 6).astype(f) * f(0.05)).reshape(1, t, hk, dk)
    k = (((i % 11) - 5).astype(f) * f(0.05)).reshape(1, t, hk, dk)
    j = np.arange(t * hv * dv)
    v = (((j % 7) - 3).astype(f) * f(0.1)).reshape(1, t, hv, dv)
    n = np.arange(t * hv)
    g = (f(0.9) + (n % 3).astype(f) * f(0.03)).reshape(1, t, hv)
    beta = (f(0.4) + (n % 2).astype(f) * f(0.1)).reshape(1, t, hv)
    s = np.arange(hv * dv * dk)
    st = (((s % 5) - 2).astype(f) * f(0.01)).reshape(1, hv, dv, dk)
    return q, k, v, g, beta, st
