"""Float64 scalar-loop forms of the hot path — TEST INFRASTRUCTURE ONLY.

Written from the mathematical definitions (not from the PyTorch op chain) to
pin ``oracle.roserlhf_oracle``: a dropped term, a wrong sign, a transposed
index or a wrong tie rule in the restatement shows up as a mismatch here.

  * ``logprob``: log p(a) = x_a - (m + log sum_v exp(x_v - m)), m = max_v x_v.
  * ``*_grad``: closed-form dL/dlogp per objective, including clamp's
    pass-through on closed intervals and minimum's half/half tie split.
  * ``returns`` / ``gae`` / ``skip_gae``: the per-step recurrences of
    docs/agentic-rl/derivations-and-code.md:269-283 and source-lab.md:215-228
    with padding treated as absent time.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np


def logprob(logits: np.ndarray, targets: np.ndarray) -> np.ndarray:
    x = np.asarray(logits, dtype=np.float64)
    flat = x.reshape(-1, x.shape[-1])
    tg = np.asarray(targets).reshape(-1)
    out = np.empty(flat.shape[0])
    for r in range(flat.shape[0]):
        row = flat[r]
        m = max(row)
        s = 0.0
        for v in row:
            s += math.exp(v - m)
        out[r] = row[int(tg[r])] - (m + math.log(s))
    return out.reshape(np.asarray(targets).shape)


def softmax_rows(logits: np.ndarray) -> np.ndarray:
    x = np.asarray(logits, dtype=np.float64)
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)


def dlogits_from_g(logits: np.ndarray, targets: np.ndarray, g: np.ndarray) -> np.ndarray:
    """dL/dx[v] = g * (onehot(a)[v] - softmax(x)[v]) per row."""

    p = softmax_rows(logits)
    oh = np.zeros_like(p)
    np.put_along_axis(oh, np.asarray(targets)[..., None].astype(np.int64), 1.0, axis=-1)
    return np.asarray(g, dtype=np.float64)[..., None] * (oh - p)


def _pass(x: float, lo: float, hi: float) -> float:
    return 1.0 if lo <= x <= hi else 0.0


def _min_share(a: float, b: float) -> float:
    if a < b:
        return 1.0
    if b < a:
        return 0.0
    return 0.5


def _clip_surr_grad(r: float, A: float, lo: float, hi: float) -> float:
    """d min(r A, clip(r, lo, hi) A) / d r."""

    c = min(max(r, lo), hi)
    sh = _min_share(r * A, c * A)
    return sh * A + (1.0 - sh) * A * _pass(r, lo, hi)


def ppo_objective_grad(cur, old, adv, w, *, clip_low, clip_high, K=20.0):
    """(objective, d objective / d cur) for the clipped loss, weights w = mask values."""

    cur, old, adv, w = (np.asarray(a, dtype=np.float64).reshape(-1) for a in (cur, old, adv, w))
    lo, hi = 1.0 - clip_low, 1.0 + clip_high
    M = w.sum()
    obj = 0.0
    g = np.zeros_like(cur)
    for i in range(cur.size):
        x = cur[i] - old[i]
        r = math.exp(min(max(x, -K), K))
        c = min(max(r, lo), hi)
        obj += w[i] * min(r * adv[i], c * adv[i])
        g[i] = (w[i] / M) * _clip_surr_grad(r, adv[i], lo, hi) * r * _pass(x, -K, K)
    return obj / M, g


def sao_objective_grad(cur, roll, adv, m, *, clip_low, clip_high, detach=True, K=20.0):
    cur, roll, adv = (np.asarray(a, dtype=np.float64).reshape(-1) for a in (cur, roll, adv))
    m = np.asarray(m).reshape(-1).astype(bool)
    lo, hi = 1.0 - clip_low, 1.0 + clip_high
    M = float(m.sum())
    obj = 0.0
    g = np.zeros_like(cur)
    for i in range(cur.size):
        x = cur[i] - roll[i]
        r = math.exp(min(max(x, -K), K))
        if lo < r < hi and m[i]:
            obj += r * adv[i] * cur[i]
            d = r * adv[i]
            if not detach:
                d += cur[i] * adv[i] * r * _pass(x, -K, K)
            g[i] = d / M
    return obj / M, g


def gspo_objective_grad(cur, roll, seq_adv, m, *, clip_low, clip_high, K=20.0):
    cur, roll = (np.asarray(a, dtype=np.float64) for a in (cur, roll))
    m = np.asarray(m).astype(bool)
    A = np.asarray(seq_adv, dtype=np.float64)
    B, T = cur.shape
    lo, hi = 1.0 - clip_low, 1.0 + clip_high
    obj = 0.0
    g = np.zeros_like(cur)
    for b in range(B):
        n = m[b].sum()
        y = sum(cur[b, t] - roll[b, t] for t in range(T) if m[b, t]) / n
        s = math.exp(min(max(y, -K), K))
        c = min(max(s, lo), hi)
        obj += min(s * A[b], c * A[b]) / B
        dy = _clip_surr_grad(s, A[b], lo, hi) * s * _pass(y, -K, K) / B
        for t in range(T):
            if m[b, t]:
                g[b, t] = dy / n
    return obj, g


def gspo_token_objective_grad(cur, roll, tok_adv, m, *, clip_low, clip_high, K=20.0):
    cur, roll, A = (np.asarray(a, dtype=np.float64) for a in (cur, roll, tok_adv))
    m = np.asarray(m).astype(bool)
    B, T = cur.shape
    lo, hi = 1.0 - clip_low, 1.0 + clip_high
    obj = 0.0
    g = np.zeros_like(cur)
    for b in range(B):
        n = m[b].sum()
        y = sum(cur[b, t] - roll[b, t] for t in range(T) if m[b, t]) / n
        s = math.exp(min(max(y, -K), K))
        c = min(max(s, lo), hi)
        for t in range(T):
            if m[b, t]:
                obj += min(s * A[b, t], c * A[b, t]) / n / B
                g[b, t] = _clip_surr_grad(s, A[b, t], lo, hi) * s / n / B
    return obj, g


def sapo_objective_grad(cur, roll, tok_adv, m, *, tau_positive=1.0, tau_negative=1.05, K=20.0):
    cur, roll, A = (np.asarray(a, dtype=np.float64) for a in (cur, roll, tok_adv))
    m = np.asarray(m).astype(bool)
    B, T = cur.shape
    obj = 0.0
    g = np.zeros_like(cur)
    for b in range(B):
        n = m[b].sum()
        for t in range(T):
            if not m[b, t]:
                continue
            x = cur[b, t] - roll[b, t]
            r = math.exp(min(max(x, -K), K))
            tau = tau_positive if A[b, t] > 0 else tau_negative
            p = 1.0 / (1.0 + math.exp(-tau * (r - 1.0)))
            obj += (4.0 / tau) * p * A[b, t] / n / B
            g[b, t] = 4.0 * p * (1.0 - p) * A[b, t] * r * _pass(x, -K, K) / n / B
    return obj, g


def _opt(a: Optional[np.ndarray], shape, default) -> np.ndarray:
    if a is None:
        return np.full(shape, default, dtype=bool)
    return np.asarray(a).astype(bool)


def returns(rewards, *, gamma=1.0, terminated=None, valid=None, bootstrap=None):
    r = np.asarray(rewards, dtype=np.float64)
    r2 = r.reshape(-1, r.shape[-1])
    d = _opt(terminated, r.shape, False).reshape(r2.shape)
    v = _opt(valid, r.shape, True).reshape(r2.shape)
    boot = np.zeros(r2.shape[0]) if bootstrap is None else np.asarray(bootstrap, np.float64).reshape(-1)
    out = np.zeros_like(r2)
    for b in range(r2.shape[0]):
        R = boot[b]
        for t in range(r2.shape[1] - 1, -1, -1):
            if not v[b, t]:
                continue
            R = r2[b, t] + gamma * (0.0 if d[b, t] else 1.0) * R
            out[b, t] = R
    return out.reshape(r.shape)


def gae(rewards, values, *, gamma=1.0, lam=1.0, terminated=None, valid=None, bootstrap=None):
    r = np.asarray(rewards, dtype=np.float64)
    V = np.asarray(values, dtype=np.float64).reshape(-1, r.shape[-1])
    r2 = r.reshape(-1, r.shape[-1])
    d = _opt(terminated, r.shape, False).reshape(r2.shape)
    v = _opt(valid, r.shape, True).reshape(r2.shape)
    boot = np.zeros(r2.shape[0]) if bootstrap is None else np.asarray(bootstrap, np.float64).reshape(-1)
    adv = np.zeros_like(r2)
    for b in range(r2.shape[0]):
        v_next, a_next = boot[b], 0.0
        for t in range(r2.shape[1] - 1, -1, -1):
            if not v[b, t]:
                continue
            c = 0.0 if d[b, t] else 1.0
            delta = r2[b, t] + gamma * c * v_next - V[b, t]
            a_next = delta + gamma * lam * c * a_next
            adv[b, t] = a_next
            v_next = V[b, t]
    tgt = np.where(v, adv + V, 0.0)
    return adv.reshape(r.shape), tgt.reshape(r.shape)


def skip_gae(rewards, end_values, next_values, *, gamma=1.0, lam=1.0, terminated=None,
             valid=None):
    r = np.asarray(rewards, dtype=np.float64)
    r2 = r.reshape(-1, r.shape[-1])
    E = np.asarray(end_values, dtype=np.float64).reshape(r2.shape)
    N = np.asarray(next_values, dtype=np.float64).reshape(r2.shape)
    d = _opt(terminated, r.shape, False).reshape(r2.shape)
    v = _opt(valid, r.shape, True).reshape(r2.shape)
    adv = np.zeros_like(r2)
    for b in range(r2.shape[0]):
        a_next = 0.0
        for i in range(r2.shape[1] - 1, -1, -1):
            if not v[b, i]:
                continue
            c = 0.0 if d[b, i] else 1.0
            a_next = r2[b, i] + gamma * c * N[b, i] - E[b, i] + gamma * lam * c * a_next
            adv[b, i] = a_next
    tgt = np.where(v, adv + E, 0.0)
    return adv.reshape(r.shape), tgt.reshape(r.shape)


def group_standardize(rewards, eps=1e-8):
    r = np.asarray(rewards, dtype=np.float64)
    out = np.zeros_like(r)
    for gi in np.ndindex(r.shape[:-1]):
        row = r[gi]
        mu = sum(row) / len(row)
        sd = math.sqrt(sum((x - mu) ** 2 for x in row) / len(row))
        out[gi] = [(x - mu) / max(sd, eps) if sd > eps else 0.0 for x in row]
    return out


def leave_one_out(rewards):
    r = np.asarray(rewards, dtype=np.float64)
    out = np.zeros_like(r)
    G = r.shape[-1]
    for gi in np.ndindex(r.shape[:-1]):
        row = r[gi]
        out[gi] = [row[i] - (sum(row) - row[i]) / (G - 1) for i in range(G)]
    return out


def turn_broadcast(turn_adv, turn_ids, mask):
    A = np.asarray(turn_adv, dtype=np.float64)
    ids = np.asarray(turn_ids)
    m = np.asarray(mask).astype(bool)
    out = np.zeros(ids.shape)
    for b in range(ids.shape[0]):
        for t in range(ids.shape[1]):
            if m[b, t]:
                out[b, t] = A[b, ids[b, t]]
    return out


def whiten(values, mask, eps=1e-8):
    x = np.asarray(values, dtype=np.float64)
    m = np.asarray(mask).astype(bool)
    sel = [float(v) for v, k in zip(x.reshape(-1), m.reshape(-1)) if k]
    mu = sum(sel) / len(sel)
    sd = math.sqrt(sum((v - mu) ** 2 for v in sel) / len(sel))
    return np.where(m, (x - mu) / (sd + eps), 0.0)


def gather_rows(seq: Sequence[float]) -> np.ndarray:
    return np.asarray(seq, dtype=np.float64)


def nll_grad(labels, *, ignore_index=-100, reduction="mean") -> np.ndarray:
    """d loss / d logp of the SFT cross-entropy per token: -1/n for each of the
    n labels that differ from ignore_index ("mean"), -1 ("sum"), 0 for an
    ignored label."""

    y = np.asarray(labels).reshape(-1)
    n = sum(1 for v in y if v != ignore_index)
    out = np.zeros(y.shape[0])
    for i, v in enumerate(y):
        if v != ignore_index:
            out[i] = -1.0 if reduction == "sum" else -1.0 / n
    return out.reshape(np.asarray(labels).shape)


def nll_loss(logits, labels, *, ignore_index=-100, reduction="mean") -> float:
    """Scalar-loop SFT loss: -sum over kept tokens of log p(label) (/ n)."""

    x = np.asarray(logits, dtype=np.float64)
    flat = x.reshape(-1, x.shape[-1])
    y = np.asarray(labels).reshape(-1)
    total, n = 0.0, 0
    for r in range(flat.shape[0]):
        if y[r] == ignore_index:
            continue
        row = flat[r]
        m = max(row)
        s = 0.0
        for v in row:
            s += math.exp(v - m)
        total += row[int(y[r])] - (m + math.log(s))
        n += 1
    if reduction == "sum":
        return -total
    return -total / n if n else float("nan")
