"""CPU restatement of next-token sampling with behaviour log-probs — TEST
INFRASTRUCTURE ONLY.

Follows roseinfer/engine.py:1103-1171 (InferenceEngine._sample_next_token_batch,
its PyTorch path) on the float64 upcast of the logits:

* greedy (not do_sample or temperature <= 0): lowest index of the maximum;
* scaled = x / T; candidates = the top_k largest when 0 < top_k < V (ties at
  the k-th value lowest index first), else all V; p = softmax over them;
* 0 < top_p < 1: descending order (ties lowest index first), a candidate is
  kept iff its inclusive cumulative p is <= top_p, the first always (the
  reference's ``mask = cum_probs > top_p; mask[..., 0] = False``);
* q = max(p * kept, 1e-9) on the candidates (``masked_fill`` then
  ``clamp_min(1e-9)``), 0 elsewhere; with top-k or top-p active the token is
  the first index, in vocabulary order, whose inclusive cumulative q exceeds
  u * sum(q);
* without top-k and top-p (the reference's ``softmax(...).clamp_min(1e-9)``
  branch) q = p + g with g = max(1e-9 - p, 0) is drawn as a mixture: the
  floor's excess g when u1 < G / (S + G) (S = sum p = 1, G = sum g), else p;
  the token is the first index whose inclusive cumulative weight of that
  component exceeds u times the component's total.  Both rules sample q / sum q
  exactly: (S / (S + G)) p / S + (G / (S + G)) g / G = q / (S + G).

The uniforms of row r come from Philox4x32-10 (Salmon, Moraes, Dror, Shaw,
SC 2011) of counter (r, r >> 32, offset, offset >> 32) and key
(seed, seed >> 32), words w0..w3: u = (w0 >> 8) * 2^-24 and
u1 = ((w1 << 21) | (w2 >> 11)) * 2^-53.  ``philox4x32_10`` is pinned by the
known-answer vectors published with the Random123 library; the distribution
by a direct restatement of the reference's torch op chain and the mixture
identity (tests/test_oracle_sampler.py).
"""

from __future__ import annotations

import math
from typing import Dict, Tuple

import numpy as np

M32 = 0xFFFFFFFF
PHILOX_M = (0xD2511F53, 0xCD9E8D57)
PHILOX_W = (0x9E3779B9, 0xBB67AE85)


def philox4x32_10(ctr, key) -> Tuple[int, int, int, int]:
    """Ten Philox4x32 rounds: (c0, c1, c2, c3) -> (hi(M1*c2)^c1^k0, lo(M1*c2),
    hi(M0*c0)^c3^k1, lo(M0*c0)), the key bumped by the Weyl constants between
    rounds."""

    c0, c1, c2, c3 = (int(v) & M32 for v in ctr)
    k0, k1 = (int(v) & M32 for v in key)
    for _ in range(10):
        p0 = PHILOX_M[0] * c0
        p1 = PHILOX_M[1] * c2
        c0, c1, c2, c3 = ((p1 >> 32) ^ c1 ^ k0) & M32, p1 & M32, ((p0 >> 32) ^ c3 ^ k1) & M32, p0 & M32
        k0 = (k0 + PHILOX_W[0]) & M32
        k1 = (k1 + PHILOX_W[1]) & M32
    return c0, c1, c2, c3


def row_uniforms(seed: int, offset: int, row: int) -> Tuple[float, float]:
    """(u, u1) of row r: the position uniform (24 bits) and the component
    uniform (53 bits)."""

    w = philox4x32_10((row & M32, (row >> 32) & M32, offset & M32, (offset >> 32) & M32),
                      (seed & M32, (seed >> 32) & M32))
    return (w[0] >> 8) * 2.0 ** -24, (((w[1] << 21) | (w[2] >> 11)) & ((1 << 53) - 1)) * 2.0 ** -53


def row_uniform(seed: int, offset: int, row: int) -> float:
    return row_uniforms(seed, offset, row)[0]


def mixture_parts(p: np.ndarray) -> Tuple[np.ndarray, np.ndarray, float]:
    """(p, g = max(1e-9 - p, 0), pi = G / (S + G)) of a full softmax p: the
    two components of max(p, 1e-9) and the probability of the floor's."""

    g = np.maximum(1e-9 - p, 0.0)
    S, G = float(p.sum()), float(g.sum())
    return p, g, (G / (S + G) if G > 0.0 else 0.0)


def inverse_cdf(w: np.ndarray, u: float) -> Tuple[int, float]:
    """(first index whose inclusive cumulative w exceeds u * sum(w), the
    distance of u * sum(w) to the nearest boundary relative to sum(w));
    rounding past the end takes the last positive entry."""

    cdf = np.cumsum(w)
    total = cdf[-1]
    tgt = u * total
    tok = int(np.searchsorted(cdf, tgt, side="right"))
    if tok >= w.size:
        tok = int(np.nonzero(w > 0)[0][-1])
    lo = cdf[tok - 1] if tok > 0 else 0.0
    return tok, min(tgt - lo, cdf[tok] - tgt) / total


def mixture_draw(p: np.ndarray, u: float, u1: float) -> Tuple[int, float]:
    """(token, margin) of the mixture rule; the margin is the smaller of the
    position margin inside the chosen component and |u1 - pi| / pi."""

    rho, g, pi = mixture_parts(p)
    tok, pos = inverse_cdf(g if u1 < pi else rho, u)
    comp = abs(u1 - pi) / pi if pi > 0.0 else math.inf
    return tok, min(pos, comp)


def _descending(x: np.ndarray) -> np.ndarray:
    """Indices by descending value, ties lowest index first."""

    return np.lexsort((np.arange(x.size), -x))


def sampling_distribution(x: np.ndarray, temperature: float, top_k: int, top_p: float
                          ) -> Tuple[np.ndarray, np.ndarray]:
    """(q over the vocabulary (unnormalised, 0 off the candidates), candidate
    mask) for one row of logits."""

    V = x.size
    s = x.astype(np.float64) / float(temperature)
    cand = np.ones(V, dtype=bool)
    if 0 < top_k < V:
        order = _descending(s)
        cand[:] = False
        cand[order[:top_k]] = True
    m = s[cand].max()
    e = np.where(cand, np.exp(np.where(cand, s - m, 0.0)), 0.0)
    p = e / e.sum()
    kept = cand.copy()
    if 0.0 < top_p < 1.0:
        order = _descending(s)
        order = order[cand[order]]
        cum = np.cumsum(p[order])
        drop = cum > top_p
        drop[0] = False
        kept[order[drop]] = False
    q = np.where(cand, np.maximum(np.where(kept, p, 0.0), 1e-9), 0.0)
    return q, cand


def top_p_margin(x: np.ndarray, temperature: float, top_k: int, top_p: float) -> float:
    """Distance of top_p from the cumulative masses on either side of the
    nucleus cut (the last kept candidate's and the first dropped one's),
    in probability; inf without top-p.  A cut closer than float32 rounding
    of the probabilities (the kernels form them in float32, as the
    reference's softmax does) can keep one token more or less."""

    if not 0.0 < top_p < 1.0:
        return math.inf
    V = x.size
    s = x.astype(np.float64) / float(temperature)
    cand = np.ones(V, dtype=bool)
    if 0 < top_k < V:
        cand[:] = False
        cand[_descending(s)[:top_k]] = True
    m = s[cand].max()
    e = np.where(cand, np.exp(np.where(cand, s - m, 0.0)), 0.0)
    p = e / e.sum()
    order = _descending(s)
    order = order[cand[order]]
    cum = np.cumsum(p[order])
    drop = np.nonzero(cum > top_p)[0]
    near = [cum[drop[0]]] if drop.size else []
    if drop.size and drop[0] > 0:
        near.append(cum[drop[0] - 1])
    return float(min((abs(c - top_p) for c in near), default=math.inf))


def sample_rows(logits: np.ndarray, *, temperature: float, top_k: int, top_p: float,
                do_sample: bool, seed: int, offset: int) -> Dict[str, np.ndarray]:
    """Per row: token, logp = log_softmax(x/T)[token] (T = 1 when greedy),
    logq = log(q[token]/sum q) (0 when greedy), margin = the distance of
    the draw's target to the nearest cumulative boundary relative to the
    total drawn over, or of u1 to the mixture's pi relative to pi, and
    p_margin = top_p_margin (decisions closer than float32 rounding can go
    either way)."""

    x = np.asarray(logits, dtype=np.float64)
    B, V = x.shape
    greedy = (not do_sample) or temperature <= 0.0
    T = 1.0 if greedy else float(temperature)
    out = {k: np.zeros(B) for k in ("logp", "logq", "margin")}
    out["p_margin"] = np.full(B, math.inf)
    out["token"] = np.zeros(B, dtype=np.int64)
    for r in range(B):
        row = x[r]
        if greedy:
            tok = int(np.argmax(row))
            out["margin"][r] = math.inf
        else:
            q, _ = sampling_distribution(row, T, top_k, top_p)
            u, u1 = row_uniforms(seed, offset, r)
            if 0 < top_k < V or 0.0 < top_p < 1.0:
                tok, margin = inverse_cdf(q, u)
            else:
                s = row / T
                e = np.exp(s - s.max())
                tok, margin = mixture_draw(e / e.sum(), u, u1)
            out["margin"][r] = margin
            out["p_margin"][r] = top_p_margin(row, T, top_k, top_p)
            out["logq"][r] = math.log(q[tok] / q.sum())
        s = row / T
        mx = s.max()
        out["logp"][r] = s[tok] - (mx + math.log(np.exp(s - mx).sum()))
        out["token"][r] = tok
    return out
