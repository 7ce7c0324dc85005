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
  ``clamp_min(1e-9)``), 0 elsewhere; the token is the first index, in
  vocabulary order, whose inclusive cumulative q exceeds u * sum(q).

The uniform of row r is Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC 2011)
of counter (r, r >> 32, offset, offset >> 32) and key (seed, seed >> 32):
u = (first word >> 8) * 2^-24.  ``philox4x32_10`` is pinned by the known-answer
vectors published with the Random123 library; the distribution by a direct
restatement of the reference's torch op chain (tests/test_oracle_sampler.py).
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


def row_uniform(seed: int, offset: int, row: int) -> float:
    w = philox4x32_10((row & M32, (row >> 32) & M32, offset & M32, (offset >> 32) & M32),
                      (seed & M32, (seed >> 32) & M32))
    return (w[0] >> 8) * 2.0 ** -24


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


def sample_rows(logits: np.ndarray, *, temperature: float, top_k: int, top_p: float,
                do_sample: bool, seed: int, offset: int) -> Dict[str, np.ndarray]:
    """Per row: token, logp = log_softmax(x/T)[token] (T = 1 when greedy),
    logq = log(q[token]/sum q) (0 when greedy), and margin = the distance of
    u*sum(q) to the nearest cumulative boundary relative to sum(q) (decisions
    closer than float32 rounding can go either way)."""

    x = np.asarray(logits, dtype=np.float64)
    B, V = x.shape
    greedy = (not do_sample) or temperature <= 0.0
    T = 1.0 if greedy else float(temperature)
    out = {k: np.zeros(B) for k in ("logp", "logq", "margin")}
    out["token"] = np.zeros(B, dtype=np.int64)
    for r in range(B):
        row = x[r]
        if greedy:
            tok = int(np.argmax(row))
            out["margin"][r] = math.inf
        else:
            q, _ = sampling_distribution(row, T, top_k, top_p)
            cdf = np.cumsum(q)
            total = cdf[-1]
            tgt = row_uniform(seed, offset, r) * total
            tok = int(np.searchsorted(cdf, tgt, side="right"))
            tok = min(tok, V - 1)
            lo = cdf[tok - 1] if tok > 0 else 0.0
            out["margin"][r] = min(tgt - lo, cdf[tok] - tgt) / total
            out["logq"][r] = math.log(q[tok] / total)
        s = row / T
        mx = s.max()
        out["logp"][r] = s[tok] - (mx + math.log(np.exp(s - mx).sum()))
        out["token"][r] = tok
    return out
