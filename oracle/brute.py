"""Brute-force fp64 disentangled attention, written from the math (not from
the eager code) — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Per (b, h), with s = 1/sqrt(D * scale_factor), t(i, j) the relative position
clamped to [-A, A], c = clamp(t + A, 0, 2A-1), p = clamp(A - t, 0, 2A-1)
(reference: deberta_v2_native.py:377, 395, 407, 604, 615-644):

  S_ij  = s * (q_i.k_j + q_i.Kr[c] + k_j.Qr[p])
  S_ij  = -inf if the pair is masked;  row i is dead if not live_i
  P     = softmax_j(S) on live rows, 0 on dead rows;   O_i = sum_j P_ij v_j

With the position-to-position term (p2p, deberta_v2_native.py:298-347) the
score also holds s * Qr[A + min(i, A-1)].Kr[c]: the query's position row
from the positive half of Qr, clamped to its A rows, against the same c2p
row of Kr.

Backward (Delta_i = dO_i.O_i, dS_ij = P_ij (dO_i.v_j - Delta_i)):
  dv_j  += P_ij dO_i
  dq_i  += s dS_ij (k_j + Kr[c])       dk_j += s dS_ij (q_i + Qr[p])
  dKr[c] += s dS_ij q_i                 dQr[p] += s dS_ij k_j
  p2p:  dKr[c] += s dS_ij Qr[r_i],      dQr[r_i] += s dS_ij Kr[c],  r_i = A + min(i, A-1)
Small shapes only (pure Python loops over (b, h, i, j)).
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np


def _rows(rel: np.ndarray, A: int) -> tuple[np.ndarray, np.ndarray]:
    t = np.clip(rel, -A, A)
    return np.clip(t + A, 0, 2 * A - 1), np.clip(A - t, 0, 2 * A - 1)


def _liveness(keep: Optional[np.ndarray], B: int, Lq: int, Lk: int, pairwise: bool) -> tuple[np.ndarray, np.ndarray]:
    """keep: None, (B, Lk) key mask, or (B, Lq, Lk) pair mask -> (pair keep, live)."""
    if keep is None:
        return np.ones((B, Lq, Lk), dtype=bool), np.ones((B, Lq), dtype=bool)
    if not pairwise:
        pk = np.broadcast_to(keep[:, None, :], (B, Lq, Lk)).astype(bool)
        return pk, keep[:, :Lq].astype(bool)
    pk = keep.astype(bool)
    return pk, np.stack([np.diag(pk[b]) for b in range(B)])


def forward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    kr: Optional[np.ndarray],
    qr: Optional[np.ndarray],
    rel: Optional[np.ndarray],
    keep: Optional[np.ndarray],
    pairwise: bool,
    scale: float,
    A: int,
    p2p: bool = False,
    c2p: bool = True,
    p2c: bool = True,
) -> tuple[np.ndarray, np.ndarray]:
    """q, k, v: (B, H, L, D) fp64; kr, qr: (H, 2A, D) or None; rel (Lq, Lk).
    c2p / p2c use kr / qr when given (``c2p`` / ``p2c`` False leave a table
    given for p2p out of those terms); ``p2p`` adds the position-to-position
    term (needs both tables).  Returns (O (B, H, Lq, D), P (B, H, Lq, Lk))."""
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    pk, live = _liveness(keep, B, Lq, Lk, pairwise)
    c = p = None
    if rel is not None:
        c, p = _rows(rel, A)
    O = np.zeros((B, H, Lq, D))
    P = np.zeros((B, H, Lq, Lk))
    for b in range(B):
        for h in range(H):
            for i in range(Lq):
                if not live[b, i]:
                    continue
                s_row = np.full(Lk, -np.inf)
                for j in range(Lk):
                    if not pk[b, i, j]:
                        continue
                    acc = float(q[b, h, i] @ k[b, h, j])
                    if kr is not None and c2p:
                        acc += float(q[b, h, i] @ kr[h, c[i, j]])
                    if qr is not None and p2c:
                        acc += float(k[b, h, j] @ qr[h, p[i, j]])
                    if p2p:
                        acc += float(qr[h, A + min(i, A - 1)] @ kr[h, c[i, j]])
                    s_row[j] = scale * acc
                m = np.max(s_row)
                e = np.exp(s_row - m)
                P[b, h, i] = e / e.sum()
                O[b, h, i] = P[b, h, i] @ v[b, h]
    return O, P


def backward(
    dO: np.ndarray,
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    kr: Optional[np.ndarray],
    qr: Optional[np.ndarray],
    rel: Optional[np.ndarray],
    keep: Optional[np.ndarray],
    pairwise: bool,
    scale: float,
    A: int,
    p2p: bool = False,
    c2p: bool = True,
    p2c: bool = True,
) -> dict[str, np.ndarray]:
    """Analytic gradients from the formulas in the module docstring."""
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    O, P = forward(q, k, v, kr, qr, rel, keep, pairwise, scale, A, p2p=p2p, c2p=c2p, p2c=p2c)
    pk, live = _liveness(keep, B, Lq, Lk, pairwise)
    c = p = None
    if rel is not None:
        c, p = _rows(rel, A)
    g = {
        "q": np.zeros_like(q),
        "k": np.zeros_like(k),
        "v": np.zeros_like(v),
        "kr": None if kr is None else np.zeros_like(kr),
        "qr": None if qr is None else np.zeros_like(qr),
    }
    for b in range(B):
        for h in range(H):
            for i in range(Lq):
                if not live[b, i]:
                    continue
                delta = float(dO[b, h, i] @ O[b, h, i])
                for j in range(Lk):
                    pij = P[b, h, i, j]
                    if pij == 0.0:
                        continue
                    g["v"][b, h, j] += pij * dO[b, h, i]
                    ds = pij * (float(dO[b, h, i] @ v[b, h, j]) - delta)
                    g["q"][b, h, i] += scale * ds * k[b, h, j]
                    g["k"][b, h, j] += scale * ds * q[b, h, i]
                    if kr is not None and c2p:
                        g["q"][b, h, i] += scale * ds * kr[h, c[i, j]]
                        g["kr"][h, c[i, j]] += scale * ds * q[b, h, i]
                    if qr is not None and p2c:
                        g["k"][b, h, j] += scale * ds * qr[h, p[i, j]]
                        g["qr"][h, p[i, j]] += scale * ds * k[b, h, j]
                    if p2p:
                        r = A + min(i, A - 1)
                        g["kr"][h, c[i, j]] += scale * ds * qr[h, r]
                        g["qr"][h, r] += scale * ds * kr[h, c[i, j]]
    return g


def bucket_exact(d: int, bucket_size: int, max_position: int) -> tuple[int, bool]:
    """Log bucket of one offset in double precision, and whether the value
    before ``ceil`` lies within 1e-4 of an integer (where fp32 rounding may
    pick either side).  Written from the published formula: clamp to
    ±(max_position-1); identity below bucket_size//2; else
    sign * (mid + ceil(log(|d|/mid) / log(max(max_position-1, mid+1)/mid) * (mid-1)))."""
    if max_position > 0:
        d = max(min(d, max_position - 1), 1 - max_position)
    mid = bucket_size // 2
    if mid <= 1:
        return d, False
    base = math.log(max(max_position - 1, mid + 1) / mid)
    if base <= 0:
        return d, False
    a = max(abs(d), 1)
    sgn = (d > 0) - (d < 0)
    if a < mid:
        return sgn * a, False
    x = math.log(a / mid) / base * (mid - 1)
    near_int = abs(x - round(x)) < 1e-4
    return sgn * (mid + math.ceil(x)), near_int
