"""f64 closed-form attention (TEST INFRASTRUCTURE).

The reference pins its ring operator against dense softmax attention plus
``logsumexp`` (ring.rs:2435-2444; ``full_attention_reference`` in
rust/src/smoke/reference_algo.rs:134-167, there non-causal).  This module is the
same closed form in f64 numpy, with global-position causal masking
(``q_pos >= k_pos``, ring.rs:262) and the GQA head map ``kv = h // (Hq/Hkv)``
(ring.rs:1962-1984).  Rows with no visible key give (o = 0, lse = -inf), the
fully-future-source convention of ring.rs:553-569.

Layouts are token-major, as drawn: q [Sq, Hq, D], k/v [Sk, Hkv, D].
"""
from __future__ import annotations

import numpy as np


def attention_f64(q, k, v, q_pos, k_pos, scale: float, causal: bool = True,
                  rows: np.ndarray | None = None):
    """Dense attention in f64.  Returns (o [R,Hq,D], lse [R,Hq]) for the selected rows.

    ``rows`` selects query rows (indices into q); default all rows.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    q_pos = np.asarray(q_pos, dtype=np.int64)
    k_pos = np.asarray(k_pos, dtype=np.int64)
    if rows is None:
        rows = np.arange(q.shape[0])
    hq, hkv = q.shape[1], k.shape[1]
    rep = hq // hkv
    out = np.zeros((len(rows), hq, q.shape[2]), dtype=np.float64)
    lse = np.full((len(rows), hq), -np.inf, dtype=np.float64)
    for g in range(hkv):
        kg = k[:, g, :]  # [Sk, D]
        vg = v[:, g, :]
        for h in range(g * rep, (g + 1) * rep):
            qh = q[rows, h, :]  # [R, D]
            s = (qh @ kg.T) * scale  # [R, Sk]
            if causal:
                vis = q_pos[rows][:, None] >= k_pos[None, :]
                s = np.where(vis, s, -np.inf)
            m = s.max(axis=1)
            ok = np.isfinite(m)
            m_safe = np.where(ok, m, 0.0)
            w = np.exp(s - m_safe[:, None])
            den = w.sum(axis=1)
            den_safe = np.where(den > 0, den, 1.0)
            out[:, h, :] = np.where(ok[:, None], (w @ vg) / den_safe[:, None], 0.0)
            lse[:, h] = np.where(ok, m_safe + np.log(den_safe), -np.inf)
    return out, lse


def merge_partials_f64(os_, lses):
    """Closed-form LSE merge of partials (o_i [.., D], lse_i [..]).

    ``m = max lse_i``; ``o = sum e^{lse_i - m} o_i / sum e^{lse_i - m}``;
    ``lse = m + ln sum e^{lse_i - m}``; all -inf gives (0, -inf).  This is the
    two-partial identity behind positioned_merge_compact_partial (ring.rs:574-603)
    extended to n partials.
    """
    lses = [np.asarray(x, dtype=np.float64) for x in lses]
    os_ = [np.asarray(x, dtype=np.float64) for x in os_]
    L = np.stack(lses)  # [n, ...]
    m = L.max(axis=0)
    ok = np.isfinite(m)
    m_safe = np.where(ok, m, 0.0)
    w = np.exp(L - m_safe)
    w = np.where(np.isfinite(L), w, 0.0)
    den = w.sum(axis=0)
    den_safe = np.where(den > 0, den, 1.0)
    num = sum(w[i][..., None] * os_[i] for i in range(len(os_)))
    o = np.where(ok[..., None], num / den_safe[..., None], 0.0)
    lse = np.where(ok, m_safe + np.log(den_safe), -np.inf)
    return o, lse


def ring_pairs(chunks):
    """Non-empty (target, source) pairs of a causal vanilla ring, in ring order.

    Domain d visits sources (d - s) mod N for s = 0..N-1 (local first, then the
    predecessor chain, ring.rs:1208-1311 with mock.rs:143-149); a source entirely in
    the future of the target (offset[src] > last position of d) contributes nothing.
    """
    n = len(chunks)
    offs = [sum(chunks[:i]) for i in range(n)]
    pairs = []
    for d in range(n):
        for s in range(n):
            src = (d - s) % n
            if offs[src] <= offs[d] + chunks[d] - 1:
                pairs.append((d, src))
    return pairs
