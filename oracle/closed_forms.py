"""ORACLE — test infrastructure only (the checker, never the product).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package. Nothing under pdum_dsl_amd/ may import it.

Closed-form float64 numpy restatements of the denotations the reference's
fusion templates compute. Each function cites the reference lines it
follows (paths relative to the reference repository root):

  np_softmax         packages/tensorlib/src/pdum/tl/zoo/zoo_common.py:33-35
  np_layernorm       packages/tensorlib/src/pdum/tl/zoo/zoo_common.py:69-72
  attention          packages/tensorlib/src/pdum/tl/zoo/tiles.py:254-257 (the flash
                     oracle: softmax(where(mask, q k^T, -1e9)) v) and the artifact
                     semantics of fusion.py:542-615 (m = running max from -1e30,
                     den = sum exp(sm - m), yield order (out, m, den))
  attention_bwd      the closed form of autodiff.grad over the naive twin
                     (autodiff.py:102-122; tiles.py:238-252): dV = P^T dO,
                     dP = dO V^T, D = rowsum(dO * O), dS = P (dP - D),
                     dQ = scale dS K, dK = scale dS^T Q
  combine_partials   the flashsm combine, zoo/attention.py:40-46

Inputs are upcast to float64 before any arithmetic, so a bf16 input is
seen by the oracle exactly as the kernel sees it (rounding happens once,
at the input), and the oracle's error is far below any kernel tolerance.
"""

from __future__ import annotations

import numpy as np

FILL = -1e9  # the reference's mask fill (fusion.py:508-512, zoo/tiles.py:220)
M0 = -1e30  # the reference's running-max identity (fusion.py:562; zoo/attention.py:57-62)


def np_softmax(s, axis):
    s = np.asarray(s, dtype=np.float64)
    e = np.exp(s - s.max(axis=axis, keepdims=True))
    return e / e.sum(axis=axis, keepdims=True)


def np_layernorm(x, g=None, beta=None, eps=1e-5, axis=-1):
    x = np.asarray(x, dtype=np.float64)
    mu = x.mean(axis=axis, keepdims=True)
    v = ((x - mu) ** 2).mean(axis=axis, keepdims=True)
    y = (x - mu) / np.sqrt(v + eps)
    if g is not None:
        y = y * np.asarray(g, dtype=np.float64)
    if beta is not None:
        y = y + np.asarray(beta, dtype=np.float64)
    return y


def band_live(t_idx, s_idx, lo=None, hi=None):
    """Boolean live mask of the band lo <= s - t <= hi (None = unbounded)."""
    d = np.asarray(s_idx)[None, :] - np.asarray(t_idx)[:, None]
    live = np.ones(d.shape, dtype=bool)
    if lo is not None:
        live &= d >= lo
    if hi is not None:
        live &= d <= hi
    return live


def attention(q, k, v, *, scale=1.0, band=None, fill=FILL, row_block=512):
    """One instance: q [T, E], k [S, E], v [S, OD] -> (out, m, den, lse).

    sc = scale * q k^T; masked entries take ``fill``; m = max(M0, max_s sc);
    den = sum_s exp(sc - m); out = sum_s exp(sc - m) v / den; lse = m + log den.
    ``band`` is None (all live) or (lo, hi). Rows are processed in blocks so
    memory stays O(row_block * S)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    T, S = q.shape[0], k.shape[0]
    out = np.empty((T, v.shape[1]))
    m_all = np.empty(T)
    den_all = np.empty(T)
    for r0 in range(0, T, row_block):
        r1 = min(T, r0 + row_block)
        sc = scale * (q[r0:r1] @ k.T)
        if band is not None:
            sc = np.where(band_live(np.arange(r0, r1), np.arange(S), *band), sc, fill)
        m = np.maximum(M0, sc.max(axis=1))
        p = np.exp(sc - m[:, None])
        den = p.sum(axis=1)
        out[r0:r1] = (p @ v) / den[:, None]
        m_all[r0:r1] = m
        den_all[r0:r1] = den
    return out, m_all, den_all, m_all + np.log(den_all)


def attention_bwd(q, k, v, do, *, scale=1.0, band=None, fill=FILL, row_block=512):
    """One instance: gradients (dq, dk, dv) of out = attention(q, k, v) seeded by do."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(do, dtype=np.float64)
    T, S = q.shape[0], k.shape[0]
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for r0 in range(0, T, row_block):
        r1 = min(T, r0 + row_block)
        sc = scale * (q[r0:r1] @ k.T)
        live = None
        if band is not None:
            live = band_live(np.arange(r0, r1), np.arange(S), *band)
            sc = np.where(live, sc, fill)
        p = np_softmax(sc, axis=1)
        o = p @ v
        dv += p.T @ do[r0:r1]
        dp = do[r0:r1] @ v.T
        dd = (do[r0:r1] * o).sum(axis=1, keepdims=True)
        ds = p * (dp - dd)
        if live is not None:  # the fill is a constant: no gradient flows to masked scores
            ds = np.where(live, ds, 0.0)
        dq[r0:r1] = scale * (ds @ k)
        dk += scale * (ds.T @ q[r0:r1])
    return dq, dk, dv


def attention_batched(q, k, v, *, scale=1.0, band=None, fill=FILL, heads=None):
    """[B, Hq, T, E] / [B, Hkv, S, E] grouped-query batch (query head h reads
    kv head h // (Hq / Hkv)); ``heads`` optionally restricts to a list of
    (b, h) instances. Returns dict (b, h) -> (out, m, den, lse)."""
    B, Hq = q.shape[:2]
    Hkv = k.shape[1]
    rep = Hq // Hkv
    todo = heads if heads is not None else [(b, h) for b in range(B) for h in range(Hq)]
    return {
        (b, h): attention(q[b, h], k[b, h // rep], v[b, h // rep], scale=scale, band=band, fill=fill)
        for (b, h) in todo
    }


def combine_partials(parts):
    """Fold (m, den, o) partial states with the associative online-softmax
    combine (zoo/attention.py:40-46): m = max; den, o rescaled by exp(m_i - m)."""
    m, den, o = parts[0]
    for mr, denr, orr in parts[1:]:
        mm = np.maximum(m, mr)
        sl, sr = np.exp(m - mm), np.exp(mr - mm)
        m, den, o = mm, den * sl + denr * sr, o * sl[..., None] + orr * sr[..., None]
    return m, den, o
