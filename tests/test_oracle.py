"""Pinning the oracle (CPU). The reference ships no golden vectors, so each
oracle function is checked against something that does not restate its
formula: brute-force Python loops on tiny inputs, library routines
(scipy.special.logsumexp, torch.autograd in float64), finite differences,
invariants (shift invariance, rows summing to one, the associative combine),
and the committed fixtures (tests/golden/, regression pins)."""

from pathlib import Path

import math

import numpy as np
import pytest
import torch
from scipy.special import logsumexp

from oracle import closed_forms as cf

GOLD = Path(__file__).resolve().parent / "golden"


def _brute_attention(q, k, v, live, fill=cf.FILL):
    """Pure-Python loops: per row, the masked scores, their softmax, the weighted sum."""
    T, S = q.shape[0], k.shape[0]
    out = np.zeros((T, v.shape[1]))
    for t in range(T):
        sc = []
        for s in range(S):
            dot = sum(q[t, e] * k[s, e] for e in range(q.shape[1]))
            sc.append(dot if live(t, s) else fill)
        mx = max(sc)
        w = [math.exp(x - mx) for x in sc]
        z = sum(w)
        for o in range(v.shape[1]):
            out[t, o] = sum(w[s] * v[s, o] for s in range(S)) / z
    return out


@pytest.mark.parametrize(
    "band,live",
    [
        ((None, 0), lambda t, s: s <= t),
        ((None, -1), lambda t, s: s < t),
        ((-2, 0), lambda t, s: s <= t and t - s < 3),
        (None, lambda t, s: True),
    ],
)
def test_attention_matches_brute_force_loops(band, live):
    rng = np.random.default_rng(1)
    q, k, v = rng.standard_normal((5, 3)), rng.standard_normal((7, 3)), rng.standard_normal((7, 2))
    out, m, den, lse = cf.attention(q, k, v, band=band)
    np.testing.assert_allclose(out, _brute_attention(q, k, v, live), rtol=1e-12, atol=1e-12)
    sc = q @ k.T
    sm = np.array([[sc[t, s] if live(t, s) else cf.FILL for s in range(7)] for t in range(5)])
    np.testing.assert_allclose(lse, logsumexp(sm, axis=1), rtol=1e-12)
    np.testing.assert_allclose(m, sm.max(axis=1), rtol=0)
    np.testing.assert_allclose(den, np.exp(sm - sm.max(axis=1, keepdims=True)).sum(axis=1), rtol=1e-12)


def test_fully_masked_row_is_uniform():
    rng = np.random.default_rng(2)
    q, k, v = rng.standard_normal((4, 3)), rng.standard_normal((4, 3)), rng.standard_normal((4, 2))
    out, m, den, _ = cf.attention(q, k, v, band=(None, -1))
    np.testing.assert_allclose(out[0], v.mean(axis=0), rtol=1e-12)
    assert m[0] == cf.FILL and den[0] == 4.0


def test_scale_and_row_blocking_are_transparent():
    rng = np.random.default_rng(3)
    q, k, v = rng.standard_normal((37, 8)), rng.standard_normal((50, 8)), rng.standard_normal((50, 4))
    a = cf.attention(q, k, v, scale=0.25, band=(None, 5), row_block=7)[0]
    b = cf.attention(0.25 * q, k, v, band=(None, 5), row_block=1000)[0]
    np.testing.assert_allclose(a, b, rtol=1e-12)


def test_attention_bwd_matches_torch_autograd_f64():
    rng = np.random.default_rng(4)
    T, S, E = 6, 9, 4
    q, k, v, do = (rng.standard_normal(s) for s in ((T, E), (S, E), (S, 3), (T, 3)))
    for band in ((None, 0), (-3, 1), None):
        tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
        sc = 0.5 * tq @ tk.T
        if band is not None:
            live = torch.as_tensor(cf.band_live(np.arange(T), np.arange(S), *band))
            sc = torch.where(live, sc, torch.tensor(cf.FILL, dtype=torch.float64))
        (torch.softmax(sc, dim=1) @ tv).backward(torch.tensor(do))
        dq, dk, dv = cf.attention_bwd(q, k, v, do, scale=0.5, band=band)
        np.testing.assert_allclose(dq, tq.grad.numpy(), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(dk, tk.grad.numpy(), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(dv, tv.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_attention_bwd_matches_finite_differences():
    rng = np.random.default_rng(5)
    q, k, v, do = (rng.standard_normal(s) for s in ((4, 3), (5, 3), (5, 2), (4, 2)))
    dq, dk, dv = cf.attention_bwd(q, k, v, do, band=(None, 1))

    def loss(qq, kk, vv):
        return float((cf.attention(qq, kk, vv, band=(None, 1))[0] * do).sum())

    h = 1e-6
    for arr, grad, which in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            ap, am = arr.copy(), arr.copy()
            ap[idx] += h
            am[idx] -= h
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[which], args_m[which] = ap, am
            num[idx] = (loss(*args_p) - loss(*args_m)) / (2 * h)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)


def test_split_key_partials_combine_to_the_whole():
    """The flashsm combine over key chunks reproduces the full softmax-weighted sum."""
    rng = np.random.default_rng(6)
    q, k, v = rng.standard_normal((3, 4)), rng.standard_normal((20, 4)), rng.standard_normal((20, 5))
    parts = []
    for c0 in range(0, 20, 6):
        sc = q @ k[c0:c0 + 6].T
        m = sc.max(axis=1)
        p = np.exp(sc - m[:, None])
        parts.append((m, p.sum(axis=1), p @ v[c0:c0 + 6]))
    m, den, o = cf.combine_partials(parts)
    out, mm, dd, _ = cf.attention(q, k, v)
    np.testing.assert_allclose(o / den[:, None], out, rtol=1e-12)
    np.testing.assert_allclose(m, mm, rtol=0)
    np.testing.assert_allclose(den, dd, rtol=1e-12)


def test_softmax_and_layernorm_invariants():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 11)) * 4
    y = cf.np_softmax(x, axis=1)
    np.testing.assert_allclose(y.sum(axis=1), 1.0, rtol=1e-14)
    np.testing.assert_allclose(cf.np_softmax(x + 123.0, axis=1), y, rtol=1e-12)
    np.testing.assert_allclose(cf.np_softmax(np.zeros((2, 4)), axis=1), 0.25)
    z = cf.np_layernorm(x, eps=0.0)
    np.testing.assert_allclose(z.mean(axis=1), 0.0, atol=1e-14)
    np.testing.assert_allclose((z**2).mean(axis=1), 1.0, rtol=1e-12)
    g, b = rng.standard_normal(11), rng.standard_normal(11)
    ln = torch.nn.functional.layer_norm(torch.tensor(x), (11,), torch.tensor(g), torch.tensor(b), eps=1e-5)
    np.testing.assert_allclose(cf.np_layernorm(x, g, b, 1e-5), ln.numpy(), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("name", sorted(p.name for p in GOLD.glob("*.npz")))
def test_oracle_reproduces_the_committed_fixtures(name):
    d = np.load(GOLD / name)
    if name.startswith("softmax"):
        np.testing.assert_allclose(cf.np_softmax(d["x"], axis=1), d["y"], rtol=1e-13)
    elif name.startswith("layernorm"):
        np.testing.assert_allclose(cf.np_layernorm(d["x"], d["g"], d["b"], 1e-5), d["y"], rtol=1e-13)
    elif name.endswith("_bwd.npz"):
        dq, dk, dv = cf.attention_bwd(d["q"], d["k"], d["v"], d["dout"], band=(None, 0))
        for a, b in ((dq, d["dq"]), (dk, d["dk"]), (dv, d["dv"])):
            np.testing.assert_allclose(a, b, rtol=1e-13, atol=1e-15)
    else:
        band = {"causal": (None, 0), "strict": (None, -1), "window3": (-2, 0), "all": None}[
            name.rsplit("_", 1)[1][:-4]
        ]
        out, m, den, lse = cf.attention(d["q"], d["k"], d["v"], band=band)
        for a, b in ((out, d["out"]), (m, d["m"]), (den, d["den"]), (lse, d["lse"])):
            np.testing.assert_allclose(a, b, rtol=1e-13, atol=1e-15)


def test_region_evaluator_agrees_with_closed_forms_and_the_planner_interpreter():
    """The torch-f64 region evaluator (oracle) on the naive twins equals the
    closed forms; on the generated tile programs it equals the planner's
    numpy interpreter (two independent implementations)."""
    from oracle import region_eval as re_
    from pdum_dsl_amd.tl import fusion, zoo
    from pdum_dsl_amd.tl.interp import run_region

    for subj in (
        zoo.attention(T=8, E=3, OD=2, mask="causal"),
        zoo.attention(T=8, E=3, OD=2, mask=("window", 3)),
        zoo.attention(T=7, S=9, E=4, OD=3, mask="all"),
        zoo.row_softmax(),
        zoo.layernorm(),
    ):
        vals = [re_.value(f.arr, p.type) for f, p in zip(subj.inputs, subj.region.params)]
        got = re_.evaluate(subj.region, vals).numpy()
        np.testing.assert_allclose(got, subj.oracle(subj.numpy_inputs()), rtol=1e-12, atol=1e-12)
        (g,) = fusion.plan_region(subj.region).groups
        tile_o = re_.evaluate(g.kernel, vals)
        tile_i = run_region(g.kernel, subj.inputs)
        np.testing.assert_allclose(tile_o.numpy(tile_i.names), tile_i.arr, rtol=1e-13, atol=1e-13)
