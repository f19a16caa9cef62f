"""Parity at the benchmark configs' full sizes (one MI355X), where the float64
oracle cannot evaluate everything: sampled instances and rows against the
closed forms (oracle/closed_forms.py), plus size-independent properties that
a plausible indexing or masking mistake breaks:

  C3 causal forward   row 0 attends to key 0 only, so out[0] == v[0] bit for
                      bit and lse[0] == scale * q0.k0; every output feature
                      lies inside the range of v's feature (a convex mix)
  C5 causal backward  the softmax rows sum to one, so sum_s dV[s] == sum_t
                      dO[t]; the rows of dS sum to zero, so sum_s dK[s] == 0
  C4 decode           sampled rows of every group of the grouped-query heads
  C2 rows             softmax rows sum to one; (layernorm - beta) / gamma has
                      zero mean and unit variance per row

Tolerances: the north-star ones (bf16 2e-2 of scale, fp32 1e-5 relative),
scaled where a property sums many bf16 terms (stated at each check)."""

import numpy as np
import pytest

from oracle import closed_forms as cf
from tests.tolerances import assert_lse

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _host(t):
    return t.detach().double().cpu().numpy()


def test_c3_causal_forward_at_full_size():
    from pdum_dsl_amd import kernels as K

    B, H, S, D = 8, 32, 4096, 128
    g = torch.Generator(device="cuda").manual_seed(3)
    q, k, v = (torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16) for _ in range(3))
    scale = D ** -0.5
    res = K.flash_fwd(q, k, v, scale=scale, band=K.CAUSAL)
    torch.cuda.synchronize()
    # row 0 sees key 0 only: the output is v[0] exactly, the lse the one score
    assert torch.equal(res.o[:, :, 0, :], v[:, :, 0, :])
    s00 = (q[:, :, 0, :].double() * k[:, :, 0, :].double()).sum(-1) * scale
    assert_lse(_host(res.lse[:, :, 0]), s00.cpu().numpy(), what="C3 row-0 lse")
    # a convex combination of v's rows stays inside v's per-feature range
    vmin, vmax = v.float().amin(dim=2, keepdim=True), v.float().amax(dim=2, keepdim=True)
    o = res.o.float()
    assert bool(((o >= vmin - 1e-2) & (o <= vmax + 1e-2)).all())
    assert torch.isfinite(res.lse).all()
    # sampled instances and rows against the float64 closed form
    rows = np.array([0, 1, 31, 32, 1000, 2047, 2048, 4095])
    for b, h in ((0, 0), (3, 17), (7, 31)):
        qi, ki, vi = _host(q[b, h]), _host(k[b, h]), _host(v[b, h])
        for r in rows:  # causal: row r sees keys 0..r
            sc = scale * qi[r] @ ki[: r + 1].T
            p = np.exp(sc - sc.max())
            w = p @ vi[: r + 1] / p.sum()
            got = _host(res.o[b, h, r])
            assert np.abs(got - w).max() <= 2e-2 * max(1.0, np.abs(w).max()), f"({b},{h}) row {r}"
            lse = sc.max() + np.log(p.sum())
            assert_lse(float(res.lse[b, h, r]), lse, what=f"lse ({b},{h}) row {r}")


def test_c5_causal_backward_at_full_size():
    from pdum_dsl_amd import kernels as K

    B, H, S, D = 4, 16, 2048, 64
    g = torch.Generator(device="cuda").manual_seed(5)
    q, k, v, do = (torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16) for _ in range(4))
    scale = D ** -0.5
    fw = K.flash_fwd(q, k, v, scale=scale, band=K.CAUSAL)
    dq, dk, dv = K.flash_bwd(q, k, v, fw.o, do, fw.lse, scale=scale, band=K.CAUSAL)
    torch.cuda.synchronize()
    # The identities hold for the fp32 results the kernel rounds to bf16; rounding moves each
    # element by at most 2^-8 of itself, so each sum over s may move by 2^-8 sum_s |x_s|.
    # sum_s dV[s] = sum_s sum_t P[t,s] dO[t] = sum_t dO[t] (rows of P sum to one)
    sdv, sdo = dv.double().sum(dim=2), do.double().sum(dim=2)
    assert bool(((sdv - sdo).abs() <= 2.0 ** -8 * dv.double().abs().sum(dim=2) + 1e-3).all())
    # rows of dS = P (dP - delta) sum to zero, so sum_s dK[s] = scale sum_t (sum_s dS[t,s]) q[t] = 0
    sdk = dk.double().sum(dim=2)
    assert bool((sdk.abs() <= 2.0 ** -8 * dk.double().abs().sum(dim=2) + 1e-3).all())
    # a sampled instance against the closed form
    b, h = 2, 9
    wq, wk, wv = cf.attention_bwd(_host(q[b, h]), _host(k[b, h]), _host(v[b, h]), _host(do[b, h]), scale=scale,
                                  band=(None, 0))
    for got, want in ((dq, wq), (dk, wk), (dv, wv)):
        assert np.abs(_host(got[b, h]) - want).max() <= 2e-2 * max(1.0, np.abs(want).max())


def test_c4_decode_at_full_size():
    from pdum_dsl_amd import kernels as K

    B, Hq, Hkv, S, D = 64, 32, 8, 8192, 128
    g = torch.Generator(device="cuda").manual_seed(4)
    q = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(torch.bfloat16)
    o, lse = K.attn_decode(q, k, v)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(lse).all()
    scale = D ** -0.5
    for b, hq in ((0, 0), (17, 3), (63, 31), (40, 12)):
        hk = hq // (Hq // Hkv)
        want, _m, _d, wlse = cf.attention(_host(q[b, hq]), _host(k[b, hk]), _host(v[b, hk]), scale=scale, band=None)
        assert np.abs(_host(o[b, hq]) - want).max() <= 2e-2 * max(1.0, np.abs(want).max())
        assert_lse(float(lse[b, hq, 0]), float(wlse[0]), what=f"C4 lse ({b},{hq})")


def test_c2_rows_at_full_size():
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn((8192, 4096), generator=g, device="cuda")
    gam = 1 + 0.1 * torch.randn((4096,), generator=g, device="cuda")
    bet = 0.1 * torch.randn((4096,), generator=g, device="cuda")
    y = K.row_softmax(x)
    z = K.layernorm(x, gam, bet, eps=1e-5)
    torch.cuda.synchronize()
    assert (y.double().sum(dim=1) - 1).abs().max().item() < 1e-5  # every row of 4096 fp32 probabilities
    # (z - beta) / gamma has zero mean and unit (biased) variance per row
    zn = (z.double() - bet.double()) / gam.double()
    assert zn.mean(dim=1).abs().max().item() < 1e-5
    assert (zn.var(dim=1, unbiased=False) - 1).abs().max().item() < 1e-3
    rows = [0, 1, 4095, 8191]
    xs = x[rows].double().cpu().numpy()
    np.testing.assert_allclose(y[rows].double().cpu().numpy(), cf.np_softmax(xs, axis=1), rtol=1e-5, atol=1e-9)
