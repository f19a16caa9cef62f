"""Backward parity on the GPU: dQ, dK, dV from libpdhip against the
closed-form gradients of the flash joint (oracle.closed_forms.attention_bwd,
the textbook FA backward that equals autodiff.grad over the naive twin,
autodiff.py:102-122, by softmax shift invariance)."""

import numpy as np
import pytest

from oracle import closed_forms as cf
from tests.tolerances import assert_lowp

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _host(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "B,H,T,D,band",
    [
        (1, 2, 128, 64, (None, 0)),
        (2, 1, 256, 64, None),
        (1, 2, 200, 64, (None, 0)),  # ragged
        (1, 1, 96, 128, (None, 0)),
        (1, 2, 160, 128, None),
        (1, 1, 130, 64, (None, -1)),  # row 0 fully masked: uniform softmax, no pruning
        (1, 1, 300, 64, (-63, 0)),  # sliding window
        (1, 1, 256, 64, (None, 5)),  # unbounded below, keys past the diagonal live
        (1, 1, 256, 128, (-40, None)),  # unbounded above
        # instances in multiples of 32: the shader-engine-balanced block order
        (2, 16, 256, 64, (None, 0)),
        (1, 32, 128, 128, None),
    ],
)
def test_flash_bwd_matches_oracle(dtype, B, H, T, D, band):
    from pdum_dsl_amd import kernels as K

    rng = np.random.default_rng(T + D + (0 if band is None else 1))
    q, k, v, do = (
        torch.as_tensor(rng.standard_normal((B, H, T, D))).to(dtype=dtype, device="cuda") for _ in range(4)
    )
    scale = D**-0.5
    kb = K.Band(*band) if band is not None else None
    fw = K.flash_fwd(q, k, v, scale=scale, band=kb, want_artifacts=True)
    grads_lse = K.flash_bwd(q, k, v, fw.o, do, fw.lse, scale=scale, band=kb)
    grads_art = K.flash_bwd(q, k, v, fw.o, do, fw.lse, m=fw.m, den=fw.den, scale=scale, band=kb)
    torch.cuda.synchronize()
    Q, Kh, V, dO = _host(q), _host(k), _host(v), _host(do)
    for b in range(B):
        for h in range(H):
            wq, wk, wv = cf.attention_bwd(Q[b, h], Kh[b, h], V[b, h], dO[b, h], scale=scale, band=band)
            for tag, (dq, dk, dv) in (("lse", grads_lse), ("m,den", grads_art)):
                assert_lowp(_host(dq)[b, h], wq, what=f"dq[{b},{h}] from {tag}")
                assert_lowp(_host(dk)[b, h], wk, what=f"dk[{b},{h}] from {tag}")
                assert_lowp(_host(dv)[b, h], wv, what=f"dv[{b},{h}] from {tag}")


def test_bwd_refuses_heads_that_do_not_group():
    from pdum_dsl_amd import kernels as K

    q = torch.zeros((1, 4, 64, 64), dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros((1, 3, 64, 64), dtype=torch.bfloat16, device="cuda")
    lse = torch.zeros((1, 4, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="multiple of key/value heads"):
        K.flash_bwd(q, kv, kv, q, q, lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize(
    "B,Hq,Hkv,T,D,band",
    [
        (1, 4, 1, 256, 64, (None, 0)),
        (2, 8, 2, 200, 128, (None, 0)),  # ragged
        (1, 6, 3, 160, 64, None),
        (1, 4, 2, 300, 64, (-63, 0)),  # sliding window
        (1, 32, 8, 128, 128, (None, 0)),  # the decode config's head grouping
    ],
)
def test_grouped_query_backward_matches_oracle(dtype, B, Hq, Hkv, T, D, band):
    """Grouped-query attention (query head h reads K / V head h // (Hq / Hkv),
    the reference's (g, r) heads over repeated K / V, zoo/llama.py:7-8):
    dQ per query head from its group's K / V; dK and dV of a K / V head are
    the sums over the query heads of its group (the repeat's adjoint)."""
    from pdum_dsl_amd import kernels as K

    rng = np.random.default_rng(Hq * T + D)
    q, do = (torch.as_tensor(rng.standard_normal((B, Hq, T, D))).to(dtype=dtype, device="cuda") for _ in range(2))
    k, v = (torch.as_tensor(rng.standard_normal((B, Hkv, T, D))).to(dtype=dtype, device="cuda") for _ in range(2))
    scale = D**-0.5
    kb = K.Band(*band) if band is not None else None
    fw = K.flash_fwd(q, k, v, scale=scale, band=kb)
    dq, dk, dv = K.flash_bwd(q, k, v, fw.o, do, fw.lse, scale=scale, band=kb)
    torch.cuda.synchronize()
    Q, Kh, V, dO = _host(q), _host(k), _host(v), _host(do)
    grp = Hq // Hkv
    wk_sum = np.zeros((B, Hkv, T, D))
    wv_sum = np.zeros((B, Hkv, T, D))
    for b in range(B):
        for h in range(Hq):
            wq, wk, wv = cf.attention_bwd(Q[b, h], Kh[b, h // grp], V[b, h // grp], dO[b, h], scale=scale, band=band)
            wk_sum[b, h // grp] += wk
            wv_sum[b, h // grp] += wv
            if dtype == torch.float32:
                np.testing.assert_allclose(_host(dq)[b, h], wq, rtol=0, atol=1e-5 * max(1.0, np.abs(wq).max()))
            else:
                assert_lowp(_host(dq)[b, h], wq, what=f"dq[{b},{h}]")
    for b in range(B):
        for hk in range(Hkv):
            for got, want, nm in ((dk, wk_sum, "dk"), (dv, wv_sum, "dv")):
                w = want[b, hk]
                if dtype == torch.float32:
                    np.testing.assert_allclose(_host(got)[b, hk], w, rtol=0, atol=1e-5 * max(1.0, np.abs(w).max()))
                else:
                    assert_lowp(_host(got)[b, hk], w, what=f"{nm}[{b},{hk}]")
