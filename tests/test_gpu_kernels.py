"""Kernel-level parity on the GPU: every libpdhip entry point against the
float64 oracle (oracle/closed_forms.py) on seeded inputs, plus the
reference's structural laws (pruned == unpruned bit-exact,
fusion.py:659-690 / conformance/test_fusion_triton.py:140-159; the
fully-masked row keeps uniform-softmax semantics, test_launch.py:82-111)."""

import numpy as np
import pytest

from oracle import closed_forms as cf
from tests.tolerances import assert_fp32, assert_lowp, assert_lse

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def K():
    from pdum_dsl_amd import kernels

    return kernels


def _dev(a, dtype=torch.float32):
    return torch.as_tensor(np.ascontiguousarray(a)).to(dtype=dtype, device="cuda")


def _host(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


# ------------------------------------------------------------------ MFMA probe


def test_mfma_lane_layouts_match_a_matmul(K):
    rng = np.random.default_rng(0)
    a32, b32 = rng.standard_normal((32, 16)), rng.standard_normal((16, 32))
    a16, b16 = rng.standard_normal((16, 32)), rng.standard_normal((32, 16))
    ta32, tb32, ta16, tb16 = (_dev(x, torch.bfloat16) for x in (a32, b32, a16, b16))
    c32, c16 = K.probe_mfma(ta32, tb32, ta16, tb16)
    torch.cuda.synchronize()
    want32 = _host(ta32) @ _host(tb32)
    want16 = _host(ta16) @ _host(tb16)
    np.testing.assert_allclose(_host(c32), want32, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(_host(c16), want16, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- row kernels


@pytest.mark.parametrize(
    "rows,cols",
    [(1, 1), (3, 7), (64, 256), (37, 1000), (128, 4096), (5, 4099), (8, 12000), (2, 64)],
)
def test_row_softmax_matches_oracle(K, rows, cols):
    rng = np.random.default_rng(rows * 7919 + cols)
    x = rng.standard_normal((rows, cols)) * 3.0
    y = K.row_softmax(_dev(x))
    torch.cuda.synchronize()
    xf = x.astype(np.float32).astype(np.float64)
    assert_fp32(_host(y), cf.np_softmax(xf, axis=1), what=f"softmax {rows}x{cols}")


def test_row_softmax_strided_rows(K):
    rng = np.random.default_rng(5)
    base = _dev(rng.standard_normal((16, 300)))
    x = base[:, 10:266]  # row stride 300, 16-byte misaligned start -> streaming kernel
    y = K.row_softmax(x)
    torch.cuda.synchronize()
    assert_fp32(_host(y), cf.np_softmax(_host(x), axis=1), what="strided softmax")


@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize(
    "rows,cols", [(4, 4), (33, 768), (64, 4096), (3, 5000), (7, 129), (7, 4096), (1, 2048), (9, 2048)]
)
def test_layernorm_matches_oracle(K, rows, cols, affine):
    rng = np.random.default_rng(rows + 31 * cols)
    x = rng.standard_normal((rows, cols)) + 0.5
    g = 1 + 0.1 * rng.standard_normal(cols) if affine else None
    b = 0.1 * rng.standard_normal(cols) if affine else None
    y = K.layernorm(_dev(x), None if g is None else _dev(g), None if b is None else _dev(b), eps=1e-5)
    torch.cuda.synchronize()
    f = lambda a: None if a is None else a.astype(np.float32).astype(np.float64)  # noqa: E731
    want = cf.np_layernorm(f(x), f(g), f(b), eps=1e-5)
    assert_fp32(_host(y), want, rtol=1e-5, atol=1e-5, what=f"layernorm {rows}x{cols}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(7, 4096), (8, 2048), (33, 768)])
def test_layernorm_16bit_storage_matches_oracle(K, dtype, rows, cols):
    """bf16 / f16 storage, fp32 arithmetic: odd and even row counts through the
    one- and two-rows-per-wave kernels, against the float64 oracle on the same
    rounded inputs."""
    rng = np.random.default_rng(rows * 7 + cols)
    x = _dev(rng.standard_normal((rows, cols)) + 0.5, dtype)
    g = _dev(1 + 0.1 * rng.standard_normal(cols), dtype)
    b = _dev(0.1 * rng.standard_normal(cols), dtype)
    y = K.layernorm(x, g, b, eps=1e-5)
    torch.cuda.synchronize()
    want = cf.np_layernorm(_host(x), _host(g), _host(b), eps=1e-5)
    assert_lowp(_host(y), want, what=f"layernorm {dtype} {rows}x{cols}")


# ---------------------------------------------------------- flash forward


def _qkv(rng, B, Hq, Hkv, T, S, E, OD, dtype):
    q = _dev(rng.standard_normal((B, Hq, T, E)), dtype)
    k = _dev(rng.standard_normal((B, Hkv, S, E)), dtype)
    v = _dev(rng.standard_normal((B, Hkv, S, OD)), dtype)
    return q, k, v


def _check_fwd(res, q, k, v, scale, band, lowp):
    Q, Kh, V = _host(q), _host(k), _host(v)
    want = cf.attention_batched(Q, Kh, V, scale=scale, band=band)
    o, lse = _host(res.o), _host(res.lse)
    m = _host(res.m) if res.m is not None else None
    den = _host(res.den) if res.den is not None else None
    for (b, h), (wo, wm, wden, wlse) in want.items():
        if lowp:
            assert_lowp(o[b, h], wo, what=f"out[{b},{h}]")
        else:
            assert_fp32(o[b, h], wo, rtol=1e-5, atol=1e-5, what=f"out[{b},{h}]")
        assert_lse(lse[b, h], wlse, what=f"lse[{b},{h}]")
        if m is not None:
            np.testing.assert_allclose(m[b, h], wm, rtol=1e-5, atol=1e-5, err_msg=f"m[{b},{h}]")
            np.testing.assert_allclose(den[b, h], wden, rtol=1e-4, atol=1e-5, err_msg=f"den[{b},{h}]")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "B,Hq,Hkv,T,S,D,causal,growth",
    [
        (1, 2, 2, 256, 256, 128, True, 1.0),
        (1, 2, 1, 77, 333, 64, False, 1.0),
        (2, 4, 4, 128, 1024, 128, False, 1.0),
        # key rows scaled up along the key axis: a row's scores keep outgrowing
        # the running reference by far more than 2^8, so full tiles take the
        # exact path (row max, rescale, exponentials again) over and over
        (1, 2, 2, 512, 512, 128, True, 6.0),
        (1, 2, 2, 64, 2048, 128, False, 6.0),
        (1, 2, 2, 300, 700, 64, False, 6.0),
    ],
)
def test_the_lse_only_forward_matches_the_oracle_and_the_artifact_launch(K, dtype, B, Hq, Hkv, T, S, D, causal, growth):
    """A launch without the (m, den) artifacts refers full tiles' exponentials
    to the running reference without a per-tile row max and takes the exact
    path only when a lane's partial sum leaves (0, 2^8]. Its o and lse must
    match the float64 closed form and the launch that keeps the max on every
    tile (the reference's recurrence, fusion.py:542-615)."""
    rng = np.random.default_rng(B * 100 + T + S + D + int(growth))
    q = _dev(rng.standard_normal((B, Hq, T, D)), dtype)
    ramp = 1.0 + (growth - 1.0) * np.linspace(0.0, 1.0, S)[:, None]  # key s scaled by 1 .. growth
    k = _dev(rng.standard_normal((B, Hkv, S, D)) * ramp, dtype)
    v = _dev(rng.standard_normal((B, Hkv, S, D)), dtype)
    band = (None, 0) if causal else None
    scale = 1.0 / np.sqrt(D)
    kb = K.Band(*band) if band else None
    lse_only = K.flash_fwd(q, k, v, scale=scale, band=kb)
    full = K.flash_fwd(q, k, v, scale=scale, band=kb, want_artifacts=True)
    torch.cuda.synchronize()
    assert lse_only.m is None and full.m is not None
    _check_fwd(lse_only, q, k, v, scale, band, lowp=True)
    assert_lowp(_host(lse_only.o), _host(full.o), what="lse-only vs artifact launch: out")
    np.testing.assert_allclose(_host(lse_only.lse), _host(full.lse), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "B,Hq,Hkv,T,S,D,causal",
    [
        (1, 2, 2, 128, 128, 128, True),
        (2, 2, 2, 256, 256, 128, False),
        (1, 4, 2, 200, 200, 128, True),  # ragged rows and keys, GQA
        (1, 2, 1, 77, 333, 64, False),
        (2, 1, 1, 384, 384, 64, True),
        (1, 1, 1, 1, 1, 128, True),
        # instances in multiples of 32: the shader-engine-balanced block order
        (2, 16, 4, 256, 256, 128, True),
        (1, 32, 8, 128, 300, 64, False),
    ],
)
def test_flash_fwd_m16_matches_oracle(K, dtype, B, Hq, Hkv, T, S, D, causal):
    rng = np.random.default_rng(B * 1000 + T + S + D)
    q, k, v = _qkv(rng, B, Hq, Hkv, T, S, D, D, dtype)
    band = (None, 0) if causal else None
    scale = 1.0 / np.sqrt(D)
    res = K.flash_fwd(q, k, v, scale=scale, band=K.Band(*band) if band else None, want_artifacts=True)
    torch.cuda.synchronize()
    _check_fwd(res, q, k, v, scale, band, lowp=True)


@pytest.mark.parametrize(
    "T,S,E,OD,causal",
    [(6, 6, 3, 2, True), (256, 256, 64, 64, False), (100, 70, 33, 17, True), (5, 130, 8, 200, False)],
)
def test_flash_fwd_fp32_generic_matches_oracle(K, T, S, E, OD, causal):
    rng = np.random.default_rng(T * 31 + S)
    q, k, v = _qkv(rng, 1, 2, 2, T, S, E, OD, torch.float32)
    band = (None, 0) if causal else None
    res = K.flash_fwd(q, k, v, scale=0.125, band=K.Band(*band) if band else None, want_artifacts=True)
    torch.cuda.synchronize()
    _check_fwd(res, q, k, v, 0.125, band, lowp=False)


@pytest.mark.parametrize(
    "B,Hq,Hkv,T,S,D,band",
    [(1, 1, 1, 256, 256, 64, None), (1, 2, 2, 300, 290, 64, (None, 0)), (2, 4, 2, 130, 1000, 32, None),
     (1, 2, 1, 200, 333, 64, (-70, 5)), (1, 3, 3, 65, 64, 32, (None, 600)), (1, 2, 2, 129, 129, 64, (None, -1)),
     (4, 16, 8, 1024, 1024, 64, (None, 0)), (2, 32, 32, 500, 700, 32, None)],
)
def test_flash_fwd_fp32_row_kernel_matches_oracle(K, B, Hq, Hkv, T, S, D, band):
    """e = od = 32 or 64 at fp32 take the row kernel (lane = query row, K / V
    chunks staged through LDS, the key range split over eight waves on grids
    under one workgroup per CU, four on the last two cases' larger grids):
    causal, windowed, half-open and fully-masked-row bands (the last disables
    the prune), grouped heads, row and key tails, the artifacts."""
    rng = np.random.default_rng(T * 7 + S + D)
    q, k, v = _qkv(rng, B, Hq, Hkv, T, S, D, D, torch.float32)
    res = K.flash_fwd(q, k, v, scale=D**-0.5, band=K.Band(*band) if band else None, want_artifacts=True)
    torch.cuda.synchronize()
    _check_fwd(res, q, k, v, D**-0.5, band, lowp=False)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_pruned_sweep_is_bit_equal_to_the_full_sweep(K, dtype):
    rng = np.random.default_rng(11)
    D = 128 if dtype != torch.float32 else 40
    q, k, v = _qkv(rng, 1, 2, 2, 320, 320, D, D, dtype)
    full = K.flash_fwd(q, k, v, band=K.CAUSAL, prune=False, want_artifacts=True)
    pruned = K.flash_fwd(q, k, v, band=K.CAUSAL, prune=True, want_artifacts=True)
    torch.cuda.synchronize()
    assert torch.equal(full.o, pruned.o)
    assert torch.equal(full.m, pruned.m) and torch.equal(full.den, pruned.den)


@pytest.mark.parametrize("B,H,T", [(1, 2, 320), (8, 32, 256)])
def test_the_row_kernel_prunes_bit_exactly(K, B, H, T):
    """The fp32 row kernel at both wave counts (a grid under one workgroup
    per CU, and one over): a causal prune leaves every bit as the full sweep."""
    rng = np.random.default_rng(12)
    q, k, v = _qkv(rng, B, H, H, T, T, 64, 64, torch.float32)
    full = K.flash_fwd(q, k, v, band=K.CAUSAL, prune=False, want_artifacts=True)
    pruned = K.flash_fwd(q, k, v, band=K.CAUSAL, prune=True, want_artifacts=True)
    torch.cuda.synchronize()
    assert torch.equal(full.o, pruned.o)
    assert torch.equal(full.m, pruned.m) and torch.equal(full.den, pruned.den)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_a_fully_masked_row_keeps_uniform_softmax(K, dtype):
    """Strict causal (lt) masks row 0 entirely: its softmax is uniform over
    the fill, so the kernel must sweep every tile for it (no pruning)."""
    rng = np.random.default_rng(3)
    D = 64
    q, k, v = _qkv(rng, 1, 1, 1, 130, 130, D, D, dtype)
    band = (None, -1)
    res = K.flash_fwd(q, k, v, scale=0.125, band=K.Band(*band), prune=True, want_artifacts=True)
    torch.cuda.synchronize()
    _check_fwd(res, q, k, v, 0.125, band, lowp=dtype != torch.float32)
    np.testing.assert_allclose(_host(res.o)[0, 0, 0], _host(v)[0, 0].mean(axis=0), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("band", [(None, 5), (None, 100), (3, None), (-40, None), (None, 1500)])
def test_half_open_bands(K, dtype, band):
    """Bands with one unbounded end: the masked tiles' per-key limits are
    computed from the bounded end only (an unbounded end entering the
    subtraction would wrap and mask every key of those tiles)."""
    rng = np.random.default_rng(41)
    D = 64 if dtype != torch.float32 else 40
    q, k, v = _qkv(rng, 1, 2, 2, 200, 600, D, D, dtype)
    res = K.flash_fwd(q, k, v, scale=0.125, band=K.Band(*band), want_artifacts=True, nsplit=1)
    torch.cuda.synchronize()
    _check_fwd(res, q, k, v, 0.125, band, lowp=dtype != torch.float32)


def test_sliding_window_band(K):
    rng = np.random.default_rng(21)
    q, k, v = _qkv(rng, 1, 2, 2, 300, 300, 128, 128, torch.bfloat16)
    band = (-63, 0)  # t - s < 64
    res = K.flash_fwd(q, k, v, band=K.Band(*band), want_artifacts=True)
    torch.cuda.synchronize()
    _check_fwd(res, q, k, v, 1 / np.sqrt(128), band, lowp=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "B,Hq,Hkv,T,S,D,band,nsplit",
    [
        (1, 12, 12, 1024, 1024, 64, (None, 0), 4),  # gpt2's attention, the split the picker chooses
        (2, 3, 3, 700, 900, 128, None, 3),  # ragged rows and keys, every key live
        (1, 4, 2, 1000, 1000, 64, (-200, 0), 5),  # a window (most splits of a block empty), GQA
        (1, 2, 2, 600, 600, 128, (None, -1), 2),  # strict causal: row 0 fully masked, no pruning
        (1, 1, 1, 64, 2048, 128, (None, 1500), 7),  # one query block, splits ragged at the key tail
    ],
)
def test_the_key_split_forward_matches_the_oracle_and_the_unsplit_sweep(K, dtype, B, Hq, Hkv, T, S, D, band,
                                                                         nsplit):
    """pdh_flash_fwd_split: the splits' partial (o, max, den) merged by the
    online-softmax combine. Against the float64 closed form (bf16 / f16
    tolerance), and against the unsplit sweep: the m artifact is a max, so
    bit-equal; lse and den within fp32 rounding; o within two 16-bit ulps."""
    rng = np.random.default_rng(T + S + D + nsplit)
    q, k, v = _qkv(rng, B, Hq, Hkv, T, S, D, D, dtype)
    scale = 1.0 / np.sqrt(D)
    kb = K.Band(*band) if band else None
    one = K.flash_fwd(q, k, v, scale=scale, band=kb, want_artifacts=True, nsplit=1)
    res = K.flash_fwd(q, k, v, scale=scale, band=kb, want_artifacts=True, nsplit=nsplit)
    torch.cuda.synchronize()
    _check_fwd(res, q, k, v, scale, band, lowp=True)
    assert torch.equal(one.m, res.m)
    assert_lse(_host(res.lse), _host(one.lse), what="split vs unsplit lse")
    assert ((one.den - res.den).abs() / one.den.abs()).max().item() < 1e-4
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    assert (one.o.float() - res.o.float()).abs().max().item() <= 2 * ulp * max(1.0, one.o.float().abs().max().item())


def test_the_key_split_refuses_a_short_workspace(K):
    import ctypes as C

    from pdum_dsl_amd import _lib as L

    q, k, v = _qkv(np.random.default_rng(1), 1, 2, 2, 256, 1024, 64, 64, torch.bfloat16)
    o = torch.empty_like(q)
    g = K._geom(q, k, v, o)
    need = L.lib().pdh_flash_fwd_workspace(C.byref(g), 4)
    assert need == 4 * 2 * 256 * (64 + 3) * 4
    ws = torch.empty(need // 4, dtype=torch.float32, device="cuda")
    with pytest.raises(Exception, match="ws must"):
        L.call("pdh_flash_fwd_split", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), None, None, None,
               C.byref(g), 1, C.c_float(0.125), C.c_float(-1e9), 0, 0, 0, 1, 4, ws.data_ptr(), C.c_size_t(need - 16),
               None)


# ------------------------------------------------------------------- decode


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "B,Hq,Hkv,T,S,D,nsplit",
    [(2, 8, 2, 1, 1000, 128, 3), (1, 4, 4, 1, 64, 64, 1), (3, 32, 8, 1, 2048, 128, None), (1, 4, 1, 2, 777, 128, 4),
     # 16 query rows per kv head (the MFMA's full width), t > 1 at D = 64, a cache shorter than one
     # 32-key block, and splits past the cache's end (S = 33 in 4 splits of 32 keys: two are empty)
     (1, 16, 1, 1, 300, 128, 2), (2, 4, 2, 3, 100, 64, 3), (1, 2, 2, 1, 5, 128, 1), (1, 8, 2, 1, 33, 128, 4)],
)
def test_decode_matches_oracle(K, dtype, B, Hq, Hkv, T, S, D, nsplit):
    rng = np.random.default_rng(S + Hq)
    q, k, v = _qkv(rng, B, Hq, Hkv, T, S, D, D, dtype)
    o, lse = K.attn_decode(q, k, v, nsplit=nsplit)
    torch.cuda.synchronize()
    want = cf.attention_batched(_host(q), _host(k), _host(v), scale=1 / np.sqrt(D))
    O, L = _host(o), _host(lse)
    for (b, h), (wo, _, _, wlse) in want.items():
        assert_lowp(O[b, h], wo, what=f"decode out[{b},{h}]")
        assert_lse(L[b, h], wlse, what=f"decode lse[{b},{h}]")


def test_entry_points_refuse_bad_shapes_without_launching(K):
    from pdum_dsl_amd._lib import PdhError

    q = torch.zeros((1, 1, 8, 96), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(PdhError, match="e == od"):
        K.flash_fwd(q, q, q)
    with pytest.raises(ValueError, match="f32, bf16 or f16"):
        K.row_softmax(q.double())


@pytest.mark.parametrize("dtype,D,band", [(torch.float32, 64, None), (torch.bfloat16, 128, (None, 0))])
def test_the_prepared_forward_call_equals_the_wrapper(K, dtype, D, band):
    """flash_fwd_prepared binds geometry, pointers and stream once; each call
    launches the same kernel as flash_fwd (bit-equal output and lse)."""
    rng = np.random.default_rng(21)
    q, k, v = _qkv(rng, 1, 2, 2, 256, 256, D, D, dtype)
    b = K.Band(*band) if band else None
    want = K.flash_fwd(q, k, v, scale=D**-0.5, band=b, nsplit=1)
    call = K.flash_fwd_prepared(q, k, v, scale=D**-0.5, band=b)
    for _ in range(3):
        o = call()
    torch.cuda.synchronize()
    assert torch.equal(o, want.o) and torch.equal(call.lse, want.lse)
