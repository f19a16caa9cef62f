"""The allocation-free decode (pdh_attn_decode_noalloc) on the GPU: the split
partials in the library's per-GPU scratch array instead of a caller
workspace. Its output must equal pdh_attn_decode's bit for bit (the same
kernels over the same partial order), on two calls in a row, the second
smaller than the first, so stale contents of the shared array from the first
call cannot leak into the second; the first call's partials fill 95% of the
array. And the entry does what it is for: it replays in a captured graph."""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _inputs(rng, B, Hq, Hkv, S, D, dtype):
    q = torch.as_tensor(rng.standard_normal((B, Hq, 1, D))).to(dtype=dtype, device="cuda")
    k = torch.as_tensor(rng.standard_normal((B, Hkv, S, D))).to(dtype=dtype, device="cuda")
    v = torch.as_tensor(rng.standard_normal((B, Hkv, S, D))).to(dtype=dtype, device="cuda")
    return q, k, v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_static_scratch_decode_equals_the_workspace_decode(dtype):
    from pdum_dsl_amd import kernels as K

    from pdum_dsl_amd import _lib

    rng = np.random.default_rng(11)
    g = torch.Generator(device="cuda").manual_seed(11)
    # the first call fills 95% of the array; the second, smaller, reuses it
    first = (64, 32, 8, 1024, 128, 15)
    geom = _lib.AttnGeom()
    geom.batch, geom.heads_q, geom.heads_kv, geom.t, geom.s, geom.e, geom.od = 64, 32, 8, 1, 1024, 128, 128
    need = _lib.lib().pdh_attn_decode_workspace(C.byref(geom), first[5])
    assert 0.9 * _lib.DECODE_SCRATCH_BYTES < need <= _lib.DECODE_SCRATCH_BYTES
    for B, Hq, Hkv, S, D, nsplit in (first, (3, 8, 2, 1000, 64, 3)):
        if B == 64:  # large: drawn on the device
            q = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(dtype)
            k = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(dtype)
            v = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(dtype)
        else:
            q, k, v = _inputs(rng, B, Hq, Hkv, S, D, dtype)
        o_ref, lse_ref = K.attn_decode(q, k, v, nsplit=nsplit)
        o = torch.full_like(o_ref, float("nan"))
        lse = torch.full_like(lse_ref, float("nan"))
        K.attn_decode_static(q, k, v, o, lse, nsplit=nsplit)
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), f"out differs at B={B} S={S} D={D}"
        assert torch.equal(lse, lse_ref), f"lse differs at B={B} S={S} D={D}"


def test_static_scratch_decode_refuses_an_oversized_request():
    from pdum_dsl_amd import _lib

    lib = _lib.lib()
    g = _lib.AttnGeom()
    g.batch, g.heads_q, g.heads_kv, g.t, g.s, g.e, g.od = 64, 32, 8, 1, 8192, 128, 128
    need = lib.pdh_attn_decode_workspace(C.byref(g), 64)
    assert need > _lib.DECODE_SCRATCH_BYTES
    rc = lib.pdh_attn_decode_noalloc(None, None, None, None, None, C.byref(g), _lib.PDH_BF16, 1.0, 64, None)
    assert rc == _lib.PDH_EINVAL and "scratch array holds" in _lib.last_error()


def test_static_scratch_decode_replays_in_a_graph():
    """The point of the allocation-free entry: capture it in a graph. Each
    replay, with eager work and new query values between replays, equals the
    workspace decode of the current inputs bit for bit."""
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(29)
    B, Hq, Hkv, S, D, nsplit = 4, 16, 4, 2048, 128, 4
    q = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(torch.bfloat16)
    o = torch.empty((B, Hq, 1, D), device="cuda", dtype=torch.bfloat16)
    lse = torch.empty((B, Hq, 1), device="cuda", dtype=torch.float32)
    K.attn_decode_static(q, k, v, o, lse, nsplit=nsplit)  # resolves the scratch address before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        K.attn_decode_static(q, k, v, o, lse, nsplit=nsplit)
    torch.cuda.synchronize()
    for rep in range(3):
        q.copy_(torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(torch.bfloat16))
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        o_ref, lse_ref = K.attn_decode(q, k, v, nsplit=nsplit)  # eager, between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), f"replay {rep}: out differs"
        assert torch.equal(lse, lse_ref), f"replay {rep}: lse differs"
