"""The allocation-free decode (pdh_attn_decode_noalloc) on the GPU: the split
partials in the library's per-GPU scratch array instead of a caller
workspace. Its output must equal pdh_attn_decode's bit for bit (the same
kernels over the same partial order), on two calls in a row, the second
smaller than the first, so stale contents of the shared array from the first
call cannot leak into the second."""

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

    rng = np.random.default_rng(11)
    # the first call fills much of the array; the second, smaller, reuses it
    for B, Hq, Hkv, S, D, nsplit in ((16, 32, 8, 8192, 128, 6), (3, 8, 2, 1000, 64, 3)):
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
