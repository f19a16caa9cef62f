"""pdh_contract_views on silicon: fp32 contractions whose operands are read in
place, k contiguous or rows contiguous (a transposed tensor), any k.

Against float64 numpy on the same fp32 inputs; and, since an element's bf16
planes and the order of the matrix-core sums do not depend on how the operand
was laid out in memory, bit for bit against the k-contiguous layout of the
same values and against pdh_contract_strided where both apply."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

MODES = {6: "bf16x6", 3: "bf16x3", 0: "fma"}


def _identity(B, M, N):
    from pdum_dsl_amd import _lib as L

    p = L.EwProgram()
    p.n_insns, p.n_operands, p.ndim, p.out_reg = 1, 0, 3, 0
    for d, (ext, st) in enumerate(zip((B, M, N), (M * N, N, 1))):
        p.shape[d], p.out_stride[d] = ext, st
    p.insns[0].op = L.EW["ACC"]
    return p


def _lay(x, layout, pad=3):
    """x [B, R, K] (fp32, device) stored k-contiguous ('k': rows of K + pad)
    or rows-contiguous ('r': [B, K, R + pad]); returns (tensor, strides)."""
    B, R, Kd = x.shape
    if layout == "k":
        t = torch.full((B, R, Kd + pad), float("nan"), device="cuda")
        t[..., :Kd] = x
        return t, (R * (Kd + pad), Kd + pad, 1)
    t = torch.full((B, Kd, R + pad), float("nan"), device="cuda")
    t[..., :R] = x.transpose(1, 2)
    return t, (Kd * (R + pad), 1, R + pad)


def _views(a, sa, bt, sb, shape, mode=6, ksplit=1):
    from pdum_dsl_amd import kernels as K

    B, M, N, _k = shape
    out = torch.empty(B * ksplit, M, N, device="cuda")
    K.contract_views(a, sa, bt, sb, shape, _identity(B * ksplit, M, N), [], out, f32_mode=MODES[mode],
                     ksplit=ksplit)
    torch.cuda.synchronize()
    return out


def _inputs(B, M, N, Kd, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(B, M, Kd, device="cuda", generator=g),
            torch.randn(B, N, Kd, device="cuda", generator=g) * 3.0)


# (B, M, N, K): 64 x 64 tiles with k under one tile, ragged everything; 128 x
# 128 tiles (B * 9 * 9 >= 256 workgroups) with k not a multiple of 4
SHAPES = [(2, 70, 90, 40), (2, 300, 260, 200), (4, 1100, 1030, 333)]


@pytest.mark.parametrize("la,lb", [("k", "k"), ("r", "k"), ("k", "r"), ("r", "r")])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("mode", [6, 0])
def test_views_against_float64(la, lb, shape, mode):
    """Every layout pair, ragged m, n and k (the padding past k holds NaN,
    which must never be read), against float64 numpy."""
    B, M, N, Kd = shape
    x, y = _inputs(B, M, N, Kd, seed=21)
    (a, sa), (bt, sb) = _lay(x, la), _lay(y, lb)
    got = _views(a, sa, bt, sb, shape, mode).double().cpu().numpy()
    want = np.einsum("bmk,bnk->bmn", x.double().cpu().numpy(), y.double().cpu().numpy())
    tol = 1e-5 * np.abs(want).max() * max(1.0, (Kd / 64) ** 0.5)  # fp32 grade per sqrt of summation depth
    assert np.isfinite(got).all() and np.abs(got - want).max() <= tol


@pytest.mark.parametrize("shape", SHAPES)
def test_the_layout_does_not_change_a_bit(shape):
    """The same values read k-contiguous or rows-contiguous give identical
    outputs (the planes and the summation order are the layout's invariants),
    and a 64-aligned k-contiguous case is pdh_contract_strided's result."""
    from pdum_dsl_amd import kernels as K

    B, M, N, Kd = shape
    x, y = _inputs(B, M, N, Kd, seed=22)
    ref = _views(*_lay(x, "k"), *_lay(y, "k"), shape)
    for la, lb in (("r", "k"), ("k", "r"), ("r", "r")):
        (a, sa), (bt, sb) = _lay(x, la), _lay(y, lb)
        assert torch.equal(_views(a, sa, bt, sb, shape), ref), (la, lb)
    K64 = Kd // 64 * 64
    if K64:
        xs, ys = x[..., :K64].contiguous(), y[..., :K64].contiguous()
        via = torch.empty(B, M, N, device="cuda")
        K.contract_strided(xs, (M * K64, K64), ys, (N * K64, K64), (B, M, N, K64), _identity(B, M, N), [], via,
                           f32_mode="bf16x6")
        (a, sa), (bt, sb) = _lay(xs, "r"), _lay(ys, "r")
        assert torch.equal(_views(a, sa, bt, sb, (B, M, N, K64)), via)


@pytest.mark.parametrize("la,lb", [("k", "k"), ("r", "r"), ("r", "k")])
@pytest.mark.parametrize("S", [2, 3, 4])
def test_ragged_k_slices_are_the_slices_products(la, lb, S):
    """ksplit slices of whole 64-column tiles, the last one ragged: index
    e * S + s is bit for bit the unsplit product over slice s's columns
    alone, and the slices sum to the whole product."""
    B, M, N, Kd = 2, 150, 130, 1000
    x, y = _inputs(B, M, N, Kd, seed=23)
    (a, sa), (bt, sb) = _lay(x, la), _lay(y, lb)
    parts = _views(a, sa, bt, sb, (B, M, N, Kd), ksplit=S).view(B, S, M, N)
    tiles = -(-Kd // 64)
    kc = -(-tiles // S) * 64  # columns per slice: whole 64-column tiles
    for s in range(S):
        k0, ks = s * kc, min(kc, Kd - s * kc)
        (a1, sa1), (b1, sb1) = _lay(x[..., k0:k0 + ks], la), _lay(y[..., k0:k0 + ks], lb)
        assert torch.equal(parts[:, s], _views(a1, sa1, b1, sb1, (B, M, N, ks))), s
    want = np.einsum("bmk,bnk->bmn", x.double().cpu().numpy(), y.double().cpu().numpy())
    got = parts.double().sum(1).cpu().numpy()
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() * 4


def test_broadcast_strides():
    """A stride of 0 reads one row (k-contiguous a, sa_r = 0) or one column
    for every k (rows-contiguous bt, sb_k = 0)."""
    B, M, N, Kd = 1, 100, 120, 300
    g = torch.Generator(device="cuda").manual_seed(24)
    row = torch.randn(Kd, device="cuda", generator=g)
    col = torch.randn(N, device="cuda", generator=g)
    got = _views(row, (0, 0, 1), col, (0, 1, 0), (B, M, N, Kd)).double().cpu().numpy()
    want = np.broadcast_to(row.double().sum().item() * col.double().cpu().numpy(), (B, M, N))
    # the terms cancel: fp32 grade is relative to the sum of their magnitudes
    scale = row.double().abs().sum().item() * col.double().abs().max().item()
    assert np.abs(got - want).max() <= 1e-6 * scale


@pytest.mark.parametrize("mode", [6, 3])
def test_non_finite_values_of_a_transposed_operand(mode):
    """A workgroup that loads a non-finite value recomputes its tile by fp32
    fma through the same strides: infs and NaNs land where IEEE arithmetic
    puts them, rows-contiguous operands included."""
    g = torch.Generator(device="cuda").manual_seed(25)
    B, M, N, Kd = 1, 700, 600, 250
    x = torch.randn(B, M, Kd, device="cuda", generator=g)
    y = torch.randn(B, N, Kd, device="cuda", generator=g).round()  # exact in bf16: zero lower planes
    y[y == 0] = 1.0
    x[0, 5, 17] = float("inf")
    x[0, 650, 3] = -float("inf")
    y[0, 333, 40] = float("nan")
    (a, sa), (bt, sb) = _lay(x, "r"), _lay(y, "r")
    got = _views(a, sa, bt, sb, (B, M, N, Kd), mode).double().cpu().numpy()
    want = np.einsum("bmk,bnk->bmn", x.double().cpu().numpy(), y.double().cpu().numpy())
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.isnan(want).sum() == M
    assert np.array_equal(np.isinf(got), np.isinf(want)) and np.array_equal(got[np.isinf(got)], want[np.isinf(want)])
    fin = np.isfinite(want)
    tol = (1e-5 if mode == 6 else 5e-5) * np.abs(want[fin]).max() * 2.0
    assert np.abs(got[fin] - want[fin]).max() <= tol
