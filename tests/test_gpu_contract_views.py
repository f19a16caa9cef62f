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


def _softmax_stat_program(B, T, S, scale, with_max):
    """The pointwise chain of a causal softmax statistic over the scores
    acc[b, t, s]: where(s <= t, scale acc, -1e9), less the row max m[b, t]
    (operand 0) and exponentiated when ``with_max``."""
    from pdum_dsl_amd import _lib as L

    p = L.EwProgram()
    p.ndim = 3
    for d, (ext, st) in enumerate(zip((B, T, S), (T * S, S, 1))):
        p.shape[d], p.out_stride[d] = ext, st
    ins = [("ACC", 0, 0, 0, 0, 0.0), ("CONST", 1, 0, 0, 0, scale), ("MUL", 0, 0, 1, 0, 0.0),
           ("IOTA", 2, 2, 0, 0, 0.0), ("IOTA", 3, 1, 0, 0, 0.0), ("LE", 4, 2, 3, 0, 0.0),
           ("CONST", 5, 0, 0, 0, -1e9), ("WHERE", 6, 4, 0, 5, 0.0)]
    if with_max:
        ins += [("LOAD", 7, 0, 0, 0, 0.0), ("SUB", 8, 6, 7, 0, 0.0), ("EXP", 9, 8, 0, 0, 0.0)]
        p.n_operands = 1
        for d, st in enumerate((T, 1, 0)):
            p.in_stride[0][d] = st
    for i, (op, dst, a, b, c, imm) in enumerate(ins):
        q = p.insns[i]
        q.op, q.dst, q.a, q.b, q.c, q.imm = L.EW[op], dst, a, b, c, imm
    p.n_insns, p.out_reg = len(ins), ins[-1][1]
    return p


@pytest.mark.parametrize("la,lb", [("k", "k"), ("r", "r")])
@pytest.mark.parametrize("mode", [6, 0])
@pytest.mark.parametrize("B,T,S,E", [(3, 200, 300, 64), (2, 1024, 1024, 64)])
def test_row_partials_of_softmax_statistics(la, lb, mode, B, T, S, E):
    """pdh_contract_views_rowred: per 32-column run, the max of the masked
    scaled scores and the sum of their exponentials less the row max, against
    float64 numpy; ragged runs (S = 300) leave out the columns past S."""
    from pdum_dsl_amd import kernels as K

    x, y = _inputs(B, T, S, E, seed=26)
    (a, sa), (bt, sb) = _lay(x, la), _lay(y, lb)
    scale = E ** -0.5
    sc = np.einsum("bte,bse->bts", x.double().cpu().numpy(), y.double().cpu().numpy()) * scale
    causal = np.arange(S)[None, None, :] <= np.arange(T)[None, :, None]
    masked = np.where(causal, sc, -1e9)
    nblk = -(-S // 32)
    pad = np.full((B, T, nblk * 32), -np.inf)
    pad[..., :S] = masked
    want_max = pad.reshape(B, T, nblk, 32).max(-1)
    part = torch.empty(B, T, nblk, device="cuda")
    K.contract_views_rowred(a, sa, bt, sb, (B, T, S, E), _softmax_stat_program(B, T, S, scale, False), [], "max",
                            part, f32_mode=MODES[mode])
    torch.cuda.synchronize()
    got = part.double().cpu().numpy()
    assert np.abs(got - want_max).max() <= 1e-5 * np.abs(sc).max()
    m = torch.tensor(masked.max(-1), device="cuda", dtype=torch.float32)
    e = np.exp(masked - m.double().cpu().numpy()[..., None])
    pad = np.zeros((B, T, nblk * 32))
    pad[..., :S] = e
    want_sum = pad.reshape(B, T, nblk, 32).sum(-1)
    K.contract_views_rowred(a, sa, bt, sb, (B, T, S, E), _softmax_stat_program(B, T, S, scale, True), [m], "sum",
                            part, f32_mode=MODES[mode])
    torch.cuda.synchronize()
    got = part.double().cpu().numpy()
    assert np.abs(got - want_sum).max() <= 1e-5 * 32 * max(1.0, np.abs(sc).max())


def test_row_partials_propagate_nan_and_leave_clean_runs_alone():
    """A NaN in one score poisons its row's max run (as the row reduction's
    max does) and only that run; min is the max's mirror."""
    from pdum_dsl_amd import kernels as K

    B, T, S, E = 1, 130, 100, 64
    x, y = _inputs(B, T, S, E, seed=27)
    x[0, 7, 5] = float("nan")
    (a, sa), (bt, sb) = _lay(x, "k"), _lay(y, "k")
    part = torch.empty(B, T, 4, device="cuda")
    ident = _identity(B, T, S)
    for red in ("max", "min"):
        K.contract_views_rowred(a, sa, bt, sb, (B, T, S, E), ident, [], red, part)
        torch.cuda.synchronize()
        got = part.double().cpu().numpy()
        nan = np.isnan(got)
        assert nan[0, 7].all() and nan.sum() == 4  # row 7: every run reads the NaN through the product
        sc = np.einsum("bte,bse->bts", x.double().cpu().numpy(), y.double().cpu().numpy())
        pad = np.full((B, T, 128), -np.inf if red == "max" else np.inf)
        pad[..., :S] = sc
        want = getattr(pad.reshape(B, T, 4, 32), red)(-1)
        ok = ~nan
        assert np.abs(got[ok] - want[ok]).max() <= 1e-5 * np.abs(sc[np.isfinite(sc)]).max()
