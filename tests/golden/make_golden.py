"""Regenerate the golden fixtures (small .npz files) from the float64 oracle.

The reference ships no golden-vector files (every pin in its suites is a
seeded inline draw against a closed form), so these fixtures are this
build's: seeded inputs drawn with the SAME seeds the reference's own tests
use (default_rng(7) for flash_tile, zoo/tiles.py:143; default_rng(9) for the
row-normalization subject, test_fusion.py:105; default_rng(6) for
flash_attention, zoo/attention.py:167), and the oracle's outputs.

    python tests/golden/make_golden.py
"""

from pathlib import Path
import sys

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import closed_forms as cf  # noqa: E402


def main():
    # flash_tile's subject: T=6, E=3, OD=2, causal, seed 7 (q, k, v drawn in that order)
    rng = np.random.default_rng(7)
    q, k, v = rng.standard_normal((6, 3)), rng.standard_normal((6, 3)), rng.standard_normal((6, 2))
    out, m, den, lse = cf.attention(q, k, v, band=(None, 0))
    np.savez(HERE / "flash_tile_T6_causal.npz", q=q, k=k, v=v, out=out, m=m, den=den, lse=lse)
    dout = np.random.default_rng(70).standard_normal((6, 2))
    dq, dk, dv = cf.attention_bwd(q, k, v, dout, band=(None, 0))
    np.savez(HERE / "flash_tile_T6_causal_bwd.npz", q=q, k=k, v=v, dout=dout, dq=dq, dk=dk, dv=dv)

    # flash_attention's subject: T=5, E=3, OD=2, causal, seed 6
    rng = np.random.default_rng(6)
    q, k, v = rng.standard_normal((5, 3)), rng.standard_normal((5, 3)), rng.standard_normal((5, 2))
    out, m, den, lse = cf.attention(q, k, v, band=(None, 0))
    np.savez(HERE / "flash_attention_T5_causal.npz", q=q, k=k, v=v, out=out, m=m, den=den, lse=lse)

    # strict causal (row 0 fully masked: uniform over the fill) and a window of 3
    rng = np.random.default_rng(3)
    q, k, v = rng.standard_normal((8, 4)), rng.standard_normal((8, 4)), rng.standard_normal((8, 3))
    for tag, band in (("strict", (None, -1)), ("window3", (-2, 0)), ("all", None)):
        out, m, den, lse = cf.attention(q, k, v, band=band)
        np.savez(HERE / f"attention_T8_{tag}.npz", q=q, k=k, v=v, out=out, m=m, den=den, lse=lse)

    # the row-normalization subject: X (4, 6), seed 9
    x = np.random.default_rng(9).standard_normal((4, 6))
    np.savez(HERE / "softmax_4x6.npz", x=x, y=cf.np_softmax(x, axis=1))

    # layernorm with gamma ~ N(1, 0.1), beta ~ N(0, 0.1), eps 1e-5, seed 2
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 6))
    g = 1 + 0.1 * rng.standard_normal(6)
    b = 0.1 * rng.standard_normal(6)
    np.savez(HERE / "layernorm_4x6.npz", x=x, g=g, b=b, y=cf.np_layernorm(x, g, b, 1e-5))


if __name__ == "__main__":
    main()
