"""The executor's k-split choice for fp32 contractions (host logic, no GPU):
candidates never leave a k slice empty, a GEMM that fills the chip is not
split, and long-k contractions with few output tiles are."""

from pdum_dsl_amd.executor import _big_tiles, _ksplit_est, _ksplit_order


def test_candidates_leave_no_slice_empty():
    for kt in (4, 5, 12, 16, 48, 786):
        for S in _ksplit_order(1, 1024, 768, kt):
            kc = -(-kt // S)
            assert (S - 1) * kc < kt and (S == 1 or kc >= 2), (kt, S)


def test_the_order_is_by_estimated_cost():
    order = _ksplit_order(1, 768, 768, 16)
    costs = [_ksplit_est(1, 768, 768, 16, S) for S in order]
    assert costs == sorted(costs)


def test_chip_filling_and_long_k_shapes():
    # gpt2-small's logits (1024 x 50257, k = 768): 3144 big tiles, no split
    assert _ksplit_order(1, 1024, 50257, 12)[0] == 1
    # its input gradient (1024 x 768, k = 50257): 48 tiles, k split about tenfold
    assert 8 <= _ksplit_order(1, 1024, 768, 786)[0] <= 12
    # 768 x 768 weight gradients over 1024 tokens: split
    assert _ksplit_order(1, 768, 768, 16)[0] > 1


def test_the_tile_rule_avoids_half_empty_tiles():
    assert _big_tiles(12 * 4, 1024, 1024)
    assert not _big_tiles(12 * 4, 1024, 64)  # an output side of 64: 64 x 64 tiles
    assert not _big_tiles(1, 1024, 768)  # 48 big tiles cannot fill 256 compute units
