"""Declared deviations (the reference's license schema,
packages/tensorlib/src/pdum/tl/licenses.py:1-90): a license names the kind
of deviation a lowering takes (closed taxonomy), the claim, and the
tolerance it is certified at. The HIP column adds one precision-demotion
row for its 16-bit MFMA attention, at the north-star tolerance."""

from __future__ import annotations

from dataclasses import dataclass

KINDS = ("none", "reassociation", "precision-demotion")


@dataclass(frozen=True)
class License:
    name: str
    kind: str
    equivalence: str
    rtol: float
    atol: float
    input_domain: str
    notes: str = ""

    def __post_init__(self):
        if self.kind not in KINDS:
            raise ValueError(f"license kind must be one of {KINDS}, got {self.kind!r} — the taxonomy is closed")


FLASH_ONLINE_SOFTMAX = (
    License(
        name="flash.online-softmax",
        kind="reassociation",
        equivalence="softmax.V over s re-bracketed by tile (so, si) with running-max rescale (online-softmax lemma)",
        rtol=1e-6,
        atol=1e-7,
        input_domain="finite masked scores; the -1e9 mask fill (exp underflows exactly to 0)",
    ),
)

GEMM_K_REASSOC = (
    License(
        name="gemm.k-reassoc",
        kind="reassociation",
        equivalence="sum over k re-bracketed by tile (ko, ki)",
        rtol=1e-6,
        atol=1e-7,
        input_domain="finite operands",
    ),
)

# the HIP column's 16-bit attention: q/k/v/P read at bf16 (or f16) into
# v_mfma_f32_32x32x16, every accumulation and the softmax statistics at fp32
HIP_ATTN_BF16 = (
    License(
        name="hip.attn.bf16tile.f32acc",
        kind="precision-demotion",
        equivalence="q, k, v and P rounded to bf16 at the MFMA operands; scores, max, denominator and the "
        "output accumulator in fp32; output rounded once to bf16",
        rtol=2e-2,
        atol=2e-2,
        input_domain="finite inputs within bf16 range; max-abs-err relative to max(1, |reference|)",
    ),
)
