"""Process-wide switches of the HIP realizer front end.

Fusion (the reference's packages/browsergrad-jit/src/python/_fusion_config.py:
20-50): fusion is on by default; ``use_fusion(False)`` turns it off for the
process, and the environment variable ``BG_DISABLE_FUSION`` set to 1 / true /
yes / on turns it off whatever the Python switch says.  Off means the walker
and the plan builder see the cast-inserted graph as built: neither the
reference's chain / softmax fusion nor this package's subgraph rewrites
(GEMM epilogues, fused attention, elementwise + reduce programs) run.

Attention score rounding (no reference counterpart): the reference's AMP
graph rounds the score matrix Q K^T to the narrow dtype before scaling
(_realize.py:395-412).  The fused attention kernel keeps S in f32 by default,
which is at least as accurate and stays inside the 16-bit parity tolerance;
``exact_attention_score_rounding(True)`` (or ``BG_ATTN_EXACT_ROUNDING=1``)
makes the walker ask the kernel for the reference's rounding instead
(``round_scores`` of bg_attention_ex), at some cost in speed.

The element ceiling per tensor (_ir.py:360-368) lives in ir.py as
``set_max_elements`` and is re-exported here.
"""
from __future__ import annotations

import os

from .ir import set_max_elements

_TRUE = ("1", "true", "yes", "on")

_fusion_on = True
_exact_scores = False


def _env_flag(name: str) -> bool:
    return os.environ.get(name, "").strip().lower() in _TRUE


def use_fusion(enabled: bool) -> None:
    """Turn fusion on or off for this process (``BG_DISABLE_FUSION`` wins)."""
    global _fusion_on
    _fusion_on = bool(enabled)


def fusion_enabled() -> bool:
    return _fusion_on and not _env_flag("BG_DISABLE_FUSION")


def exact_attention_score_rounding(enabled: bool) -> None:
    """Ask the fused attention kernel to round S to the narrow dtype before
    scaling, as the reference graph does (``BG_ATTN_EXACT_ROUNDING=1`` also
    turns it on)."""
    global _exact_scores
    _exact_scores = bool(enabled)


def attention_rounds_scores() -> bool:
    return _exact_scores or _env_flag("BG_ATTN_EXACT_ROUNDING")


__all__ = ["use_fusion", "fusion_enabled", "exact_attention_score_rounding", "attention_rounds_scores",
           "set_max_elements"]
