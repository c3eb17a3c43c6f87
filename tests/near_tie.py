"""Greedy-token agreement under the reference's near-tie rule (research/phase5/benchmark_review.py:46, 54-67).

Two greedy decodes agree if their tokens are equal, or if they first diverge at a
step where the reference's top-1 / top-2 logit margin is a near-tie. The
reference's bound is 1e-2 on fp32 logits; Qwen3 logits here are bf16, whose spacing
at the top logit is 2^(e-7), so the bound is the larger of 1e-2 and two bf16 ulps
of the top logit (a one-ulp difference in each of the two competing logits).
"""

import math

NEAR_TIE_LOGIT_MARGIN = 1e-2


def near_tie_bound(top1):
    a = abs(float(top1))
    ulp = 2.0 ** (math.floor(math.log2(a)) - 7) if a > 0 else 0.0
    return max(NEAR_TIE_LOGIT_MARGIN, 2 * ulp)


def first_divergence(ref, got):
    for i, (a, b) in enumerate(zip(ref, got)):
        if a != b:
            return i
    return None if len(ref) == len(got) else min(len(ref), len(got))


def near_tie_match(ref, got, margins, tops):
    """(ok, index): `margins[i]` / `tops[i]` are the reference's top-1 minus top-2 and top-1 at step i."""
    i = first_divergence(ref, got)
    if i is None:
        return True, None
    if i >= len(margins):
        return False, i
    return margins[i] < near_tie_bound(tops[i]), i
