"""Greedy speculative acceptance (reference: chomikgrad/generation.py:15-28)."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence, Tuple


@dataclass(frozen=True)
class GreedyVerification:
    """Decision for one greedy speculative block."""

    emitted_tokens: Tuple[int, ...]
    accepted_draft_tokens: int


def verify_greedy_candidates(
    draft_tokens: Sequence[int], target_tokens: Sequence[int]
) -> GreedyVerification:
    """Accept the longest draft prefix that equals the target's greedy choice;
    at the first mismatch emit the target token instead."""
    draft = tuple(int(token) for token in draft_tokens)
    target = tuple(int(token) for token in target_tokens)
    if not draft:
        raise ValueError("speculative verification requires at least one token")
    if len(draft) != len(target):
        raise ValueError("draft and target blocks must have equal lengths")
    accepted = 0
    while accepted < len(draft) and draft[accepted] == target[accepted]:
        accepted += 1
    if accepted == len(draft):
        return GreedyVerification(draft, accepted)
    return GreedyVerification(draft[:accepted] + (target[accepted],), accepted)


def verify_greedy_block_with_bonus(
    draft_tokens: Sequence[int], target_tokens: Sequence[int]
) -> GreedyVerification:
    """Verify ``k`` draft tokens against ``k + 1`` target predictions.

    The target block is ``[last, d1, ..., dk]``, so its last prediction
    follows ``dk``: when every draft token is accepted it is emitted as a
    bonus token.  No reference counterpart: the reference verifies ``k``
    positions ``[last, d1, ..., d_{k-1}]`` (generate_tinyllama.py:607-614).
    """
    target = tuple(int(token) for token in target_tokens)
    if len(target) != len(draft_tokens) + 1:
        raise ValueError("the target block must hold one more prediction than the draft")
    decision = verify_greedy_candidates(draft_tokens, target[:-1])
    if decision.accepted_draft_tokens == len(draft_tokens):
        return GreedyVerification(decision.emitted_tokens + (target[-1],), len(draft_tokens))
    return decision
