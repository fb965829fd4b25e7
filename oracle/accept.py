"""Greedy acceptance and cache-length restatements (oracle; test infrastructure only)."""
from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np

from .attention import _np


def argmax_first(row) -> int:
    """torch.argmax over one row: the first maximum; any NaN counts as the
    maximum (first NaN wins); -0.0 equals +0.0. Used by the reference at
    std_qwen25vl.py:107-108 and :806."""
    x = _np(row).ravel()
    nan = np.isnan(x)
    if nan.any():
        return int(np.argmax(nan))
    return int(np.argmax(x))


def greedy_prefix(draft_tokens: Sequence[int], predictions: Sequence[int]) -> Tuple[int, int]:
    """(accepted_prefix_length, bonus): predictions holds one prediction per
    draft token plus the one after the last draft token.
    Restates src/std_repro/hsd_spike.py:30-43 (including its ValueError)."""
    if len(predictions) != len(draft_tokens) + 1:
        raise ValueError("predictions must contain one bonus row after the draft")
    accepted = 0
    while accepted < len(draft_tokens) and int(draft_tokens[accepted]) == int(predictions[accepted]):
        accepted += 1
    return accepted, int(predictions[accepted])


def verify_predictions(logits, has_pending: bool, dense_next: int = -1) -> List[int]:
    """Prediction list of the parallel verify (std_qwen25vl.py:806-810): the
    argmax of every verify row, preceded by the prefill's dense_next when no
    bonus token was pending (the first round)."""
    x = _np(logits)
    if x.ndim == 3:
        x = x[0]
    preds = [argmax_first(x[r]) for r in range(x.shape[0])]
    return preds if has_pending else [int(dense_next)] + preds


def verify_accept(logits, draft: Sequence[int], has_pending: bool, dense_next: int = -1) -> Tuple[int, int, List[int]]:
    """(accept_len, bonus, predictions) of one verify round (std_qwen25vl.py:806-815)."""
    preds = verify_predictions(logits, has_pending, dense_next)
    a, bonus = greedy_prefix(draft, preds)
    return a, bonus, preds


def rollback_lengths(dense_cached_len: int, n_pending: int, sparse_prev_len: int, accept_len: int) -> Tuple[int, int]:
    """Cache lengths after a round (std_qwen25vl.py:923-928): the dense cache
    keeps the previous pending token and the accepted prefix, the sparse cache
    keeps the accepted prefix; the new bonus is appended later."""
    return dense_cached_len + n_pending + accept_len, sparse_prev_len + accept_len
