"""Verification fallback policies of the generate loop, with the names and
meaning of the reference's std_repro/verification_policy.py (its functions
positional_token_metrics, min_prediction_margin and needs_sequential_fallback,
lines 10-64). They decide on the host, from one round's verify result, whether
that round is replayed sequentially; nothing here runs on the decode hot path
itself."""
from __future__ import annotations

from typing import Dict, Iterable, Optional

import torch

SEQUENTIAL_FALLBACKS = ("sequential_guard", "sequential_on_low_margin", "sequential_on_reject",
                        "sequential_on_low_accept")
VERIFY_FALLBACKS = ("none",) + SEQUENTIAL_FALLBACKS


def positional_token_metrics(reference: torch.Tensor, candidate: torch.Tensor) -> Dict[str, float]:
    """Token-by-token disagreement of two token sequences (any shapes, read
    flat): positions where both have a token and the tokens differ, plus every
    position only one of them has. token_level_agreement is 1 minus that count
    over the longer length (1.0 for two empty sequences)."""
    ref = reference.reshape(-1).tolist()
    cand = candidate.reshape(-1).tolist()
    longer = max(len(ref), len(cand))
    mismatches = sum(a != b for a, b in zip(ref, cand)) + abs(len(ref) - len(cand))
    return {"mismatch_token_count": mismatches,
            "token_level_agreement": (1.0 - mismatches / longer) if longer else 1.0}


def min_prediction_margin(logits: torch.Tensor, prediction_indices: Iterable[int],
                          has_dense_pending: bool) -> Optional[float]:
    """Smallest gap between the two largest logits over the verify rows that
    produced the committed predictions. logits is the verify forward's
    [1, rows, vocab]. Prediction i comes from row i when a pending token led
    the verify input, else from row i - 1 (prediction 0 is then the token the
    previous step already produced, with no row in this verify); indices with
    no row are skipped. None when no index has a row."""
    n_rows = int(logits.shape[1])
    shift = 0 if has_dense_pending else 1
    rows = sorted({int(i) - shift for i in prediction_indices if 0 <= int(i) - shift < n_rows})
    if not rows:
        return None
    picked = logits[0, rows, :].float()
    top2 = torch.topk(picked, 2, dim=-1).values
    return float((top2[:, 0] - top2[:, 1]).min())


def needs_sequential_fallback(mode: str, *, accept_len: int, draft_len: int, sequential_fallback_max_accept: int,
                              low_margin: bool) -> bool:
    """Whether a round verified in parallel is replayed one token at a time:
    always ("sequential_guard"), when a committed prediction had a low margin
    ("sequential_on_low_margin"), when a draft token was rejected
    ("sequential_on_reject"), or when one was rejected after at most
    sequential_fallback_max_accept accepted ones ("sequential_on_low_accept");
    never for "none" or any other mode."""
    rejected = accept_len < draft_len
    if mode == "sequential_guard":
        return True
    if mode == "sequential_on_low_margin":
        return bool(low_margin)
    if mode == "sequential_on_reject":
        return rejected
    if mode == "sequential_on_low_accept":
        return rejected and accept_len <= sequential_fallback_max_accept
    return False
