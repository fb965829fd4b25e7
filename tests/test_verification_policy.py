"""The verification fallback policies of the generate loop
(std_amd/verification_policy.py) against the reference's own known answers
(tests/test_verification_fallback.py:13-84, restated as data in
golden/reference_kats.json), plus the cases those leave open: a margin over
rows without a logit row, every mode name, length-only differences."""
import json
import os

import pytest
import torch

from std_amd.verification_policy import (VERIFY_FALLBACKS, min_prediction_margin, needs_sequential_fallback,
                                         positional_token_metrics)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def test_needs_sequential_fallback_kats():
    table = _kats()["needs_sequential_fallback"]
    for case in table["cases"]:
        got = needs_sequential_fallback(case["mode"], accept_len=case["accept_len"], draft_len=case["draft_len"],
                                        sequential_fallback_max_accept=table["sequential_fallback_max_accept"],
                                        low_margin=case["low_margin"])
        assert got is case["expected"], case


def test_needs_sequential_fallback_every_mode_on_a_full_accept_and_a_rejection():
    # a fully accepted draft replays only under the guard (or a low margin)
    assert [needs_sequential_fallback(m, accept_len=9, draft_len=9, sequential_fallback_max_accept=9,
                                      low_margin=False) for m in VERIFY_FALLBACKS] == [False, True, False, False, False]
    # a rejection at 0 accepted replays under every mode but "none" and the margin mode without a low margin
    assert [needs_sequential_fallback(m, accept_len=0, draft_len=9, sequential_fallback_max_accept=0,
                                      low_margin=False) for m in VERIFY_FALLBACKS] == [False, True, False, True, True]
    assert not needs_sequential_fallback("unknown", accept_len=0, draft_len=9, sequential_fallback_max_accept=1,
                                         low_margin=True)


def test_min_prediction_margin_kats():
    for case in _kats()["min_prediction_margin"]:
        got = min_prediction_margin(torch.tensor(case["logits"]), case["prediction_indices"],
                                    has_dense_pending=case["has_dense_pending"])
        assert got == pytest.approx(case["expected"])


def test_min_prediction_margin_without_rows_and_with_a_tie():
    logits = torch.tensor([[[1.0, 1.0, 0.0], [7.0, 2.0, 0.0]]])
    # without a pending token prediction 0 has no row: None when it is the only one
    assert min_prediction_margin(logits, [0], has_dense_pending=False) is None
    assert min_prediction_margin(logits, [5, 6], has_dense_pending=True) is None
    # an exact tie for the top logit has margin 0
    assert min_prediction_margin(logits, [0, 1], has_dense_pending=True) == 0.0
    assert min_prediction_margin(logits, [2], has_dense_pending=False) == pytest.approx(5.0)


def test_positional_token_metrics_kats_and_length_only_differences():
    for case in _kats()["positional_token_metrics"]:
        m = positional_token_metrics(torch.tensor(case["reference"]), torch.tensor(case["candidate"]))
        assert m["mismatch_token_count"] == case["mismatch_token_count"]
        assert m["token_level_agreement"] == pytest.approx(case["token_level_agreement"])
    m = positional_token_metrics(torch.tensor([5, 6]), torch.tensor([5, 6, 7, 8]))
    assert m["mismatch_token_count"] == 2 and m["token_level_agreement"] == pytest.approx(0.5)
    m = positional_token_metrics(torch.tensor([], dtype=torch.long), torch.tensor([], dtype=torch.long))
    assert m == {"mismatch_token_count": 0, "token_level_agreement": 1.0}
