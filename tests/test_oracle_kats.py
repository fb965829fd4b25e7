"""The reference's own known-answer tests for this path, restated against the oracle.

Sources: tests/test_hsd_spike.py:6-18 (greedy prefix),
tests/test_sparse_verify_spike.py:34-80 (offset-causal mask, batched ==
sequential, no future leakage), tests/test_verification_fallback.py:45-73
(prediction-row convention with and without a pending token),
tests/test_sparse_cache_refresh.py:30-49 (unique-valued compaction fixture).
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import accept, attention, selection

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def test_greedy_prefix_kats():
    for case in _kats()["greedy_prefix"]:
        assert accept.greedy_prefix(case["draft"], case["predictions"]) == tuple(case["expected"])


def test_greedy_prefix_missing_bonus_raises():
    for case in _kats()["greedy_prefix_invalid"]:
        with pytest.raises(ValueError):
            accept.greedy_prefix(case["draft"], case["predictions"])


def test_offset_mask_kat():
    kat = _kats()["offset_causal_mask"]
    mask = attention.offset_causal_mask(kat["q_len"], kat["kv_len"])
    assert mask.shape == (1, 1, kat["q_len"], kat["kv_len"])
    for row, visible in enumerate(kat["visible_prefix"]):
        assert np.all(mask[0, 0, row, :visible] == 0)
        assert np.all(np.isneginf(mask[0, 0, row, visible:]))
    assert attention.offset_causal_mask(1, 4) is None
    with pytest.raises(ValueError):
        attention.offset_causal_mask(5, 4)


def test_batched_verify_matches_sequential():
    torch.manual_seed(7)
    q = torch.randn(1, 4, 3, 8)
    k = torch.randn(1, 2, 7, 8)
    v = torch.randn(1, 2, 7, 8)
    batched = attention.verify_attention(q, k, v)
    offset = k.shape[-2] - q.shape[-2]
    rows = [attention.verify_attention(q[:, :, i:i + 1], k[:, :, :offset + i + 1], v[:, :, :offset + i + 1])
            for i in range(q.shape[-2])]
    np.testing.assert_allclose(batched, np.concatenate(rows, axis=2), atol=1e-5, rtol=1e-5)


def test_verify_has_no_future_leakage():
    torch.manual_seed(11)
    q = torch.randn(1, 2, 2, 4)
    k = torch.randn(1, 1, 5, 4)
    v = torch.randn(1, 1, 5, 4)
    base = attention.verify_attention(q, k, v)
    changed = v.clone()
    changed[:, :, -1] += 10000
    altered = attention.verify_attention(q, k, changed)
    np.testing.assert_allclose(base[:, :, :1], altered[:, :, :1], atol=1e-5, rtol=1e-5)
    assert not np.allclose(base[:, :, 1:], altered[:, :, 1:], atol=1e-5, rtol=1e-5)


def test_prediction_rows_with_and_without_pending():
    kat = _kats()["prediction_rows"]
    logits = torch.tensor(kat["logits"])
    assert accept.verify_predictions(logits, has_pending=True) == kat["with_pending"]
    assert accept.verify_predictions(logits, has_pending=False, dense_next=kat["dense_next"]) == kat["without_pending"]


def test_compaction_unique_valued_fixture():
    """Unique KV values make a wrong head, layer or slot visible."""
    non_visual = np.array([0, 4, 8])
    topk = np.array([[[1, 3, 7], [2, 5, 7]], [[1, 5, 6], [2, 3, 6]]])  # [layer][head][k]
    layers, heads, k = topk.shape
    batch, capacity, dim = 1, 14, 3
    for layer in range(layers):
        for kv in range(2):
            data = np.arange(batch * heads * capacity * dim).reshape(batch, heads, capacity, dim)
            data = data + layer * 100_000 + kv * 10_000
            index = np.stack([selection.compact_index(non_visual, topk[layer, h]) for h in range(heads)])
            assert index.shape == (heads, len(non_visual) + k)
            out = selection.compact_kv(data, index)
            for h in range(heads):
                positions = sorted(non_visual.tolist() + topk[layer, h].tolist())
                np.testing.assert_array_equal(out[0, h], data[0, h, positions])


def test_selection_k_rule():
    assert selection.selection_k(4096, 3968, 3968, 1024) == 896
    assert selection.selection_k(65536, 65408, 65408, 4096) == 3968
    assert selection.selection_k(300, 200, 200, 1024) == 200          # clamped to the visual count
    assert selection.selection_k(300, 299, 299, 1024, explicit_k=5) == 5
    assert selection.last_video_index([1, 9, 9, 2, 3], 9) == 2
    assert selection.last_video_index([1, 2], 9) == -1
