"""Pin the oracle with what the mathematics fixes: closed forms, invariants,
brute-force loops on tiny inputs and constructed ties. Each check is chosen so
that a plausible mistake (wrong head mapping, off-by-one causal limit, missing
scale, transposed operand, wrong tie order) fails it."""
import math

import numpy as np
import pytest
import torch

from oracle import accept, attention, brute, selection


def _rand(*shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape)


# ---------------------------------------------------------------- attention
def test_decode_uniform_keys_gives_mean_of_values():
    q = _rand(1, 6, 1, 16, seed=1)
    k = np.repeat(_rand(1, 2, 1, 16, seed=2), 9, axis=2)        # every key identical
    v = _rand(1, 2, 9, 16, seed=3)
    out = attention.gqa_sdpa(q, k, v)
    for h in range(6):
        np.testing.assert_allclose(out[0, h, 0], v[0, h // 3].mean(axis=0), rtol=1e-12, atol=1e-12)


def test_decode_dominant_key_selects_its_value_row_and_head_mapping():
    d = 16
    q = np.zeros((1, 4, 1, d))
    k = np.zeros((1, 2, 5, d))
    v = _rand(1, 2, 5, d, seed=4)
    for h in range(4):
        q[0, h, 0, 0] = 50.0
    k[0, 0, 3, 0] = 50.0       # KV head 0 -> row 3 dominates
    k[0, 1, 1, 0] = 50.0       # KV head 1 -> row 1 dominates
    out = attention.gqa_sdpa(q, k, v)
    for h in range(4):
        row = 3 if h // 2 == 0 else 1
        np.testing.assert_allclose(out[0, h, 0], v[0, h // 2, row], atol=1e-12)


def test_decode_scale_is_inverse_sqrt_head_dim():
    q = _rand(1, 2, 1, 64, seed=5)
    k = _rand(1, 1, 7, 64, seed=6)
    v = _rand(1, 1, 7, 64, seed=7)
    s = (q[0, :, 0] @ k[0, 0].T) / math.sqrt(64)
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(attention.gqa_sdpa(q, k, v)[0, :, 0], p @ v[0, 0], rtol=1e-12)


def test_attention_matches_brute_force_loops():
    q = _rand(1, 6, 3, 8, seed=8)
    k = _rand(1, 2, 11, 8, seed=9)
    v = _rand(1, 2, 11, 8, seed=10)
    ref_dec = brute.attention_loops(q[0, :, :1].tolist(), k[0].tolist(), v[0].tolist())
    np.testing.assert_allclose(attention.gqa_sdpa(q[:, :, :1], k, v)[0], np.array(ref_dec), rtol=1e-12, atol=1e-12)
    ref_ver = brute.attention_loops(q[0].tolist(), k[0].tolist(), v[0].tolist(), causal_offset=11 - 3)
    np.testing.assert_allclose(attention.verify_attention(q, k, v)[0], np.array(ref_ver), rtol=1e-12, atol=1e-12)


def test_verify_last_row_equals_decode_over_everything():
    q = _rand(1, 4, 5, 8, seed=11)
    k = _rand(1, 2, 9, 8, seed=12)
    v = _rand(1, 2, 9, 8, seed=13)
    full = attention.verify_attention(q, k, v)
    np.testing.assert_allclose(full[:, :, -1], attention.gqa_sdpa(q[:, :, -1:], k, v)[:, :, 0], rtol=1e-12)
    # first row sees exactly kv_len - q_len + 1 keys
    np.testing.assert_allclose(full[:, :, 0], attention.gqa_sdpa(q[:, :, :1], k[:, :, :5], v[:, :, :5])[:, :, 0],
                               rtol=1e-12)


# ---------------------------------------------------------------- selection
def test_selection_scores_match_brute_force():
    q = _rand(1, 4, 3, 8, seed=14)
    k = _rand(1, 2, 10, 8, seed=15)
    text_start = 7
    ref = np.array(brute.selection_scores_loops(q[0].tolist(), k[0, :, :10].tolist(), text_start))
    got = selection.selection_scores(q, k, text_start)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-15)
    # chunked evaluation equals the single-chunk one bit-for-bit where it matters
    np.testing.assert_allclose(selection.selection_scores(q, k, text_start, chunk=3), got, rtol=1e-13)


def test_selection_invariants():
    q = torch.randn(1, 6, 5, 16, generator=torch.Generator().manual_seed(1))
    k = torch.randn(1, 3, 40, 16, generator=torch.Generator().manual_seed(2))
    text_start = 35
    s = selection.selection_scores(q, k, text_start)
    assert s.shape == (3, 40)
    assert np.all(s >= 0)
    # each (head, row) distributes probability 1 -> per KV head the sum is group * T
    np.testing.assert_allclose(s.sum(axis=1), np.full(3, 2 * 5), rtol=1e-12)
    # the last text row alone sees the last column: its score is < group (one row per head)
    assert np.all(s[:, -1] < 2.0)


def test_selection_causal_limit_matters():
    """Text row i must not see keys after text_start + i: moving the last key
    changes only the rows that can see it."""
    q = _rand(1, 2, 4, 8, seed=16)
    k = _rand(1, 1, 12, 8, seed=17)
    base = selection.selection_scores(q, k, 8)
    k2 = k.copy()
    k2[0, 0, 11] *= 5.0                  # only row 3 (position 11) sees key 11
    changed = selection.selection_scores(q, k2, 8)
    ref = np.array(brute.selection_scores_loops(q[0].tolist(), k2[0].tolist(), 8))
    np.testing.assert_allclose(changed, ref, rtol=1e-12, atol=1e-15)
    assert not np.allclose(base, changed)


def test_topk_lowest_index_wins_exact_ties():
    scores = np.array([[0.5, 0.9, 0.9, 0.1, 0.9, 0.3]])
    vis = np.arange(6)
    np.testing.assert_array_equal(selection.topk_positions(scores, vis, 2), [[1, 2]])
    np.testing.assert_array_equal(selection.topk_positions(scores, vis, 3), [[1, 2, 4]])
    np.testing.assert_array_equal(selection.topk_positions(scores, vis, 4), [[0, 1, 2, 4]])
    np.testing.assert_array_equal(selection.topk_positions(scores, vis, 6), [vis])


def test_topk_restricted_to_visual_positions_and_sorted():
    scores = np.array([[9.0, 1.0, 2.0, 8.0, 3.0, 7.0]])
    vis = np.array([1, 2, 4, 5])
    np.testing.assert_array_equal(selection.topk_positions(scores, vis, 2), [[4, 5]])


def test_duplicated_key_columns_tie_exactly():
    gen = torch.Generator().manual_seed(3)
    q = torch.randn(1, 4, 6, 16, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, 2, 50, 16, generator=gen).to(torch.bfloat16)
    k[0, :, 30] = k[0, :, 7]
    k[0, :, 41] = k[0, :, 7]
    s = selection.selection_scores(q, k, 44)
    for g in range(2):
        assert s[g, 7] == s[g, 30] == s[g, 41]


def test_full_pipeline_dict():
    gen = torch.Generator().manual_seed(5)
    ids = [7] * 20 + [1, 2, 3]
    q = [torch.randn(1, 4, 3, 16, generator=gen) for _ in range(2)]
    k = [torch.randn(1, 2, 23, 16, generator=gen) for _ in range(2)]
    sel = selection.build_sparse_selection(q, k, ids, video_token_id=7, target_k_plus_text=8)
    assert sel["k"] == 5 and sel["text_len"] == 3 and sel["visual_len"] == 20
    np.testing.assert_array_equal(sel["non_visual_positions"], [20, 21, 22])
    for layer in range(2):
        t = sel["topk_positions"][layer]
        assert t.shape == (2, 5) and np.all(np.diff(t, axis=1) > 0) and t.max() < 20


# ---------------------------------------------------------------- accept
def test_argmax_semantics():
    assert accept.argmax_first([1.0, 3.0, 3.0, 2.0]) == 1
    assert accept.argmax_first([1.0, float("nan"), 5.0, float("nan")]) == 1
    assert accept.argmax_first([-0.0, 0.0, -1.0]) == 0
    assert accept.argmax_first([float("-inf"), float("-inf")]) == 0
    x = torch.tensor([[0.0, 2.0, 2.0, float("nan"), 1.0], [1.0, 1.0, 0.5, -3.0, 1.0]])
    for r in range(2):
        assert accept.argmax_first(x[r]) == int(torch.argmax(x[r]))


def test_verify_accept_and_rollback_invariant():
    logits = torch.full((4, 6), -1.0)
    for r, tok in enumerate([2, 5, 1, 4]):
        logits[r, tok] = 1.0
    a, bonus, preds = accept.verify_accept(logits, [2, 5, 0], has_pending=True)
    assert (a, bonus, preds) == (2, 1, [2, 5, 1, 4])
    a, bonus, preds = accept.verify_accept(logits[:3], [3, 2, 5], has_pending=False, dense_next=3)
    assert (a, bonus) == (3, 1)
    prompt_len, generated, pending = 100, 7, 1
    dense_cached = prompt_len + generated - pending
    dense_len, sparse_len = accept.rollback_lengths(dense_cached, pending, 40 + generated, 2)
    # after the round the bonus joins `generated` and stays pending
    assert dense_len + 1 == prompt_len + generated + 2 + 1
    assert sparse_len == 40 + generated + 2
