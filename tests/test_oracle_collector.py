"""Pins oracle.collector.verification_scores (the restatement of
VerificationCollectorV3._hook, src/std_repro/dynamic_selection.py:504-519)
with checks that share no code with it."""
import numpy as np
import pytest

from oracle import brute
from oracle.collector import verification_scores


def _case(seed, n_q=6, n_kv=2, q_len=3, kv_len=14, d=8):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((1, n_q, q_len, d))
    k = rng.standard_normal((1, n_kv, kv_len, d))
    return q, k


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_matches_brute_force_loops(seed):
    q, k = _case(seed)
    vis = list(range(3, 11))
    got = verification_scores(q, k, vis)
    want = brute.verification_scores_loops(q[0].tolist(), k[0].tolist(), vis)
    np.testing.assert_allclose(got, np.array(want), rtol=1e-12, atol=1e-14)


def test_each_position_contributes_a_distribution():
    q, k = _case(5, q_len=4)
    s = verification_scores(q, k, range(0, 12))
    assert (s >= 0).all()
    np.testing.assert_allclose(s.sum(axis=1), 4.0, rtol=1e-12)


def test_mean_query_logits_equal_mean_of_head_logits():
    """The collector's logits are linear in the query: q_bar . k equals the
    mean over the group's heads of q_h . k, computed here per head."""
    q, k = _case(7, n_q=8, n_kv=2, q_len=2, d=16)
    vis = np.arange(2, 13)
    d = q.shape[-1]
    s = np.zeros((2, vis.size))
    for g in range(2):
        for i in range(2):
            per_head = [q[0, g * 4 + h, i] @ k[0, g, vis].T for h in range(4)]
            logits = np.mean(per_head, axis=0) / np.sqrt(d)
            w = np.exp(logits - logits.max())
            s[g] += w / w.sum()
    np.testing.assert_allclose(verification_scores(q, k, vis), s, rtol=1e-12)


def test_identical_visual_keys_share_the_mass_evenly():
    q, k = _case(9, q_len=5)
    k[0, :, 2:10] = k[0, :, 2:3]
    s = verification_scores(q, k, range(2, 10))
    np.testing.assert_allclose(s, 5.0 / 8, rtol=1e-12)


def test_one_dominant_key_takes_every_position():
    q, k = _case(11, n_q=4, n_kv=1, q_len=3)
    qbar = q[0].reshape(1, 4, 3, -1).mean(axis=1)[0]          # [3, D]
    k[0, 0, 6] = 500.0 * np.linalg.pinv(qbar) @ np.ones(3)   # qbar_i . k_6 = 500 for every position i
    s = verification_scores(q, k, range(0, 12))
    assert s[0, 6] > 3.0 - 1e-6


def test_keys_outside_the_visual_set_change_nothing():
    q, k = _case(13)
    vis = range(4, 9)
    a = verification_scores(q, k, vis)
    k[0, :, :4] += 100.0
    k[0, :, 9:] -= 100.0
    np.testing.assert_allclose(verification_scores(q, k, vis), a, rtol=1e-13)


def test_probability_scores_equal_the_exact_score_path():
    """scores_from_probs on the causal text-row probabilities (built here from
    q and k) equals selection_scores, which never materialises them."""
    from oracle.selection import scores_from_probs, selection_scores
    rng = np.random.default_rng(3)
    n_q, n_kv, T, P, d = 6, 2, 5, 19, 8
    q = rng.standard_normal((1, n_q, T, d))
    k = rng.standard_normal((1, n_kv, P, d))
    text_start = P - T
    probs = np.zeros((1, n_q, T, P))
    for h in range(n_q):
        g = h // (n_q // n_kv)
        for t in range(T):
            lim = text_start + t
            z = q[0, h, t] @ k[0, g, :lim + 1].T / np.sqrt(d)
            w = np.exp(z - z.max())
            probs[0, h, t, :lim + 1] = w / w.sum()
    np.testing.assert_allclose(scores_from_probs(probs, n_kv), selection_scores(q, k, text_start), rtol=1e-12,
                               atol=1e-15)


def test_probability_scores_are_exact_sums_of_fp16_values():
    """fp16 probabilities: the fp64 group sum is exact, so any summation order
    gives the same bits (the device sums in another order)."""
    import torch
    from oracle.selection import scores_from_probs
    g = torch.Generator().manual_seed(5)
    probs = torch.rand(1, 7, 33, 101, generator=g).to(torch.float16)
    s = scores_from_probs(probs, 1)
    a = probs.double().numpy()[0]
    rev = a[::-1, ::-1].sum(axis=(0, 1))           # the rows in reverse order
    assert np.array_equal(s[0], rev)


def test_torch_cpu_restatements_match_the_numpy_oracle():
    """The torch-CPU operators timed as the CPU baseline agree with the fp64
    numpy oracle (fp32 tolerance) on decode, offset-causal verify and accept."""
    import torch
    from oracle import accept as np_accept
    from oracle import attention as np_attn
    from oracle import torch_cpu
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 28, 1, 128, generator=g)
    k = torch.randn(1, 4, 300, 128, generator=g)
    v = torch.randn(1, 4, 300, 128, generator=g)
    np.testing.assert_allclose(torch_cpu.gqa_sdpa(q, k, v).double().numpy(), np_attn.gqa_sdpa(q, k, v),
                               rtol=1e-5, atol=1e-6)
    qv = torch.randn(1, 28, 10, 128, generator=g)
    np.testing.assert_allclose(torch_cpu.verify_attention(qv, k, v).double().numpy(),
                               np_attn.verify_attention(qv, k, v), rtol=1e-5, atol=1e-6)
    logits = torch.randn(10, 1000, generator=g)
    preds = np_accept.verify_predictions(logits.numpy(), True)
    draft = preds[:3] + [(preds[3] + 1) % 1000] + preds[4:9]
    assert torch_cpu.greedy_accept(logits, draft, True) == (3, preds[3])
    a, bonus, _ = np_accept.verify_accept(logits.numpy(), draft, True)
    assert (a, bonus) == (3, preds[3])


def test_torch_cpu_selection_matches_the_numpy_oracle():
    """The CPU baseline's selection restatement (causal text-row softmax,
    group and row sums, top-k over the visual positions) picks the oracle's
    positions; 16 keys per head are boosted along the group's mean query so
    that the top-k is far from any tie at fp32 precision."""
    import torch
    from oracle import selection as np_sel
    from oracle import torch_cpu
    g = torch.Generator().manual_seed(12)
    T, V, k = 20, 280, 16
    q = torch.randn(1, 28, T, 128, generator=g)
    key = torch.randn(1, 4, V + T, 128, generator=g)
    for h in range(4):
        u = q[0, 7 * h:7 * h + 7].reshape(-1, 128).mean(0)
        pos = torch.randperm(V, generator=g)[:k]
        key[0, h, pos] += 3.0 * u / u.norm()
    want = np_sel.topk_positions(np_sel.selection_scores(q, key, V), range(V), k)
    got = torch_cpu.select_topk(q, key, V, k).numpy()
    np.testing.assert_array_equal(got, want)
