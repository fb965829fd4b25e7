"""The oracle reproduces the committed golden fixtures (tests/golden/
oracle_cases.npz, written by tests/golden/make_golden.py), and the fixtures
carry the properties they were built to exercise."""
import os

import numpy as np
import pytest
import torch

from oracle import accept as ref_accept
from oracle import attention as ref_attn
from oracle import selection as ref_sel

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_cases.npz")


@pytest.fixture(scope="module")
def z():
    return np.load(GOLDEN)


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits).view(torch.bfloat16)


def test_decode_cases(z):
    out = ref_attn.gqa_sdpa(z["decode_f32_q"], z["decode_f32_k"], z["decode_f32_v"])
    np.testing.assert_allclose(out, z["decode_f32_out"], rtol=1e-12, atol=1e-12)
    out = ref_attn.gqa_sdpa(bf16(z["decode_bf16_q"]), bf16(z["decode_bf16_k"]), bf16(z["decode_bf16_v"]))
    np.testing.assert_allclose(out, z["decode_bf16_out"], rtol=1e-12, atol=1e-12)


def test_verify_case(z):
    out = ref_attn.verify_attention(bf16(z["verify_bf16_q"]), bf16(z["verify_bf16_k"]), bf16(z["verify_bf16_v"]))
    np.testing.assert_allclose(out, z["verify_bf16_out"], rtol=1e-12, atol=1e-12)
    # the last query row sees every key: it equals single-query decode over all keys
    q = bf16(z["verify_bf16_q"])
    last = ref_attn.gqa_sdpa(q[:, :, -1:], bf16(z["verify_bf16_k"]), bf16(z["verify_bf16_v"]))
    np.testing.assert_allclose(z["verify_bf16_out"][:, :, -1:], last, rtol=1e-12, atol=1e-12)


def test_selection_case_and_boundary_ties(z):
    P, T, k = (int(x) for x in z["select_meta"])
    scores = ref_sel.selection_scores(bf16(z["select_q_text"]), bf16(z["select_key"]), P - T)
    np.testing.assert_allclose(scores, z["select_scores"], rtol=1e-13, atol=0)
    top = ref_sel.topk_positions(scores, np.arange(P - T), k)
    np.testing.assert_array_equal(top, z["select_topk"])
    for h in range(top.shape[0]):
        sel = set(top[h].tolist())
        boundary = min(z["select_scores"][h, c] for c in sel)
        tied = [c for c in range(P - T) if z["select_scores"][h, c] == boundary]
        assert len(tied) >= 2 and tied[0] in sel and tied[-1] not in sel     # lowest position wins the tie
    # every text row's probabilities sum to 1: each head's scores sum to 7 heads x T rows
    np.testing.assert_allclose(z["select_scores"].sum(axis=1), 7 * T, rtol=1e-12)
    for h in range(top.shape[0]):
        np.testing.assert_array_equal(z["compact_index"][h], ref_sel.compact_index(np.arange(P - T, P), top[h]))


def test_accept_cases(z):
    logits = z["accept_logits"]
    draft = z["accept_draft"].tolist()
    a, bonus, _ = ref_accept.verify_accept(logits, draft, True)
    assert [a, bonus] == z["accept_pending"].tolist() and a == 4
    rows = int(z["accept_no_pending_logits_rows"])
    a2, bonus2, _ = ref_accept.verify_accept(logits[:rows], draft, False, int(z["accept_no_pending_dense_next"]))
    assert [a2, bonus2] == z["accept_no_pending"].tolist()
