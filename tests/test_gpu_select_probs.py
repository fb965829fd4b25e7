"""GPU parity of the selection from materialised attention probabilities
(std_select_topk_probs; the reference's build_sparse_selection input,
src/std_repro/std_qwen25vl.py:175-231) against the oracle: fp64 group and
text-row sums, then lowest-position top-k."""
import numpy as np
import pytest
import torch

from oracle import selection as ref_sel
from std_amd import ops
from std_amd.std_qwen25vl import build_sparse_selection
from tests.gpu_helpers import announce, dev

pytestmark = pytest.mark.gpu


def _probs(n_q, T, P, dtype, seed, dup_frac=0.0):
    g = torch.Generator().manual_seed(seed)
    p = torch.rand(1, n_q, T, P, generator=g) ** 4          # skewed, nonnegative
    if dup_frac:
        n = int(dup_frac * P)
        perm = torch.randperm(P - T, generator=g)
        p[..., perm[:n]] = p[..., perm[n:2 * n]]             # duplicated visual columns tie exactly
    return p.to(dtype)


@pytest.mark.parametrize("dtype,P,dup", [(torch.float16, 4096, 0.05), (torch.float16, 16384, 0.0),
                                         (torch.bfloat16, 4096, 0.05), (torch.float32, 4096, 0.05)])
def test_select_topk_probs_matches_oracle(dtype, P, dup):
    n_q, n_kv, T = 28, 4, 128
    V = P - T
    k = 896
    announce(f"select from probs {dtype} P={P} dup={dup}")
    probs = _probs(n_q, T, P, dtype, P + 7, dup)
    vis = torch.arange(V, dtype=torch.int32)
    topk, scores = ops.select_topk_probs(probs.to(dev()), vis.to(dev()), k, n_kv, return_scores=True)
    torch.cuda.synchronize()
    want_scores = ref_sel.scores_from_probs(probs, n_kv)
    want = ref_sel.topk_positions(want_scores, np.arange(V), k)
    np.testing.assert_array_equal(topk.cpu().numpy(), want)
    if dtype == torch.float16:
        assert np.array_equal(scores.cpu().numpy(), want_scores)        # exact sums
    else:
        np.testing.assert_allclose(scores.cpu().numpy(), want_scores, rtol=1e-13)


def test_select_topk_probs_strided_view():
    """A [1, n_q, T, P] view cut from a longer allocation (row stride > P)."""
    n_q, n_kv, T, P = 14, 2, 64, 2048
    announce("select from probs, strided view")
    full = _probs(n_q, T, P + 64, torch.float16, 3)
    probs = full[..., :P]
    vis = torch.arange(P - T, dtype=torch.int32)
    topk = ops.select_topk_probs(probs.to(dev()), vis.to(dev()), 500, n_kv)
    torch.cuda.synchronize()
    want = ref_sel.topk_positions(ref_sel.scores_from_probs(probs, n_kv), np.arange(P - T), 500)
    np.testing.assert_array_equal(topk.cpu().numpy(), want)


@pytest.mark.parametrize("dtype,P", [(torch.float16, 4093), (torch.bfloat16, 2047), (torch.float32, 4094)])
def test_select_topk_probs_odd_prompt_length(dtype, P):
    """The reference's contiguous [1, n_q, T, P] probabilities with a prompt
    length that is not a multiple of four (row stride P): rows are not
    four-element aligned, so the column sums take element loads."""
    n_q, n_kv, T = 28, 4, 128
    V = P - T
    announce(f"select from probs {dtype} odd P={P}")
    probs = _probs(n_q, T, P, dtype, P + 11, 0.05)
    assert probs.is_contiguous() and probs.stride(2) == P
    vis = torch.arange(V, dtype=torch.int32)
    topk, scores = ops.select_topk_probs(probs.to(dev()), vis.to(dev()), 896, n_kv, return_scores=True)
    torch.cuda.synchronize()
    want_scores = ref_sel.scores_from_probs(probs, n_kv)
    np.testing.assert_array_equal(topk.cpu().numpy(), ref_sel.topk_positions(want_scores, np.arange(V), 896))
    if dtype == torch.float16:
        assert np.array_equal(scores.cpu().numpy(), want_scores)        # exact sums
    else:
        np.testing.assert_allclose(scores.cpu().numpy(), want_scores, rtol=1e-13)


def test_build_sparse_selection_reference_signature():
    """build_sparse_selection(attentions, full_input_ids, video_token_id,
    text_start, target_k_plus_text, explicit_k, num_key_value_heads) on two
    layers of fp16 probabilities equals the oracle selection record."""
    n_q, n_kv, T, P, vid = 28, 4, 128, 4096, 151656
    V = P - T
    announce("build_sparse_selection with the reference signature")
    ids = torch.cat([torch.full((V,), vid), torch.arange(T) + 10]).view(1, -1)
    layers = [_probs(n_q, T, P, torch.float16, 100 + l, 0.02) for l in range(2)]
    sel = build_sparse_selection([a.to(dev()) for a in layers], ids, vid, V, target_k_plus_text=1024,
                                 num_key_value_heads=n_kv)
    assert (sel.k, sel.text_len, sel.visual_len, sel.prompt_len) == (896, T, V, P)
    assert sel.non_visual_positions.tolist() == list(range(V, P))
    for l in range(2):
        want = ref_sel.topk_positions(ref_sel.scores_from_probs(layers[l], n_kv), np.arange(V), 896)
        np.testing.assert_array_equal(sel.topk_positions[l].numpy(), want)
