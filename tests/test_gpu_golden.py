"""The HIP path against the committed golden fixtures (tests/golden/
oracle_cases.npz): attention within the bf16/fp32 tolerances, selection,
compaction index and acceptance bit-exact."""
import os

import numpy as np
import pytest
import torch

from std_amd import ops
from tests.gpu_helpers import announce, assert_close, cache_buffer, dev

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_cases.npz")


@pytest.fixture(scope="module")
def z():
    return np.load(GOLDEN)


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits).view(torch.bfloat16)


def test_golden_decode(z):
    announce("golden decode fp32/bf16 14/2 heads S=96")
    for dt in ("f32", "bf16"):
        conv = torch.from_numpy if dt == "f32" else bf16
        q, k, v = (conv(z[f"decode_{dt}_{n}"]) for n in "qkv")
        kb, vb = cache_buffer(k, 100), cache_buffer(v, 100)
        out = ops.gqa_decode(q.to(dev()), kb[:, :, :96], vb[:, :, :96])
        torch.cuda.synchronize()
        assert_close(out, z[f"decode_{dt}_out"], q.dtype)


def test_golden_verify(z):
    announce("golden verify bf16 q_len 6 kv 100")
    q, k, v = (bf16(z[f"verify_bf16_{n}"]) for n in "qkv")
    out = ops.verify_attention(q.to(dev()), k.to(dev()), v.to(dev()))
    torch.cuda.synchronize()
    assert_close(out, z["verify_bf16_out"], torch.bfloat16)


def test_golden_selection_and_compaction(z):
    announce("golden selection bf16 P=160 k=24 with boundary ties")
    P, T, k = (int(x) for x in z["select_meta"])
    q_text, key = bf16(z["select_q_text"]), bf16(z["select_key"])
    vis = torch.arange(P - T, dtype=torch.int32, device=dev())
    top, scores = ops.select_topk(q_text.to(dev()), cache_buffer(key, P + 3), P - T, vis, k, return_scores=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(top.cpu().numpy(), z["select_topk"])
    np.testing.assert_allclose(scores.cpu().numpy(), z["select_scores"], rtol=1e-12, atol=1e-15)
    idx = ops.build_compact_index(torch.arange(P - T, P, dtype=torch.int32, device=dev()), top)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(idx.cpu().numpy(), z["compact_index"])


def test_golden_accept(z):
    announce("golden greedy accept 10 x 1000")
    logits = torch.from_numpy(z["accept_logits"]).to(dev())
    draft = torch.from_numpy(z["accept_draft"]).to(dev())
    res = ops.greedy_accept(logits, draft, has_pending=True)
    rows = int(z["accept_no_pending_logits_rows"])
    nxt = torch.tensor([int(z["accept_no_pending_dense_next"])], dtype=torch.int32, device=dev())
    res2 = ops.greedy_accept(logits[:rows], draft, has_pending=False, dense_next=nxt)
    torch.cuda.synchronize()
    assert res[:2].tolist() == z["accept_pending"].tolist()
    assert res2[:2].tolist() == z["accept_no_pending"].tolist()
