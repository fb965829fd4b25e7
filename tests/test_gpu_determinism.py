"""Run-to-run determinism of the hot path on the GPU: the same inputs give
bit-identical selection scores and indices, verify outputs, collector scores
and acceptance results on every call. Every floating-point reduction is done
in a fixed order (the only atomics are the radix select's integer histogram
counts), so these hold exactly, not within a tolerance."""
import numpy as np
import pytest
import torch

from std_amd import ops
from std_amd.workloads import WORKLOADS, make_layer, make_logits, visual_positions
from tests.gpu_helpers import announce, cache_buffer, dev

pytestmark = pytest.mark.gpu

RUNS = 10


def test_selection_is_deterministic():
    w = WORKLOADS["c2"]
    x = make_layer(w, 3)
    P, T = w.prompt_len, w.text_len
    kb = cache_buffer(x["k"], P + 40)
    vis = visual_positions(w, "cuda")
    q = x["q_text"].to(dev())
    announce(f"selection determinism c2 P={P} x{RUNS}")
    runs = [ops.select_topk(q, kb, P - T, vis, w.k_plus_text - T, return_scores=True) for _ in range(RUNS)]
    torch.cuda.synchronize()
    for topk, scores in runs[1:]:
        assert torch.equal(topk, runs[0][0])
        assert np.array_equal(scores.cpu().numpy().view(np.uint64), runs[0][1].cpu().numpy().view(np.uint64))


def test_verify_and_collector_are_deterministic():
    w = WORKLOADS["c2"]
    x = make_layer(w, 4)
    k = torch.cat([x["k"], x["new_k"]], 2)
    v = torch.cat([x["v"], x["new_v"]], 2)
    kv = k.shape[2]
    kb, vb = cache_buffer(k, kv + 9)[:, :, :kv], cache_buffer(v, kv + 9)[:, :, :kv]
    q = x["q_verify"].to(dev())
    announce(f"verify + collector determinism c2 kv={kv} x{RUNS}")
    outs = [ops.verify_attention(q, kb, vb) for _ in range(RUNS)]
    colls = [ops.verify_attention_collect(q, kb, vb, 0, w.prompt_len - w.text_len, kv_len=kv) for _ in range(5)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    for o, s in colls:
        assert torch.equal(o, outs[0])
        assert torch.equal(s.view(torch.int32), colls[0][1].view(torch.int32))


def test_acceptance_is_deterministic():
    w = WORKLOADS["c2"]
    logits = make_logits(w, w.gamma + 1, seed=w.seed_base + 91).to(dev())
    preds = logits.float().argmax(-1).to(torch.int32)
    draft = preds[:w.gamma].clone()
    draft[5] = (draft[5] + 1) % w.vocab                # reject at the sixth draft token
    announce(f"acceptance determinism c2 vocab={w.vocab} x{RUNS}")
    outs = []
    for _ in range(RUNS):
        lens = torch.tensor([5000, 1100], dtype=torch.int32, device=dev())
        outs.append((ops.greedy_accept(logits, draft, True, rollback_lengths=lens), lens))
    torch.cuda.synchronize()
    first = outs[0][0].cpu().tolist()
    assert first[0] == 5 and first[1] == int(preds[5])
    for out, lens in outs:
        assert out.cpu().tolist() == first
        assert lens.cpu().tolist() == [5000 - (w.gamma - 5), 1100 - (w.gamma - 5)]
