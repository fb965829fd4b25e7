"""GPU parity of top-K selection and sparse-cache compaction: selected
positions bit-exact against the oracle (ties to the lowest position), column
scores to fp64 round-off, compacted rows bit-exact."""
import numpy as np
import pytest
import torch

from oracle import selection as ref
from std_amd import ops
from std_amd.workloads import WORKLOADS, make_layer, non_visual_positions, visual_positions
from tests.gpu_helpers import announce, cache_buffer, dev

pytestmark = pytest.mark.gpu


def _run_select(w, x, prompt_len=None):
    P = prompt_len or w.prompt_len
    T = w.text_len
    text_start = P - T
    k_sel = min(max(1, w.k_plus_text - T), P - T)
    kb = cache_buffer(x["k"], P + 40)
    vis = visual_positions(w, "cuda", prompt_len=P)
    topk, scores = ops.select_topk(x["q_text"].to(dev()), kb, text_start, vis, k_sel, return_scores=True)
    torch.cuda.synchronize()
    return topk.cpu().numpy(), scores.cpu().numpy(), text_start, k_sel


def _check_against_oracle(w, x, prompt_len=None):
    topk, scores, text_start, k_sel = _run_select(w, x, prompt_len)
    P = text_start + w.text_len
    ref_scores = ref.selection_scores(x["q_text"], x["k"], text_start)
    np.testing.assert_allclose(scores, ref_scores, rtol=1e-11, atol=1e-300)
    ref_topk = ref.topk_positions(ref_scores, np.arange(P - w.text_len), k_sel)
    np.testing.assert_array_equal(topk, ref_topk)
    # invariants that hold at any size
    np.testing.assert_allclose(scores.sum(axis=1), (w.n_q // w.n_kv) * w.text_len, rtol=1e-12)
    assert np.all(np.diff(topk, axis=1) > 0)
    return topk, scores


def test_select_c1_fp32():
    w = WORKLOADS["c1"]
    announce("select c1 fp32 P=4096 k=896")
    _check_against_oracle(w, make_layer(w, 0))


@pytest.mark.parametrize("layer", [0, 27])
def test_select_c2_bf16(layer):
    w = WORKLOADS["c2"]
    announce(f"select c2 bf16 P=16384 k=896 layer={layer}")
    x = make_layer(w, layer)
    topk, _ = _check_against_oracle(w, x)
    print(f"selected {topk.size} positions", flush=True)


def test_select_c4_tie_variant_reduced():
    """C4 recipe (log-normal key norms, 5% bit-exact duplicated keys) at P=8192."""
    w = WORKLOADS["c4"]
    P = 8192
    announce(f"select c4-tie bf16 P={P}")
    x = make_layer(w, 0, tie=True, prompt_len=P)
    topk, scores = _check_against_oracle(w, x, prompt_len=P)
    # every duplicated pair that straddles the selection boundary keeps the lower position
    kk = x["k"][0].view(torch.int16).numpy()
    for g in range(w.n_kv):
        rows = {}
        for j in range(P - w.text_len):
            rows.setdefault(kk[g, j].tobytes(), []).append(j)
        chosen = set(topk[g].tolist())
        for members in rows.values():
            if len(members) > 1:
                picked = [m in chosen for m in members]
                assert picked == sorted(picked, reverse=True), (g, members)
                assert len({scores[g, m] for m in members}) == 1


def test_select_c4_tie_full_one_layer():
    """Full 131072-position C4 tie variant for one layer."""
    w = WORKLOADS["c4"]
    announce("select c4-tie bf16 P=131072 k=896 layer=0")
    _check_against_oracle(w, make_layer(w, 0, tie=True))


def test_select_c3_one_layer():
    w = WORKLOADS["c3"]
    announce("select c3 bf16 P=65536 k=3968 layer=0")
    _check_against_oracle(w, make_layer(w, 0))


def test_select_is_deterministic():
    w = WORKLOADS["c2"]
    x = make_layer(w, 3)
    announce("select determinism c2 x3")
    runs = [_run_select(w, x)[:2] for _ in range(3)]
    for t, s in runs[1:]:
        np.testing.assert_array_equal(t, runs[0][0])
        np.testing.assert_array_equal(s, runs[0][1])


def test_compact_index_and_gather_bit_exact():
    w = WORKLOADS["c2"]
    x = make_layer(w, 2)
    P = w.prompt_len
    announce("compact index + gather c2 bf16")
    kb, vb = cache_buffer(x["k"], P + 10), cache_buffer(x["v"], P + 10)
    topk = ops.select_topk(x["q_text"].to(dev()), kb, P - w.text_len, visual_positions(w, "cuda"), w.k)
    nonvis = non_visual_positions(w, "cuda")
    idx = ops.build_compact_index(nonvis, topk)
    cap = w.compact_len + 64
    sk = torch.full((1, w.n_kv, cap, w.head_dim), float("nan"), dtype=w.dtype, device=dev())
    sv = torch.full_like(sk, float("nan"))
    ops.compact_kv(kb, vb, sk, sv, idx)
    torch.cuda.synchronize()
    idx_h, topk_h = idx.cpu().numpy(), topk.cpu().numpy()
    for g in range(w.n_kv):
        np.testing.assert_array_equal(idx_h[g], ref.compact_index(nonvis.cpu().numpy(), topk_h[g]))
    exp_k = ref.compact_kv(x["k"], idx_h)
    exp_v = ref.compact_kv(x["v"], idx_h)
    assert torch.equal(sk[:, :, :w.compact_len].cpu().view(torch.int16), exp_k.view(torch.int16))
    assert torch.equal(sv[:, :, :w.compact_len].cpu().view(torch.int16), exp_v.view(torch.int16))
    assert torch.isnan(sk[:, :, w.compact_len:].float()).all()       # nothing written past compact_len


def test_compaction_unique_valued_fixture_on_gpu():
    """The reference's unique-valued cache pattern (tests/test_sparse_cache_refresh.py:30-49)
    at head_dim 128: every row is distinguishable, so a wrong head or slot shows."""
    n_kv, cap, D = 2, 14, 128
    non_visual = torch.tensor([0, 4, 8], dtype=torch.int32)
    topk = torch.tensor([[1, 3, 7], [2, 5, 7]], dtype=torch.int32)
    base = torch.arange(n_kv * cap * D, dtype=torch.float32).reshape(1, n_kv, cap, D)
    announce("compaction unique-valued fixture fp32")
    dk, dv = base.to(dev()), (base + 10_000).to(dev())
    idx = ops.build_compact_index(non_visual.to(dev()), topk.to(dev()))
    sk = torch.full((1, n_kv, 8, D), -1.0, device=dev())
    sv = torch.full((1, n_kv, 8, D), -1.0, device=dev())
    ops.compact_kv(dk, dv, sk, sv, idx)
    torch.cuda.synchronize()
    for h in range(n_kv):
        positions = sorted(non_visual.tolist() + topk[h].tolist())
        assert idx[h].cpu().tolist() == positions
        assert torch.equal(sk[0, h, :6].cpu(), base[0, h, positions])
        assert torch.equal(sv[0, h, :6].cpu(), base[0, h, positions] + 10_000)
        assert torch.all(sk[0, h, 6:] == -1)
