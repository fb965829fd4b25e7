"""The hot path with fp16 caches and logits, the dtype the reference loads its
model in (scripts/benchmark_std.py:66): decode and verify attention (plain,
fused append, batched, index-addressed, device length, allocation-free)
against the fp64 oracle, greedy acceptance and selection bit-exact, the
compaction a bit copy, the rotary embedding + append against the oracle's
fp16 rounding."""
import math

import numpy as np
import pytest
import torch

from oracle import accept as ref_accept
from oracle import attention as ref
from oracle import rope as ref_rope
from oracle import selection as ref_sel
from std_amd import ops
from tests.gpu_helpers import announce, assert_close, cache_buffer, dev

pytestmark = pytest.mark.gpu

F16 = torch.float16
D, NQ, NKV = 128, 28, 4


def _kvq(kv, q_len, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(1, NKV, kv, D, generator=g).to(F16)
    v = torch.randn(1, NKV, kv, D, generator=g).to(F16)
    q = torch.randn(1, NQ, q_len, D, generator=g).to(F16)
    return q, k, v


@pytest.mark.parametrize("kv", [1, 65, 320, 321, 1034, 16384, 131072])
def test_decode_matches_oracle(kv):
    q, k, v = _kvq(kv, 1, 100 + kv)
    announce(f"fp16 decode kv={kv}")
    out = ops.gqa_decode(q.to(dev()), cache_buffer(k, kv + 37)[:, :, :kv], cache_buffer(v, kv + 37)[:, :, :kv])
    torch.cuda.synchronize()
    assert out.dtype == F16
    assert_close(out, ref.gqa_sdpa(q, k, v), F16)


@pytest.mark.parametrize("kv", [4106, 16394, 131082])
def test_verify_matches_oracle(kv):
    q, k, v = _kvq(kv, 10, 200 + kv)
    announce(f"fp16 verify kv={kv}")
    out = ops.verify_attention(q.to(dev()), cache_buffer(k, kv + 7)[:, :, :kv], cache_buffer(v, kv + 7)[:, :, :kv])
    torch.cuda.synchronize()
    assert_close(out, ref.verify_attention(q, k, v), F16)


@pytest.mark.parametrize("kind,kv", [("decode", 16384), ("decode", 131072), ("verify", 16394), ("verify", 131082)])
def test_large_magnitudes_stay_finite_and_accurate(kind, kv):
    """fp16 tops out at 65504: values near it in V and logits sharpened about
    16x (q and k scaled by 4, so the softmax is dominated by a few keys) must
    neither overflow an intermediate (split partials, the key-split combine,
    the merge) nor lose accuracy. Bound: the fp16 tolerance with the absolute
    part scaled by the value scale."""
    g = torch.Generator().manual_seed(700 + kv)
    rows = 1 if kind == "decode" else 10
    vscale = 15000.0
    k = (torch.randn(1, NKV, kv, D, generator=g) * 4).to(F16)
    v = (torch.randn(1, NKV, kv, D, generator=g) * vscale).clamp(-60000, 60000).to(F16)
    q = (torch.randn(1, NQ, rows, D, generator=g) * 4).to(F16)
    announce(f"fp16 large magnitudes {kind} kv={kv}")
    kb, vb = cache_buffer(k, kv + 7)[:, :, :kv], cache_buffer(v, kv + 7)[:, :, :kv]
    if kind == "decode":
        out, want = ops.gqa_decode(q.to(dev()), kb, vb), ref.gqa_sdpa(q, k, v)
    else:
        out, want = ops.verify_attention(q.to(dev()), kb, vb), ref.verify_attention(q, k, v)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, rtol=5e-3, atol=5e-4 * vscale)


@pytest.mark.parametrize("kv", [130, 16394])
def test_append_paths_write_the_rows_and_match_oracle(kv):
    Q = 10
    q, k, v = _kvq(kv, Q, 300 + kv)
    announce(f"fp16 verify_append / decode_append kv={kv}")
    kb, vb = cache_buffer(k[:, :, :kv - Q], kv + 7), cache_buffer(v[:, :, :kv - Q], kv + 7)
    out = ops.verify_attention_append(q.to(dev()), kb, vb, k[:, :, kv - Q:].to(dev()), v[:, :, kv - Q:].to(dev()), kv)
    torch.cuda.synchronize()
    assert torch.equal(kb[:, :, kv - Q:kv].cpu(), k[:, :, kv - Q:])
    assert torch.equal(vb[:, :, kv - Q:kv].cpu(), v[:, :, kv - Q:])
    assert torch.isnan(vb[:, :, kv:].float()).all()
    assert_close(out, ref.verify_attention(q, k, v), F16)
    kb, vb = cache_buffer(k[:, :, :kv - 1], kv + 7), cache_buffer(v[:, :, :kv - 1], kv + 7)
    out = ops.gqa_decode_append(q[:, :, :1].to(dev()), kb, vb, k[:, :, kv - 1:].to(dev()), v[:, :, kv - 1:].to(dev()),
                                kv)
    sep = ops.gqa_decode(q[:, :, :1].to(dev()), kb[:, :, :kv], vb[:, :, :kv])
    torch.cuda.synchronize()
    assert torch.equal(out, sep)
    assert_close(out, ref.gqa_sdpa(q[:, :, :1], k, v), F16)


def test_batched_matches_oracle_and_single_problem():
    B, S = 28, 1034
    g = torch.Generator().manual_seed(401)
    k = torch.randn(B, 1, NKV, S, D, generator=g).to(F16)
    v = torch.randn(B, 1, NKV, S, D, generator=g).to(F16)
    q = torch.randn(B, 1, NQ, 1, D, generator=g).to(F16)
    announce(f"fp16 decode_batched B={B} S={S}")
    out = ops.gqa_decode_batched(q.to(dev()), k.to(dev()), v.to(dev()))
    one = ops.gqa_decode_batched(q[:1].to(dev()), k[:1].to(dev()), v[:1].to(dev()))
    single = ops.gqa_decode(q[0].to(dev()), k[0].to(dev()), v[0].to(dev()))
    torch.cuda.synchronize()
    for b in (0, 13, 27):
        assert_close(out[b], ref.gqa_sdpa(q[b], k[b], v[b]), F16)
    assert torch.equal(one[0], single)


def test_indexed_equals_compacted():
    P, n_index, n_tail = 8192, 1024, 9
    g = torch.Generator().manual_seed(402)
    kd = torch.randn(1, NKV, P + 64, D, generator=g).to(F16).to(dev())
    vd = torch.randn(1, NKV, P + 64, D, generator=g).to(F16).to(dev())
    index = torch.stack([torch.sort(torch.randperm(P, generator=g)[:n_index]).values for _ in range(NKV)]).int()
    tail_k = torch.randn(1, NKV, n_tail, D, generator=g).to(F16).to(dev())
    tail_v = torch.randn(1, NKV, n_tail, D, generator=g).to(F16).to(dev())
    q = torch.randn(1, NQ, 1, D, generator=g).to(F16).to(dev())
    S = n_index + n_tail
    announce(f"fp16 indexed vs compacted n_index={n_index}")
    ck = torch.cat([torch.stack([kd[0, h, index[h].long()] for h in range(NKV)])[None], tail_k], 2)
    cv = torch.cat([torch.stack([vd[0, h, index[h].long()] for h in range(NKV)])[None], tail_v], 2)
    tk = torch.full((1, NKV, S + 40, D), float("nan"), dtype=F16, device=dev())
    tv = torch.full_like(tk, float("nan"))
    tk[:, :, n_index:S], tv[:, :, n_index:S] = tail_k, tail_v
    want = ops.gqa_decode(q, ck.contiguous(), cv.contiguous())
    got = ops.gqa_decode_indexed(q, kd, vd, ops.pad_index(index.to(dev())), n_index, tk, tv, kv_len=S)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_device_length_and_allocation_free_entry():
    kv, cap, Q = 4106, 4500, 10
    q, k, v = _kvq(cap, Q, 403)
    kd, vd = k.to(dev()), v.to(dev())
    announce("fp16 attention_devlen and gqa_decode_noalloc")
    length = torch.tensor([kv - Q], dtype=torch.int32, device=dev())
    got = ops.attention_devlen(q.to(dev()), kd, vd, length, max_kv_len=cap)
    want = ops.verify_attention(q.to(dev()), kd[:, :, :kv], vd[:, :, :kv])
    a = ops.gqa_decode(q[:, :, :1].to(dev()), kd[:, :, :1034], vd[:, :, :1034])
    b = ops.gqa_decode_noalloc(q[:, :, :1].to(dev()), kd[:, :, :1034], vd[:, :, :1034])
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(a, b)


def test_accept_matches_oracle_with_ties():
    vocab, n_draft = 152064, 9
    g = torch.Generator().manual_seed(404)
    logits = torch.randn(n_draft + 1, vocab, generator=g).to(F16)
    logits[2, 500] = logits[2, 90000] = 30.0            # duplicated row maximum: the lower index wins
    preds = ref_accept.verify_predictions(logits, True)
    a = 4
    draft = [int(p) for p in preds[:n_draft]]
    draft[a] = (preds[a] + 1) % vocab
    want = ref_accept.verify_accept(logits, draft, True)
    announce("fp16 greedy_accept")
    lens = torch.tensor([5000, 1100], dtype=torch.int32, device=dev())
    out = ops.greedy_accept(logits.to(dev()), torch.tensor(draft, dtype=torch.int32, device=dev()), True,
                            None, lens)
    torch.cuda.synchronize()
    out = out.cpu().tolist()
    assert out[0] == want[0] == a and out[1] == want[1] and out[2:] == want[2] and want[2][2] == 500
    assert lens.cpu().tolist() == [5000 - (n_draft - a), 1100 - (n_draft - a)]


def test_selection_and_compaction():
    P, T, K = 4096, 128, 896
    g = torch.Generator().manual_seed(405)
    q_text = torch.randn(1, NQ, T, D, generator=g).to(F16)
    k = torch.randn(1, NKV, P, D, generator=g).to(F16)
    v = torch.randn(1, NKV, P, D, generator=g).to(F16)
    text_start = P - T
    announce(f"fp16 select_topk P={P} k={K} + compaction")
    kb, vb = cache_buffer(k, P + 40), cache_buffer(v, P + 40)
    vis = torch.arange(text_start, dtype=torch.int32, device=dev())
    topk, scores = ops.select_topk(q_text.to(dev()), kb, text_start, vis, K, return_scores=True)
    torch.cuda.synchronize()
    ref_scores = ref_sel.selection_scores(q_text, k, text_start)
    np.testing.assert_allclose(scores.cpu().numpy(), ref_scores, rtol=1e-11, atol=1e-300)
    np.testing.assert_array_equal(topk.cpu().numpy(), ref_sel.topk_positions(ref_scores, np.arange(text_start), K))
    nonvis = torch.arange(text_start, P, dtype=torch.int32, device=dev())
    idx = ops.build_compact_index(nonvis, topk)
    sk = torch.zeros(1, NKV, K + T + 16, D, dtype=F16, device=dev())
    sv = torch.zeros_like(sk)
    ops.compact_kv(kb, vb, sk, sv, idx)
    torch.cuda.synchronize()
    rows = idx.cpu().long()
    for h in range(NKV):
        assert torch.equal(sk[0, h, :K + T].cpu(), k[0, h, rows[h]])
        assert torch.equal(sv[0, h, :K + T].cpu(), v[0, h, rows[h]])


def test_rope_append_matches_oracle():
    n, cap, length, pos = 10, 300, 137, 131000
    g = torch.Generator().manual_seed(406)
    qkv = torch.randn(1, n, (NQ + 2 * NKV) * D, generator=g).to(F16)
    kc = torch.full((1, NKV, cap, D), float("nan"), dtype=F16, device=dev())
    vc = torch.full_like(kc, float("nan"))
    inv = ref_rope.inv_freq(1e6, D)
    announce("fp16 rope_append")
    one = lambda x: torch.tensor([x], dtype=torch.int32, device=dev())     # noqa: E731
    q = ops.rope_append(qkv.to(dev()), NQ, kc, vc, one(length), one(pos), torch.from_numpy(inv).to(dev()))
    torch.cuda.synchronize()
    x = qkv[0].float().numpy().reshape(n, NQ + 2 * NKV, D)
    cos, sin = ref_rope.cos_sin(pos + np.arange(n), inv, "fp16")
    want_q = ref_rope.apply_rope(x[:, :NQ].transpose(1, 0, 2), cos, sin, "fp16")
    want_k = ref_rope.apply_rope(x[:, NQ:NQ + NKV].transpose(1, 0, 2), cos, sin, "fp16")
    rows = {"q": (q[0].float().cpu().numpy(), want_q, x[:, :NQ].transpose(1, 0, 2)),
            "k": (kc[0, :, length:length + n].float().cpu().numpy(), want_k, x[:, NQ:NQ + NKV].transpose(1, 0, 2))}
    for name, (got, want, xin) in rows.items():
        diff = np.abs(got - want)
        # exact except where the device's and the oracle's cos/sin round to
        # neighbouring fp16 values; then each product term moves by about an
        # fp16 ulp of its own size (|x| |cos| + |rotate_half(x)| |sin| bounds both)
        rot = np.concatenate([-xin[..., D // 2:], xin[..., :D // 2]], axis=-1)
        bound = (np.abs(xin) + np.abs(rot)) * 2.0 ** -9 + 2.0 ** -24
        print(f"[{name}] exact {(diff == 0).mean():.5f}, max diff {diff.max():.3g}", flush=True)
        assert (diff == 0).mean() > 0.995 and (diff <= bound).all()
    np.testing.assert_array_equal(vc[0, :, length:length + n].float().cpu().numpy(), x[:, NQ + NKV:].transpose(1, 0, 2))


# -- the whole loop with an fp16 model ------------------------------------------
# The tiny random decoder in fp16: projections go through torch (the HIP GEMVs
# are bf16 only), every attention, rotary/append, norm, selection, compaction
# and acceptance step through the library in fp16.

def _tiny16():
    from std_amd.decoder import DecoderConfig, RandomDecoder
    cfg = DecoderConfig.tiny(layers=2)
    return cfg, RandomDecoder(cfg, dev(), F16, seed=7)


def _loop_inputs(cfg, seed, n_visual=1000, n_text=24):
    g = torch.Generator().manual_seed(seed)
    text = torch.randint(0, cfg.vocab_size - 2, (n_text,), generator=g)
    ids = torch.cat([torch.full((n_visual,), cfg.video_token_id), text]).view(1, -1)
    vis = torch.randn(n_visual, cfg.hidden_size, generator=g)
    return {"input_ids": ids.to(dev()), "visual_embeds": vis.to(dev(), F16)}


def test_loop_selection_and_compaction_from_fp16_prefill():
    """Selection on an fp16 prefill's captured text queries equals the oracle
    bit-exactly (fp64 scores of fp16 values); compact rows are bit copies."""
    from std_amd.kv_cache import initialize_past_key_values
    from std_amd.std_qwen25vl import (build_sparse_selection_from_queries, compact_sparse_prompt_cache,
                                      prefill_prompt)
    cfg, model = _tiny16()
    inputs = _loop_inputs(cfg, 11)
    P = inputs["input_ids"].shape[1]
    announce(f"fp16 loop: selection from prefill P={P}")
    pkv, _, _ = initialize_past_key_values(cfg, dev(), F16, P + 8)
    prompt_ids, _, _, text_start = prefill_prompt(model, inputs, pkv, cfg.video_token_id, capture_text_queries=True)
    queries = list(model.captured_queries)
    assert queries[0].dtype == F16 and torch.isfinite(queries[0]).all()
    sel = build_sparse_selection_from_queries(queries, [layer[0].data for layer in pkv], prompt_ids,
                                              cfg.video_token_id, text_start, target_k_plus_text=256,
                                              num_key_value_heads=1)
    want = ref_sel.build_sparse_selection([q.cpu() for q in queries], [layer[0].data[:, :, :P].cpu() for layer in pkv],
                                          prompt_ids[0].cpu().tolist(), cfg.video_token_id, target_k_plus_text=256)
    assert (sel.k, sel.prompt_len) == (want["k"], want["prompt_len"])
    for layer in range(cfg.num_hidden_layers):
        np.testing.assert_array_equal(sel.topk_positions[layer].numpy(), want["topk_positions"][layer])
    sparse, _, sparse_len = initialize_past_key_values(cfg, dev(), F16, sel.compact_len + 4)
    n = compact_sparse_prompt_cache(sparse, sparse_len, sel, pkv)
    torch.cuda.synchronize()
    for layer in range(cfg.num_hidden_layers):
        idx = ref_sel.compact_index(want["non_visual_positions"], want["topk_positions"][layer][0])
        for kind in range(2):
            assert torch.equal(sparse[layer][kind].data[0, 0, :n].cpu(),
                               pkv[layer][kind].data[0, 0, torch.as_tensor(idx)].cpu())


def test_loop_graph_rounds_equal_eager_rounds_fp16():
    """fp16 model: the graph-replayed rounds give the eager rounds' tokens and
    accept lengths; lengths stay consistent; generation stops at EOS."""
    from std_amd.std_qwen25vl import first_divergence, std_generate_qwen25vl
    cfg, model = _tiny16()
    inputs = _loop_inputs(cfg, 9)
    announce("fp16 loop: STD eager vs graph rounds, 32 tokens, gamma 9")
    kw = dict(max_new_tokens=32, gamma=9, target_k_plus_text=256, ignore_eos=True)
    eager, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, use_graphs=False, **kw)
    graph, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, use_graphs=True, **kw)
    assert eager.generate_len == graph.generate_len == 32 and graph.decode_rounds >= 3
    assert all(0 <= a <= p for a, p in zip(graph.accept_lengths, graph.proposed_lengths))
    assert graph.accept_lengths == eager.accept_lengths
    assert first_divergence(graph.output_ids, eager.output_ids) is None
    gen = graph.output_ids[0, -graph.generate_len:].tolist()
    eos = gen[5]
    stop, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, eos, use_graphs=True,
                                    **dict(kw, ignore_eos=False))
    assert stop.output_ids[0, -stop.generate_len:].tolist() == gen[:gen.index(eos) + 1]


def test_loop_indexed_sparse_kv_equals_compact_fp16():
    from std_amd.std_qwen25vl import std_generate_qwen25vl
    cfg, model = _tiny16()
    inputs = _loop_inputs(cfg, 9)
    announce("fp16 loop: sparse_kv indexed vs compact, graphs")
    kw = dict(max_new_tokens=24, gamma=9, target_k_plus_text=256, ignore_eos=True, use_graphs=True)
    comp, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, **kw)
    idx, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, sparse_kv="indexed", **kw)
    assert torch.equal(idx.output_ids, comp.output_ids) and idx.accept_lengths == comp.accept_lengths
