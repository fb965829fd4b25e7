"""GPU parity of the visual-attention collector that rides the verify pass
(std_verify_attn_collect) against the oracle restatement of
VerificationCollectorV3._hook (src/std_repro/dynamic_selection.py:504-519),
and bit-equality of its attention output with the plain verify launch."""
import numpy as np
import pytest
import torch

from oracle import collector as ref_coll
from std_amd import ops
from std_amd.workloads import WORKLOADS, make_layer
from tests.gpu_helpers import announce, cache_buffer, dev

pytestmark = pytest.mark.gpu

# Scores: fp32 sums of exp2 of fp32 logits whose queries carry the fp32 mean
# (bf16 head + bf16 remainder; fp16 head + fp16 remainder for fp16 caches),
# against fp64: relative 2e-4.
RTOL, ATOL = 2e-4, 1e-9


def _layer(wname, layer, prompt_len=None, q_len=None, dtype=torch.bfloat16):
    w = WORKLOADS[wname]
    x = make_layer(w, layer, prompt_len=prompt_len)
    if q_len is not None and q_len != x["q_verify"].shape[2]:
        x = dict(x, q_verify=x["q_verify"][:, :, :q_len].contiguous(), new_k=x["new_k"][:, :, :q_len].contiguous(),
                 new_v=x["new_v"][:, :, :q_len].contiguous())
    if dtype != torch.bfloat16:
        x = {n: x[n].to(dtype) for n in ("q_verify", "k", "v", "new_k", "new_v")}
    k = torch.cat([x["k"], x["new_k"]], 2)
    v = torch.cat([x["v"], x["new_v"]], 2)
    return w, x, k, v


def _check(wname, layer, vis_begin, vis_end, prompt_len=None, q_len=None, append=False, dtype=torch.bfloat16,
           rtol=RTOL):
    w, x, k, v = _layer(wname, layer, prompt_len, q_len, dtype)
    q = x["q_verify"]
    Q, kv_len = q.shape[2], k.shape[2]
    announce(f"collector {wname} layer={layer} kv_len={kv_len} q_len={Q} visual=[{vis_begin},{vis_end}) "
             f"append={append} dtype={dtype}")
    kb = cache_buffer(k, kv_len + 29)
    vb = cache_buffer(v, kv_len + 29)
    qd = q.to(dev())
    want_out = ops.verify_attention(qd, kb[:, :, :kv_len], vb[:, :, :kv_len])
    if append:
        kb2 = cache_buffer(x["k"], kv_len + 29)
        vb2 = cache_buffer(x["v"], kv_len + 29)
        out, scores = ops.verify_attention_collect(qd, kb2, vb2, vis_begin, vis_end, new_key=x["new_k"].to(dev()),
                                                   new_value=x["new_v"].to(dev()), kv_len=kv_len)
        torch.cuda.synchronize()
        assert torch.equal(kb2[:, :, :kv_len], kb[:, :, :kv_len]) and torch.equal(vb2[:, :, :kv_len],
                                                                                    vb[:, :, :kv_len])
    else:
        out, scores = ops.verify_attention_collect(qd, kb, vb, vis_begin, vis_end, kv_len=kv_len)
    torch.cuda.synchronize()
    assert torch.equal(out, want_out), "collector launch changed the verify output"
    want = ref_coll.verification_scores(q, k, np.arange(vis_begin, vis_end))
    got = scores.double().cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, rtol=rtol, atol=ATOL)
    np.testing.assert_allclose(got.sum(axis=1), Q, rtol=1e-4)


def test_collector_c2():
    w = WORKLOADS["c2"]
    _check("c2", 0, 0, w.prompt_len - w.text_len)


def test_collector_c2_append_first_round_rows():
    """Nine verify rows (the first round, no pending token) and the fused append."""
    w = WORKLOADS["c2"]
    _check("c2", 1, 0, w.prompt_len - w.text_len, q_len=9, append=True)


def test_collector_unaligned_visual_range():
    """Visual keys not starting at 0 nor on a 4-key boundary (a system prompt before the video)."""
    _check("c2", 2, 13, 3003, prompt_len=4096)


def test_collector_c4_full_context_lognormal_keys():
    """131082 keys with heavy-tailed key norms, the 128k-context verify."""
    w = WORKLOADS["c4"]
    _check("c4", 0, 0, w.prompt_len - w.text_len, append=True)


@pytest.mark.parametrize("wname", ["c2", "c4"])
def test_collector_fp16(wname):
    """fp16 caches and queries (the dtype the reference loads its model in):
    the same workloads' values converted to fp16, with the fused append. An
    fp16 head + fp16 remainder carries about 22 bits of the mean, so the
    bound is 2e-5 relative (1.9e-6 measured at 131082 keys); a head formed
    twice with different roundings left 4e4 scores beyond 1e-5."""
    w = WORKLOADS[wname]
    _check(wname, 0, 0, w.prompt_len - w.text_len, append=True, dtype=torch.float16, rtol=2e-5)


def test_collector_class_on_a_decoder_verify_forward():
    """VerificationCollectorV3 (the reference's interface) around a bf16 verify
    forward of a two-layer decoder: per-layer scores equal the oracle on that
    forward's rotated queries and cached keys, and the verify logits are the
    same with and without the collector."""
    from std_amd.decoder import DecoderConfig, RandomDecoder
    from std_amd.kv_cache import initialize_past_key_values
    from std_amd.std_qwen25vl import VerificationCollectorV3, prefill_prompt

    announce("collector class on a tiny bf16 decoder verify forward")
    cfg = DecoderConfig.tiny(layers=2)
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=5003)
    gen = torch.Generator().manual_seed(17)
    n_vis, n_text, Q = 1000, 24, 10
    ids = torch.cat([torch.full((n_vis,), cfg.video_token_id),
                     torch.randint(0, cfg.vocab_size - 2, (n_text,), generator=gen)]).view(1, -1).to(dev())
    vis = torch.randn(n_vis, cfg.hidden_size, generator=gen).to(dev(), torch.bfloat16)
    P = n_vis + n_text
    step = torch.randint(0, cfg.vocab_size - 2, (1, Q), generator=gen).to(dev())
    results = []
    for with_collector in (False, True):
        pkv, _, _ = initialize_past_key_values(cfg, dev(), torch.bfloat16, P + 32)
        prefill_prompt(model, {"input_ids": ids, "visual_embeds": vis}, pkv, cfg.video_token_id)
        coll = None
        if with_collector:
            coll = VerificationCollectorV3(model, torch.arange(n_vis))
            coll.install()
            coll.begin_verification(0)
        model.capture_text_queries = True
        logits = model(step, pkv, all_logits=True)
        model.capture_text_queries = False
        if coll is not None:
            coll.end_verification()
            coll.uninstall()
        torch.cuda.synchronize()
        results.append((logits, coll, [q.clone() for q in model.captured_queries], pkv))
    assert torch.equal(results[0][0], results[1][0]), "the collector changed the verify logits"
    _, coll, queries, pkv = results[1]
    scores = coll.latest_scores()
    assert scores.shape == (cfg.num_hidden_layers, cfg.num_key_value_heads, n_vis)
    for li in range(cfg.num_hidden_layers):
        keys = pkv[li][0].data[:, :, :P + Q]
        want = ref_coll.verification_scores(queries[li], keys, np.arange(n_vis))
        np.testing.assert_allclose(scores[li].double().numpy(), want, rtol=RTOL, atol=ATOL)


# --- any visual position set, longer verifies, device lengths, graph rounds ---

def _verify_rows(w, x, q_len, seed):
    """q_len verify rows: the workload's ten, then seeded N(0, 1) rows."""
    q, nk, nv = x["q_verify"], x["new_k"], x["new_v"]
    if q_len > q.shape[2]:
        g = torch.Generator().manual_seed(seed)
        extra = q_len - q.shape[2]
        q = torch.cat([q, torch.randn(1, w.n_q, extra, 128, generator=g).to(q.dtype)], 2)
        nk = torch.cat([nk, torch.randn(1, w.n_kv, extra, 128, generator=g).to(q.dtype)], 2)
        nv = torch.cat([nv, torch.randn(1, w.n_kv, extra, 128, generator=g).to(q.dtype)], 2)
    return q[:, :, :q_len].contiguous(), nk[:, :, :q_len].contiguous(), nv[:, :, :q_len].contiguous()


def _check_positions(wname, layer, positions, prompt_len=None, q_len=10, append=False, dtype=torch.bfloat16,
                     bit_equal_verify=True, rtol=RTOL):
    w = WORKLOADS[wname]
    x = make_layer(w, layer, prompt_len=prompt_len)
    q, nk, nv = _verify_rows(w, x, q_len, 900 + layer)
    if dtype != torch.bfloat16:
        x = {n: x[n].to(dtype) for n in ("k", "v")}
        q, nk, nv = q.to(dtype), nk.to(dtype), nv.to(dtype)
    k = torch.cat([x["k"], nk], 2)
    v = torch.cat([x["v"], nv], 2)
    kv_len = k.shape[2]
    pos = np.asarray(positions)
    announce(f"collector {wname} layer={layer} kv_len={kv_len} q_len={q_len} n_visual={pos.size} "
             f"span=[{pos[0]},{pos[-1]}] append={append} dtype={dtype}")
    visual = ops.visual_keys(torch.as_tensor(pos), dev())
    qd = q.to(dev())
    kb = cache_buffer(k, kv_len + 29)
    vb = cache_buffer(v, kv_len + 29)
    want_out = ops.verify_attention(qd, kb[:, :, :kv_len], vb[:, :, :kv_len])
    if append:
        kb2 = cache_buffer(x["k"], kv_len + 29)
        vb2 = cache_buffer(x["v"], kv_len + 29)
        out, scores = ops.verify_attention_collect(qd, kb2, vb2, visual=visual, new_key=nk.to(dev()),
                                                   new_value=nv.to(dev()), kv_len=kv_len)
        torch.cuda.synchronize()
        assert torch.equal(kb2[:, :, :kv_len], kb[:, :, :kv_len]) and torch.equal(vb2[:, :, :kv_len],
                                                                                    vb[:, :, :kv_len])
    else:
        out, scores = ops.verify_attention_collect(qd, kb, vb, visual=visual, kv_len=kv_len)
    torch.cuda.synchronize()
    if bit_equal_verify:
        assert torch.equal(out, want_out), "collector launch changed the verify output"
    else:
        from oracle import attention as ref_attn
        from tests.gpu_helpers import assert_close
        assert_close(out, ref_attn.verify_attention(q, k, v), dtype)
    want = ref_coll.verification_scores(q, k, pos)
    got = scores.double().cpu().numpy()
    assert got.shape == want.shape and np.isfinite(got).all()
    np.testing.assert_allclose(got, want, rtol=rtol, atol=ATOL)
    np.testing.assert_allclose(got.sum(axis=1), q_len, rtol=1e-4)
    return out, scores


def test_collector_two_visual_segments_c2():
    """Video tokens in two segments split by 100 text tokens (a prompt that
    interleaves text and video): the hook gathers the keys at exactly those
    positions (dynamic_selection.py:515)."""
    w = WORKLOADS["c2"]
    V = w.prompt_len - w.text_len
    pos = np.concatenate([np.arange(0, 6000), np.arange(6100, V)])
    _check_positions("c2", 3, pos)


def test_collector_two_visual_segments_c4_full_context():
    """131082 keys with two visual segments (the second starting off a 64-key
    tile boundary) and the fused append."""
    w = WORKLOADS["c4"]
    V = w.prompt_len - w.text_len
    pos = np.concatenate([np.arange(17, 65000), np.arange(65037, V)])
    _check_positions("c4", 1, pos, append=True)


def test_collector_scattered_visual_positions():
    """An irregular visual set: every third key of one range, a dense run,
    and single keys (mask words with isolated bits, tiles with no visual key)."""
    g = np.random.default_rng(5)
    pos = np.unique(np.concatenate([np.arange(40, 1500, 3), np.arange(2000, 2400), g.choice(np.arange(2600, 3900), 50,
                                                                                           replace=False)]))
    _check_positions("c2", 4, pos, prompt_len=4096)


@pytest.mark.parametrize("q_len", [11, 13])
def test_collector_more_rows_than_one_launch(q_len):
    """gamma = 10 and 12 at seven query heads per KV head: (7 + 1) q_len > 80,
    so the verify runs in chunks of positions (each chunk's rows see the same
    keys they would in one launch); the attention output is held to the
    oracle and the scores sum over all q_len positions."""
    w = WORKLOADS["c2"]
    _check_positions("c2", 5, np.arange(0, w.prompt_len - w.text_len), q_len=q_len, append=True,
                     bit_equal_verify=False)


def test_collector_more_rows_fp16_two_segments():
    w = WORKLOADS["c2"]
    V = w.prompt_len - w.text_len
    pos = np.concatenate([np.arange(0, 8000), np.arange(8064, V)])
    _check_positions("c2", 6, pos, q_len=12, dtype=torch.float16, bit_equal_verify=False, rtol=2e-5)


def test_collector_device_length_equals_host_length():
    """With the cache length read on the device (graph-replayed verify steps)
    the launch is the host-length launch when planned for the same key count:
    bit-equal outputs and scores; planned for a larger capacity, still the
    oracle's scores."""
    w = WORKLOADS["c2"]
    x = make_layer(w, 7)
    q, nk, nv = _verify_rows(w, x, 10, 907)
    k = torch.cat([x["k"], nk], 2)
    v = torch.cat([x["v"], nv], 2)
    kv_len = k.shape[2]
    V = w.prompt_len - w.text_len
    pos = np.concatenate([np.arange(0, 5000), np.arange(5050, V)])
    visual = ops.visual_keys(torch.as_tensor(pos), dev())
    announce(f"collector device length c2 kv_len={kv_len}")
    kb = cache_buffer(k, kv_len + 300)
    vb = cache_buffer(v, kv_len + 300)
    qd = q.to(dev())
    length = torch.tensor([kv_len - 10], dtype=torch.int32, device=dev())
    host_out, host_scores = ops.verify_attention_collect(qd, kb, vb, visual=visual, kv_len=kv_len)
    dev_out, dev_scores = ops.verify_attention_collect(qd, kb, vb, visual=visual, kv_len=kv_len, length=length)
    cap_out, cap_scores = ops.verify_attention_collect(qd, kb, vb, visual=visual, kv_len=kv_len + 300, length=length)
    torch.cuda.synchronize()
    assert torch.equal(dev_out, host_out) and torch.equal(dev_scores, host_scores)
    want = ref_coll.verification_scores(q, k, pos)
    np.testing.assert_allclose(cap_scores.double().cpu().numpy(), want, rtol=RTOL, atol=ATOL)
    from oracle import attention as ref_attn
    from tests.gpu_helpers import assert_close
    assert_close(cap_out, ref_attn.verify_attention(q, k, v), torch.bfloat16)


def _two_segment_inputs(cfg, seed):
    gen = torch.Generator().manual_seed(seed)
    vid = cfg.video_token_id
    ids = torch.cat([torch.full((400,), vid), torch.randint(0, cfg.vocab_size - 2, (20,), generator=gen),
                     torch.full((600,), vid), torch.randint(0, cfg.vocab_size - 2, (24,), generator=gen)]).view(1, -1)
    vis = torch.randn(1000, cfg.hidden_size, generator=gen)
    return {"input_ids": ids.to(dev()), "visual_embeds": vis.to(dev(), torch.bfloat16)}


@pytest.mark.parametrize("gamma", [9, 10])
def test_collector_in_graph_replayed_rounds(gamma):
    """VerificationCollectorV3 on the generate loop, installed on the model and
    as the trace collector (which brackets every verify step), with video
    tokens in two segments: the graph-replayed rounds (use_graphs=True) give
    the same tokens and, round for round, the same scores bit for bit as the
    eager rounds; each round's scores sum to the verify positions per KV head.
    gamma = 10 verifies eleven positions per round, in chunks."""
    from std_amd.std_qwen25vl import VerificationCollectorV3, set_trace_collector, std_generate_qwen25vl
    from std_amd.decoder import DecoderConfig, RandomDecoder

    cfg = DecoderConfig.tiny(layers=2)
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=5005)
    inputs = _two_segment_inputs(cfg, 31)
    positions = torch.nonzero(inputs["input_ids"][0] == cfg.video_token_id).flatten().cpu()
    runs = {}
    for use_graphs in (False, True):
        announce(f"collector in generate rounds, gamma={gamma}, graphs={use_graphs}")
        coll = VerificationCollectorV3(model, positions)
        coll.install()
        set_trace_collector(coll)
        try:
            res, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=40,
                                           gamma=gamma, target_k_plus_text=256, ignore_eos=True,
                                           use_graphs=use_graphs)
        finally:
            set_trace_collector(None)
            coll.uninstall()
        torch.cuda.synchronize()
        runs[use_graphs] = (res, coll)
    (eager, ce), (graph, cg) = runs[False], runs[True]
    assert torch.equal(eager.output_ids, graph.output_ids)
    assert eager.accept_lengths == graph.accept_lengths
    assert len(ce.rounds) == eager.decode_rounds and len(cg.rounds) == graph.decode_rounds
    assert graph.decode_rounds >= 3, "too few rounds to replay a captured verify"
    for r, (a, b) in enumerate(zip(ce.rounds, cg.rounds)):
        assert a.shape == (cfg.num_hidden_layers, cfg.num_key_value_heads, positions.numel())
        assert torch.equal(a, b), f"round {r}: graph-replayed scores differ from the eager round's"
        q_rows = graph.proposed_lengths[r] + graph.pending_lengths[r]
        np.testing.assert_allclose(b.double().sum(-1).numpy(), q_rows, rtol=1e-4)


def test_collector_records_every_round_of_a_long_verify():
    """gamma = 13 at seven query heads per KV head: fourteen verify positions
    (98 query rows per KV head) take the decoder's unfused verify path; the
    collector still records one round per verification (the reference's hook
    runs in every verify forward), each summing to the round's positions."""
    from std_amd.std_qwen25vl import VerificationCollectorV3, set_trace_collector, std_generate_qwen25vl
    from std_amd.decoder import DecoderConfig, RandomDecoder

    cfg = DecoderConfig.tiny(layers=2)
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=5006)
    inputs = _two_segment_inputs(cfg, 37)
    positions = torch.nonzero(inputs["input_ids"][0] == cfg.video_token_id).flatten().cpu()
    announce("collector rounds, gamma=13, eager")
    coll = VerificationCollectorV3(model, positions)
    coll.install()
    set_trace_collector(coll)
    try:
        res, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=30,
                                       gamma=13, target_k_plus_text=256, ignore_eos=True)
    finally:
        set_trace_collector(None)
        coll.uninstall()
    assert len(coll.rounds) == res.decode_rounds >= 2
    for r, sc in enumerate(coll.rounds):
        q_rows = res.proposed_lengths[r] + res.pending_lengths[r]
        assert sc.shape == (cfg.num_hidden_layers, cfg.num_key_value_heads, positions.numel())
        np.testing.assert_allclose(sc.double().sum(-1).numpy(), q_rows, rtol=1e-4)


def test_collector_class_takes_positions_in_any_order_with_repeats():
    """The reference's hook gathers key_states at visual_positions as given
    (dynamic_selection.py:515), so a collector built on a shuffled position
    list with repeats reports, position for position, the scores that the
    collector on the sorted distinct list reports for those positions (bit for
    bit: the launches score the sorted distinct set either way)."""
    from std_amd.decoder import DecoderConfig, RandomDecoder
    from std_amd.kv_cache import initialize_past_key_values
    from std_amd.std_qwen25vl import VerificationCollectorV3, prefill_prompt

    announce("collector class: visual positions shuffled, with repeats")
    cfg = DecoderConfig.tiny(layers=2)
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=5007)
    gen = torch.Generator().manual_seed(23)
    n_vis, n_text, Q = 900, 24, 10
    ids = torch.cat([torch.full((n_vis,), cfg.video_token_id),
                     torch.randint(0, cfg.vocab_size - 2, (n_text,), generator=gen)]).view(1, -1).to(dev())
    vis = torch.randn(n_vis, cfg.hidden_size, generator=gen).to(dev(), torch.bfloat16)
    P = n_vis + n_text
    step = torch.randint(0, cfg.vocab_size - 2, (1, Q), generator=gen).to(dev())
    sorted_pos = torch.arange(0, n_vis, 3)                       # every third visual position (a bit mask)
    given = torch.cat([sorted_pos[torch.randperm(sorted_pos.numel(), generator=gen)], sorted_pos[:17].flip(0)])
    scores = []
    for positions in (sorted_pos, given):
        pkv, _, _ = initialize_past_key_values(cfg, dev(), torch.bfloat16, P + 32)
        prefill_prompt(model, {"input_ids": ids, "visual_embeds": vis}, pkv, cfg.video_token_id)
        coll = VerificationCollectorV3(model, positions)
        coll.install()
        coll.begin_verification(0)
        model(step, pkv, all_logits=True)
        coll.end_verification()
        coll.uninstall()
        scores.append(coll.latest_scores())
        assert coll.visual_len == positions.numel()
    base, got = scores
    assert got.shape == (cfg.num_hidden_layers, cfg.num_key_value_heads, given.numel())
    rank = torch.searchsorted(sorted_pos, given)
    assert torch.equal(got, base[:, :, rank])
