"""End-to-end self-speculative decode on a tiny random decoder with the HIP
hot path (selection, compaction, sparse draft, parallel verify, greedy
acceptance, rollback): the std_qwen25vl.py loop through libstdhip.so."""
import numpy as np
import pytest
import torch

from oracle import selection as ref_sel
from std_amd.decoder import DecoderConfig, RandomDecoder
from std_amd.kv_cache import initialize_past_key_values
from std_amd.std_qwen25vl import (SparseSelection, ar_generate_qwen25vl, build_sparse_selection_from_queries,
                                  compact_sparse_prompt_cache, first_divergence, prefill_prompt,
                                  std_generate_qwen25vl)
from tests.gpu_helpers import announce, dev

pytestmark = pytest.mark.gpu

N_VISUAL, N_TEXT, TARGET = 1000, 24, 256


def _inputs(cfg, seed, n_visual=N_VISUAL, n_text=N_TEXT, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    text = torch.randint(0, cfg.vocab_size - 2, (n_text,), generator=gen)
    ids = torch.cat([torch.full((n_visual,), cfg.video_token_id), text]).view(1, -1)
    vis = torch.randn(n_visual, cfg.hidden_size, generator=gen)
    return {"input_ids": ids.to(dev()), "visual_embeds": vis.to(dev(), dtype)}


@pytest.fixture(scope="module")
def tiny32():
    cfg = DecoderConfig.tiny(layers=2)
    return cfg, RandomDecoder(cfg, dev(), torch.float32, seed=5001)


def test_selection_and_compaction_from_prefill(tiny32):
    """Selection on the captured text queries equals the oracle bit-exactly;
    the compact cache rows are bit copies of the dense rows."""
    cfg, model = tiny32
    inputs = _inputs(cfg, 11)
    P = inputs["input_ids"].shape[1]
    announce(f"e2e selection tiny fp32 P={P}")
    pkv, _, _ = initialize_past_key_values(cfg, dev(), torch.float32, P + 8)
    prompt_ids, _, _, text_start = prefill_prompt(model, inputs, pkv, cfg.video_token_id, capture_text_queries=True)
    queries = list(model.captured_queries)
    assert text_start == N_VISUAL and queries[0].shape == (1, 7, N_TEXT, 128)
    sel = build_sparse_selection_from_queries(queries, [layer[0].data for layer in pkv], prompt_ids,
                                              cfg.video_token_id, text_start, target_k_plus_text=TARGET,
                                              num_key_value_heads=1)
    want = ref_sel.build_sparse_selection([q.cpu() for q in queries], [layer[0].data[:, :, :P].cpu() for layer in pkv],
                                          prompt_ids[0].cpu().tolist(), cfg.video_token_id, target_k_plus_text=TARGET)
    assert (sel.k, sel.text_len, sel.visual_len, sel.prompt_len) == (want["k"], want["text_len"],
                                                                      want["visual_len"], want["prompt_len"])
    for layer in range(cfg.num_hidden_layers):
        np.testing.assert_array_equal(sel.topk_positions[layer].numpy(), want["topk_positions"][layer])
    sparse, _, sparse_len = initialize_past_key_values(cfg, dev(), torch.float32, sel.compact_len + 4)
    n = compact_sparse_prompt_cache(sparse, sparse_len, sel, pkv)
    torch.cuda.synchronize()
    assert n == N_TEXT + sel.k and all(int(x) == n for x in sparse_len)
    for layer in range(cfg.num_hidden_layers):
        idx = ref_sel.compact_index(want["non_visual_positions"], want["topk_positions"][layer][0])
        for kind in range(2):
            got = sparse[layer][kind].data[0, 0, :n].cpu()
            assert torch.equal(got, pkv[layer][kind].data[0, 0, torch.as_tensor(idx)].cpu())


def test_compaction_from_a_reference_built_selection(tiny32):
    """A SparseSelection built as the reference builds it (per-layer CPU
    position tensors) compacts exactly as the selection kernels' own."""
    cfg, model = tiny32
    inputs = _inputs(cfg, 12)
    P = inputs["input_ids"].shape[1]
    announce(f"e2e compaction from a reference-built selection P={P}")
    pkv, _, _ = initialize_past_key_values(cfg, dev(), torch.float32, P + 8)
    prompt_ids, _, _, text_start = prefill_prompt(model, inputs, pkv, cfg.video_token_id, capture_text_queries=True)
    sel = build_sparse_selection_from_queries(list(model.captured_queries), [layer[0].data for layer in pkv],
                                              prompt_ids, cfg.video_token_id, text_start, target_k_plus_text=TARGET,
                                              num_key_value_heads=1)
    ref_built = SparseSelection([t.clone() for t in sel.topk_positions], sel.non_visual_positions, sel.prompt_len,
                                sel.visual_len, sel.text_len, sel.k)
    caches = []
    for s in (sel, ref_built):
        sparse, data, lengths = initialize_past_key_values(cfg, dev(), torch.float32, sel.compact_len + 4)
        n = compact_sparse_prompt_cache(sparse, lengths, s, pkv)
        caches.append((n, data))
    torch.cuda.synchronize()
    assert caches[0][0] == caches[1][0] == sel.compact_len
    assert torch.equal(caches[0][1], caches[1][1])


def test_std_tokens_equal_dense_ar_fp32(tiny32):
    """Greedy STD with exact dense verification reproduces dense AR decoding."""
    cfg, model = tiny32
    inputs = _inputs(cfg, 5)
    announce("e2e STD vs AR tiny fp32, 40 tokens, gamma 9")
    ar = ar_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=40, ignore_eos=True)
    std, sel = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=40, gamma=9,
                                     target_k_plus_text=TARGET, ignore_eos=True)
    assert ar.generate_len == std.generate_len == 40
    assert first_divergence(std.output_ids, ar.output_ids) is None
    assert std.decode_rounds == len(std.accept_lengths) == len(std.proposed_lengths)
    assert std.accepted_draft_tokens == sum(std.accept_lengths)
    assert std.proposed_draft_tokens == sum(std.proposed_lengths)
    assert all(0 <= a <= p for a, p in zip(std.accept_lengths, std.proposed_lengths))
    # every round but the last appends accept + 1 tokens
    assert sum(a + 1 for a in std.accept_lengths[:-1]) < 40 <= sum(a + 1 for a in std.accept_lengths)
    assert std.pending_lengths[0] == 0 and all(x == 1 for x in std.pending_lengths[1:])
    assert sel.k == TARGET - N_TEXT


def test_std_runs_bf16_with_eos_stop():
    """bf16 tiny decoder: the loop's invariants hold and generation stops at
    the first EOS when ignore_eos is False."""
    cfg = DecoderConfig.tiny(layers=2)
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=7)
    inputs = _inputs(cfg, 9, dtype=torch.bfloat16)
    announce("e2e STD tiny bf16, 32 tokens")
    std, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=32, gamma=9,
                                   target_k_plus_text=TARGET, ignore_eos=True)
    gen = std.output_ids[0, -std.generate_len:].tolist()
    assert std.generate_len == 32 and std.accepted_draft_tokens == sum(std.accept_lengths)
    eos = gen[5]                       # pretend the sixth generated token is EOS
    stop, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, eos, max_new_tokens=32, gamma=9,
                                    target_k_plus_text=TARGET, ignore_eos=False)
    got = stop.output_ids[0, -stop.generate_len:].tolist()
    assert got == gen[:gen.index(eos) + 1]


def test_full_selection_draft_equals_dense(tiny32):
    """With k = every visual position the compact cache equals the dense
    prompt cache, so the sparse draft (original positions, fused append,
    rollback, bonus append) must reproduce the dense model: every drafted
    token is accepted."""
    cfg, model = tiny32
    inputs = _inputs(cfg, 21, n_visual=300, n_text=20)
    announce("e2e STD tiny fp32, k = all visual positions")
    std, sel = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=36, gamma=5,
                                     explicit_k=300, ignore_eos=True)
    assert sel.k == 300 and sel.compact_len == 320
    assert std.accept_lengths == std.proposed_lengths, (std.accept_lengths, std.proposed_lengths)
    assert std.acceptance_rate == 1.0
    ar = ar_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=36, ignore_eos=True)
    assert first_divergence(std.output_ids, ar.output_ids) is None
    # "math_on_full_accept": every round accepts its whole draft, so every
    # round counts one math re-verification, which changes nothing
    math, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=36, gamma=5,
                                    explicit_k=300, ignore_eos=True, verify_attn_backend="math_on_full_accept")
    assert torch.equal(math.output_ids, std.output_ids) and math.accept_lengths == std.accept_lengths
    assert math.fallback_count == math.decode_rounds and math.fallback_accepted_extra == 0
    assert std.fallback_count == 0


def test_graph_rounds_equal_eager_rounds_fp32(tiny32):
    """The graph-replayed loops (cache lengths and positions on the device,
    rolled back by the acceptance kernel; one captured draft, verify and
    bonus graph replayed per round) give the eager loops' tokens and accept
    lengths, and STD still equals dense AR."""
    cfg, model = tiny32
    inputs = _inputs(cfg, 5)
    announce("e2e graph vs eager, STD and AR, tiny fp32, 40 tokens, gamma 4")
    kw = dict(max_new_tokens=40, ignore_eos=True)
    std_e, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, gamma=4,
                                     target_k_plus_text=TARGET, use_graphs=False, **kw)
    std_g, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, gamma=4,
                                     target_k_plus_text=TARGET, use_graphs=True, **kw)
    assert std_g.decode_rounds >= 3                       # rounds 2.. replay the captured graphs
    assert std_g.accept_lengths == std_e.accept_lengths and std_g.proposed_lengths == std_e.proposed_lengths
    assert first_divergence(std_g.output_ids, std_e.output_ids) is None
    ar_e = ar_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, use_graphs=False, **kw)
    ar_g = ar_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, use_graphs=True, **kw)
    assert first_divergence(ar_g.output_ids, ar_e.output_ids) is None
    assert first_divergence(std_g.output_ids, ar_g.output_ids) is None


def test_graph_full_selection_accepts_every_draft(tiny32):
    """Full selection with the graph-replayed rounds: any error in the device
    positions, lengths or rollback would reject drafts."""
    cfg, model = tiny32
    inputs = _inputs(cfg, 21, n_visual=300, n_text=20)
    announce("e2e graph rounds, tiny fp32, k = all visual positions")
    std, sel = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=40, gamma=5,
                                     explicit_k=300, ignore_eos=True, use_graphs=True)
    assert sel.compact_len == 320 and std.decode_rounds >= 4
    assert std.accept_lengths == std.proposed_lengths, (std.accept_lengths, std.proposed_lengths)
    ar = ar_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=40, ignore_eos=True,
                              use_graphs=True)
    assert first_divergence(std.output_ids, ar.output_ids) is None


def test_graph_rounds_bf16_with_eos_stop():
    cfg = DecoderConfig.tiny(layers=2)
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=7)
    inputs = _inputs(cfg, 9, dtype=torch.bfloat16)
    announce("e2e graph rounds tiny bf16, 32 tokens, EOS stop")
    std, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=32, gamma=9,
                                   target_k_plus_text=TARGET, ignore_eos=True, use_graphs=True)
    gen = std.output_ids[0, -std.generate_len:].tolist()
    assert std.generate_len == 32 and all(0 <= a <= p for a, p in zip(std.accept_lengths, std.proposed_lengths))
    eos = gen[5]
    stop, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, eos, max_new_tokens=32, gamma=9,
                                    target_k_plus_text=TARGET, ignore_eos=False, use_graphs=True)
    got = stop.output_ids[0, -stop.generate_len:].tolist()
    assert got == gen[:gen.index(eos) + 1]


@pytest.mark.parametrize("use_graphs", [False, True])
def test_indexed_sparse_kv_tokens_equal_compact(use_graphs):
    """The index-addressed sparse cache (the draft reads the selected prompt
    rows from the dense cache through the index lists) sees the same keys in
    the same order as the compacted cache: identical tokens and acceptance."""
    cfg = DecoderConfig.tiny(layers=2)
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=7)
    inputs = _inputs(cfg, 9, dtype=torch.bfloat16)
    announce(f"e2e STD tiny bf16, sparse_kv indexed vs compact, graphs={use_graphs}")
    kw = dict(max_new_tokens=32, gamma=9, target_k_plus_text=TARGET, ignore_eos=True, use_graphs=use_graphs)
    comp, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, **kw)
    idx, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, sparse_kv="indexed", **kw)
    assert torch.equal(idx.output_ids, comp.output_ids)
    assert idx.accept_lengths == comp.accept_lengths and idx.generate_len == 32


@pytest.mark.parametrize("use_graphs", [False, True])
def test_trace_collector_brackets_prefill_and_each_verify(tiny32, use_graphs):
    """set_trace_collector: one prefill bracket, then one verify bracket per
    round carrying the round number, opened and closed in order; removing
    the collector stops the calls (std_qwen25vl.py:30-38, 693-698, 799-805)."""
    from std_amd.std_qwen25vl import set_trace_collector
    cfg, model = tiny32
    inputs = _inputs(cfg, 5)
    events = []

    class Recorder:
        def begin_prefill(self):
            events.append("bp")

        def end_prefill(self):
            events.append("ep")

        def begin_verification(self, round_idx):
            events.append(("bv", round_idx))

        def end_verification(self):
            events.append("ev")

    announce(f"e2e trace collector brackets, graphs={use_graphs}")
    set_trace_collector(Recorder())
    try:
        std, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=20, gamma=4,
                                       target_k_plus_text=TARGET, ignore_eos=True, use_graphs=use_graphs)
    finally:
        set_trace_collector(None)
    want = ["bp", "ep"]
    for r in range(1, std.decode_rounds + 1):
        want += [("bv", r), "ev"]
    assert events == want
    events.clear()
    std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=4, gamma=2,
                          target_k_plus_text=TARGET, ignore_eos=True, use_graphs=use_graphs)
    assert events == []


@pytest.mark.parametrize("use_graphs", [False, True])
def test_cache_overflow_raises_instead_of_dropping_rows(tiny32, monkeypatch, use_graphs):
    """Caches sized too small for the decode: the reference's KVCache.cat
    raises (kv_cache.py:54-69). Here the device-length appends skip the rows
    past the capacity and mark the model's status word, which the round's
    readback turns into the same RuntimeError (with graphs), or the host
    length check raises it first (eager)."""
    import std_amd.std_qwen25vl as stdq
    cfg, model = tiny32
    inputs = _inputs(cfg, 13, n_visual=300, n_text=20)
    announce(f"e2e cache overflow reported, graphs={use_graphs}")
    monkeypatch.setattr(stdq, "_cache_capacity", lambda p, n, g: p + 12)
    with pytest.raises(RuntimeError, match="KV cache overflow"):
        std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=40, gamma=5,
                              target_k_plus_text=TARGET, ignore_eos=True, use_graphs=use_graphs)
    torch.cuda.synchronize()
    monkeypatch.undo()
    # the status word is cleared by the next call, which runs normally
    std, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=12, gamma=5,
                                   target_k_plus_text=TARGET, ignore_eos=True, use_graphs=use_graphs)
    assert std.generate_len == 12 and int(model.decode_status) == 0


@pytest.mark.parametrize("n_text", [N_TEXT, 9])
def test_prefill_output_attentions_feed_the_reference_selection(tiny32, n_text):
    """prefill_prompt(..., output_attentions=True) returns, as the reference's
    does (std_qwen25vl.py:150-172), each layer's text-suffix probabilities
    [1, n_q, T, P]: the causal softmax of the captured queries against the
    cached keys (fp64 recomputation, zero past each row's limit), and
    build_sparse_selection on them selects what the oracle selects from the
    same probabilities. Nine text rows fit the fused decode launch, which a
    prefill asked for its probabilities must not take."""
    from oracle import selection as ref_sel
    from std_amd.std_qwen25vl import build_sparse_selection
    cfg, model = tiny32
    inputs = _inputs(cfg, 17, n_text=n_text)
    P = inputs["input_ids"].shape[1]
    announce(f"prefill output_attentions tiny fp32 P={P} T={n_text}")
    pkv, _, _ = initialize_past_key_values(cfg, dev(), torch.float32, P + 8)
    prompt_ids, nxt, attn, text_start = prefill_prompt(model, inputs, pkv, cfg.video_token_id, True,
                                                       capture_text_queries=True)
    assert text_start == N_VISUAL and len(attn) == cfg.num_hidden_layers
    pkv2, _, _ = initialize_past_key_values(cfg, dev(), torch.float32, P + 8)
    _, nxt2, none, _ = prefill_prompt(model, inputs, pkv2, cfg.video_token_id)
    assert none is None and torch.equal(nxt, nxt2)
    g = cfg.num_attention_heads // cfg.num_key_value_heads
    for li in range(cfg.num_hidden_layers):
        a = attn[li]
        assert a.shape == (1, cfg.num_attention_heads, n_text, P) and a.dtype == torch.float32
        q = model.captured_queries[li].double().cpu()                   # [1, n_q, T, D]
        k = pkv[li][0].data[:, :, :P].double().cpu()                     # [1, n_kv, P, D]
        s = (q @ k.repeat_interleave(g, dim=1).transpose(-1, -2)) / np.sqrt(q.shape[-1])
        rows = torch.arange(text_start, P)[:, None]
        s = s.masked_fill(torch.arange(P)[None, :] > rows, float("-inf"))
        np.testing.assert_allclose(a.double().cpu().numpy(), torch.softmax(s, -1).numpy(), rtol=1e-4, atol=1e-6)
    sel = build_sparse_selection(attn, prompt_ids, cfg.video_token_id, text_start, target_k_plus_text=TARGET,
                                 num_key_value_heads=cfg.num_key_value_heads)
    for li in range(cfg.num_hidden_layers):
        scores = ref_sel.scores_from_probs(attn[li].double().cpu().numpy(), cfg.num_key_value_heads)
        want = ref_sel.topk_positions(scores, np.arange(text_start), sel.k)
        np.testing.assert_array_equal(sel.topk_positions[li].numpy(), want)


def test_use_compile_runs_the_graph_replayed_rounds(tiny32):
    """use_compile=True (the reference's CUDA-graph-compiled sparse step,
    std_qwen25vl.py:456-464) takes the graph-replayed rounds: the same tokens
    and accept lengths as use_graphs=True and as the eager loop."""
    cfg, model = tiny32
    inputs = _inputs(cfg, 5)
    announce("e2e use_compile vs use_graphs vs eager, tiny fp32")
    kw = dict(max_new_tokens=24, gamma=4, target_k_plus_text=TARGET, ignore_eos=True)
    eager, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, **kw)
    graphs, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, use_graphs=True, **kw)
    comp, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, use_compile=True, **kw)
    for r in (graphs, comp):
        assert torch.equal(r.output_ids, eager.output_ids) and r.accept_lengths == eager.accept_lengths


def test_use_compile_beyond_the_device_state_rows_runs_eagerly(tiny32):
    """With gamma = 13 the verify carries 14 x 7 = 98 rows per KV head, more
    than the device-state launches serve: use_compile then keeps the eager
    loop (the reference's compiled step has no such limit) and matches it."""
    cfg, model = tiny32
    inputs = _inputs(cfg, 6)
    announce("e2e use_compile at gamma 13 (eager rounds), tiny fp32")
    kw = dict(max_new_tokens=30, gamma=13, target_k_plus_text=TARGET, ignore_eos=True)
    assert not model.fused_rows(14)
    eager, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, **kw)
    comp, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, use_compile=True, **kw)
    assert torch.equal(comp.output_ids, eager.output_ids) and comp.accept_lengths == eager.accept_lengths
