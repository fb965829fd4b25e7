"""Host-side logic of the std_qwen25vl / kv_cache mirror (CPU only: no
kernel is launched)."""
import types

import pytest
import torch

from std_amd import kv_cache
from std_amd.decoder import DecoderConfig
from std_amd.std_qwen25vl import (GenerateResult, SparseDraftController, SparseSelection, first_divergence,
                                  get_last_video_idx, selection_k, split_video_text_inputs, std_generate_qwen25vl)


def test_last_video_idx_matches_reverse_scan():
    """utils.py:8-15: last occurrence, -1 when absent."""
    assert get_last_video_idx([5, 9, 9, 3, 9, 1], 9) == 4
    assert get_last_video_idx([1, 2, 3], 9) == -1
    assert get_last_video_idx(torch.tensor([9]), 9) == 0


@pytest.mark.parametrize("prompt_len,text_start,n_visual,target,explicit,expect", [
    (4096, 3968, 3968, 1024, None, (128, 896)),        # C1/C2/C4 layout
    (65536, 65408, 65408, 4096, None, (128, 3968)),    # C3
    (200, 190, 190, 1024, None, (10, 190)),            # k capped by the visual count
    (100, 100, 100, 1024, None, (1, 100)),             # text_len floors at 1
    (4096, 3968, 3968, 1024, 7, (128, 7)),             # explicit k wins
    (4096, 3968, 3968, 100, None, (128, 1)),           # k floors at 1
])
def test_selection_k_rule(prompt_len, text_start, n_visual, target, explicit, expect):
    """std_qwen25vl.py:190-195."""
    assert selection_k(prompt_len, text_start, n_visual, target, explicit) == expect


def test_split_video_text_inputs():
    ids = torch.tensor([[7, 7, 1, 7, 2, 3]])
    text_start, video, text = split_video_text_inputs(ids, 7)
    assert text_start == 4
    assert video.tolist() == [[7, 7, 1, 7]] and text.tolist() == [[2, 3]]
    with pytest.raises(ValueError, match="No video token"):
        split_video_text_inputs(torch.tensor([[1, 2]]), 7)


def test_kv_cache_cat_copy_and_overflow():
    """kv_cache.py:42-69 semantics on CPU tensors."""
    cfg = DecoderConfig.tiny(layers=2)
    pkv, data, lengths = kv_cache.initialize_past_key_values(cfg, torch.device("cpu"), torch.float32, 8)
    assert data.shape == (4, 1, 1, 8, 128) and lengths.shape == (4,) and lengths.dtype == torch.long
    assert pkv[1][0].data.data_ptr() == data[2].data_ptr() and pkv[1][1].current_length is not None
    kc = pkv[0][0]
    rows = torch.arange(3 * 128, dtype=torch.float32).view(1, 1, 3, 128)
    view = kc.cat(rows)
    assert kc.length == 3 and view.shape == (1, 1, 3, 128) and torch.equal(view, rows)
    assert int(lengths[0]) == 3 and int(lengths[1]) == 0          # K and V lengths are independent
    assert kc.shape == (1, 1, 3, 128)
    kc.copy(torch.tensor([2, 0]), prev_length=1)
    assert kc.length == 3
    assert torch.equal(kc.data[0, 0, 1], rows[0, 0, 2]) and torch.equal(kc.data[0, 0, 2], rows[0, 0, 0])
    with pytest.raises(RuntimeError, match="overflow"):
        kc.cat(torch.zeros(1, 1, 6, 128))
    with pytest.raises(RuntimeError, match="overflow"):
        kc.advance(6)
    kv_cache.fill_cache_length(lengths, 5)
    assert all(int(x) == 5 for x in lengths) and kc.length == 5


def test_default_max_cache_len(monkeypatch):
    monkeypatch.delenv("SPECVLM_MAX_CACHE_LEN", raising=False)
    assert kv_cache.default_max_cache_len(128000) == 16384
    assert kv_cache.default_max_cache_len(4096) == 8192
    monkeypatch.setenv("SPECVLM_MAX_CACHE_LEN", "1000")
    assert kv_cache.default_max_cache_len(128000) == 1000


def test_sparse_selection_host_mirror():
    topk = torch.tensor([[[3, 5], [1, 4]], [[0, 2], [6, 7]]], dtype=torch.int32)
    sel = SparseSelection(topk_device=topk, non_visual_positions=torch.tensor([8, 9]), prompt_len=10,
                          visual_len=8, text_len=2, k=2)
    host = sel.topk_positions
    assert len(host) == 2 and host[1].dtype == torch.int64 and host[1].tolist() == [[0, 2], [6, 7]]
    assert sel.topk_positions is host and sel.compact_len == 4


def test_controller_validates_mode():
    """std_qwen25vl.py:239-240 raises ValueError on an unknown mode; the
    reference's three mode names are accepted (each runs the HIP kernel) as
    well as "hip", and the reference's default needs no argument change."""
    class Model:
        sparse_controller = None
    sel = SparseSelection(torch.zeros(1, 1, 1, dtype=torch.int32), torch.tensor([0]), 2, 1, 1, 1)
    with pytest.raises(ValueError, match="sparse_attn_mode"):
        SparseDraftController(Model(), sel, sparse_attn_mode="flash")
    for mode in ("hip", "gqa_sdpa", "triton_gqa", "repeat_sdpa"):
        m = Model()
        c = SparseDraftController(m, sel, sparse_attn_mode=mode)
        c.install()
        assert m.sparse_controller is c and not c.enabled
    c.set_enabled(True)
    assert c.enabled
    assert SparseDraftController(Model(), sel, use_compile=True).use_compile      # the reference's flag is taken


@pytest.mark.parametrize("kwargs", [dict(verify_mode="tree"), dict(verify_fallback="always"),
                                    dict(sequential_fallback_max_accept=-1),
                                    dict(verify_fallback="sequential_on_low_margin"),
                                    dict(verify_margin_threshold=-0.5),
                                    dict(verify_mode="sequential", use_graphs=True),
                                    dict(verify_fallback="sequential_on_reject", use_graphs=True),
                                    dict(verify_margin_threshold=0.5, use_graphs=True),
                                    dict(adaptive_gamma_min=0), dict(verify_attn_backend="flash"),
                                    dict(sparse_kv="paged")])
def test_std_generate_rejects_unsupported_options(kwargs):
    with pytest.raises(ValueError):
        std_generate_qwen25vl(None, {"input_ids": torch.zeros(1, 4, dtype=torch.long)}, 7, 8, **kwargs)


@pytest.mark.parametrize("kwargs", [dict(verify_mode="sequential"), dict(verify_fallback="sequential_on_reject"),
                                    dict(verify_fallback="sequential_on_low_accept",
                                         sequential_fallback_max_accept=0),
                                    dict(verify_fallback="sequential_guard"),
                                    dict(verify_fallback="sequential_on_low_margin", verify_margin_threshold=0.1),
                                    dict(verify_margin_threshold=0.0), dict(copy_sparse_prefill=False),
                                    dict(use_compile=True), dict(use_compile=True, verify_mode="sequential")])
def test_std_generate_accepts_the_reference_verify_options(kwargs):
    """The reference's verify modes, fallbacks, margin threshold
    (std_qwen25vl.py:634-660), copy_sparse_prefill=False and use_compile pass
    validation: the call then fails on the missing model, not on the option."""
    with pytest.raises(AttributeError):
        std_generate_qwen25vl(None, {"input_ids": torch.zeros(1, 4, dtype=torch.long)}, 7, 8, **kwargs)


def test_math_on_full_accept_is_accepted_and_counts_full_accepts():
    """verify_attn_backend="math_on_full_accept" (std_qwen25vl.py:111-116,
    657-658, 843-858) is a valid option, and a round counts as one math
    re-verification exactly when its whole draft was accepted."""
    from std_amd.std_qwen25vl import math_reverify_count
    assert math_reverify_count("math_on_full_accept", 9, 9) == 1
    assert math_reverify_count("math_on_full_accept", 3, 3) == 1
    assert math_reverify_count("math_on_full_accept", 8, 9) == 0
    assert math_reverify_count("math_on_full_accept", 0, 9) == 0
    for backend in ("default", "math"):
        assert math_reverify_count(backend, 9, 9) == 0
    # validation passes (the call then fails on the missing model, not on the option)
    with pytest.raises(AttributeError):
        std_generate_qwen25vl(None, {"input_ids": torch.zeros(1, 4, dtype=torch.long)}, 7, 8,
                              verify_attn_backend="math_on_full_accept")


def test_indexed_sparse_kv_needs_a_16_bit_model():
    fp32_model = types.SimpleNamespace(dtype=torch.float32)
    with pytest.raises(ValueError):
        std_generate_qwen25vl(fp32_model, {"input_ids": torch.zeros(1, 4, dtype=torch.long)}, 7, 8,
                              sparse_kv="indexed")


def test_generate_result_fields_and_rate():
    r = GenerateResult(torch.zeros(1, 3), 1.0, 2.0, 3, accepted_draft_tokens=6, proposed_draft_tokens=8)
    assert r.acceptance_rate == 0.75
    assert GenerateResult(torch.zeros(1), 0.0, 0.0, 0).acceptance_rate == 0.0
    for name in ("accept_lengths", "proposed_lengths", "pending_lengths", "gamma_history", "draft_time",
                 "verify_time", "bonus_time", "selection_time", "sparse_cache_time"):
        assert hasattr(r, name)


def test_first_divergence():
    assert first_divergence(torch.tensor([1, 2, 3]), torch.tensor([1, 2, 3])) is None
    assert first_divergence(torch.tensor([1, 2, 3]), torch.tensor([1, 5, 3])) == 1
    assert first_divergence(torch.tensor([1, 2]), torch.tensor([1, 2, 3])) == 2


def test_7b_config_shapes():
    """Qwen2.5-VL-7B language model: 6.53 B layer + 0.545 B lm_head parameters."""
    c = DecoderConfig.qwen25vl_7b()
    d = c.head_dim
    per_layer = ((c.num_attention_heads + 2 * c.num_key_value_heads) * d * (c.hidden_size + 1)
                 + c.hidden_size * c.num_attention_heads * d + 3 * c.hidden_size * c.intermediate_size
                 + 2 * c.hidden_size)
    assert d == 128 and c.num_attention_heads // c.num_key_value_heads == 7
    assert abs(per_layer * c.num_hidden_layers / 1e9 - 6.53) < 0.01
    assert abs(c.vocab_size * c.hidden_size / 1e9 - 0.545) < 0.001


def test_same_layout_ignores_size_one_strides():
    """A projection's K (made contiguous after RoPE) and V (a transposed view)
    of one decode token differ only in the unused stride of the size-1 row dim."""
    from std_amd.ops import same_layout
    k = torch.randn(1, 4, 1, 128)
    v = torch.randn(1, 1, 4, 128).transpose(1, 2)
    assert k.stride() != v.stride() and v.is_contiguous()
    assert same_layout(k, v)
    kk = torch.randn(1, 4, 3, 128)
    vv = torch.randn(1, 3, 4, 128).transpose(1, 2)
    assert not same_layout(kk, vv)
    assert not same_layout(k, kk)


def test_generated_suffix_and_tokens_equal():
    from std_amd.std_qwen25vl import generated_suffix, tokens_equal
    ids = torch.tensor([[5, 6, 7, 8, 9]])
    assert generated_suffix(ids, 3).tolist() == [[8, 9]]
    assert tokens_equal(ids, ids.clone()) and not tokens_equal(ids, ids[:, :4])
    assert not tokens_equal(ids, torch.tensor([[5, 6, 7, 8, 0]]))


def test_copy_prompt_cache_copies_the_prefix_and_sets_lengths():
    from std_amd.std_qwen25vl import copy_prompt_cache
    cfg = DecoderConfig.tiny(layers=2)
    src, src_data, src_len = kv_cache.initialize_past_key_values(cfg, torch.device("cpu"), torch.float32, 16)
    dst, dst_data, dst_len = kv_cache.initialize_past_key_values(cfg, torch.device("cpu"), torch.float32, 12)
    src_data.copy_(torch.randn(src_data.shape, generator=torch.Generator().manual_seed(3)))
    src_len.fill_(10)
    copy_prompt_cache(src, dst, dst_len, 7)
    assert torch.equal(dst_data[:, :, :, :7], src_data[:, :, :, :7])
    assert not dst_data[:, :, :, 7:].any()
    assert dst_len.tolist() == [7] * len(dst_len) and all(c.length == 7 for layer in dst for c in layer)
    with pytest.raises(RuntimeError):
        copy_prompt_cache(src, dst, dst_len, 11)             # longer than the source's 10 rows


def test_initialize_past_key_values_takes_the_model_as_the_reference_does(monkeypatch):
    cfg = DecoderConfig.tiny(layers=2)
    model = types.SimpleNamespace(config=cfg, device=torch.device("cpu"), dtype=torch.bfloat16)
    monkeypatch.setenv("SPECVLM_MAX_CACHE_LEN", "96")
    pkv, data, lengths = kv_cache.initialize_past_key_values(model)
    assert data.dtype == torch.bfloat16 and data.device.type == "cpu"
    assert tuple(data.shape) == (4, 1, cfg.num_key_value_heads, 96, cfg.hidden_size // cfg.num_attention_heads)
    assert len(pkv) == 2 and pkv[1][1].capacity == 96 and lengths.tolist() == [0, 0, 0, 0]
    with pytest.raises(ValueError):
        kv_cache.initialize_past_key_values(cfg)          # a bare config needs a device and a dtype


def test_sparse_selection_is_built_as_the_reference_builds_it():
    layers = [torch.tensor([[1, 4, 6]]), torch.tensor([[0, 2, 5]])]          # per-layer [Hkv, k], CPU int64
    sel = SparseSelection(layers, torch.tensor([7, 8]), 9, 7, 2, 3)            # positional, as the reference's test
    assert sel.topk_device.dtype == torch.int32 and tuple(sel.topk_device.shape) == (2, 1, 3)
    assert all(torch.equal(a, b) for a, b in zip(sel.topk_positions, layers)) and sel.compact_len == 5
    kw = SparseSelection(topk_positions=layers, non_visual_positions=[7, 8], prompt_len=9, visual_len=7, text_len=2,
                         k=3)
    assert torch.equal(kw.topk_device, sel.topk_device) and kw.non_visual_positions.dtype == torch.int64
    with pytest.raises(ValueError):
        SparseSelection(layers, torch.tensor([7, 8]), 9, 7, 2, 3, topk_device=sel.topk_device)
    with pytest.raises(ValueError):
        SparseSelection(None, torch.tensor([7, 8]), 9, 7, 2, 3)


def test_initialize_past_key_values_takes_the_model_as_the_reference_passes_it():
    """initialize_past_key_values(model) (kv_cache.py:72): config, device and
    dtype from the model, positionally or by the reference's keyword."""
    cfg = DecoderConfig.tiny(layers=2)

    class Model:
        config = cfg
        device = torch.device("cpu")
        dtype = torch.float16

    for pkv, data, lengths in (kv_cache.initialize_past_key_values(Model(), max_cache_len=8),
                               kv_cache.initialize_past_key_values(model=Model(), max_cache_len=8)):
        assert data.shape == (4, 1, 1, 8, 128) and data.dtype == torch.float16 and lengths.shape == (4,)
        assert len(pkv) == 2 and pkv[1][1].capacity == 8
    with pytest.raises(ValueError):
        kv_cache.initialize_past_key_values(cfg, max_cache_len=8)          # a bare config needs device and dtype
