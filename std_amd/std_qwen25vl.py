"""Sparse-to-Dense decoding with the HIP hot path, keeping the interface of
the reference's std_repro/std_qwen25vl.py.

Same flow and names as the reference: sparse visual KV selection after the
prompt prefill, a gamma-token draft with sparse attention over a compact
cache, one parallel dense verification, greedy acceptance, rollback and the
bonus-token append. What changes underneath:

* selection keeps the selected indices on the device
  (``SparseSelection.topk_device``; the reference's per-layer CPU lists are a
  lazily built host mirror). ``build_sparse_selection`` takes the reference's
  input, the materialised attention probabilities; the generate loop uses
  ``build_sparse_selection_from_queries``, which reads each layer's
  text-suffix queries and the dense key cache and never materialises them;
* compaction gathers straight from the dense cache into the sparse cache
  (no full-prompt copy);
* every attention call of the decode loop is a libstdhip.so launch with the
  KV append fused in, whichever ``sparse_attn_mode`` is named (the
  reference's default ``"gqa_sdpa"``, its other modes, or ``"hip"``);
* acceptance and rollback are computed on the device, and draft tokens stay
  on the device, so a round reads back a handful of int32 values once.

``verify_mode="sequential"``, the sequential verify fallbacks and the
margin checks (std_qwen25vl.py:780-893) run as the reference runs them, one
dense q_len = 1 forward per verified token, in the eagerly launched loop
(use_graphs=False, the default); the margin re-verification with the math
SDPA backend is counted, since the HIP verify computes that definition.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import ops
from .kv_cache import KVCache, fill_cache_length, initialize_past_key_values
from .verification_policy import VERIFY_FALLBACKS, min_prediction_margin, needs_sequential_fallback

# "hip" and the reference's three mode names (std_qwen25vl.py:239-240), which
# all compute the same draft attention: each runs the HIP decode kernel here.
SPARSE_ATTN_MODES = {"hip", "gqa_sdpa", "triton_gqa", "repeat_sdpa"}
# "compact": the selected prompt rows are copied into the sparse cache
# (compact_sparse_prompt_cache, std_qwen25vl.py:265-298); "indexed": the draft
# reads them from the dense cache through the per-head index lists (no copy;
# a selection refresh rewrites the indices only).
SPARSE_KV_MODES = {"compact", "indexed"}

_TRACE_COLLECTOR = None


def set_trace_collector(collector) -> None:
    """Install (None removes) an object whose ``begin_prefill()`` /
    ``end_prefill()`` bracket the prompt prefill of std_generate_qwen25vl and
    whose ``begin_verification(round)`` / ``end_verification()`` bracket each
    round's verify step (std_qwen25vl.py:30-38, 693-698, 799-805). The
    brackets run on the host around the step; with ``use_graphs=True`` a
    verify step is a graph replay, inside which no Python hook runs."""
    global _TRACE_COLLECTOR
    _TRACE_COLLECTOR = collector


class SparseSelection:
    """Per-layer sparse visual KV choices (std_qwen25vl.py:41-50).

    Built as the reference builds it, ``SparseSelection(topk_positions,
    non_visual_positions, prompt_len, visual_len, text_len, k)`` with the
    per-layer ascending [Hkv, k] position tensors (a list, or one [L, Hkv, k]
    tensor), or with ``topk_device=`` an int32 [L, Hkv, k] device tensor in
    place of ``topk_positions`` (what the selection kernels produce; the
    per-layer CPU tensors are then built on first access of
    ``topk_positions``). Compaction moves the indices to the cache's device."""

    def __init__(self, topk_positions=None, non_visual_positions=None, prompt_len: int = 0, visual_len: int = 0,
                 text_len: int = 0, k: int = 0, *, topk_device: Optional[torch.Tensor] = None):
        if (topk_positions is None) == (topk_device is None):
            raise ValueError("SparseSelection needs exactly one of topk_positions and topk_device")
        self._host: Optional[List[torch.Tensor]] = None
        if topk_device is None:
            if isinstance(topk_positions, torch.Tensor):
                topk_positions = list(topk_positions.unbind(0))
            layers = [torch.as_tensor(t) for t in topk_positions]
            topk_device = torch.stack(layers).to(torch.int32)
            self._host = [t.to("cpu", torch.int64) for t in layers]
        self.topk_device = topk_device
        self.non_visual_positions = torch.as_tensor(non_visual_positions).to("cpu", torch.int64)
        self.prompt_len = int(prompt_len)
        self.visual_len = int(visual_len)
        self.text_len = int(text_len)
        self.k = int(k)

    @property
    def topk_positions(self) -> List[torch.Tensor]:
        if self._host is None:
            host = self.topk_device.to("cpu", torch.int64)
            self._host = [host[i] for i in range(host.shape[0])]
        return self._host

    @property
    def compact_len(self) -> int:
        return int(self.non_visual_positions.numel()) + self.k

    def __repr__(self) -> str:
        return (f"SparseSelection(layers={self.topk_device.shape[0]}, heads={self.topk_device.shape[1]}, k={self.k}, "
                f"prompt_len={self.prompt_len}, visual_len={self.visual_len}, text_len={self.text_len})")


@dataclass
class GenerateResult:
    """Same fields as the reference's GenerateResult (std_qwen25vl.py:53-89)."""

    output_ids: torch.Tensor
    decoding_time: float
    inference_time: float
    generate_len: int
    accepted_draft_tokens: int = 0
    proposed_draft_tokens: int = 0
    mean_accept_length: float = 0.0
    decode_rounds: int = 0
    final_gamma: int = 0
    fallback_count: int = 0
    fallback_accepted_extra: int = 0
    verify_margin_reruns: int = 0
    min_verify_margin: float = 0.0
    gamma_history: List[int] = field(default_factory=list)
    proposed_lengths: List[int] = field(default_factory=list)
    accept_lengths: List[int] = field(default_factory=list)
    pending_lengths: List[int] = field(default_factory=list)
    draft_time: float = 0.0
    verify_time: float = 0.0
    bonus_time: float = 0.0
    cache_adjust_time: float = 0.0
    cache_init_time: float = 0.0
    prefill_time: float = 0.0
    selection_prefill_time: float = 0.0
    selection_time: float = 0.0
    dense_prefill_time: float = 0.0
    sparse_cache_time: float = 0.0

    @property
    def acceptance_rate(self) -> float:
        if self.proposed_draft_tokens == 0:
            return 0.0
        return self.accepted_draft_tokens / self.proposed_draft_tokens


# ---------------------------------------------------------------------------
# Prompt layout and the selection size rule.

def get_last_video_idx(input_ids, video_token_id: int) -> int:
    """Last position of video_token_id, or -1 (specvlm/utils/utils.py:8-15)."""
    ids = torch.as_tensor(input_ids).reshape(-1)
    hits = torch.nonzero(ids == video_token_id, as_tuple=False)
    return int(hits[-1]) if hits.numel() else -1


def selection_k(prompt_len: int, text_start: int, n_visual: int, target_k_plus_text: int = 1024,
                explicit_k: Optional[int] = None) -> Tuple[int, int]:
    """(text_len, k) with text_len = max(1, P - text_start) and
    k = min(explicit_k or max(1, target - text_len), n_visual)
    (std_qwen25vl.py:190-195)."""
    text_len = max(1, int(prompt_len) - int(text_start))
    k = int(explicit_k) if explicit_k is not None else max(1, int(target_k_plus_text) - text_len)
    return text_len, min(k, int(n_visual))


def split_video_text_inputs(input_ids: torch.Tensor, video_token_id: int) -> Tuple[int, torch.Tensor, torch.Tensor]:
    """(text_start, video-prefix ids, text-suffix ids) (std_qwen25vl.py:125-147)."""
    last = get_last_video_idx(input_ids[0], video_token_id)
    if last < 0:
        raise ValueError("No video token found in the prompt; STD visual KV selection requires video input.")
    text_start = last + 1
    return text_start, input_ids[:, :text_start], input_ids[:, text_start:]


def prefill_prompt(model, inputs: Dict[str, torch.Tensor], past_key_values, video_token_id: int,
                   output_attentions: bool = False, capture_text_queries: bool = False):
    """Video-prefix prefill, then the text suffix (std_qwen25vl.py:150-172).
    Returns, as the reference does, (prompt ids, next token [1, 1] on the
    device, attentions, text_start): with output_attentions the text suffix's
    per-layer softmax probabilities [1, n_q, T, P] in the model dtype (the
    input of build_sparse_selection), else None. With capture_text_queries
    the text suffix's per-layer queries are kept on the model instead, for
    build_sparse_selection_from_queries (which never materialises the
    probabilities)."""
    input_ids = inputs["input_ids"].to(model.device)
    visual = inputs.get("visual_embeds")
    text_start, video_ids, text_ids = split_video_text_inputs(input_ids, video_token_id)
    model(video_ids, past_key_values, visual_embeds=visual)
    model.capture_text_queries = capture_text_queries
    model.output_attentions = bool(output_attentions)
    try:
        logits = model(text_ids, past_key_values)
    finally:
        model.capture_text_queries = False
        model.output_attentions = False
    attentions = None
    if output_attentions:
        attentions = tuple(model.captured_attentions)
        model.captured_attentions = [None] * len(model.captured_attentions)
    next_token = _token_argmax(logits)
    return input_ids, next_token, attentions, text_start


# ---------------------------------------------------------------------------
# Selection and compaction.

def build_sparse_selection(attentions, full_input_ids: torch.Tensor, video_token_id: int, text_start: int,
                           target_k_plus_text: int = 1024, explicit_k: Optional[int] = None,
                           num_key_value_heads: int = 4) -> SparseSelection:
    """Top-k visual positions per (layer, KV head) from the prefill's
    materialised attention probabilities: the reference's signature and input
    (std_qwen25vl.py:175-231). attentions[l]: [1, Hq, T, P] probabilities of
    the text suffix's rows over the prompt (fp16 as the reference's attention
    returns them, bf16 or fp32), on the device. Each layer's group and
    text-row sums (fp64) and the top-k run on the device; ties go to the
    lowest position. build_sparse_selection_from_queries is the fast path that
    never materialises the probabilities."""
    prompt_ids = full_input_ids[0]
    if len(attentions) == 0:
        raise ValueError("no attention layers")
    dev = attentions[0].device
    visual = torch.nonzero(prompt_ids == video_token_id, as_tuple=False).flatten()
    if visual.numel() == 0:
        raise ValueError("Cannot build sparse selection without visual/video token positions.")
    non_visual = torch.nonzero(prompt_ids != video_token_id, as_tuple=False).flatten()
    prompt_len = int(prompt_ids.numel())
    text_len, k = selection_k(prompt_len, text_start, visual.numel(), target_k_plus_text, explicit_k)
    visual_i32 = visual.to(dev, torch.int32)
    layers = []
    for layer_attn in attentions:
        attn = layer_attn.detach()
        if attn.shape[-1] != prompt_len:
            raise ValueError(f"attention columns {attn.shape[-1]} != prompt length {prompt_len}")
        layers.append(ops.select_topk_probs(attn, visual_i32, k, num_key_value_heads))
    return SparseSelection(topk_device=torch.stack(layers), non_visual_positions=non_visual.to("cpu", torch.int64),
                           prompt_len=prompt_len, visual_len=int(visual.numel()), text_len=text_len, k=k)


def build_sparse_selection_from_queries(text_queries, key_caches, full_input_ids: torch.Tensor, video_token_id: int,
                                        text_start: int, target_k_plus_text: int = 1024,
                                        explicit_k: Optional[int] = None,
                                        num_key_value_heads: int = 4) -> SparseSelection:
    """Top-k visual positions per (layer, KV head) (std_qwen25vl.py:175-231)
    without materialising the probabilities.

    text_queries[l]: [1, Hq, T, D] text-suffix queries of layer l (RoPE
    applied); key_caches[l]: [1, Hkv, >= P, D] cache view of layer l. The
    scores are the reference's head-group and text-row sums of the causal
    softmax probabilities, computed exactly (fp64) on the device; ties go to
    the lowest position."""
    prompt_ids = full_input_ids[0]
    dev = key_caches[0].device
    visual = torch.nonzero(prompt_ids == video_token_id, as_tuple=False).flatten()
    if visual.numel() == 0:
        raise ValueError("Cannot build sparse selection without visual/video token positions.")
    non_visual = torch.nonzero(prompt_ids != video_token_id, as_tuple=False).flatten()
    prompt_len = int(prompt_ids.numel())
    text_len, k = selection_k(prompt_len, text_start, visual.numel(), target_k_plus_text, explicit_k)
    visual_i32 = visual.to(dev, torch.int32)
    layers = []
    for q_text, key in zip(text_queries, key_caches):
        if q_text.shape[1] % num_key_value_heads or key.shape[1] != num_key_value_heads:
            raise ValueError(
                f"Query heads ({q_text.shape[1]}) must be divisible by KV heads ({num_key_value_heads}).")
        if q_text.shape[2] != text_len:
            raise ValueError(f"text queries hold {q_text.shape[2]} rows, the prompt has {text_len}")
        layers.append(ops.select_topk(q_text.contiguous(), key, int(text_start), visual_i32, k))
    return SparseSelection(topk_device=torch.stack(layers), non_visual_positions=non_visual.to("cpu", torch.int64),
                           prompt_len=prompt_len, visual_len=int(visual.numel()), text_len=text_len, k=k)


def compact_sparse_prompt_cache(past_key_values, current_length_data: torch.Tensor, selection: SparseSelection,
                                dense_past_key_values) -> int:
    """Fill the sparse cache with each head's sorted union of non-visual and
    selected positions (std_qwen25vl.py:265-298), gathered straight from the
    dense prompt cache (which replaces copy_prompt_cache, :301-320)."""
    compact_len = selection.compact_len
    dev = past_key_values[0][0].data.device
    non_visual = selection.non_visual_positions.to(dev, torch.int32)
    for layer_idx, (sparse_layer, dense_layer) in enumerate(zip(past_key_values, dense_past_key_values)):
        index = ops.build_compact_index(non_visual, selection.topk_device[layer_idx].to(dev))
        if index.shape[1] != compact_len:
            raise RuntimeError("Compacted sparse KV produced an unexpected length.")
        ops.compact_kv(dense_layer[0].data, dense_layer[1].data, sparse_layer[0].data, sparse_layer[1].data, index)
    fill_cache_length(current_length_data, compact_len)
    return compact_len


def index_sparse_prompt_cache(past_key_values, current_length_data: torch.Tensor, selection: SparseSelection,
                              dense_past_key_values):
    """The index-addressed counterpart of compact_sparse_prompt_cache: builds
    each layer's sorted per-head key list (padded for the indexed decode),
    copies nothing, and sets the sparse length to compact_len as if the rows
    were there. Returns (compact_len, per-layer (dense K, dense V, index))."""
    compact_len = selection.compact_len
    dev = past_key_values[0][0].data.device
    non_visual = selection.non_visual_positions.to(dev, torch.int32)
    gathers = []
    for layer_idx, dense_layer in enumerate(dense_past_key_values):
        index = ops.build_compact_index(non_visual, selection.topk_device[layer_idx].to(dev))
        if index.shape[1] != compact_len:
            raise RuntimeError("Sparse key list has an unexpected length.")
        gathers.append((dense_layer[0].data, dense_layer[1].data, ops.pad_index(index)))
    fill_cache_length(current_length_data, compact_len)
    return compact_len, gathers


class SparseDraftController:
    """Routes the model's q_len = 1 attention to the sparse cache with the
    HIP decode kernel while enabled (std_qwen25vl.py:234-262); with index
    lists set (index-addressed sparse KV) the first compact_len keys of each
    layer are read from the dense cache through them."""

    def __init__(self, model, selection: SparseSelection, sparse_attn_mode: str = "gqa_sdpa",
                 use_compile: bool = False):
        if sparse_attn_mode not in SPARSE_ATTN_MODES:
            raise ValueError(f"Unsupported sparse_attn_mode={sparse_attn_mode!r}.")
        # use_compile: the reference compiles the sparse step with
        # torch.compile(mode="reduce-overhead"), i.e. CUDA-graph replay
        # (std_qwen25vl.py:456-464); here the generate loop captures the step
        # in a HIP graph instead (std_generate_qwen25vl turns use_graphs on)
        self.use_compile = bool(use_compile)
        self.model = model
        self.selection = selection
        self.sparse_attn_mode = sparse_attn_mode
        self.enabled = False
        self._installed = False
        self.compiled_forward = None
        self.gathers = None               # per layer (dense K, dense V, index) in the indexed mode
        self.n_index = 0

    def gather_for(self, layer_idx: int):
        """(dense K, dense V, index, n_index) of a layer, or None (compacted cache)."""
        if self.gathers is None:
            return None
        dk, dv, index = self.gathers[layer_idx]
        return dk, dv, index, self.n_index

    def install(self) -> None:
        if self._installed:
            return
        self.model.sparse_controller = self
        self._installed = True

    def set_enabled(self, enabled: bool) -> None:
        self.enabled = enabled


class VerificationCollectorV3:
    """Per-round visual relevance from the dense verify forward, with the
    interface of the reference's VerificationCollectorV3
    (src/std_repro/dynamic_selection.py:447-519): install / uninstall,
    begin_verification / end_verification around a verify forward, and
    ``rounds`` / ``latest_scores()`` holding fp32 [num_layers, kv_heads,
    visual_len] on the CPU (one readback per round).

    Where the reference's hook recomputes the group-mean queries against the
    gathered visual keys in separate GEMMs, each layer's scores here come out
    of the verify attention launch itself (``ops.verify_attention_collect``):
    the collector's query rows ride the verify kernel's padding rows, so the
    visual keys are read once. Any set of visual positions is served, in any
    order and with repeats, as the hook gathers key_states at visual_positions:
    the launches score the sorted distinct positions and the readback puts
    their scores in the caller's order (a repeated position repeats its
    score); a verify of more
    positions than one launch carries ((group + 1) * q_len > 80, e.g. gamma >=
    10 at seven query heads per KV head) runs in chunks of positions. Each
    layer's scores land in one persistent device buffer, so a verify step
    captured in a HIP graph (std_generate_qwen25vl(use_graphs=True)) writes
    them on every replay and end_verification reads them back with the round.
    begin_prefill / end_prefill do nothing, so the collector can also be
    installed with set_trace_collector, which brackets every verify step."""

    def __init__(self, model, visual_positions: torch.Tensor):
        pos = torch.as_tensor(visual_positions).to(torch.long).cpu().reshape(-1)
        if pos.numel() == 0:
            raise ValueError("no visual positions")
        self.model = model
        self.visual_positions = pos
        self.visual_len = int(pos.numel())
        self.num_kv_heads = model.config.num_key_value_heads
        # the launches score the sorted distinct positions; _order maps them
        # back to the caller's order (None: the positions are already that)
        distinct, inverse = torch.unique(pos, sorted=True, return_inverse=True)
        self._order = None if distinct.numel() == pos.numel() and torch.equal(distinct, pos) else inverse
        self.visual = ops.visual_keys(distinct, model.device)
        self.vis_begin, self.vis_end = self.visual.begin, self.visual.end
        self.scores_dev = torch.zeros(model.config.num_hidden_layers, self.num_kv_heads, int(distinct.numel()),
                                      dtype=torch.float32, device=model.device)
        self.rounds: List[torch.Tensor] = []
        self.active = False
        self.capturing = False            # set while a verify graph with the collector is captured
        self.graph_layers: List[int] = []
        self._layers: List[int] = []
        self.collect_time = 0.0

    @property
    def collecting(self) -> bool:
        return self.active or self.capturing

    def install(self) -> None:
        self.model.verify_collector = self

    def uninstall(self) -> None:
        if getattr(self.model, "verify_collector", None) is self:
            self.model.verify_collector = None

    def begin_prefill(self) -> None:
        pass

    def end_prefill(self) -> None:
        pass

    def begin_verification(self, round_id: int) -> None:
        self.active = True
        self._layers = []

    def scores_out(self, layer_idx: int) -> torch.Tensor:
        """The device buffer [kv_heads, visual_len] that a verify forward's
        layer writes its scores into."""
        return self.scores_dev[layer_idx]

    def record(self, layer_idx: int) -> None:
        """Called by the verify forward once layer layer_idx has written its scores."""
        if self.capturing:
            self.graph_layers.append(layer_idx)
        else:
            self._layers.append(layer_idx)

    def note_replay(self) -> None:
        """A captured verify graph with the collector was replayed: its layers
        wrote this round's scores."""
        if self.active:
            self._layers = list(self.graph_layers)

    def end_verification(self) -> None:
        self.active = False
        if not self._layers:
            return
        t0 = time.perf_counter()
        order = sorted(set(self._layers))
        if order == list(range(self.scores_dev.shape[0])):
            stacked = self.scores_dev.cpu()                                  # single sync
        else:
            stacked = self.scores_dev[torch.tensor(order, device=self.scores_dev.device)].cpu()
        if self._order is not None:
            stacked = stacked[:, :, self._order]
        self.collect_time += time.perf_counter() - t0
        self.rounds.append(stacked)
        self._layers = []

    def latest_scores(self) -> Optional[torch.Tensor]:
        return self.rounds[-1] if self.rounds else None


def math_reverify_count(verify_attn_backend: str, accept_len: int, draft_len: int) -> int:
    """1 if the reference would re-verify this round with the math SDPA
    backend, else 0. With "math_on_full_accept" the reference re-runs a fully
    accepted draft's verification with math attention and counts it in
    fallback_count (std_qwen25vl.py:843-858). The HIP verify already computes
    the math definition, so that re-run returns the same predictions: the
    round is counted, the accepted length and bonus stay, and
    fallback_accepted_extra gains nothing."""
    return int(verify_attn_backend == "math_on_full_accept" and accept_len == draft_len)


def _decode_status(model, dev) -> torch.Tensor:
    """The model's device status word (cleared), or a zero stand-in for a
    model without one."""
    status = getattr(model, "decode_status", None)
    if status is None:
        return torch.zeros(1, dtype=torch.int32, device=dev)
    status.zero_()
    return status


def _check_decode_status(value: int) -> None:
    """Raise as the reference's KVCache.cat does (kv_cache.py:54-69) when a
    device-length step reported a cache overflow."""
    if int(value) & ops.STATUS_CACHE_OVERFLOW:
        raise RuntimeError("KV cache overflow: a decode step's device length placed rows past a cache's capacity "
                           "(nothing was written there; the cache was sized too small for this decode)")


def _token_argmax(logits: torch.Tensor) -> torch.Tensor:
    """[1, 1] int64 next token of the last row (graph-capture safe argmax)."""
    return ops.argmax_rows(logits[0, -1:, :]).view(1, 1)


def _profile_mark(enabled: bool) -> float:
    if enabled:
        torch.cuda.synchronize()
    return time.time()


def _draft_tokens(model, first_token: torch.Tensor, gamma: int, past_key_values,
                  sparse_controller: SparseDraftController, start_position: int) -> torch.Tensor:
    """gamma sequential sparse forwards (std_qwen25vl.py:531-550); token i is
    fed at position start_position + i. Returns the drafted tokens as a device
    int64 tensor [gamma] (no per-token host sync)."""
    token = first_token.reshape(1, 1)
    drafted = []
    sparse_controller.set_enabled(True)
    try:
        for offset in range(gamma):
            drafted.append(token.reshape(1))
            logits = model(token, past_key_values, start_position=start_position + offset)
            token = _token_argmax(logits)
    finally:
        sparse_controller.set_enabled(False)
    return torch.cat(drafted)


def _append_dense_tokens(model, tokens, past_key_values) -> torch.Tensor:
    """One dense forward over ``tokens`` at the cache's length; returns the
    [1, 1] next token (std_qwen25vl.py:467-471)."""
    ids = torch.as_tensor(list(tokens) if not torch.is_tensor(tokens) else tokens, dtype=torch.long)
    return _token_argmax(model(ids.reshape(1, -1).to(model.device), past_key_values))


def _sequential_verify(model, draft: torch.Tensor, dense_next: torch.Tensor, dense_pkv) -> torch.Tensor:
    """Verify the drafted tokens one dense q_len = 1 forward at a time from a
    cache that holds everything before them (std_qwen25vl.py:885-893): the
    accepted length a is the longest prefix of the draft that the dense model
    predicts token by token, starting from dense_next; each accepted token is
    forwarded (its K/V cached), and the prediction after the last one is the
    bonus. Returns the device int32 pair (a, bonus)."""
    drafted = draft.reshape(-1).tolist()
    nxt = dense_next.reshape(1, 1)
    a = 0
    while a < len(drafted) and drafted[a] == int(nxt.reshape(-1)[0]):
        nxt = _token_argmax(model(draft.reshape(-1)[a:a + 1].reshape(1, 1).to(torch.long), dense_pkv))
        a += 1
    return torch.tensor([a, int(nxt.reshape(-1)[0])], dtype=torch.int32, device=model.device)


def _sequential_verify_draft(model, draft: torch.Tensor, dense_pending: Sequence[int], dense_next: torch.Tensor,
                             dense_pkv, dense_lengths: torch.Tensor, dense_cached_len: int) -> Tuple[int, int]:
    """Replay one round's verification sequentially (std_qwen25vl.py:504-528):
    roll the dense cache back to dense_cached_len, cache the pending tokens
    with one dense forward (its prediction replaces dense_next), then verify
    the draft one token at a time. Returns (accepted length, bonus token)."""
    fill_cache_length(dense_lengths, dense_cached_len)
    nxt = _append_dense_tokens(model, dense_pending, dense_pkv) if dense_pending else dense_next
    a, bonus = _sequential_verify(model, draft, nxt, dense_pkv).tolist()
    return int(a), int(bonus)


def _append_sparse_tokens(model, tokens: torch.Tensor, past_key_values, sparse_controller: SparseDraftController,
                          start_position: int) -> torch.Tensor:
    """Cache the bonus token in the sparse cache (std_qwen25vl.py:474-494)."""
    sparse_controller.set_enabled(True)
    try:
        next_token = None
        for offset in range(tokens.numel()):
            logits = model(tokens.reshape(-1)[offset:offset + 1].reshape(1, 1), past_key_values,
                           start_position=start_position + offset)
            next_token = _token_argmax(logits)
    finally:
        sparse_controller.set_enabled(False)
    if next_token is None:
        raise ValueError("Cannot append an empty sparse token sequence.")
    return next_token


def _contains_eos(tokens, eos_token_id: int) -> Optional[int]:
    for idx, token in enumerate(tokens):
        if int(token) == eos_token_id:
            return idx
    return None


def _cache_capacity(prompt_len: int, max_new_tokens: int, gamma: int) -> int:
    return prompt_len + max_new_tokens + gamma + 2


# ---------------------------------------------------------------------------
# HIP-graph capture of device-state decode steps.

def _warm_and_capture(run_all, restore, phases):
    """Run `run_all` once on a side stream (lazy library set-up stays out of
    the capture), undo its effect on the decode state with `restore`, then
    capture each phase (fn, args) in order into its own HIP graph. Returns
    [(graph, outputs)]; capturing executes nothing, so every phase reads the
    static outputs of the phases before it only when replayed in order."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_all()
    torch.cuda.current_stream().wait_stream(side)
    restore()
    torch.cuda.synchronize()
    captured = []
    for fn, args in phases:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = fn(*[a() if callable(a) else a for a in args])
        captured.append((graph, out))
    return captured


# ---------------------------------------------------------------------------
# Orchestrators.

@torch.inference_mode()
def ar_generate_qwen25vl(model, inputs: Dict[str, torch.Tensor], video_token_id: int, eos_token_id: int,
                         max_new_tokens: int = 256, output_attentions: bool = False, profile_prefill: bool = False,
                         ignore_eos: bool = False, use_graphs: bool = False) -> GenerateResult:
    """Greedy dense decoding with the same two-stage prefill
    (std_qwen25vl.py:553-606); every decode step runs the HIP rope/append and
    attention launches of each layer over the full dense cache. With
    use_graphs the step (cache length and position on the device) is captured
    once in a HIP graph and replayed per token. output_attentions is taken and
    changes nothing: the reference sets it so that the AR prefill runs the
    STD selection prefill's attention path (std_qwen25vl.py:565-568), and here
    both loops prefill through the same path without it."""
    del output_attentions
    torch.cuda.synchronize()
    start = time.time()
    prompt_len = int(inputs["input_ids"].shape[1])
    stage = _profile_mark(profile_prefill)
    pkv, _, lengths = initialize_past_key_values(model.config, model.device, model.dtype,
                                                 _cache_capacity(prompt_len, max_new_tokens, 0))
    cache_init_time = _profile_mark(profile_prefill) - stage if profile_prefill else 0.0
    stage = _profile_mark(profile_prefill)
    prompt_ids, next_token, _, _ = prefill_prompt(model, inputs, pkv, video_token_id)
    prefill_time = _profile_mark(profile_prefill) - stage if profile_prefill else 0.0

    generated: List[torch.Tensor] = []
    status = _decode_status(model, model.device)
    step = None
    if use_graphs and max_new_tokens > 1:
        state = torch.tensor([prompt_len, prompt_len], dtype=torch.int32).to(model.device)   # (length, position)
        token = next_token.reshape(1, 1).clone()

        def ar_step():
            token.copy_(_token_argmax(model(token, pkv, step_state=state)))
            return token

        snap = (state.clone(), token.clone())

        def restore():
            state.copy_(snap[0])
            token.copy_(snap[1])

        (graph, _), = _warm_and_capture(ar_step, restore, [(ar_step, ())])
        next_token = token
        step = graph.replay
    torch.cuda.synchronize()
    decode_start = time.time()
    while len(generated) < max_new_tokens:
        generated.append(next_token.reshape(1).clone() if step is not None else next_token.reshape(1))
        if not ignore_eos and int(next_token) == eos_token_id:
            break
        if len(generated) == max_new_tokens:
            break
        if step is not None:
            step()
        else:
            next_token = _token_argmax(model(next_token, pkv))
    if step is not None:
        fill_cache_length(lengths, prompt_len + len(generated) - 1)
    torch.cuda.synchronize()
    end = time.time()
    _check_decode_status(int(status[0]))
    gen = torch.cat(generated) if generated else torch.empty(0, dtype=torch.long, device=model.device)
    out = torch.cat([prompt_ids, gen.reshape(1, -1)], dim=1)
    return GenerateResult(out, end - decode_start, end - start, int(gen.numel()), cache_init_time=cache_init_time,
                          prefill_time=prefill_time)


@torch.inference_mode()
def std_generate_qwen25vl(model, inputs: Dict[str, torch.Tensor], video_token_id: int, eos_token_id: int,
                          max_new_tokens: int = 256, gamma: int = 9, target_k_plus_text: int = 1024,
                          explicit_k: Optional[int] = None, verify_mode: str = "parallel",
                          verify_fallback: str = "none", sequential_fallback_max_accept: int = 1,
                          profile_decode: bool = False, sparse_attn_mode: str = "gqa_sdpa",
                          adaptive_gamma_min: Optional[int] = None, adaptive_gamma_mode: str = "accept_len",
                          copy_sparse_prefill: bool = True, profile_prefill: bool = False,
                          verify_attn_backend: str = "default", verify_margin_threshold: Optional[float] = None,
                          use_compile: bool = False, ignore_eos: bool = False, use_graphs: bool = False,
                          sparse_kv: str = "compact", round_hook=None) -> Tuple[GenerateResult, SparseSelection]:
    """Sparse-to-Dense greedy decoding (std_qwen25vl.py:609-978).

    use_graphs: keep both caches' lengths and positions on the device (the
    acceptance kernel rolls them back) and replay each full-gamma round with a
    pending token as three captured HIP graphs (gamma sparse draft steps; the
    dense verify forward with greedy acceptance; the sparse bonus step), with
    one readback per round; the first round and any shorter round run the same
    device-state steps eagerly. With a VerificationCollectorV3 installed on the
    model when the call begins, a second verify graph carries its kernels and
    replaces the plain one in the rounds where the collector is active.

    verify_attn_backend: "default", "math" and "math_on_full_accept" all run
    the exact HIP verify (the math definition). With "math_on_full_accept" a
    fully accepted draft counts in ``fallback_count``, as the reference's
    math re-verification does (std_qwen25vl.py:843-858); that re-run would
    return the same predictions, so ``fallback_accepted_extra`` stays 0.

    use_compile: the reference compiles its sparse step into CUDA-graph
    replays (std_qwen25vl.py:456-464); here it turns on use_graphs, unless a
    sequential verify, fallback or margin check needs the eager loop or the
    verify rows exceed the device-state launches (more than 96 per KV head).

    verify_mode="sequential", verify_fallback and verify_margin_threshold:
    as in the reference (std_qwen25vl.py:780-893): sequential verification
    and the sequential replay of a round (counted in ``fallback_count``, its
    extra accepted tokens in ``fallback_accepted_extra``) run one dense
    q_len = 1 forward per verified token; a round whose smallest committed
    top-1/top-2 logit margin falls below the threshold counts a math
    re-verification in ``verify_margin_reruns`` (the HIP verify is that
    definition already), and ``min_verify_margin`` is the smallest margin
    seen. These host-side decisions need the eager loop: with use_graphs=True
    they raise ValueError.

    sparse_kv: "compact" gathers the selected prompt rows into the sparse
    cache; "indexed" (bf16, fp16) has the draft read them from the dense cache
    through the per-head index lists instead (same keys, same results).

    round_hook (a test probe; None adds nothing): called once per round after
    the rollback with a dict holding that round's verify logits [Q, vocab]
    (device; with graphs the captured graph's own buffer), draft, has_pending,
    dense_next, the kernel's accept_len and bonus, the pre-round lengths
    (dense_cached_len, n_pending, sparse_prev_len) and the rolled-back
    (dense, sparse) lengths: the device lengths with graphs, else the host
    lengths."""
    if sparse_kv not in SPARSE_KV_MODES:
        raise ValueError(f"Unsupported sparse_kv={sparse_kv!r}; choose one of {sorted(SPARSE_KV_MODES)}.")
    if sparse_kv == "indexed" and model.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("the index-addressed sparse cache serves bf16 and fp16 models")
    if verify_mode not in {"parallel", "sequential"}:
        raise ValueError(f"Unsupported verify_mode={verify_mode!r}; expected 'parallel' or 'sequential'.")
    if verify_fallback not in VERIFY_FALLBACKS:
        raise ValueError("verify_fallback must be 'none', 'sequential_on_reject', "
                         "'sequential_on_low_accept', 'sequential_on_low_margin', or 'sequential_guard'.")
    if sequential_fallback_max_accept < 0:
        raise ValueError("sequential_fallback_max_accept must be non-negative.")
    if verify_fallback == "sequential_on_low_margin" and verify_margin_threshold is None:
        raise ValueError("sequential_on_low_margin requires verify_margin_threshold.")
    if verify_attn_backend not in {"default", "math", "math_on_full_accept"}:
        raise ValueError("verify_attn_backend must be 'default', 'math', or 'math_on_full_accept'.")
    if verify_margin_threshold is not None and verify_margin_threshold < 0:
        raise ValueError("verify_margin_threshold must be non-negative.")
    host_policies = verify_mode != "parallel" or verify_fallback != "none" or verify_margin_threshold is not None
    if use_graphs and host_policies:
        raise ValueError("use_graphs=True replays the parallel verify with no host-side fallback; run "
                         "verify_mode='sequential', verify fallbacks and margin checks with use_graphs=False")
    # the reference's use_compile (a CUDA-graph-compiled sparse step) maps to
    # the graph-replayed rounds, where the round has no host-side decision and
    # the verify rows fit the device-state launches
    if use_compile and not use_graphs and not host_policies:
        fits = getattr(model, "fused_rows", None)
        use_graphs = fits is not None and fits(gamma + 1)
    if adaptive_gamma_min is not None and not (1 <= adaptive_gamma_min <= gamma):
        raise ValueError("adaptive_gamma_min must be between 1 and gamma.")
    if adaptive_gamma_mode not in {"accept_len", "conservative"}:
        raise ValueError("adaptive_gamma_mode must be 'accept_len' or 'conservative'.")
    # copy_sparse_prefill=False: the reference prefills the prompt a second
    # time into the sparse cache instead of copying the dense rows
    # (std_qwen25vl.py:735-739); the prefill is deterministic here, so those
    # rows equal the dense prefill's, from which compaction gathers either way
    del copy_sparse_prefill
    dev = model.device

    torch.cuda.synchronize()
    start = time.time()
    prompt_len = int(inputs["input_ids"].shape[1])
    stage = _profile_mark(profile_prefill)
    dense_pkv, _, dense_lengths = initialize_past_key_values(model.config, dev, model.dtype,
                                                             _cache_capacity(prompt_len, max_new_tokens, gamma))
    cache_init_time = _profile_mark(profile_prefill) - stage if profile_prefill else 0.0

    stage = _profile_mark(profile_prefill)
    trace = _TRACE_COLLECTOR
    if trace is not None:
        trace.begin_prefill()
    prompt_ids, dense_next, _, text_start = prefill_prompt(model, inputs, dense_pkv, video_token_id,
                                                        capture_text_queries=True)
    if trace is not None:
        trace.end_prefill()
    selection_prefill_time = _profile_mark(profile_prefill) - stage if profile_prefill else 0.0

    stage = _profile_mark(profile_prefill)
    queries = model.captured_queries
    model.captured_queries = [None] * model.config.num_hidden_layers
    selection = build_sparse_selection_from_queries(queries, [layer[0].data for layer in dense_pkv], prompt_ids,
                                                    video_token_id, text_start, target_k_plus_text=target_k_plus_text,
                                                    explicit_k=explicit_k,
                                                    num_key_value_heads=model.config.num_key_value_heads)
    del queries
    selection_time = _profile_mark(profile_prefill) - stage if profile_prefill else 0.0
    controller = SparseDraftController(model, selection, sparse_attn_mode=sparse_attn_mode, use_compile=use_compile)
    controller.install()

    stage = _profile_mark(profile_prefill)
    sparse_pkv, _, sparse_lengths = initialize_past_key_values(
        model.config, dev, model.dtype, _cache_capacity(selection.compact_len, max_new_tokens, gamma))
    if sparse_kv == "indexed":
        sparse_prompt_len, controller.gathers = index_sparse_prompt_cache(sparse_pkv, sparse_lengths, selection,
                                                                          dense_pkv)
        controller.n_index = sparse_prompt_len
    else:
        sparse_prompt_len = compact_sparse_prompt_cache(sparse_pkv, sparse_lengths, selection, dense_pkv)
    sparse_next = dense_next.clone()
    sparse_cache_time = _profile_mark(profile_prefill) - stage if profile_prefill else 0.0

    generated: List[int] = []
    accept_lengths: List[int] = []
    proposed_lengths: List[int] = []
    pending_lengths: List[int] = []
    gamma_history: List[int] = []
    dense_pending: List[int] = []
    accepted_total = proposed_total = decode_rounds = fallback_count = 0
    fallback_accepted_extra = verify_margin_reruns = 0
    verify_margins: List[float] = []
    draft_time = verify_time = bonus_time = cache_adjust_time = 0.0
    current_gamma = gamma
    dense_next_i32 = dense_next.reshape(1).to(torch.int32)

    # Device decode state for use_graphs: (dense length, dense position,
    # sparse length, sparse position). The dense position is the dense length
    # (cache_position); the sparse position is the original position of the
    # next drafted token. Both caches' pairs advance with their steps and are
    # rolled back together by the acceptance kernel.
    st4 = tok_s = pending = None
    graphs = None
    last_logits = [None]                    # the latest verify logits (round_hook)
    if use_graphs:
        st4 = torch.tensor([prompt_len, prompt_len, sparse_prompt_len, prompt_len], dtype=torch.int32).to(dev)
        tok_s = sparse_next.reshape(1, 1).clone()
        pending = torch.zeros(1, dtype=torch.long, device=dev)

    def draft_phase(n_steps: int) -> torch.Tensor:
        drafted = []
        controller.set_enabled(True)
        try:
            for _ in range(n_steps):
                drafted.append(tok_s.reshape(1).clone())
                tok_s.copy_(_token_argmax(model(tok_s, sparse_pkv, step_state=st4[2:4])))
        finally:
            controller.set_enabled(False)
        return torch.cat(drafted)

    def verify_phase(draft: torch.Tensor, has_pending: bool) -> torch.Tensor:
        ids = torch.cat([pending, draft]) if has_pending else draft
        logits = model(ids.reshape(1, -1), dense_pkv, step_state=st4[0:2], all_logits=True)
        last_logits[0] = logits[0]
        return ops.greedy_accept(logits[0], draft.to(torch.int32), has_pending=has_pending,
                                 dense_next=None if has_pending else dense_next_i32, rollback_lengths=st4)

    def bonus_phase(res: torch.Tensor) -> torch.Tensor:
        pending.copy_(res[1:2].to(torch.long))
        controller.set_enabled(True)
        try:
            tok_s.copy_(_token_argmax(model(pending.reshape(1, 1), sparse_pkv, step_state=st4[2:4])))
        finally:
            controller.set_enabled(False)
        return tok_s

    collector = getattr(model, "verify_collector", None)      # captured into the verify graph with graphs

    def verify_collect_phase(draft: torch.Tensor) -> torch.Tensor:
        # the verify forward with the installed collector's kernels in it (captured once, replayed in the
        # rounds where the collector is active)
        collector.capturing = True
        collector.graph_layers = []
        try:
            return verify_phase(draft, True)
        finally:
            collector.capturing = False

    def capture_round():
        snap = (st4.clone(), tok_s.clone(), pending.clone())

        def run_all():
            draft = draft_phase(gamma)
            state = st4.clone()
            res = verify_phase(draft, True)
            if collector is not None:        # the same verify again, with the collector (same rows, same result)
                st4.copy_(state)
                res = verify_collect_phase(draft)
            bonus_phase(res)

        def restore():
            st4.copy_(snap[0])
            tok_s.copy_(snap[1])
            pending.copy_(snap[2])

        holder = {}

        def draft_static():
            holder["draft"] = draft_phase(gamma)
            return holder["draft"]

        def verify_static(has_pending):
            holder["res"] = verify_phase(holder["draft"], has_pending)
            holder["logits"] = last_logits[0]
            return holder["res"]

        phases = [(draft_static, ()), (verify_static, (True,)), (lambda: bonus_phase(holder["res"]), ())]
        if collector is not None:
            def verify_collect_static():
                holder["res"].copy_(verify_collect_phase(holder["draft"]))     # the bonus graph reads holder["res"]
                holder["coll_logits"] = last_logits[0]
                return holder["res"]
            phases.append((verify_collect_static, ()))
        caps = _warm_and_capture(run_all, restore, phases)
        # the verify graphs' logits buffers: plain, and with the collector (or None)
        return caps, holder["draft"], holder["res"], (holder["logits"], holder.get("coll_logits"))

    status = _decode_status(model, dev)
    torch.cuda.synchronize()
    decode_start = time.time()
    while len(generated) < max_new_tokens:
        decode_rounds += 1
        remaining = max_new_tokens - len(generated)
        gamma_history.append(current_gamma)
        propose_len = min(current_gamma, remaining)
        context_len = prompt_len + len(generated)
        dense_cached_len = context_len - len(dense_pending)
        sparse_prev_len = sparse_prompt_len + len(generated)
        replay = use_graphs and bool(dense_pending) and propose_len == gamma
        if replay and graphs is None:
            graphs = capture_round()
        if verify_mode == "sequential" and dense_pending:
            # sequential verification starts from a dense cache that holds the
            # pending bonus token (std_qwen25vl.py:785-791)
            stage = _profile_mark(profile_decode)
            fill_cache_length(dense_lengths, dense_cached_len)
            dense_next = _append_dense_tokens(model, dense_pending, dense_pkv)
            dense_pending = []
            dense_cached_len = context_len
            cache_adjust_time += _profile_mark(profile_decode) - stage

        stage = _profile_mark(profile_decode)
        if replay:
            graphs[0][0][0].replay()
            draft_dev = graphs[1]
        elif use_graphs:
            draft_dev = draft_phase(propose_len)
        else:
            draft_dev = _draft_tokens(model, sparse_next, propose_len, sparse_pkv, controller,
                                      start_position=context_len)
        draft_time += _profile_mark(profile_decode) - stage
        proposed_total += propose_len
        proposed_lengths.append(propose_len)
        pending_lengths.append(len(dense_pending))

        stage = _profile_mark(profile_decode)
        trace = _TRACE_COLLECTOR if verify_mode == "parallel" else None
        if trace is not None:
            trace.begin_verification(decode_rounds)
        current = getattr(model, "verify_collector", None)
        collecting = current is not None and current.active
        if replay and collecting and (len(graphs[0]) < 4 or current is not collector):
            # a collector installed after the call began has no captured verify: this round's verify runs
            # eagerly (device state), and the captured bonus step reads its result from the verify graph's buffer
            graphs[2].copy_(verify_phase(draft_dev, True))
            res = graphs[2]
        elif replay and collecting:
            graphs[0][3][0].replay()
            collector.note_replay()
            res = graphs[2]
            last_logits[0] = graphs[3][1]
        elif replay:
            graphs[0][1][0].replay()
            res = graphs[2]
            last_logits[0] = graphs[3][0]
        elif use_graphs:
            res = verify_phase(draft_dev, bool(dense_pending))
        elif verify_mode == "sequential":
            res = _sequential_verify(model, draft_dev, dense_next, dense_pkv)
        else:
            if dense_pending:
                pend = torch.tensor(dense_pending, dtype=torch.long).to(dev, non_blocking=True)
                verify_ids = torch.cat([pend, draft_dev]).reshape(1, -1)
            else:
                verify_ids = draft_dev.reshape(1, -1)
            logits = model(verify_ids, dense_pkv, all_logits=True)
            last_logits[0] = logits[0]
            res = ops.greedy_accept(logits[0], draft_dev.to(torch.int32), has_pending=bool(dense_pending),
                                    dense_next=None if dense_pending else dense_next_i32)
        if trace is not None:
            trace.end_verification()
        host = torch.cat([res[:2], status, draft_dev.to(torch.int32)]).tolist()     # the round's one readback
        accept_len, bonus_token, draft = host[0], host[1], host[3:]
        _check_decode_status(host[2])
        if verify_mode == "parallel":
            low_margin = False
            if verify_margin_threshold is not None:
                margin = min_prediction_margin(last_logits[0].unsqueeze(0), range(accept_len + 1),
                                               has_dense_pending=bool(dense_pending))
                if margin is not None:
                    verify_margins.append(margin)
                low_margin = margin is not None and margin < verify_margin_threshold
                if low_margin and verify_fallback != "sequential_on_low_margin":
                    # the reference re-verifies with the math SDPA backend
                    # (std_qwen25vl.py:824-840); the HIP verify computes the
                    # math definition, so that re-run predicts these tokens
                    verify_margin_reruns += 1
            fallback_count += math_reverify_count(verify_attn_backend, accept_len, propose_len)
            if needs_sequential_fallback(verify_fallback, accept_len=accept_len, draft_len=len(draft),
                                         sequential_fallback_max_accept=sequential_fallback_max_accept,
                                         low_margin=low_margin):
                fallback_count += 1
                if low_margin and verify_fallback == "sequential_on_low_margin":
                    verify_margin_reruns += 1
                seq_accept, seq_bonus = _sequential_verify_draft(model, draft_dev, dense_pending, dense_next,
                                                                 dense_pkv, dense_lengths, dense_cached_len)
                fallback_accepted_extra += max(0, seq_accept - accept_len)
                accept_len, bonus_token = seq_accept, seq_bonus
        verify_time += _profile_mark(profile_decode) - stage
        accept_lengths.append(accept_len)
        accepted_total += accept_len
        if adaptive_gamma_min is not None:
            if accept_len < propose_len:
                if adaptive_gamma_mode == "accept_len":
                    current_gamma = max(adaptive_gamma_min, accept_len if accept_len > 0 else adaptive_gamma_min)
                else:
                    ratio = accept_len / propose_len if propose_len else 0.0
                    if accept_len == 0:
                        current_gamma = max(adaptive_gamma_min, current_gamma - 2)
                    elif ratio < 0.5:
                        current_gamma = max(adaptive_gamma_min, current_gamma - 1)
            elif current_gamma < gamma:
                current_gamma = min(gamma, current_gamma + 1)

        full_append = draft[:accept_len] + [bonus_token]
        eos_index = None if ignore_eos else _contains_eos(full_append, eos_token_id)
        if eos_index is not None:
            full_append = full_append[:eos_index + 1]
        to_append = full_append[:remaining]
        generated.extend(int(x) for x in to_append)
        if len(generated) >= max_new_tokens or (not ignore_eos and to_append and to_append[-1] == eos_token_id):
            break

        stage = _profile_mark(profile_decode)
        # Keep the previous pending token and the accepted draft prefix; the
        # new bonus stays pending until the next verification caches it.
        fill_cache_length(dense_lengths, dense_cached_len + len(dense_pending) + accept_len)
        fill_cache_length(sparse_lengths, sparse_prev_len + accept_len)
        cache_adjust_time += _profile_mark(profile_decode) - stage
        if round_hook is not None:
            lengths = ((int(st4[0]), int(st4[2])) if use_graphs
                       else (int(dense_lengths[0]), int(sparse_lengths[0])))
            round_hook(dict(round=decode_rounds, logits=last_logits[0], draft=draft, has_pending=bool(dense_pending),
                            dense_next=int(dense_next.reshape(-1)[0]), accept_len=accept_len, bonus=bonus_token,
                            dense_cached_len=dense_cached_len, n_pending=len(dense_pending),
                            sparse_prev_len=sparse_prev_len, lengths=lengths, replayed=replay))

        dense_pending = [bonus_token]
        stage = _profile_mark(profile_decode)
        if replay:
            graphs[0][2][0].replay()
        elif use_graphs:
            bonus_phase(res)
        else:
            bonus_dev = torch.tensor([bonus_token], dtype=torch.long).to(dev, non_blocking=True)
            sparse_next = _append_sparse_tokens(model, bonus_dev, sparse_pkv, controller,
                                                start_position=context_len + accept_len)
        if use_graphs:
            fill_cache_length(sparse_lengths, sparse_prev_len + accept_len + 1)
        bonus_time += _profile_mark(profile_decode) - stage

    torch.cuda.synchronize()
    end = time.time()
    out = torch.cat([prompt_ids, torch.tensor([generated], dtype=torch.long, device=dev)], dim=1)
    result = GenerateResult(
        output_ids=out, decoding_time=end - decode_start, inference_time=end - start, generate_len=len(generated),
        accepted_draft_tokens=accepted_total, proposed_draft_tokens=proposed_total,
        mean_accept_length=sum(accept_lengths) / len(accept_lengths) if accept_lengths else 0.0,
        decode_rounds=decode_rounds, final_gamma=current_gamma, gamma_history=gamma_history,
        proposed_lengths=proposed_lengths, accept_lengths=accept_lengths, pending_lengths=pending_lengths,
        draft_time=draft_time, verify_time=verify_time, bonus_time=bonus_time, cache_adjust_time=cache_adjust_time,
        cache_init_time=cache_init_time, prefill_time=selection_prefill_time,
        selection_prefill_time=selection_prefill_time, selection_time=selection_time, dense_prefill_time=0.0,
        sparse_cache_time=sparse_cache_time, fallback_count=fallback_count,
        fallback_accepted_extra=fallback_accepted_extra, verify_margin_reruns=verify_margin_reruns,
        min_verify_margin=min(verify_margins) if verify_margins else 0.0)
    return result, selection


def first_divergence(a: torch.Tensor, b: torch.Tensor) -> Optional[int]:
    """Index of the first differing generated token, or None (the diagnostic of
    benchmark_std.py:327-356)."""
    a, b = a.reshape(-1).tolist(), b.reshape(-1).tolist()
    for i, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return i
    return None if len(a) == len(b) else min(len(a), len(b))


def generated_suffix(output_ids: torch.Tensor, prompt_len: int) -> torch.Tensor:
    """The generated tokens of ``output_ids`` [1, prompt + generated]
    (std_qwen25vl.py:981-982)."""
    return output_ids[:, prompt_len:]


def tokens_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Same shape and the same tokens (std_qwen25vl.py:985-986)."""
    return a.shape == b.shape and bool(torch.equal(a.detach().cpu(), b.detach().cpu()))


def copy_prompt_cache(source_past_key_values, target_past_key_values, target_length_data: torch.Tensor,
                      prompt_len: int) -> None:
    """Copy the first ``prompt_len`` rows of every layer's K and V from one
    cache set into another and set the target lengths to ``prompt_len``
    (std_qwen25vl.py:301-320). The generate loop does not need it (compaction
    gathers the selected rows straight from the dense cache); it is kept for
    callers that build a second cache from a prefilled one."""
    for source_layer, target_layer in zip(source_past_key_values, target_past_key_values):
        for src, dst in zip(source_layer, target_layer):
            if src.length < prompt_len:
                raise RuntimeError(f"Cannot copy prompt cache: source length {src.length} is shorter than "
                                   f"prompt length {prompt_len}.")
            dst.data.narrow(2, 0, prompt_len).copy_(src.data.narrow(2, 0, prompt_len))
            dst.current_length.fill_(prompt_len)
    target_length_data.fill_(prompt_len)
