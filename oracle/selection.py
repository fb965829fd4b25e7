"""Sparse-KV selection and compaction restatements (oracle; test infrastructure only).

The reference selects, per layer and KV head, the k visual positions with the
largest sum of selection-prefill attention probabilities over the group's
query heads and the text rows (src/std_repro/std_qwen25vl.py:175-231). The
probabilities come from the text-suffix forward, whose rows are causally
masked: text row i (absolute position text_start + i) attends to keys
[0, text_start + i] (modeling_qwen2_5_vl.py:65-101, :1394-1399, consumed at
:1115-1123 through the custom attention of :966-995).

This oracle evaluates that definition exactly (fp64 logits from exact input
values, fp64 softmax and sums) instead of the reference's fp16 rounding of
the probabilities; torch.topk's unspecified tie order (std_qwen25vl.py:220)
is replaced by the rule "ties go to the lowest position".
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence

import numpy as np

from .attention import _np


def selection_k(prompt_len: int, text_start: int, n_visual: int, target_k_plus_text: int = 1024,
                explicit_k: Optional[int] = None) -> int:
    """k rule of std_qwen25vl.py:192-195: text_len = max(1, P - text_start),
    k = explicit_k or max(1, target - text_len), clamped to the visual count."""
    text_len = max(1, prompt_len - int(text_start))
    k = int(explicit_k) if explicit_k is not None else max(1, int(target_k_plus_text) - text_len)
    return min(k, int(n_visual))


def last_video_index(input_ids: Sequence[int], video_token_id: int) -> int:
    """Last position of video_token_id, or -1 (src/specvlm/utils/utils.py:8-15)."""
    for i in range(len(input_ids) - 1, -1, -1):
        if int(input_ids[i]) == video_token_id:
            return i
    return -1


def _bit_rows(x) -> np.ndarray:
    """Integer view of the raw input values (bf16/fp32 torch or numpy)."""
    if hasattr(x, "detach"):
        import torch

        x = x.detach().cpu().contiguous()
        return x.view(torch.int16 if x.element_size() == 2 else torch.int32).numpy()
    return np.ascontiguousarray(x)


def _duplicate_groups(k_rows: np.ndarray):
    """Columns whose key row has a bit-identical twin, and for each the index
    of the first occurrence (which maps to itself)."""
    rows = np.ascontiguousarray(k_rows)
    view = rows.view(np.dtype((np.void, rows.dtype.itemsize * rows.shape[1]))).ravel()
    _, first, inverse, counts = np.unique(view, return_index=True, return_inverse=True, return_counts=True)
    dup_cols = np.nonzero(counts[inverse] > 1)[0]
    return dup_cols, first[inverse[dup_cols]]


def selection_scores(q_text, key, text_start: int, scale: Optional[float] = None,
                     chunk: int = 8192) -> np.ndarray:
    """Column scores [n_kv, P] (P = text_start + T) in fp64.

    score[g][j] = sum_{h in group g} sum_{i: j <= text_start + i} softmax_i(q[h][i] . k[g] * scale)[j]
    Bit-identical key columns receive bit-identical scores (their logits are
    taken from one shared evaluation), so exact ties stay exact.
    q_text [1, n_q, T, D]; key [1, n_kv, >= P, D] (input dtype values).
    """
    q = _np(q_text)
    _, n_q, text_len, d = q.shape
    n_kv = key.shape[1]
    group = n_q // n_kv
    prompt_len = int(text_start) + text_len
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    limits = np.tile(int(text_start) + np.arange(text_len), group)      # row r = hl*T + i
    scores = np.zeros((n_kv, prompt_len))
    for g in range(n_kv):
        kg_raw = key[0, g, :prompt_len]
        kg = _np(kg_raw)
        dup_cols, dup_src = _duplicate_groups(_bit_rows(kg_raw))
        qg = q[0, g * group:(g + 1) * group].reshape(group * text_len, d)
        rep_cols, rep_idx = np.unique(dup_src, return_inverse=True)
        rep_logits = (qg @ kg[rep_cols].T) * scale

        def logits(c0: int, c1: int) -> np.ndarray:
            s = (qg @ kg[c0:c1].T) * scale
            sel = (dup_cols >= c0) & (dup_cols < c1)
            s[:, dup_cols[sel] - c0] = rep_logits[:, rep_idx[sel]]
            cols = np.arange(c0, c1)
            return np.where(cols[None, :] > limits[:, None], -np.inf, s)

        m = np.full(group * text_len, -np.inf)
        l = np.zeros(group * text_len)
        for c0 in range(0, prompt_len, chunk):
            s = logits(c0, min(prompt_len, c0 + chunk))
            m_new = np.maximum(m, s.max(axis=1))
            l = l * np.exp(m - m_new) + np.exp(s - m_new[:, None]).sum(axis=1)
            m = m_new
        lse = m + np.log(l)
        for c0 in range(0, prompt_len, chunk):
            c1 = min(prompt_len, c0 + chunk)
            p = np.exp(logits(c0, c1) - lse[:, None])
            scores[g, c0:c1] = p.sum(axis=0)
    return scores


def scores_from_probs(probs, n_kv: int) -> np.ndarray:
    """The reference's selection scores from materialised probabilities
    (std_qwen25vl.py:203-215): one layer's [1, n_q, T, P] attention of the
    text rows, summed over the query heads of each KV head and over the text
    rows (fp64 here; exact for fp16 inputs) -> [n_kv, P]."""
    a = probs
    if hasattr(a, "detach"):
        a = a.detach().cpu()
        if str(a.dtype) in ("torch.bfloat16", "torch.float16"):
            a = a.float()
        a = a.numpy()
    a = np.asarray(a)[0]
    n_q, t_len, p_len = a.shape
    out = np.zeros((n_kv, p_len))
    group = n_q // n_kv
    for g in range(n_kv):
        for h in range(g * group, (g + 1) * group):
            out[g] += a[h].astype(np.float64).sum(axis=0)
    return out


def topk_positions(scores: np.ndarray, visual_positions: Sequence[int], k: int) -> np.ndarray:
    """Per KV head, the k visual positions with the largest score, ties to the
    lowest position, returned sorted ascending (std_qwen25vl.py:219-222 with a
    defined tie order). scores [n_kv, P] -> int64 [n_kv, k]."""
    vis = np.asarray(visual_positions, dtype=np.int64)
    out = np.empty((scores.shape[0], k), dtype=np.int64)
    for g in range(scores.shape[0]):
        sv = scores[g, vis]
        order = np.lexsort((vis, -sv))   # primary: score descending, then position ascending
        out[g] = np.sort(vis[order[:k]])
    return out


def build_sparse_selection(q_text_layers, key_layers, input_ids: Sequence[int], video_token_id: int,
                           target_k_plus_text: int = 1024, explicit_k: Optional[int] = None) -> Dict:
    """Whole-prompt selection record, the SparseSelection of
    std_qwen25vl.py:41-50 / :175-231, from per-layer query and key states."""
    ids = np.asarray(input_ids)
    visual = np.nonzero(ids == video_token_id)[0]
    if visual.size == 0:
        raise ValueError("Cannot build sparse selection without visual/video token positions.")
    non_visual = np.nonzero(ids != video_token_id)[0]
    text_start = last_video_index(ids, video_token_id) + 1
    prompt_len = ids.size
    k = selection_k(prompt_len, text_start, visual.size, target_k_plus_text, explicit_k)
    topk: List[np.ndarray] = []
    for q_text, key in zip(q_text_layers, key_layers):
        topk.append(topk_positions(selection_scores(q_text, key, text_start), visual, k))
    return dict(topk_positions=topk, non_visual_positions=non_visual, prompt_len=prompt_len,
                visual_len=int(visual.size), text_len=max(1, prompt_len - text_start), k=k)


def compact_index(non_visual: Sequence[int], topk_head: Sequence[int]) -> np.ndarray:
    """unique(sorted(non_visual ++ topk[h])) (std_qwen25vl.py:286-291)."""
    idx = np.unique(np.concatenate([np.asarray(non_visual, np.int64), np.asarray(topk_head, np.int64)]))
    return idx


def compact_kv(dense, index: np.ndarray):
    """sparse[:, g, s] = dense[:, g, index[g][s]] (std_qwen25vl.py:292-295).
    dense [1, n_kv, >=P, D] (numpy or torch, values copied bit-exactly)."""
    index = np.asarray(index)
    if hasattr(dense, "detach"):
        import torch

        d = dense.detach().cpu()
        return torch.stack([d[0, g, torch.as_tensor(index[g], dtype=torch.long)] for g in range(d.shape[1])])[None]
    return np.stack([dense[0, g, index[g]] for g in range(dense.shape[1])])[None]
