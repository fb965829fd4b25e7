"""The reference's own torch operators for the hot path, run on the CPU in
fp32 (oracle package: test infrastructure and the timed CPU baseline only).

Each function restates the torch call the reference makes on the GPU:
  gqa_sdpa          draft decode, F.scaled_dot_product_attention(q, k, v,
                    enable_gqa=True) (src/std_repro/std_qwen25vl.py:406-417)
  verify_attention  dense verify, math SDPA with the offset-causal additive
                    mask (src/specvlm/models/modeling_qwen2_5_vl.py:1124-1132,
                    mask :65-126 and :1388-1399, verify_attn_backend="math")
  greedy_accept     argmax over the verify logits, the longest matching
                    prefix and the bonus token (std_qwen25vl.py:806-815)
  select_topk       the selection prefill's text-row attention probabilities
                    (causal softmax, modeling_qwen2_5_vl.py:966-995), summed
                    over each KV head's query heads and the text rows, top-k
                    over the visual positions, sorted (std_qwen25vl.py:200-222)
They are pinned against the fp64 numpy restatements in tests/.
"""
from __future__ import annotations

import math
from typing import List, Tuple

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel


def gqa_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """q [1, n_q, 1, D], k/v [1, n_kv, S, D] (fp32, CPU)."""
    return F.scaled_dot_product_attention(q, k, v, is_causal=False, enable_gqa=True)


def offset_causal_mask(q_len: int, kv_len: int) -> torch.Tensor:
    """Additive [q_len, kv_len] mask: row i sees keys [0, kv_len - q_len + i]."""
    rows = torch.arange(q_len).view(-1, 1) + (kv_len - q_len)
    cols = torch.arange(kv_len).view(1, -1)
    return torch.where(cols <= rows, 0.0, float("-inf"))


def verify_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """q [1, n_q, Q, D], k/v [1, n_kv, kv_len, D] (fp32, CPU), math backend."""
    mask = offset_causal_mask(q.shape[2], k.shape[2]).to(q.dtype)
    with sdpa_kernel(SDPBackend.MATH):
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)


def greedy_accept(logits: torch.Tensor, draft: List[int], has_pending: bool,
                  dense_next: int = -1) -> Tuple[int, int]:
    """logits [Q, vocab]; returns (accepted length, bonus token)."""
    pred = torch.argmax(logits, dim=-1).tolist()
    if not has_pending:
        pred = [int(dense_next)] + pred
    a = 0
    while a < len(draft) and draft[a] == pred[a]:
        a += 1
    return a, pred[a]


def select_topk(q_text: torch.Tensor, key: torch.Tensor, text_start: int, k: int) -> torch.Tensor:
    """q_text [1, n_q, T, D] (the prompt's last T rows), key [1, n_kv, P, D]
    with P = text_start + T, fp32 on the CPU; visual positions [0, text_start).
    Returns int64 [n_kv, k], ascending."""
    _, n_q, t_len, d = q_text.shape
    n_kv, p_len = key.shape[1], key.shape[2]
    group = n_q // n_kv
    rows = torch.arange(t_len).view(-1, 1) + text_start
    mask = torch.where(torch.arange(p_len).view(1, -1) <= rows, 0.0, float("-inf"))
    out = []
    for g in range(n_kv):
        s = q_text[0, g * group:(g + 1) * group] @ key[0, g].transpose(0, 1) / math.sqrt(d)   # [group, T, P]
        p = torch.softmax(s + mask, dim=-1)
        col = p.sum(dim=(0, 1))[:text_start]
        top = torch.topk(col, k).indices
        out.append(torch.sort(top).values)
    return torch.stack(out)

