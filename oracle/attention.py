"""Attention restatements in fp64 numpy (oracle; test infrastructure only).

Shapes follow the reference: query [1, n_q, q_len, D], key/value
[1, n_kv, kv_len, D]; query head h reads KV head h // (n_q // n_kv), the
repeat_kv order of src/specvlm/models/modeling_qwen2_5_vl.py:735-744.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np


def _np(x, dtype=np.float64) -> np.ndarray:
    if hasattr(x, "detach"):  # torch tensor (bf16 is upcast exactly via float32)
        x = x.detach().cpu()
        if str(x.dtype) == "torch.bfloat16":
            x = x.float()
        x = x.numpy()
    return np.asarray(x, dtype=dtype)


def offset_causal_mask(q_len: int, kv_len: int) -> Optional[np.ndarray]:
    """Additive mask for q_len appended queries: row i reads keys
    [0, kv_len - q_len + i]; None for q_len == 1.
    Follows src/std_repro/sparse_verify_spike.py:24-42."""
    if q_len < 1 or kv_len < q_len:
        raise ValueError(f"expected 1 <= q_len <= kv_len, got q_len={q_len}, kv_len={kv_len}")
    if q_len == 1:
        return None
    past = kv_len - q_len
    keys = np.arange(kv_len)[None, :]
    limits = past + np.arange(q_len)[:, None]
    mask = np.zeros((1, 1, q_len, kv_len))
    mask[0, 0][keys > limits] = -np.inf
    return mask


def _attend(q, k, v, scale, limits, dtype):
    """Core: per KV head group, softmax(q k^T * scale) over keys j <= limits[row]."""
    q = _np(q, dtype)
    k = _np(k, dtype)
    v = _np(v, dtype)
    _, n_q, q_len, d = q.shape
    n_kv, kv_len = k.shape[1], k.shape[2]
    if n_q % n_kv:
        raise ValueError("n_q must be a multiple of n_kv")
    group = n_q // n_kv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = np.empty((1, n_q, q_len, d), dtype=dtype)
    cols = np.arange(kv_len)
    for g in range(n_kv):
        qg = q[0, g * group:(g + 1) * group].reshape(group * q_len, d)
        s = (qg @ k[0, g].T) * dtype(scale)
        if limits is not None:
            lim = np.tile(limits, group)
            s = np.where(cols[None, :] > lim[:, None], -np.inf, s)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[0, g * group:(g + 1) * group] = (p @ v[0, g]).reshape(group, q_len, d)
    return out


def gqa_sdpa(query, key, value, scale: Optional[float] = None, dtype=np.float64) -> np.ndarray:
    """softmax(q k^T / sqrt(D)) v with GQA head sharing and no mask: the draft
    `gqa_sdpa` mode, F.scaled_dot_product_attention(..., is_causal=False,
    enable_gqa=True) at src/std_repro/std_qwen25vl.py:406-417 (and the
    triton_gqa kernel's contract, src/std_repro/triton_attention.py:83-112)."""
    return _attend(query, key, value, scale, None, dtype)


def verify_attention(query, key, value, scale: Optional[float] = None, dtype=np.float64) -> np.ndarray:
    """Dense verify: math SDPA with the offset-causal mask, i.e. row i sees
    keys [0, kv_len - q_len + i]. Restates the verify forward's attention
    (modeling_qwen2_5_vl.py:1096-1132 with the causal mask of :65-126 and
    :1388-1399) in the form of sparse_verify_spike.py:45-67."""
    q_len = _np(query).shape[2]
    kv_len = _np(key).shape[2]
    if q_len > kv_len:
        raise ValueError("key/value sequence cannot be shorter than query sequence")
    limits = (kv_len - q_len) + np.arange(q_len)
    return _attend(query, key, value, scale, limits, dtype)
