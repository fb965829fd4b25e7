"""Visual-attention collector restatement in fp64 numpy (oracle; test
infrastructure only).

Follows VerificationCollectorV3._hook (src/std_repro/dynamic_selection.py:
504-519), which the verify forward calls with its rotated queries and the key
cache including the new rows (src/specvlm/models/modeling_qwen2_5_vl.py:
1063-1067): per KV head, the mean of the group's query rows at each position,
a softmax (scale head_dim ** -0.5) over the visual keys only, summed over the
positions.
"""
from __future__ import annotations

import numpy as np

from .attention import _np


def verification_scores(query, key, visual_positions) -> np.ndarray:
    """query [1, n_q, q_len, D], key [1, n_kv, kv_len, D], visual_positions
    (absolute key positions) -> scores [n_kv, n_visual] (fp64)."""
    q = _np(query)[0]
    k = _np(key)[0]
    pos = np.asarray(visual_positions, dtype=np.int64)
    n_q, q_len, d = q.shape
    n_kv = k.shape[0]
    group = n_q // n_kv
    qbar = q.reshape(n_kv, group, q_len, d).mean(axis=1)                  # [n_kv, q_len, D]
    kv = k[:, pos, :]                                                    # [n_kv, V, D]
    logits = np.einsum("gid,gjd->gij", qbar, kv) * d ** -0.5             # [n_kv, q_len, V]
    logits -= logits.max(axis=-1, keepdims=True)
    w = np.exp(logits)
    w /= w.sum(axis=-1, keepdims=True)
    return w.sum(axis=1)
