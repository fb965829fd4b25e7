"""Pure-Python loop versions for tiny inputs (oracle; test infrastructure only).

They share no code with the numpy restatements, so agreement between the two
pins an indexing or masking mistake in either.
"""
from __future__ import annotations

import math
from typing import List


def attention_loops(q, k, v, causal_offset=None) -> List:
    """q [n_q][Q][D], k/v [n_kv][S][D] nested lists; row i of a query sees
    keys j <= causal_offset + i (all keys when causal_offset is None)."""
    n_q, q_len, d = len(q), len(q[0]), len(q[0][0])
    n_kv, s_len = len(k), len(k[0])
    group = n_q // n_kv
    scale = 1.0 / math.sqrt(d)
    out = []
    for h in range(n_q):
        g = h // group
        rows = []
        for i in range(q_len):
            lim = s_len - 1 if causal_offset is None else causal_offset + i
            logits = [sum(q[h][i][e] * k[g][j][e] for e in range(d)) * scale for j in range(lim + 1)]
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            tot = sum(w)
            rows.append([sum(w[j] * v[g][j][e] for j in range(lim + 1)) / tot for e in range(d)])
        out.append(rows)
    return out


def selection_scores_loops(q_text, k, text_start) -> List[List[float]]:
    """q_text [n_q][T][D], k [n_kv][P][D]; causal text rows; returns [n_kv][P]."""
    n_q, t_len, d = len(q_text), len(q_text[0]), len(q_text[0][0])
    n_kv = len(k)
    group = n_q // n_kv
    p_len = text_start + t_len
    scale = 1.0 / math.sqrt(d)
    scores = [[0.0] * p_len for _ in range(n_kv)]
    for h in range(n_q):
        g = h // group
        for i in range(t_len):
            lim = text_start + i
            logits = [sum(q_text[h][i][e] * k[g][j][e] for e in range(d)) * scale for j in range(lim + 1)]
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            tot = sum(w)
            for j in range(lim + 1):
                scores[g][j] += w[j] / tot
    return scores


def verification_scores_loops(q, k, visual_positions) -> List[List[float]]:
    """q [n_q][Q][D], k [n_kv][S][D] nested lists; per KV head, the group's
    mean query per position, softmax over the visual keys, summed over the
    positions: returns [n_kv][len(visual_positions)]."""
    n_q, q_len, d = len(q), len(q[0]), len(q[0][0])
    n_kv = len(k)
    group = n_q // n_kv
    scale = 1.0 / math.sqrt(d)
    out = []
    for g in range(n_kv):
        col = [0.0] * len(visual_positions)
        for i in range(q_len):
            qbar = [sum(q[g * group + h][i][e] for h in range(group)) / group for e in range(d)]
            logits = [sum(qbar[e] * k[g][j][e] for e in range(d)) * scale for j in visual_positions]
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            tot = sum(w)
            for c in range(len(w)):
                col[c] += w[c] / tot
        out.append(col)
    return out
