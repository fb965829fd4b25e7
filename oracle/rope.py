"""Rotary position embedding restated in numpy (oracle; test infrastructure only).

Follows Qwen2_5_VLRotaryEmbedding.forward and apply_multimodal_rotary_pos_emb
(src/specvlm/models/modeling_qwen2_5_vl.py:656-671, 690-732) for text
positions, where the three position rows are identical and the multimodal
sections therefore select one and the same 1-D table:
    inv_freq[j] = 1 / theta^(2j / D)                       (fp32 table)
    angle[p, j] = float32(p) * inv_freq[j]                 (fp32 product)
    cos, sin    = cos/sin of cat(angle, angle), rounded to the model dtype
    x_embed     = (x * cos) + (rotate_half(x) * sin)       (each op rounded to the dtype)
with rotate_half(x) = cat(-x[D/2:], x[:D/2]).

The model dtype is "bf16" (round to nearest even on the float32 value, as
torch's bfloat16 arithmetic does), "fp16" (the same to IEEE half, the dtype the
reference loads its model in, scripts/benchmark_std.py:66) or "fp32".
"""
from __future__ import annotations

import numpy as np


def inv_freq(theta: float, d: int) -> np.ndarray:
    """The fp32 inverse-frequency table (computed in fp64, rounded once)."""
    return (1.0 / (theta ** (np.arange(0, d, 2, dtype=np.float64) / d))).astype(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


def _round(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)     # IEEE half, ties to even
    return x


def cos_sin(positions: np.ndarray, inv: np.ndarray, dtype: str):
    """[n, D] cos and sin tables for integer positions, rounded to the dtype.
    cos/sin are evaluated in fp64 on the fp32 angle and rounded to fp32."""
    ang = np.asarray(positions, dtype=np.float32)[:, None] * inv[None, :]      # fp32 product
    emb = np.concatenate([ang, ang], axis=-1).astype(np.float64)
    return _round(np.cos(emb).astype(np.float32), dtype), _round(np.sin(emb).astype(np.float32), dtype)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """x [..., n, D] (values already representable in the dtype), cos/sin [n, D]."""
    x = np.asarray(x, dtype=np.float32)
    h = x.shape[-1] // 2
    rot = np.concatenate([-x[..., h:], x[..., :h]], axis=-1)
    return _round(_round(x * cos, dtype) + _round(rot * sin, dtype), dtype)
