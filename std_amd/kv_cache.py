"""KV cache slots with the reference's interface (specvlm/kv_cache/kv_cache.py).

One tensor ``[2L, 1, Hkv, max_len, D]`` holds every layer's K and V; each
``KVCache`` is a strided ``[1, Hkv, max_len, D]`` view of it plus a length.
As in the reference (kv_cache.py:131-138) the lengths live in a CPU int64
tensor ``[2L]`` so that the host always knows every length without a device
sync; the HIP attention entry points receive them by value and write the new
rows themselves (the fused append of ``gqa_decode_append`` /
``verify_attention_append``), so ``cat`` is only used on the prefill path.
"""
from __future__ import annotations

import os
from typing import List, Tuple

import torch


class KVCache:
    """A growing K or V cache (kv_cache.py:6-69).

    ``data``: ``[1, Hkv, max_len, D]`` view; ``current_length``: a 0-d CPU
    int64 tensor (an element of the shared length vector)."""

    def __init__(self, data: torch.Tensor, current_length: torch.Tensor):
        self.data = data
        self.current_length = current_length

    @property
    def length(self) -> int:
        return int(self.current_length)

    @property
    def capacity(self) -> int:
        return int(self.data.shape[2])

    @property
    def shape(self):
        """(batch, heads, current length, head_dim) (kv_cache.py:32-40)."""
        return (self.data.shape[0], self.data.shape[1], self.length, self.data.shape[3])

    def view(self) -> torch.Tensor:
        """The valid prefix ``data[:, :, :current_length]``."""
        return self.data.narrow(2, 0, self.length)

    def copy(self, indices: torch.Tensor, prev_length: int, dim: int = 2) -> None:
        """Move rows ``indices`` to ``[prev_length, ...)`` (kv_cache.py:42-52)."""
        tgt = self.data.index_select(dim, indices)
        dst = self.data.narrow(dim, prev_length, tgt.shape[dim])
        dst.copy_(tgt, non_blocking=True)
        self.current_length.fill_(prev_length + tgt.shape[dim])

    def cat(self, tensor: torch.Tensor, dim: int = 2) -> torch.Tensor:
        """Append ``tensor`` at the current length and return the valid prefix
        (kv_cache.py:54-69). Raises instead of writing past the capacity."""
        start, n = self.length, tensor.shape[dim]
        if start + n > self.capacity:
            raise RuntimeError(f"KV cache overflow: {start} + {n} > capacity {self.capacity}")
        self.data.narrow(dim, start, n).copy_(tensor)
        self.current_length.add_(n)
        return self.data.narrow(2, 0, start + n)

    def advance(self, n: int) -> None:
        """Account for ``n`` rows written in place by a fused HIP append."""
        if self.length + n > self.capacity:
            raise RuntimeError(f"KV cache overflow: {self.length} + {n} > capacity {self.capacity}")
        self.current_length.add_(n)


def default_max_cache_len(max_position_embeddings: int) -> int:
    """``SPECVLM_MAX_CACHE_LEN`` or ``min(2 * max_position_embeddings, 16384)``
    (kv_cache.py:105-106)."""
    return int(os.environ.get("SPECVLM_MAX_CACHE_LEN", min(max_position_embeddings * 2, 16384)))


def initialize_past_key_values(
    model, device: torch.device = None, dtype: torch.dtype = None, max_cache_len: int = None
) -> Tuple[List[List[KVCache]], torch.Tensor, torch.Tensor]:
    """Allocate one cache (kv_cache.py:72-165) on a single device.

    ``model`` is the model, as the reference passes it
    (``initialize_past_key_values(model)``), whose config, device and dtype
    are used, or a model config with ``device`` and ``dtype`` given. Returns
    ``(past_key_values, data [2L, 1, Hkv, max_len, D], current_length_data [2L])``;
    ``past_key_values[l] = [K cache, V cache]``. Rows are zero-initialised as
    in the reference."""
    config = model
    if hasattr(model, "config"):                      # the reference's form: a model
        config = model.config
        device = model.device if device is None else device
        dtype = model.dtype if dtype is None else dtype
    if device is None or dtype is None:
        raise ValueError("initialize_past_key_values needs a model, or a config with a device and a dtype")
    if max_cache_len is None:
        max_cache_len = default_max_cache_len(config.max_position_embeddings)
    n_layers = config.num_hidden_layers
    head_dim = config.hidden_size // config.num_attention_heads
    data = torch.zeros(2 * n_layers, 1, config.num_key_value_heads, max_cache_len, head_dim,
                       device=device, dtype=dtype)
    current_length_data = torch.zeros(2 * n_layers, dtype=torch.long, device="cpu")
    past_key_values = [[KVCache(data[2 * i + j], current_length_data[2 * i + j]) for j in range(2)]
                       for i in range(n_layers)]
    return past_key_values, data, current_length_data


def fill_cache_length(current_length_data: torch.Tensor, length: int) -> None:
    """Roll every layer's length back or forward (std_qwen25vl.py:103-104)."""
    current_length_data.fill_(int(length))
