"""Tensor-level wrappers of the HIP hot path (torch on ROCm is only the
allocator and stream provider here; all compute runs in libstdhip.so).

Every function validates dtype, device, shape and strides on the host, then
calls the C ABI on the tensors' device and current stream. Nonzero statuses
raise ``StdHipError`` (a RuntimeError), as the reference raises
RuntimeError/ValueError on unsupported calls (std_qwen25vl.py:379-402).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib

HEAD_DIM = 128
STATUS_CACHE_OVERFLOW = _lib.STD_STATUS_CACHE_OVERFLOW   # device status word bit (see _status_ptr)


def _dtype_code(t: torch.Tensor) -> int:
    """fp32, bf16 or fp16 (the reference loads its model in fp16); ops whose
    kernels lack a dtype report STD_E_DTYPE from the library."""
    if t.dtype == torch.float32:
        return _lib.STD_F32
    if t.dtype == torch.bfloat16:
        return _lib.STD_BF16
    if t.dtype == torch.float16:
        return _lib.STD_F16
    raise TypeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16")


def _check_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError("the HIP hot path needs tensors on a ROCm device (got %s)" % dev)
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _workspace(nbytes: int, dev: torch.device) -> Tuple[int, torch.Tensor]:
    """Per-call scratch (selection, acceptance): no initial contents needed."""
    if nbytes == 0:
        return 0, None
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    return buf.data_ptr(), buf


_ATTN_WS = {}
_ATTN_WS_RETIRED = []


def _attn_workspace(nbytes: int, dev: torch.device) -> int:
    """Persistent attention workspace per (device, stream): calls on one stream
    are ordered and may share it (no per-call allocation on the decode path);
    another stream gets its own. A workspace outgrown by a larger call is kept
    alive (never freed), since a captured HIP graph may still address it."""
    if nbytes == 0:
        return 0
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    buf = _ATTN_WS.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _ATTN_WS_RETIRED.append(buf)
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _ATTN_WS[key] = buf
    return buf.data_ptr()


def same_layout(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Same shape and the same stride in every dimension of size > 1 (the
    stride of a size-1 dimension is never used to address an element)."""
    return a.shape == b.shape and all(a.stride(i) == b.stride(i) for i in range(a.dim()) if a.shape[i] > 1)


def _check_cache_view(name: str, t: torch.Tensor) -> None:
    """[1, Hkv, S, D] with contiguous rows; any head stride (cache view)."""
    if t.dim() != 4 or t.shape[0] != 1:
        raise ValueError(f"{name} must be [1, n_kv, seq, head_dim], got {tuple(t.shape)}")
    if t.shape[3] != HEAD_DIM:
        raise ValueError(f"{name}: head_dim {t.shape[3]} unsupported (only {HEAD_DIM})")
    if t.stride(3) != 1 or t.stride(2) != HEAD_DIM:
        raise ValueError(f"{name}: rows must be contiguous (strides {t.stride()})")


def _check_rows_contiguous(name: str, t: torch.Tensor) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def gqa_decode(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
               scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Single-query GQA attention, the draft / AR decode step.

    query [1, n_q, 1, D]; key, value [1, n_kv, S, D] (cache views, read in
    place through their head stride). Returns [1, n_q, 1, D] in query dtype.
    Same contract as fused_gqa_attention (triton_attention.py:83-112) and
    F.scaled_dot_product_attention(q, k, v, enable_gqa=True) with q_len = 1
    (std_qwen25vl.py:409-417).
    """
    if query.dim() != 4 or query.shape[0] != 1 or query.shape[2] != 1:
        raise ValueError(f"Expected q_len=1 query [1, n_q, 1, D], got {tuple(query.shape)}")
    return _attention("std_gqa_decode", query, key, value, scale, out)


def gqa_decode_batched(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                       scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """n_batch independent single-query GQA decodes in one launch.

    query [B, 1, n_q, 1, D] (or [B, n_q, 1, D]); key, value [B, 1, n_kv, S, D]
    with any batch and head strides (e.g. one draft step's 28 layer caches).
    Each problem b equals gqa_decode(query[b], key[b], value[b]) to fp32
    rounding, bit for bit when both get the same split count (always for a
    batch of one; many problems may each stream unsplit)."""
    squeeze = query.dim() == 4
    if squeeze:
        query = query.unsqueeze(1)
    if query.dim() != 5 or query.shape[1] != 1 or query.shape[3] != 1:
        raise ValueError(f"Expected query [B, 1, n_q, 1, D], got {tuple(query.shape)}")
    if key.dim() != 5 or key.shape[0] != query.shape[0] or value.shape != key.shape:
        raise ValueError("key/value must be [B, 1, n_kv, S, D] matching the query batch")
    dev = _check_device(query, key, value)
    code = _dtype_code(query)
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise TypeError("query, key and value must share a dtype")
    _check_cache_view("key", key[0])
    _check_cache_view("value", value[0])
    if not query[0].is_contiguous():
        raise ValueError("each query problem must be contiguous")
    n_batch, _, n_q, _, d = query.shape
    n_kv, kv_len = key.shape[2], key.shape[3]
    if d != HEAD_DIM or n_q % n_kv:
        raise ValueError("unsupported head_dim or head counts")
    if out is None:
        out = torch.empty_like(query, memory_format=torch.contiguous_format)
    elif out.shape != query.shape or out.dtype != query.dtype or not out[0].is_contiguous():
        raise ValueError("out must be shaped like query with contiguous problems")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    lib = _lib.load_library()
    ws_bytes = lib.std_gqa_decode_batched_workspace_bytes(n_batch, n_q, n_kv, kv_len, d)
    ws_ptr = _attn_workspace(ws_bytes, dev)
    _lib.call("std_gqa_decode_batched", query.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr(), n_batch,
              n_q, n_kv, kv_len, d, query.stride(0), key.stride(0), value.stride(0), out.stride(0), key.stride(2),
              value.stride(2), float(scale), code, ws_ptr, ws_bytes, _stream(dev))
    return out.squeeze(1) if squeeze else out


def verify_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                     scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense verify attention for q_len appended rows with the offset-causal mask.

    query [1, n_q, Q, D]; key, value [1, n_kv, kv_len, D] including the Q new
    rows. Row i sees keys [0, kv_len - Q + i] (sparse_verify_spike.py:24-42,
    the math-SDPA verify of modeling_qwen2_5_vl.py:1096-1132).
    """
    if query.dim() != 4 or query.shape[0] != 1:
        raise ValueError(f"Expected query [1, n_q, Q, D], got {tuple(query.shape)}")
    return _attention("std_verify_attn", query, key, value, scale, out)


def gqa_decode_append(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                      new_key: torch.Tensor, new_value: torch.Tensor, kv_len: int,
                      scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """KVCache.cat of one new row at position kv_len - 1, then single-query
    attention over kv_len keys, in one launch (std_qwen25vl.py:395-417).
    key_cache/value_cache: full [1, n_kv, capacity, D] buffers; new_key/new_value
    [1, n_kv, 1, D] with contiguous head_dim."""
    if query.dim() != 4 or query.shape[0] != 1 or query.shape[2] != 1:
        raise ValueError(f"Expected q_len=1 query [1, n_q, 1, D], got {tuple(query.shape)}")
    return _attention("std_gqa_decode_append", query, key_cache, value_cache, scale, out,
                      new_key=new_key, new_value=new_value, kv_len=kv_len)


def verify_attention_append(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                            new_key: torch.Tensor, new_value: torch.Tensor, kv_len: int,
                            scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """KVCache.cat of the Q new rows at [kv_len - Q, kv_len), then the
    offset-causal verify attention over kv_len keys, in one launch
    (modeling_qwen2_5_vl.py:1057-1132). new_key/new_value [1, n_kv, Q, D]."""
    if query.dim() != 4 or query.shape[0] != 1:
        raise ValueError(f"Expected query [1, n_q, Q, D], got {tuple(query.shape)}")
    return _attention("std_verify_attn_append", query, key_cache, value_cache, scale, out,
                      new_key=new_key, new_value=new_value, kv_len=kv_len)


def _attention(fn: str, query, key, value, scale, out, new_key=None, new_value=None, kv_len=None):
    dev = _check_device(query, key, value)
    code = _dtype_code(query)
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise TypeError("query, key and value must share a dtype")
    _check_cache_view("key", key)
    _check_cache_view("value", value)
    _check_rows_contiguous("query", query)
    _, n_q, q_len, d = query.shape
    appending = new_key is not None
    if appending:
        if kv_len is None or not (q_len <= kv_len <= key.shape[2]):
            raise ValueError(f"kv_len={kv_len} must be in [q_len, cache capacity {key.shape[2]}]")
        for name, t in (("new_key", new_key), ("new_value", new_value)):
            if t.dim() != 4 or tuple(t.shape) != (1, key.shape[1], q_len, HEAD_DIM) or t.stride(3) != 1:
                raise ValueError(f"{name} must be [1, n_kv, {q_len}, {HEAD_DIM}] with contiguous rows")
            if t.dtype != query.dtype or t.device != query.device:
                raise TypeError(f"{name} must match the query dtype and device")
        if not same_layout(new_key, new_value):
            raise ValueError("new_key and new_value must share strides")
        if value.stride(1) != key.stride(1):
            raise ValueError("key and value caches must share a head stride")
    n_kv = key.shape[1]
    if not appending:
        kv_len = key.shape[2]
    if value.shape != key.shape:
        raise ValueError(f"key {tuple(key.shape)} and value {tuple(value.shape)} differ")
    if d != HEAD_DIM:
        raise ValueError(f"head_dim {d} unsupported")
    if n_q % n_kv != 0:
        raise ValueError(f"n_q={n_q} is not a multiple of n_kv={n_kv}")
    if q_len > kv_len:
        raise ValueError(f"q_len={q_len} exceeds kv_len={kv_len}")
    if out is None:
        out = torch.empty_like(query)
    elif out.shape != query.shape or out.dtype != query.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like query")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    lib = _lib.load_library()
    if q_len == 1 and fn.startswith("std_gqa_decode"):
        ws_bytes = lib.std_gqa_decode_workspace_bytes(n_q, n_kv, kv_len, d)
    else:
        ws_bytes = lib.std_verify_attn_workspace_bytes(n_q, n_kv, q_len, kv_len, d)
    ws_ptr = _attn_workspace(ws_bytes, dev)
    hs_k, hs_v = key.stride(1), value.stride(1)
    qp, kp, vp, op, st = query.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr(), _stream(dev)
    if fn == "std_gqa_decode":
        _lib.call(fn, qp, kp, vp, op, n_q, n_kv, kv_len, d, hs_k, hs_v, float(scale), code, ws_ptr, ws_bytes, st)
    elif fn == "std_verify_attn":
        _lib.call(fn, qp, kp, vp, op, n_q, n_kv, q_len, kv_len, d, hs_k, hs_v, float(scale), code, ws_ptr, ws_bytes,
                  st)
    elif fn == "std_gqa_decode_append":
        _lib.call(fn, qp, kp, vp, new_key.data_ptr(), new_value.data_ptr(), op, n_q, n_kv, kv_len, d, hs_k, hs_v,
                  new_key.stride(1), float(scale), code, ws_ptr, ws_bytes, st)
    else:
        _lib.call(fn, qp, kp, vp, new_key.data_ptr(), new_value.data_ptr(), op, n_q, n_kv, q_len, kv_len, d, hs_k,
                  hs_v, new_key.stride(1), new_key.stride(2), float(scale), code, ws_ptr, ws_bytes, st)
    return out


class ShapeAssertionError(ValueError, AssertionError):
    """A shape the reference rejects with an ``assert`` (q_len != 1, or query
    heads not a multiple of KV heads: triton_attention.py:89, 94). Catchable
    as AssertionError, as there, and as ValueError, as every shape error of
    this module."""


def fused_gqa_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """Drop-in for std_repro.triton_attention.fused_gqa_attention (same
    signature, output allocation -- a new tensor in query dtype -- and shape
    assertions)."""
    if query.dim() != 4 or query.shape[2] != 1:
        raise ShapeAssertionError(f"Expected q_len=1, got {tuple(query.shape)}")
    if key.dim() != 4 or key.shape[1] == 0 or query.shape[1] % key.shape[1] != 0:
        raise ShapeAssertionError(f"query heads {query.shape[1]} are not a multiple of KV heads in "
                                  f"{tuple(key.shape)}")
    return gqa_decode(query, key, value)


def select_topk(q_text: torch.Tensor, key: torch.Tensor, text_start: int, visual_positions: torch.Tensor,
                k: int, return_scores: bool = False):
    """Per-KV-head top-k visual positions from causal text-row attention.

    q_text [1, n_q, T, D] (text-suffix queries, RoPE applied); key
    [1, n_kv, >= P, D] cache view with P = text_start + T valid keys;
    visual_positions int32 [n_visual] sorted ascending. Returns int32
    [n_kv, k] sorted ascending (and fp64 scores [n_kv, P] if requested).
    Restates build_sparse_selection (std_qwen25vl.py:175-231) on the exact
    softmax of the selection prefill.
    """
    dev = _check_device(q_text, key, visual_positions)
    code = _dtype_code(q_text)
    if key.dtype != q_text.dtype:
        raise TypeError("q_text and key must share a dtype")
    if q_text.dim() != 4 or q_text.shape[0] != 1:
        raise ValueError(f"q_text must be [1, n_q, T, D], got {tuple(q_text.shape)}")
    _check_rows_contiguous("q_text", q_text)
    _check_cache_view("key", key)
    if visual_positions.dtype != torch.int32 or visual_positions.dim() != 1:
        raise TypeError("visual_positions must be a 1-D int32 tensor")
    visual_positions = visual_positions.contiguous()
    _, n_q, text_len, d = q_text.shape
    n_kv = key.shape[1]
    prompt_len = int(text_start) + text_len
    if key.shape[2] < prompt_len:
        raise ValueError(f"key holds {key.shape[2]} rows, prompt needs {prompt_len}")
    n_vis = visual_positions.numel()
    if not (1 <= k <= n_vis):
        raise ValueError(f"k={k} must be in [1, n_visual={n_vis}]")
    lib = _lib.load_library()
    ws_bytes = lib.std_select_topk_workspace_bytes(n_q, n_kv, text_len, prompt_len, n_vis, d)
    if ws_bytes == 0:
        raise ValueError("unsupported selection shape")
    ws_ptr, ws = _workspace(ws_bytes, dev)
    topk = torch.empty(n_kv, k, dtype=torch.int32, device=dev)
    scores = torch.empty(n_kv, prompt_len, dtype=torch.float64, device=dev) if return_scores else None
    _lib.call("std_select_topk", q_text.data_ptr(), key.data_ptr(), n_q, n_kv, text_len, prompt_len, int(text_start),
              d, key.stride(1), code, visual_positions.data_ptr(), n_vis, int(k), topk.data_ptr(),
              scores.data_ptr() if scores is not None else None, ws_ptr, ws_bytes, _stream(dev))
    return (topk, scores) if return_scores else topk


def select_topk_probs(probs: torch.Tensor, visual_positions: torch.Tensor, k: int, num_key_value_heads: int,
                      return_scores: bool = False):
    """Per-KV-head top-k visual positions from one layer's materialised
    attention probabilities, the reference's selection input
    (build_sparse_selection, std_qwen25vl.py:175-231).

    probs [1, n_q, T, P] (fp16 as the reference produces them, bf16 or fp32;
    columns contiguous, any head/row strides); visual_positions int32
    [n_visual] ascending. Returns int32 [n_kv, k] ascending (and the fp64
    group sums [n_kv, P] if requested); ties go to the lowest position."""
    dev = _check_device(probs, visual_positions)
    codes = {torch.float16: _lib.STD_F16, torch.bfloat16: _lib.STD_BF16, torch.float32: _lib.STD_F32}
    if probs.dtype not in codes:
        raise TypeError(f"unsupported probability dtype {probs.dtype}")
    if probs.dim() != 4 or probs.shape[0] != 1 or probs.stride(3) != 1:
        raise ValueError(f"probs must be [1, n_q, T, P] with contiguous columns, got {tuple(probs.shape)}")
    if visual_positions.dtype != torch.int32 or visual_positions.dim() != 1:
        raise TypeError("visual_positions must be a 1-D int32 tensor")
    visual_positions = visual_positions.contiguous()
    _, n_q, text_len, prompt_len = probs.shape
    if n_q % num_key_value_heads:
        raise ValueError(f"Query heads ({n_q}) must be divisible by KV heads ({num_key_value_heads}).")
    n_vis = visual_positions.numel()
    if not (1 <= k <= n_vis):
        raise ValueError(f"k={k} must be in [1, n_visual={n_vis}]")
    lib = _lib.load_library()
    ws_bytes = lib.std_select_topk_probs_workspace_bytes(n_q, num_key_value_heads, text_len, prompt_len, n_vis)
    ws_ptr, ws = _workspace(ws_bytes, dev)
    topk = torch.empty(num_key_value_heads, k, dtype=torch.int32, device=dev)
    scores = torch.empty(num_key_value_heads, prompt_len, dtype=torch.float64, device=dev) if return_scores else None
    _lib.call("std_select_topk_probs", probs.data_ptr(), probs.stride(1), probs.stride(2), codes[probs.dtype], n_q,
              num_key_value_heads, text_len, prompt_len, visual_positions.data_ptr(), n_vis, int(k), topk.data_ptr(),
              scores.data_ptr() if scores is not None else None, ws_ptr, ws_bytes, _stream(dev))
    return (topk, scores) if return_scores else topk


def build_compact_index(non_visual: torch.Tensor, topk: torch.Tensor) -> torch.Tensor:
    """Sorted union of the non-visual positions and each head's top-k
    (std_qwen25vl.py:286-291). Returns int32 [n_kv, n_nonvisual + k]."""
    dev = _check_device(topk, non_visual) if non_visual.numel() else _check_device(topk)
    if topk.dtype != torch.int32 or topk.dim() != 2:
        raise TypeError("topk must be int32 [n_kv, k]")
    if non_visual.dtype != torch.int32 or non_visual.dim() != 1:
        raise TypeError("non_visual must be 1-D int32")
    topk = topk.contiguous()
    non_visual = non_visual.contiguous()
    n_kv, k = topk.shape
    n_nv = non_visual.numel()
    idx = torch.empty(n_kv, n_nv + k, dtype=torch.int32, device=dev)
    _lib.call("std_build_compact_index", non_visual.data_ptr() if n_nv else None, n_nv, topk.data_ptr(), k, n_kv,
              idx.data_ptr(), _stream(dev))
    return idx


def compact_kv(dense_k: torch.Tensor, dense_v: torch.Tensor, sparse_k: torch.Tensor, sparse_v: torch.Tensor,
               index: torch.Tensor) -> None:
    """sparse[:, g, s] = dense[:, g, index[g, s]] for one layer, K and V.

    dense_*, sparse_* are full cache buffers [1, n_kv, capacity, D]; index is
    int32 [n_kv, compact_len] (std_qwen25vl.py:265-298 without the
    full-prompt copy)."""
    dev = _check_device(dense_k, dense_v, sparse_k, sparse_v, index)
    code = _dtype_code(dense_k)
    for name, t in (("dense_k", dense_k), ("dense_v", dense_v), ("sparse_k", sparse_k), ("sparse_v", sparse_v)):
        _check_cache_view(name, t)
        if t.dtype != dense_k.dtype:
            raise TypeError("all caches must share a dtype")
    if dense_v.stride(1) != dense_k.stride(1) or sparse_v.stride(1) != sparse_k.stride(1):
        raise ValueError("K and V caches must share a head stride")
    if index.dtype != torch.int32 or index.dim() != 2 or index.shape[0] != dense_k.shape[1]:
        raise TypeError("index must be int32 [n_kv, compact_len]")
    index = index.contiguous()
    n_kv, compact_len = index.shape
    if compact_len > sparse_k.shape[2]:
        raise ValueError(f"compact_len {compact_len} exceeds sparse capacity {sparse_k.shape[2]}")
    _lib.call("std_compact_kv", dense_k.data_ptr(), dense_v.data_ptr(), sparse_k.data_ptr(), sparse_v.data_ptr(),
              index.data_ptr(), n_kv, compact_len, HEAD_DIM, dense_k.stride(1), dense_k.shape[2],
              sparse_k.stride(1), sparse_k.shape[2], code, _stream(dev))


def _status_ptr(status: Optional[torch.Tensor], dev: torch.device):
    """The device status word's address (or None): an int32 tensor of at least
    one element on the op's device; kernels OR STD_STATUS_CACHE_OVERFLOW into
    element 0 when a row or length falls past the cache capacity."""
    if status is None:
        return None
    if status.dtype != torch.int32 or status.numel() < 1 or not status.is_contiguous() or status.device != dev:
        raise TypeError("status must be a contiguous int32 tensor on the op's device")
    return status.data_ptr()


def kv_append(cache_k: torch.Tensor, cache_v: torch.Tensor, new_k: torch.Tensor, new_v: torch.Tensor,
              length: torch.Tensor, status: Optional[torch.Tensor] = None) -> None:
    """Write new rows at positions length[0] + r (KVCache.cat, kv_cache.py:54-69,
    with the length on the device). cache_* [1, n_kv, capacity, D] buffers;
    new_* [1, n_kv, rows, D] with contiguous rows (any head/row stride). Rows
    that would land past the capacity are not written and mark ``status``."""
    dev = _check_device(cache_k, cache_v, new_k, new_v, length)
    code = _dtype_code(cache_k)
    _check_cache_view("cache_k", cache_k)
    _check_cache_view("cache_v", cache_v)
    if cache_v.stride(1) != cache_k.stride(1):
        raise ValueError("K and V caches must share a head stride")
    for name, t in (("new_k", new_k), ("new_v", new_v)):
        if t.dim() != 4 or t.shape[0] != 1 or t.shape[1] != cache_k.shape[1] or t.shape[3] != HEAD_DIM:
            raise ValueError(f"{name} must be [1, n_kv, rows, D], got {tuple(t.shape)}")
        if t.stride(3) != 1 or t.dtype != cache_k.dtype:
            raise ValueError(f"{name} must have contiguous head_dim and the cache dtype")
    if new_v.shape != new_k.shape or not same_layout(new_k, new_v):
        raise ValueError("new_k and new_v must share shape and strides")
    if length.dtype != torch.int32:
        raise TypeError("length must be a device int32 tensor")
    rows = new_k.shape[2]
    _lib.call("std_kv_append", cache_k.data_ptr(), cache_v.data_ptr(), new_k.data_ptr(), new_v.data_ptr(),
              cache_k.shape[1], rows, HEAD_DIM, cache_k.stride(1), new_k.stride(1), new_k.stride(2),
              cache_k.shape[2], length.data_ptr(), code, _status_ptr(status, dev), _stream(dev))


def _check_dev_scalar(name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.int32 or t.numel() < 1 or not t.is_contiguous():
        raise TypeError(f"{name} must be a contiguous device int32 tensor")


def rope_append(qkv: torch.Tensor, n_q: int, key_cache: torch.Tensor, value_cache: torch.Tensor,
                length: torch.Tensor, position: torch.Tensor, inv_freq: torch.Tensor, pos_offset: int = 0,
                q_out: Optional[torch.Tensor] = None, status: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rotary embedding of this step's rows plus the K/V cache append, with
    the length and the position read on the device (one launch).

    qkv [1, n, (n_q + 2 n_kv) D]: the fused q|k|v projection output (rows
    contiguous in the head dim). Row r has position position[0] + pos_offset
    + r; its rotated keys and its values go to cache row length[0] + r.
    Returns the rotated queries [1, n_q, n, D] (q_out if given). Restates
    apply_multimodal_rotary_pos_emb (modeling_qwen2_5_vl.py:690-732) for text
    positions and KVCache.cat (kv_cache.py:54-69); the length is not advanced.
    Rows that would land past the capacity are not written and mark
    ``status`` (see _status_ptr)."""
    dev = _check_device(qkv, key_cache, value_cache, length, position, inv_freq)
    code = _dtype_code(qkv)
    if qkv.dim() != 3 or qkv.shape[0] != 1 or qkv.stride(2) != 1:
        raise ValueError(f"qkv must be [1, n, width] with a contiguous last dim, got {tuple(qkv.shape)}")
    _check_cache_view("key_cache", key_cache)
    _check_cache_view("value_cache", value_cache)
    if value_cache.shape != key_cache.shape or value_cache.stride(1) != key_cache.stride(1):
        raise ValueError("key and value caches must share shape and head stride")
    if key_cache.dtype != qkv.dtype or value_cache.dtype != qkv.dtype:
        raise TypeError("caches must have the qkv dtype")
    n_kv = key_cache.shape[1]
    n = qkv.shape[1]
    if n_q % n_kv or qkv.shape[2] < (n_q + 2 * n_kv) * HEAD_DIM:
        raise ValueError(f"qkv width {qkv.shape[2]} too small for {n_q} + 2 x {n_kv} heads")
    _check_dev_scalar("length", length)
    _check_dev_scalar("position", position)
    if inv_freq.dtype != torch.float32 or inv_freq.numel() != HEAD_DIM // 2 or not inv_freq.is_contiguous():
        raise TypeError("inv_freq must be a contiguous float32 tensor of head_dim / 2 entries")
    if q_out is None:
        q_out = torch.empty(1, n_q, n, HEAD_DIM, dtype=qkv.dtype, device=dev)
    elif tuple(q_out.shape) != (1, n_q, n, HEAD_DIM) or q_out.dtype != qkv.dtype or not q_out.is_contiguous():
        raise ValueError("q_out must be a contiguous [1, n_q, n, D] tensor of the qkv dtype")
    _lib.call("std_rope_append", qkv.data_ptr(), qkv.stride(1), q_out.data_ptr(), key_cache.data_ptr(),
              value_cache.data_ptr(), n, n_q, n_kv, HEAD_DIM, key_cache.stride(1), key_cache.shape[2],
              length.data_ptr(), position.data_ptr(), int(pos_offset), inv_freq.data_ptr(), code,
              _status_ptr(status, dev), _stream(dev))
    return q_out


QKV_ROPE_MAX_K = 4096          # qkv_rope_append stages up to this many activations a row in LDS
QKV_ROPE_NORM_MAX_K = 3584     # ... and normalises rows up to this width in the same launch


def qkv_rope_append(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], n_q: int,
                    key_cache: torch.Tensor, value_cache: torch.Tensor, length: torch.Tensor,
                    position: torch.Tensor, inv_freq: torch.Tensor, pos_offset: int = 0,
                    norm_weight: Optional[torch.Tensor] = None, eps: float = 0.0,
                    status: Optional[torch.Tensor] = None) -> torch.Tensor:
    """rope_append(linear(x, weight, bias), ...) in one launch for up to four
    bf16 rows: x [1, n, K] (K <= 4096), weight [(n_q + 2 n_kv) D, K] the
    stacked q|k|v projection, bias [(n_q + 2 n_kv) D] or None. Same outputs,
    bit for bit, as the projection followed by rope_append: returns the
    rotated queries [1, n_q, n, D]; rotated keys and the values go to cache
    row length[0] + r. The length is not advanced. With norm_weight (one row,
    K <= 3584) x is normalised first in the same launch, exactly as
    rms_norm(x, norm_weight, eps). Rows past the capacity mark ``status``."""
    dev = _check_device(x, weight, key_cache, value_cache, length, position, inv_freq)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("qkv_rope_append: bf16 only")
    if x.dim() != 3 or x.shape[0] != 1 or x.stride(2) != 1:
        raise ValueError(f"x must be [1, n, K] with a contiguous last dim, got {tuple(x.shape)}")
    n, K = x.shape[1], x.shape[2]
    _check_cache_view("key_cache", key_cache)
    _check_cache_view("value_cache", value_cache)
    if value_cache.shape != key_cache.shape or value_cache.stride(1) != key_cache.stride(1):
        raise ValueError("key and value caches must share shape and head stride")
    if key_cache.dtype != x.dtype or value_cache.dtype != x.dtype:
        raise TypeError("caches must have the x dtype")
    n_kv = key_cache.shape[1]
    NW = (n_q + 2 * n_kv) * HEAD_DIM
    if n_q % n_kv or weight.shape != (NW, K) or weight.stride(1) != 1:
        raise ValueError(f"weight must be [{NW}, {K}] for {n_q} + 2 x {n_kv} heads")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.shape != (NW,) or not bias.is_contiguous()):
        raise ValueError(f"bias must be a contiguous bf16 [{NW}]")
    _check_dev_scalar("length", length)
    _check_dev_scalar("position", position)
    if inv_freq.dtype != torch.float32 or inv_freq.numel() != HEAD_DIM // 2 or not inv_freq.is_contiguous():
        raise TypeError("inv_freq must be a contiguous float32 tensor of head_dim / 2 entries")
    if norm_weight is not None:
        _check_device(norm_weight)
        if norm_weight.dtype != torch.bfloat16 or norm_weight.shape != (K,) or not norm_weight.is_contiguous():
            raise ValueError(f"norm weight must be a contiguous bf16 [{K}]")
    q_out = torch.empty(1, n_q, n, HEAD_DIM, dtype=x.dtype, device=dev)
    _lib.call("std_qkv_rope_append", x.data_ptr(), x.stride(1), n, K, weight.data_ptr(), weight.stride(0),
              bias.data_ptr() if bias is not None else None, n_q, n_kv, HEAD_DIM, q_out.data_ptr(),
              key_cache.data_ptr(), value_cache.data_ptr(), key_cache.stride(1), key_cache.shape[2],
              length.data_ptr(), position.data_ptr(), int(pos_offset), inv_freq.data_ptr(),
              norm_weight.data_ptr() if norm_weight is not None else None, float(eps), _lib.STD_BF16,
              _status_ptr(status, dev), _stream(dev))
    return q_out


def attention_devlen(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                     length: torch.Tensor, max_kv_len: int, scale: Optional[float] = None,
                     out: Optional[torch.Tensor] = None, status: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Offset-causal GQA attention with the cache length read on the device:
    keys [0, length[0] + q_len) are valid (this step's q_len rows last) and
    query row i sees keys [0, length[0] + i]; q_len == 1 is the decode. The
    launch is planned for max_kv_len (<= the cache capacity), so one captured
    graph serves every length up to it; a device length past
    max_kv_len - q_len yields NaN outputs and marks ``status``. query
    [1, n_q, q_len, D]."""
    dev = _check_device(query, key_cache, value_cache, length)
    code = _dtype_code(query)
    if query.dim() != 4 or query.shape[0] != 1:
        raise ValueError(f"Expected query [1, n_q, q_len, D], got {tuple(query.shape)}")
    if key_cache.dtype != query.dtype or value_cache.dtype != query.dtype:
        raise TypeError("query and caches must share a dtype")
    _check_cache_view("key_cache", key_cache)
    _check_cache_view("value_cache", value_cache)
    _check_rows_contiguous("query", query)
    _check_dev_scalar("length", length)
    if value_cache.shape != key_cache.shape:
        raise ValueError("key and value caches differ in shape")
    _, n_q, q_len, d = query.shape
    n_kv = key_cache.shape[1]
    if not (q_len <= max_kv_len <= key_cache.shape[2]):
        raise ValueError(f"max_kv_len={max_kv_len} must be in [q_len, cache capacity {key_cache.shape[2]}]")
    if d != HEAD_DIM or n_q % n_kv:
        raise ValueError("unsupported head_dim or head counts")
    if out is None:
        out = torch.empty_like(query)
    elif out.shape != query.shape or out.dtype != query.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like query")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    lib = _lib.load_library()
    ws_bytes = lib.std_verify_attn_workspace_bytes(n_q, n_kv, q_len, max_kv_len, d)
    ws_ptr = _attn_workspace(ws_bytes, dev)
    _lib.call("std_attn_devlen", query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), out.data_ptr(), n_q,
              n_kv, q_len, length.data_ptr(), int(max_kv_len), d, key_cache.stride(1), value_cache.stride(1),
              float(scale), code, ws_ptr, ws_bytes, _status_ptr(status, dev), _stream(dev))
    return out


def _gemv(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], residual: Optional[torch.Tensor],
          gated: bool, name: str, norm_weight: Optional[torch.Tensor] = None, eps: float = 0.0) -> torch.Tensor:
    dev = _check_device(x, weight)
    if norm_weight is not None:
        _check_device(norm_weight)
        K = x.shape[-1]
        if norm_weight.dtype != torch.bfloat16 or norm_weight.shape != (K,) or not norm_weight.is_contiguous():
            raise ValueError(f"{name}: norm_weight must be a contiguous bf16 [{K}]")
        one_launch = (x.numel() == K and K <= 3584 and x.is_contiguous() and x.data_ptr() % 16 == 0
                      and norm_weight.data_ptr() % 16 == 0)
        if not one_launch:      # the norm as its own launch, then the projection
            return _gemv(rms_norm(x, norm_weight, eps), weight, bias, residual, gated, name)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError(f"{name}: bf16 only")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M, (NW, Kw) = x2.shape[0], weight.shape
    if Kw != K or weight.stride(1) != 1 or x2.stride(1) != 1:
        raise ValueError(f"{name}: weight must be [N, K] and x [..., K], both contiguous in K")
    if gated and NW % 2:
        raise ValueError(f"{name}: weight must stack the gate and up rows, [2 * N, K]")
    N = NW // 2 if gated else NW
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.shape != (NW,) or not bias.is_contiguous()):
        raise ValueError(f"{name}: bias must be a contiguous bf16 [{NW}]")
    r2 = None
    if residual is not None:
        _check_device(residual)
        if residual.dtype != torch.bfloat16 or residual.shape != (*x.shape[:-1], N):
            raise ValueError(f"{name}: residual must be bf16 shaped [..., {N}] like the output")
        r2 = residual.reshape(-1, N)
        if r2.stride(1) != 1:
            raise ValueError(f"{name}: residual rows must be contiguous")
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    if norm_weight is not None:
        _lib.call("std_gemv_norm", x2.data_ptr(), norm_weight.data_ptr(), float(eps), weight.data_ptr(),
                  weight.stride(0), bias.data_ptr() if bias is not None else None,
                  r2.data_ptr() if r2 is not None else None, y.data_ptr(), N, K, int(gated), _lib.STD_BF16,
                  _stream(dev))
        return y.view(*x.shape[:-1], N)
    _lib.call("std_gemv_ex", x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0),
              bias.data_ptr() if bias is not None else None, r2.data_ptr() if r2 is not None else None,
              r2.stride(0) if r2 is not None else 0, y.data_ptr(), y.stride(0), M, N, K, int(gated), _lib.STD_BF16,
              _stream(dev))
    return y.view(*x.shape[:-1], N)


def pad_index(index: torch.Tensor) -> torch.Tensor:
    """int32 [n_kv, n] -> int32 [n_kv, n rounded up to 16] (padding entries 0):
    the row layout gqa_decode_indexed reads, 16 entries at a time."""
    if index.dtype != torch.int32 or index.dim() != 2:
        raise TypeError("index must be int32 [n_kv, n]")
    n_kv, n = index.shape
    out = torch.zeros(n_kv, (n + 15) // 16 * 16, dtype=torch.int32, device=index.device)
    out[:, :n] = index
    return out


def gqa_decode_indexed(query: torch.Tensor, dense_k: torch.Tensor, dense_v: torch.Tensor, index: torch.Tensor,
                       n_index: int, key_cache: torch.Tensor, value_cache: torch.Tensor, kv_len: Optional[int] = None,
                       length: Optional[torch.Tensor] = None, max_kv_len: Optional[int] = None,
                       scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                       status: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Draft decode whose first n_index keys per KV head are rows
    index[g, j] of the dense cache (no compaction copy); keys j >= n_index
    are rows j of the sparse cache key_cache / value_cache.

    query [1, n_q, 1, D] bf16; dense_* and key/value caches [1, n_kv, capacity, D]
    views with contiguous rows; index int32 [n_kv, >= n_index rounded up to 16]
    (see pad_index). Host length: kv_len keys. Device length: length[0] + 1
    keys (this step's row written at length[0]), planned for max_kv_len; a
    length past it marks ``status``."""
    dev = _check_device(query, dense_k, dense_v, index, key_cache, value_cache)
    if query.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("gqa_decode_indexed: bf16 or fp16")
    for name, t in (("dense_k", dense_k), ("dense_v", dense_v), ("key_cache", key_cache), ("value_cache", value_cache)):
        _check_cache_view(name, t)
        if t.dtype != query.dtype:
            raise TypeError("query and caches must share a dtype")
    if query.dim() != 4 or query.shape[0] != 1 or query.shape[2] != 1:
        raise ValueError(f"Expected query [1, n_q, 1, D], got {tuple(query.shape)}")
    _check_rows_contiguous("query", query)
    n_q, d = query.shape[1], query.shape[3]
    n_kv = key_cache.shape[1]
    if dense_k.shape[1] != n_kv or dense_v.shape != dense_k.shape or value_cache.shape != key_cache.shape:
        raise ValueError("dense and sparse caches must have the same KV heads")
    if d != HEAD_DIM or n_q % n_kv:
        raise ValueError("unsupported head_dim or head counts")
    if index.dtype != torch.int32 or index.dim() != 2 or index.shape[0] != n_kv or index.stride(1) != 1:
        raise TypeError("index must be int32 [n_kv, n] with contiguous rows")
    n_index = int(n_index)
    if not (0 <= n_index <= index.shape[1]) or index.shape[1] < (n_index + 15) // 16 * 16:
        raise ValueError("index rows must hold n_index entries rounded up to 16 (see pad_index)")
    if (length is None) == (kv_len is None):
        raise ValueError("give exactly one of kv_len (host length) and length (device length)")
    if length is not None:
        _check_device(length)
        _check_dev_scalar("length", length)
        if max_kv_len is None:
            raise ValueError("a device-length launch needs max_kv_len")
        plan = int(max_kv_len)
    else:
        plan = int(kv_len)
    if not (max(1, n_index) <= plan <= key_cache.shape[2]):
        raise ValueError(f"key count {plan} must be in [n_index, cache capacity {key_cache.shape[2]}]")
    if out is None:
        out = torch.empty_like(query)
    elif out.shape != query.shape or out.dtype != query.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like query")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    ws_bytes = _lib.load_library().std_gqa_decode_workspace_bytes(n_q, n_kv, plan, d)
    ws_ptr = _attn_workspace(ws_bytes, dev)
    _lib.call("std_gqa_decode_indexed", query.data_ptr(), dense_k.data_ptr(), dense_v.data_ptr(), dense_k.shape[2],
              dense_k.stride(1), dense_v.stride(1), index.data_ptr(), index.stride(0), n_index, key_cache.data_ptr(),
              value_cache.data_ptr(), key_cache.stride(1), value_cache.stride(1), out.data_ptr(), n_q, n_kv, plan,
              length.data_ptr() if length is not None else None, d, float(scale), _dtype_code(query), ws_ptr, ws_bytes,
              _status_ptr(status, dev), _stream(dev))
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           residual: Optional[torch.Tensor] = None, norm_weight: Optional[torch.Tensor] = None,
           eps: float = 0.0) -> torch.Tensor:
    """torch.nn.functional.linear for at most 16 bf16 rows: the HIP
    weight-streaming projection (weight [N, K] read once, fp32 accumulation,
    deterministic). x [..., K] with at most 16 rows in total. With residual
    ([..., N] bf16) it returns residual + linear(x, weight, bias), the
    decoder's residual add, rounded as torch rounds the two ops. With
    norm_weight x is first normalised as rms_norm(x, norm_weight, eps) (one
    launch for one row of at most 3584 elements: std_gemv_norm)."""
    return _gemv(x, weight, bias, residual, False, "linear", norm_weight, eps)


def gated_linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                 norm_weight: Optional[torch.Tensor] = None, eps: float = 0.0) -> torch.Tensor:
    """silu(gate) * up of gate, up = linear(x, weight, bias).chunk(2, -1) for
    at most 16 bf16 rows (the MLP's fused gate/up projection and activation,
    each op rounded to bf16 as torch rounds it): weight [2 I, K] stacks the
    gate rows over the up rows; returns [..., I]. norm_weight, eps: as in
    linear."""
    return _gemv(x, weight, bias, None, True, "gated_linear", norm_weight, eps)


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """int64 [rows] = argmax over the last dim of [rows, vocab] logits (first
    maximum; NaN wins), graph-capture safe (torch.argmax over a large vocab
    stages through a memset semaphore that captured graphs do not replay
    correctly)."""
    dev = _check_device(logits)
    code = _dtype_code(logits)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [rows, vocab] with contiguous rows")
    rows, vocab = logits.shape
    out = torch.empty(rows, dtype=torch.long, device=dev)
    ws_bytes = _lib.load_library().std_greedy_accept_workspace_bytes(rows, vocab)
    ws_ptr, ws = _workspace(ws_bytes, dev)
    _lib.call("std_argmax_rows", logits.data_ptr(), logits.stride(0), rows, vocab, code, out.data_ptr(), ws_ptr,
              ws_bytes, _stream(dev))
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen2RMSNorm (modeling_qwen2_5_vl.py:192-197) over the last dim, one
    HIP workgroup per row (graph-capture safe)."""
    dev = _check_device(x, weight)
    code = _dtype_code(x)
    if weight.dtype != x.dtype or weight.dim() != 1 or weight.shape[0] != x.shape[-1] or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [hidden] tensor of the input dtype")
    if x.stride(-1) != 1:
        raise ValueError("x must be contiguous in the last dim")
    hidden = x.shape[-1]
    x2 = x.reshape(-1, hidden)
    out = torch.empty(x2.shape, dtype=x.dtype, device=dev)
    _lib.call("std_rms_norm", x2.data_ptr(), x2.stride(0), weight.data_ptr(), out.data_ptr(), out.stride(0),
              x2.shape[0], hidden, float(eps), code, _stream(dev))
    return out.view(x.shape)


def len_add(length: torch.Tensor, delta: int) -> None:
    """length[:] += delta on the device."""
    dev = _check_device(length)
    if length.dtype != torch.int32 or not length.is_contiguous():
        raise TypeError("length must be a contiguous int32 tensor")
    _lib.call("std_len_add", length.data_ptr(), length.numel(), int(delta), _stream(dev))


def greedy_accept(logits: torch.Tensor, draft: torch.Tensor, has_pending: bool,
                  dense_next: Optional[torch.Tensor] = None,
                  rollback_lengths: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Greedy verification of a draft (std_qwen25vl.py:806-815 and rollback
    :923-928; pure form greedy_prefix, hsd_spike.py:30-43).

    logits [Q, V] (or [1, Q, V]) with Q = len(draft) + has_pending; draft int32
    [n_draft]; dense_next int32 [1] when has_pending is False. Returns int32
    [2 + n_draft + 1] = [accept_len, bonus, predictions...] on the device and
    decreases every entry of rollback_lengths by n_draft - accept_len.
    """
    if logits.dim() == 3:
        if logits.shape[0] != 1:
            raise ValueError("batch size 1 only")
        logits = logits[0]
    dev = _check_device(logits, draft)
    code = _dtype_code(logits)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [Q, vocab] with contiguous rows")
    if draft.dtype != torch.int32 or draft.dim() != 1:
        raise TypeError("draft must be 1-D int32")
    draft = draft.contiguous()
    q_rows, vocab = logits.shape
    n_draft = draft.numel()
    if q_rows != n_draft + (1 if has_pending else 0):
        raise ValueError(f"logits rows {q_rows} != n_draft {n_draft} + has_pending {int(has_pending)}")
    if not has_pending:
        if dense_next is None or dense_next.dtype != torch.int32:
            raise TypeError("dense_next (int32) is required without a pending token")
        _check_device(logits, dense_next)
    n_lens = 0
    if rollback_lengths is not None:
        if rollback_lengths.dtype != torch.int32 or not rollback_lengths.is_contiguous():
            raise TypeError("rollback_lengths must be contiguous int32")
        _check_device(logits, rollback_lengths)
        n_lens = rollback_lengths.numel()
    out = torch.empty(2 + n_draft + 1, dtype=torch.int32, device=dev)
    lib = _lib.load_library()
    ws_bytes = lib.std_greedy_accept_workspace_bytes(q_rows, vocab)
    ws_ptr, ws = _workspace(ws_bytes, dev)
    _lib.call("std_greedy_accept", logits.data_ptr(), logits.stride(0), q_rows, vocab, code, draft.data_ptr(),
              n_draft, 1 if has_pending else 0, dense_next.data_ptr() if dense_next is not None else None,
              out.data_ptr(), rollback_lengths.data_ptr() if n_lens else None, n_lens, ws_ptr, ws_bytes, _stream(dev))
    return out


STREAM_MODES = {
    0: "vector loads, contiguous chunk per workgroup",
    1: "vector loads, tiles round-robin",
    2: "LDS DMA ring (verify schedule: 8 waves, 2 tiles in flight), contiguous chunk per workgroup",
    3: "LDS DMA ring (verify schedule), tiles round-robin",
    4: "LDS DMA ring (decode key split: 4 waves, 3 tiles in flight), contiguous chunk per workgroup",
    5: "LDS DMA ring (decode key split), tiles round-robin",
    6: "LDS DMA ring (verify schedule), tiles round-robin, non-temporal loads",
    7: "LDS DMA ring (decode key split), tiles round-robin, non-temporal loads",
}


def stream_read(buf: torch.Tensor, mode: int, n_workgroups: int, sink: torch.Tensor) -> None:
    """Read all of buf once with the streaming-ceiling kernel (a measurement
    helper: nothing is computed). sink: int32, at least n_workgroups words."""
    dev = _check_device(buf, sink)
    if not buf.is_contiguous() or not sink.is_contiguous() or sink.numel() < n_workgroups:
        raise ValueError("buf and sink must be contiguous; sink needs n_workgroups words")
    nbytes = buf.numel() * buf.element_size()
    _lib.call("std_stream_read", buf.data_ptr(), nbytes, int(mode), int(n_workgroups), sink.data_ptr(), _stream(dev))


def gqa_decode_noalloc(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                       scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gqa_decode through the allocation-free entry point: the library's own
    per-GPU scratch array replaces the workspace (no allocation at all when
    `out` is given). Results equal gqa_decode's bit for bit."""
    if query.dim() != 4 or query.shape[0] != 1 or query.shape[2] != 1:
        raise ValueError(f"Expected q_len=1 query [1, n_q, 1, D], got {tuple(query.shape)}")
    dev = _check_device(query, key, value)
    code = _dtype_code(query)
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise TypeError("query, key and value must share a dtype")
    _check_cache_view("key", key)
    _check_cache_view("value", value)
    _check_rows_contiguous("query", query)
    n_q, n_kv, kv_len = query.shape[1], key.shape[1], key.shape[2]
    if value.shape != key.shape:
        raise ValueError("key and value shapes differ")
    if out is None:
        out = torch.empty_like(query)
    elif out.shape != query.shape or out.dtype != query.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like query")
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else float(scale)
    _lib.call("std_gqa_decode_noalloc", query.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr(), n_q, n_kv,
              kv_len, HEAD_DIM, key.stride(1), value.stride(1), scale, code, _stream(dev))
    return out


class VisualKeys:
    """The visual key positions a collector scores, in the form the collector
    launch reads: the first position and last + 1 (begin, end), the count n,
    and, unless the positions are the whole range [begin, end), a device
    bitmask (uint32 words as int32, bit j % 32 of word j // 32 set for a
    visual key j) with each word's rank (visual keys below it). Build it once
    per prompt with ``visual_keys(positions, device)``."""

    def __init__(self, begin: int, end: int, n: int, mask: Optional[torch.Tensor], rank: Optional[torch.Tensor],
                 positions: torch.Tensor):
        self.begin, self.end, self.n = int(begin), int(end), int(n)
        self.mask, self.rank = mask, rank
        self.positions = positions

    @property
    def contiguous(self) -> bool:
        return self.mask is None


def visual_keys(positions, device) -> VisualKeys:
    """VisualKeys of an ascending set of visual positions (a tensor or a
    sequence of ints); dynamic_selection.py:515 gathers key_states at them."""
    pos = torch.as_tensor(positions).to("cpu", torch.int64).reshape(-1)
    if pos.numel() == 0:
        raise ValueError("no visual positions")
    if int(pos[0]) < 0 or (pos.numel() > 1 and not bool((pos[1:] > pos[:-1]).all())):
        raise ValueError("visual positions must be nonnegative and strictly ascending")
    begin, end, n = int(pos[0]), int(pos[-1]) + 1, int(pos.numel())
    if n == end - begin:
        return VisualKeys(begin, end, n, None, None, pos)
    n_words = (end + 31) // 32
    bits = torch.zeros(n_words * 32, dtype=torch.int64)
    bits[pos] = 1
    weights = torch.tensor([1 << i for i in range(32)], dtype=torch.int64)
    words = (bits.view(n_words, 32) * weights).sum(1)
    words = torch.where(words >= 1 << 31, words - (1 << 32), words).to(torch.int32)     # uint32 bit pattern
    counts = bits.view(n_words, 32).sum(1)
    rank = (torch.cumsum(counts, 0) - counts).to(torch.int32)
    dev = torch.device(device)
    return VisualKeys(begin, end, n, words.to(dev), rank.to(dev), pos)


def verify_attention_collect(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                             vis_begin: Optional[int] = None, vis_end: Optional[int] = None,
                             new_key: Optional[torch.Tensor] = None, new_value: Optional[torch.Tensor] = None,
                             kv_len: Optional[int] = None, scale: Optional[float] = None,
                             out: Optional[torch.Tensor] = None, scores: Optional[torch.Tensor] = None,
                             visual: Optional[VisualKeys] = None, length: Optional[torch.Tensor] = None,
                             status: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dense verify attention plus the visual-attention collector in one pass
    (VerificationCollectorV3._hook, dynamic_selection.py:504-519, riding the
    verify forward at modeling_qwen2_5_vl.py:1063-1067).

    query [1, n_q, q_len, D] bf16 or fp16; key_cache / value_cache [1, n_kv, S, D]
    cache views (read in place). Without new_key/new_value the caches hold
    kv_len (default S) keys including this step's q_len rows; with them
    ([1, n_kv, q_len, D]) those rows are appended at kv_len - q_len first.
    With ``length`` (device int32 [1]) the cache instead holds length[0] rows
    plus this step's q_len, read on the device (a graph-replayed verify), and
    kv_len is the largest such total (default S).
    The visual keys are [vis_begin, vis_end), or any ascending set given as
    ``visual`` (see visual_keys).
    Returns (out [1, n_q, q_len, D], scores [n_kv, n_visual] fp32):
    scores[g, r] sums, over the q_len positions, the softmax over the visual
    keys of the group-mean query of KV head g, at the r-th visual key. out is
    verify_attention's result bit for bit when (group + 1) * q_len <= 80;
    longer verifies run in chunks of positions."""
    dev = _check_device(query, key_cache, value_cache)
    if query.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("the collector path is bf16 or fp16")
    if key_cache.dtype != query.dtype or value_cache.dtype != query.dtype:
        raise TypeError("query and caches must share a dtype")
    _check_cache_view("key_cache", key_cache)
    _check_cache_view("value_cache", value_cache)
    _check_rows_contiguous("query", query)
    if query.dim() != 4 or query.shape[0] != 1:
        raise ValueError(f"Expected query [1, n_q, q_len, D], got {tuple(query.shape)}")
    _, n_q, q_len, d = query.shape
    n_kv = key_cache.shape[1]
    if n_q % n_kv:
        raise ValueError(f"Query heads ({n_q}) must be divisible by KV heads ({n_kv}).")
    if n_q // n_kv + 1 > 80:
        raise ValueError(f"{n_q // n_kv} query heads per KV head exceed the collector's 79")
    if kv_len is None:
        kv_len = key_cache.shape[2]
    if not (q_len <= kv_len <= key_cache.shape[2]):
        raise ValueError(f"kv_len={kv_len} must be in [q_len, cache capacity {key_cache.shape[2]}]")
    if length is not None:
        _check_dev_scalar("length", length)
        if length.device != dev:
            raise RuntimeError("length must be on the query's device")
    appending = new_key is not None
    if appending != (new_value is not None):
        raise ValueError("new_key and new_value go together")
    if appending:
        for name, t in (("new_key", new_key), ("new_value", new_value)):
            if t.dim() != 4 or tuple(t.shape) != (1, n_kv, q_len, HEAD_DIM) or t.stride(3) != 1:
                raise ValueError(f"{name} must be [1, n_kv, {q_len}, {HEAD_DIM}] with contiguous rows")
            if t.dtype != query.dtype or t.device != query.device:
                raise TypeError(f"{name} must match the query dtype and device")
        if not same_layout(new_key, new_value):
            raise ValueError("new_key and new_value must share strides")
    if visual is None:
        if vis_begin is None or vis_end is None:
            raise ValueError("give the visual keys as vis_begin/vis_end or as visual=")
        visual = VisualKeys(vis_begin, vis_end, vis_end - vis_begin, None, None, None)
    elif vis_begin is not None or vis_end is not None:
        raise ValueError("give the visual keys once")
    elif visual.mask is not None and visual.mask.device != dev:
        raise RuntimeError("the visual key mask must be on the query's device")
    if not (0 <= visual.begin < visual.end <= kv_len - q_len):
        raise ValueError(f"visual keys [{visual.begin}, {visual.end}) must be prompt keys below {kv_len - q_len}")
    if out is None:
        out = torch.empty_like(query)
    elif out.shape != query.shape or out.dtype != query.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like query")
    if scores is None:
        scores = torch.empty(n_kv, visual.n, dtype=torch.float32, device=dev)
    elif scores.dtype != torch.float32 or scores.dim() != 2 or tuple(scores.shape) != (n_kv, visual.n) or \
            scores.stride(1) != 1:
        raise ValueError(f"scores must be float32 [{n_kv}, {visual.n}] with contiguous rows")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    lib = _lib.load_library()
    ws_bytes = lib.std_verify_attn_collect_workspace_bytes(n_q, n_kv, q_len, kv_len, d, visual.begin, visual.end)
    ws_ptr = _attn_workspace(ws_bytes, dev)
    _lib.call("std_verify_attn_collect_ex", query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
              new_key.data_ptr() if appending else None, new_value.data_ptr() if appending else None,
              out.data_ptr(), n_q, n_kv, q_len, int(kv_len), length.data_ptr() if length is not None else None, d,
              key_cache.stride(1), value_cache.stride(1), new_key.stride(1) if appending else 0,
              new_key.stride(2) if appending else 0, float(scale), _dtype_code(query), visual.begin, visual.end,
              visual.mask.data_ptr() if visual.mask is not None else None,
              visual.rank.data_ptr() if visual.rank is not None else None, visual.n, scores.data_ptr(),
              scores.stride(0), ws_ptr, ws_bytes, _status_ptr(status, dev), _stream(dev))
    return out, scores
