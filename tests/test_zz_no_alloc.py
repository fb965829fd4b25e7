"""The allocation-free decode entry point (std_gqa_decode_noalloc, which keeps
its split partials in the library's own per-GPU scratch array) against the
workspace entry point std_gqa_decode, through the C ABI: bit-equal outputs on
two calls in a row, the second with a smaller input, in bf16 and fp32."""
import math

import pytest
import torch

from std_amd import _lib, ops

from gpu_helpers import announce, dev

pytestmark = pytest.mark.gpu

D = 128


def _inputs(n_q, n_kv, kv_len, capacity, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(1, n_q, 1, D, generator=g, device="cuda").to(dtype)
    k = torch.full((1, n_kv, capacity, D), float("nan"), dtype=dtype, device=dev())
    v = torch.full_like(k, float("nan"))
    k[:, :, :kv_len] = torch.randn(1, n_kv, kv_len, D, generator=g, device="cuda").to(dtype)
    v[:, :, :kv_len] = torch.randn(1, n_kv, kv_len, D, generator=g, device="cuda").to(dtype)
    return q, k[:, :, :kv_len], v[:, :, :kv_len]


def _workspace_decode(q, k, v):
    """The existing entry point, with a caller workspace, through the C ABI."""
    lib = _lib.load_library()
    n_q, n_kv, kv_len = q.shape[1], k.shape[1], k.shape[2]
    code = {torch.bfloat16: _lib.STD_BF16, torch.float16: _lib.STD_F16}.get(q.dtype, _lib.STD_F32)
    out = torch.empty_like(q)
    ws_bytes = lib.std_gqa_decode_workspace_bytes(n_q, n_kv, kv_len, D)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev())
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("std_gqa_decode", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), n_q, n_kv, kv_len, D,
              k.stride(1), v.stride(1), 1.0 / math.sqrt(D), code, ws.data_ptr(), ws_bytes, st)
    return out


def _noalloc_decode(q, k, v):
    n_q, n_kv, kv_len = q.shape[1], k.shape[1], k.shape[2]
    code = {torch.bfloat16: _lib.STD_BF16, torch.float16: _lib.STD_F16}.get(q.dtype, _lib.STD_F32)
    out = torch.full_like(q, float("nan"))
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("std_gqa_decode_noalloc", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), n_q, n_kv, kv_len,
              D, k.stride(1), v.stride(1), 1.0 / math.sqrt(D), code, st)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_noalloc_decode_equals_workspace_decode(dtype):
    # first call: the dense 128k AR decode (64 splits per KV head, the largest
    # partial set of the decode path); second: the 1034-key sparse draft, which
    # leaves most of the first call's partials in the array
    for kv_len, seed in ((131072, 11), (1034, 12)):
        announce(f"noalloc decode {dtype} kv_len={kv_len}")
        q, k, v = _inputs(28, 4, kv_len, kv_len + 64, dtype, seed)
        want = _workspace_decode(q, k, v)
        got = _noalloc_decode(q, k, v)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), f"noalloc decode differs at kv_len={kv_len}"


def test_noalloc_ops_wrapper_matches():
    announce("noalloc decode through ops, bf16, kv_len=4096")
    q, k, v = _inputs(28, 4, 4096, 4160, torch.bfloat16, 13)
    want = ops.gqa_decode(q, k, v)
    got = ops.gqa_decode_noalloc(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
