"""The allocation-free decode entry point (std_gqa_decode_noalloc, which keeps
its split partials in the library's own per-GPU scratch array) against the
workspace entry point std_gqa_decode, through the C ABI: bit-equal outputs on
two calls in a row, the second with a smaller input, in bf16, fp16 and fp32;
and a process whose first allocation-free call is made under HIP graph
capture."""
import math
import os
import subprocess
import sys
import textwrap

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


_CAPTURE_FIRST_CALL = textwrap.dedent("""
    import math, sys
    import torch
    sys.path.insert(0, {root!r})
    from std_amd import ops
    g = torch.Generator(device="cuda").manual_seed(21)
    q = torch.randn(1, 28, 1, 128, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(1, 4, 8192, 128, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(1, 4, 8192, 128, generator=g, device="cuda").to(torch.bfloat16)
    want = ops.gqa_decode(q, k, v)          # the same kernels, launched eagerly before the capture
    torch.cuda.synchronize()
    out = torch.full_like(q, float("nan"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):           # the process's first allocation-free call, under capture
        ops.gqa_decode_noalloc(q, k, v, out=out)
    for i in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), "replay %d differs from the eager decode" % i
        ops.gqa_decode(q[:, :, :, :].clone(), k, v)       # eager work between replays
        torch.cuda.synchronize()
    print("CAPTURE_FIRST_CALL_OK", flush=True)
""")


def test_noalloc_first_call_under_graph_capture():
    """A fresh process whose first std_gqa_decode_noalloc call is recorded
    into a HIP graph (the scratch address lookup then runs during the
    capture): every replay equals the eager workspace decode bit for bit."""
    announce("noalloc decode: first call of a process under graph capture")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, "-c", _CAPTURE_FIRST_CALL.format(root=root)], capture_output=True,
                         text=True, timeout=240)
    assert res.returncode == 0 and "CAPTURE_FIRST_CALL_OK" in res.stdout, res.stdout[-2000:] + res.stderr[-4000:]
