"""The C-ABI library loads, exports every function include/std_hip.h declares,
and rejects bad arguments on the host before any device work (no GPU needed:
only validation paths and host-only queries are called here). Every call in
this file must fail validation: the pointers are placeholders, never memory."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from std_amd import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "std_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(std_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_match_binding_table():
    assert _declared() == _lib.exported_symbols()


def test_library_exports_every_declared_symbol():
    lib = _lib.load_library()
    for name in _declared():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())], capture_output=True, text=True)
    exported = set(re.findall(r" T (std_\w+)", out.stdout))
    assert set(_declared()) <= exported


def test_status_strings_and_version():
    lib = _lib.load_library()
    assert lib.std_version() == 0x000100
    assert lib.std_status_string(0) == b"success"
    for code in range(-6, 0):
        assert b"unknown" not in lib.std_status_string(code)


def test_workspace_queries():
    lib = _lib.load_library()
    assert lib.std_gqa_decode_workspace_bytes(28, 4, 1024, 128) > 0
    assert lib.std_gqa_decode_workspace_bytes(28, 4, 64, 128) == 0        # one tile: no split, no workspace
    assert lib.std_verify_attn_workspace_bytes(28, 4, 10, 131082, 128) > 0
    assert lib.std_verify_attn_workspace_bytes(28, 4, 10, 131082, 64) == 0   # unsupported head dim
    assert lib.std_select_topk_workspace_bytes(28, 4, 128, 4096, 3968, 128) > 0
    assert lib.std_greedy_accept_workspace_bytes(10, 152064) >= 10 * 75 * 8


NULL = None


@pytest.mark.parametrize("args,expected", [
    ((NULL, NULL, NULL, NULL, 28, 4, 1024, 128, 0, 0, 1.0, 1, NULL, 0, NULL), -1),
    ((16, 16, 16, 16, 28, 4, 1024, 64, 1024 * 128, 1024 * 128, 1.0, 1, NULL, 0, NULL), -3),   # head_dim
    ((16, 16, 16, 16, 28, 5, 1024, 128, 1024 * 128, 1024 * 128, 1.0, 1, NULL, 0, NULL), -3),  # 28 % 5
    ((16, 16, 16, 16, 28, 4, 1024, 128, 1024 * 128, 1024 * 128, 1.0, 7, NULL, 0, NULL), -2),  # dtype
    ((16, 16, 16, 16, 28, 4, 1024, 128, 100, 1024 * 128, 1.0, 1, NULL, 0, NULL), -3),        # head stride < rows
    ((8, 16, 16, 16, 28, 4, 1024, 128, 1024 * 128, 1024 * 128, 1.0, 1, 16, 1 << 30, NULL), -5),  # misaligned q
    ((16, 16, 16, 16, 28, 4, 1024, 128, 1024 * 128, 1024 * 128, 1.0, 1, NULL, 0, NULL), -4),  # no workspace
])
def test_decode_validation(args, expected):
    assert _lib.load_library().std_gqa_decode(*args) == expected


def test_noalloc_decode_validation():
    """The allocation-free decode rejects bad arguments, and a workspace need
    beyond its scratch array (2 MiB + 64 KiB), before any HIP call."""
    lib = _lib.load_library()
    hs = 1 << 27
    assert lib.std_gqa_decode_noalloc(NULL, 16, 16, 16, 28, 4, 1024, 128, hs, hs, 1.0, 1, NULL) == -1
    assert lib.std_gqa_decode_noalloc(16, 16, 16, 16, 28, 4, 1024, 64, hs, hs, 1.0, 1, NULL) == -3
    assert lib.std_gqa_decode_noalloc(16, 16, 16, 16, 28, 4, 1024, 128, hs, hs, 1.0, 9, NULL) == -2
    # fp32 with 16 query heads per KV head over 1M keys: 512 splits x 16 rows of partials = 4.2 MB
    assert lib.std_gqa_decode_workspace_bytes(64, 4, 1 << 20, 128) > (2 << 20) + (64 << 10)
    assert lib.std_gqa_decode_noalloc(16, 16, 16, 16, 64, 4, 1 << 20, 128, hs, hs, 1.0, 0, NULL) == -4
    # the largest bf16 need fits (256 splits x 16 rows)
    assert lib.std_gqa_decode_workspace_bytes(64, 4, 1 << 20, 128) > 0


def test_split_plan():
    """The planner's split counts at the shapes they were measured on: the
    per-layer draft (4 KV heads, 1034 keys) keeps one tile per split, dense
    decode and verify at 128k keep 64 splits per head, the 28-layer draft
    launch (112 problems) and decodes of at most five tiles stream unsplit,
    and 32 / 64 problems keep their 256-workgroup plans."""
    lib = _lib.load_library()
    bf16, f32, f16 = 1, 0, 2
    for n_prob, rows, kv_len, want in [(4, 7, 1034, 17), (4, 7, 1043, 17), (4, 7, 131072, 64), (4, 70, 131082, 64),
                                        (112, 7, 1034, 1), (112, 7, 2048, 1), (64, 7, 1034, 4), (64, 7, 2048, 4),
                                        (32, 7, 1034, 8), (32, 7, 2048, 8), (224, 7, 1034, 1), (4, 7, 320, 1),
                                        (4, 7, 400, 7), (4, 7, 64, 1), (4, 7, 1, 1), (4, 70, 4106, 64),
                                        (4, 70, 16394, 64), (4, 70, 65546, 64)]:
        assert lib.std_attn_split_count(n_prob, rows, kv_len, bf16) == want, (n_prob, rows, kv_len)
        # fp16 runs the same kernels, partials and workspace layout as bf16
        assert lib.std_attn_split_count(n_prob, rows, kv_len, f16) == want, (n_prob, rows, kv_len)
    # fp32 and multi-row-tile launches split to fill the GPU whatever the merge costs
    assert lib.std_attn_split_count(4, 7, 320, f32) == 5
    assert lib.std_attn_split_count(112, 70, 1034, bf16) == 2
    assert lib.std_attn_split_count(4, 7, 1034, 5) == -2
    assert lib.std_attn_split_count(0, 7, 1034, bf16) == -3
    assert lib.std_attn_split_count(4, 97, 1034, bf16) == -3
    assert lib.std_attn_split_count(4, 7, 0, bf16) == -3


def test_batched_decode_validation():
    """Every call here fails validation before any launch."""
    lib = _lib.load_library()
    hs = 1024 * 128
    assert lib.std_gqa_decode_batched_workspace_bytes(28, 28, 4, 1034, 128) > 0
    assert lib.std_gqa_decode_batched_workspace_bytes(0, 28, 4, 1034, 128) == 0
    args = [16, 16, 16, 16, 28, 28, 4, 1024, 128, 28 * 128, 4 * hs, 4 * hs, 28 * 128, hs, hs, 1.0, 1, NULL, 0, NULL]
    bad_batch = list(args)
    bad_batch[4] = 0
    assert lib.std_gqa_decode_batched(*bad_batch) == -3
    overlap = list(args)
    overlap[12] = 100                                      # out batch stride < n_q * d: problems overlap
    assert lib.std_gqa_decode_batched(*overlap) == -3
    misaligned = list(args)
    misaligned[10] = 4 * hs + 3                            # k batch stride not a 16-byte multiple
    assert lib.std_gqa_decode_batched(*misaligned) == -5
    # two problems of 16 tiles are split (28 of them stream unsplit and need no workspace)
    split = list(args)
    split[4] = 2
    assert lib.std_gqa_decode_batched(*split) == -4        # no workspace


def test_verify_validation():
    lib = _lib.load_library()
    hs = 4106 * 128
    assert lib.std_verify_attn(16, 16, 16, 16, 28, 4, 20, 4106, 128, hs, hs, 1.0, 1, NULL, 0, NULL) == -3  # 7*20 rows > 96
    assert lib.std_verify_attn(16, 16, 16, 16, 28, 4, 11, 10, 128, hs, hs, 1.0, 1, NULL, 0, NULL) == -3   # q > kv


def test_verify_collect_validation():
    lib = _lib.load_library()
    hs = 4106 * 128
    args = dict(q=16, k=16, v=16, nk=NULL, nv=NULL, out=16, nq=28, nkv=4, ql=10, kv=4106, d=128, khs=hs, vhs=hs,
                nhs=0, nrs=0, scale=0.088, dt=1, vb=0, ve=3968, sc=16, schs=3968, ws=16, wsb=1 << 30, st=NULL)

    def call(**kw):
        a = dict(args, **kw)
        return lib.std_verify_attn_collect(*a.values())
    assert lib.std_verify_attn_collect_workspace_bytes(28, 4, 10, 4106, 128, 0, 3968) > 0
    assert call(dt=0) == -2                     # bf16 or fp16
    assert call(dt=3) == -2
    assert call(sc=NULL) == -1
    assert call(nk=16) == -1                    # new_k without new_v
    # (7 + 1) * 11 > 80 rows: served in chunks of positions, which need room
    # for one chunk's query and output rows
    ws10 = lib.std_verify_attn_collect_workspace_bytes(28, 4, 10, 4106, 128, 0, 3968)
    ws11 = lib.std_verify_attn_collect_workspace_bytes(28, 4, 11, 4106, 128, 0, 3968)
    assert ws11 >= ws10 + 2 * 28 * 10 * 128 * 2
    assert call(ql=11, dt=2, wsb=ws10) == -4   # fp16: fp32 partials, the size the query reports
    assert call(nq=4, ql=17, wsb=10) == -4      # chunks of 16 positions
    assert lib.std_verify_attn_collect_workspace_bytes(80, 1, 2, 4106, 128, 0, 3968) == 0   # 81 > 80 rows
    assert call(nq=80, nkv=1, ql=2) == -3
    assert call(ve=4100) == -3                  # visual keys must be prompt keys
    assert call(vb=3968) == -3                  # empty visual range
    assert call(schs=100) == -3                 # score rows overlap
    assert call(wsb=10) == -4


def test_verify_collect_ex_validation():
    lib = _lib.load_library()
    hs = 4106 * 128
    args = dict(q=16, k=16, v=16, nk=NULL, nv=NULL, out=16, nq=28, nkv=4, ql=10, kv=4106, len_dev=NULL, d=128,
                khs=hs, vhs=hs, nhs=0, nrs=0, scale=0.088, dt=1, vb=0, ve=3968, mask=NULL, rank=NULL, nvis=3968,
                sc=16, schs=3968, ws=16, wsb=1 << 30, status=NULL, st=NULL)

    def call(**kw):
        a = dict(args, **kw)
        return lib.std_verify_attn_collect_ex(*a.values())
    assert call(mask=16) == -1                  # mask and rank go together
    assert call(rank=16) == -1
    assert call(nvis=3000) == -3                # a whole range counts vis_end - vis_begin keys
    assert call(mask=16, rank=16, nvis=0) == -3
    assert call(mask=16, rank=16, nvis=3969) == -3   # more than the range holds
    assert call(mask=16, rank=16, nvis=100, schs=99) == -3
    assert call(mask=16, rank=16, nvis=100, wsb=10) == -4
    assert call(dt=0) == -2


def test_select_probs_validation():
    lib = _lib.load_library()
    P, T = 4096, 128
    assert lib.std_select_topk_probs_workspace_bytes(28, 4, T, P, P - T) > 0
    ok = dict(p=16, hs=T * P, rs=P, dt=2, nq=28, nkv=4, t=T, pl=P, vis=16, nv=P - T, k=896, out=16, sc=NULL, ws=16,
              wsb=1 << 30, st=NULL)

    def call(**kw):
        a = dict(ok, **kw)
        return lib.std_select_topk_probs(*a.values())
    assert call(dt=5) == -2
    assert call(vis=NULL) == -1
    assert call(k=P) == -3                      # k above the visual count
    assert call(rs=P - 1) == -3                 # rows overlap
    assert call(nkv=5) == -3                    # 28 % 5
    assert call(p=17) == -5                     # fp16 elements must be 2-byte aligned
    assert call(wsb=100) == -4


def test_select_validation():
    lib = _lib.load_library()
    hs = 4096 * 128
    # k > n_visual, and prompt_len != text_start + text_len
    assert lib.std_select_topk(16, 16, 28, 4, 128, 4096, 3968, 128, hs, 1, 16, 3968, 4000, 16, NULL, 16, 1 << 30,
                               NULL) == -3
    assert lib.std_select_topk(16, 16, 28, 4, 128, 4096, 3900, 128, hs, 1, 16, 3968, 896, 16, NULL, 16, 1 << 30,
                               NULL) == -3
    assert lib.std_select_topk(16, 16, 28, 4, 128, 4096, 3968, 128, hs, 1, 16, 3968, 896, 16, NULL, 16, 10,
                               NULL) == -4
    # K is read in 16-byte chunks: a misaligned base or head stride is rejected
    assert lib.std_select_topk(16, 8, 28, 4, 128, 4096, 3968, 128, hs, 1, 16, 3968, 896, 16, NULL, 16, 1 << 30,
                               NULL) == -5
    assert lib.std_select_topk(16, 16, 28, 4, 128, 4096, 3968, 128, hs + 4, 1, 16, 3968, 896, 16, NULL, 16, 1 << 30,
                               NULL) == -5


def test_indexed_decode_validation():
    lib = _lib.load_library()
    hs = 128 * 4096
    # fp32 is not served; the index must be present, aligned and padded to 16 entries per row
    args = dict(q=16, dk=16, dv=16, rows=4096, dks=hs, dvs=hs, idx=16, ihs=1024, n=1024, k=16, v=16, ks=hs, vs=hs,
                out=16, nq=28, nkv=4, kv=1100, ld=NULL, d=128, scale=0.088, dt=1, ws=16, wsb=1 << 30, status=NULL,
                st=NULL)

    def call(**kw):
        a = dict(args, **kw)
        return lib.std_gqa_decode_indexed(*a.values())
    assert call(dt=0) == -2
    assert call(idx=NULL) == -1
    assert call(idx=20) == -5
    assert call(ihs=1000) == -3                 # below n_index
    assert call(n=2000) == -3                   # more indexed keys than keys
    assert call(ihs=1026, n=1024) == -5         # row stride not a multiple of 4 entries


def test_gemv_validation():
    lib = _lib.load_library()
    # K must be a multiple of 32; at most 16 rows; bf16 only; 16-byte aligned rows
    assert lib.std_gemv_ex(16, 100, 16, 100, NULL, NULL, 0, 16, 64, 1, 64, 100, 0, 1, NULL) == -3
    assert lib.std_gemv_ex(16, 128, 16, 128, NULL, NULL, 0, 16, 64, 17, 64, 128, 0, 1, NULL) == -3
    assert lib.std_gemv_ex(16, 128, 16, 128, NULL, NULL, 0, 16, 64, 1, 64, 128, 0, 0, NULL) == -2
    assert lib.std_gemv_ex(16, 128, 16, 128, NULL, NULL, 0, 16, 64, 1, 64, 128, 0, 2, NULL) == -2
    assert lib.std_gemv_ex(16, 128, 16, 128, NULL, 16, 10, 16, 64, 1, 64, 128, 0, 1, NULL) == -3  # residual stride
    assert lib.std_gemv_ex(16, 132, 16, 128, NULL, NULL, 0, 16, 64, 2, 64, 128, 1, 1, NULL) == -5  # x row stride
    assert lib.std_gemv(NULL, 128, 16, 128, NULL, 16, 64, 1, 64, 128, 1, NULL, 0, NULL) == -1
    # the projection with the input RMSNorm: one row of at most 3584, bf16, 16-byte aligned
    assert lib.std_gemv_norm(NULL, 16, 1e-6, 16, 3584, NULL, NULL, 16, 64, 3584, 0, 1, NULL) == -1
    assert lib.std_gemv_norm(16, NULL, 1e-6, 16, 3584, NULL, NULL, 16, 64, 3584, 0, 1, NULL) == -1
    assert lib.std_gemv_norm(16, 16, 1e-6, 16, 3616, NULL, NULL, 16, 64, 3616, 0, 1, NULL) == -3
    assert lib.std_gemv_norm(16, 16, 1e-6, 16, 3584, NULL, NULL, 16, 64, 3500, 1, 1, NULL) == -3
    assert lib.std_gemv_norm(16, 16, 1e-6, 16, 100, NULL, NULL, 16, 64, 128, 0, 1, NULL) == -3
    assert lib.std_gemv_norm(16, 16, 1e-6, 16, 3584, NULL, NULL, 16, 64, 3584, 0, 0, NULL) == -2
    assert lib.std_gemv_norm(16, 24, 1e-6, 16, 3584, NULL, NULL, 16, 64, 3584, 0, 1, NULL) == -5
    assert lib.std_gemv_norm(16, 16, 1e-6, 16, 3588, NULL, NULL, 16, 64, 3584, 0, 1, NULL) == -5
    # the fused q|k|v projection: bf16 only
    qkv = [16, 3584, 1, 3584, 16, 3584, NULL, 28, 4, 128, 16, 16, 16, 128 * 1024, 1024, 16, 16, 0, 16, NULL, 1e-6]
    assert lib.std_qkv_rope_append(*qkv, 2, NULL, NULL) == -2
    assert lib.std_qkv_rope_append(*qkv, 0, NULL, NULL) == -2


def test_accept_and_append_validation():
    lib = _lib.load_library()
    # q_rows must be n_draft + has_pending
    assert lib.std_greedy_accept(16, 152064, 9, 152064, 1, 16, 9, 1, NULL, 16, NULL, 0, 16, 1 << 20, NULL) == -3
    # dense_next is required without a pending token
    assert lib.std_greedy_accept(16, 152064, 9, 152064, 1, 16, 9, 0, NULL, 16, NULL, 0, 16, 1 << 20, NULL) == -1
    assert lib.std_kv_append(16, 16, 16, 16, 4, 1, 128, 128 * 100, 128, 512, 100, NULL, 1, NULL, NULL) == -1
    assert lib.std_kv_append(16, 16, 16, 16, 4, 1, 128, 128 * 100, 128, 3, 100, 16, 1, NULL, NULL) == -5  # row stride
    assert lib.std_compact_kv(16, 16, 16, 16, 16, 4, 2000, 128, 128 * 4096, 4096, 128 * 1024, 1024, 1, NULL) == -6


def test_python_shim_rejects_cpu_tensors_before_the_library():
    q = torch.zeros(1, 28, 1, 128)
    k = torch.zeros(1, 4, 64, 128)
    with pytest.raises(RuntimeError, match="ROCm device"):
        ops.gqa_decode(q, k, k)
    with pytest.raises(RuntimeError, match="ROCm device"):
        ops.verify_attention(torch.zeros(1, 28, 10, 128), k, k)


def test_python_shim_shape_errors():
    # shape checks run before the device check only for q_len, mirroring the
    # reference's q_len assertion (triton_attention.py:89)
    with pytest.raises(ValueError, match="q_len=1"):
        ops.gqa_decode(torch.zeros(1, 28, 2, 128), torch.zeros(1, 4, 8, 128), torch.zeros(1, 4, 8, 128))
    # the reference's drop-in asserts its shapes (triton_attention.py:89, 94): the error is both kinds
    kv = torch.zeros(1, 4, 8, 128)
    for q, k in ((torch.zeros(1, 28, 2, 128), kv), (torch.zeros(1, 30, 1, 128), kv)):
        with pytest.raises(AssertionError):
            ops.fused_gqa_attention(q, k, kv)
        with pytest.raises(ValueError):
            ops.fused_gqa_attention(q, k, kv)


def test_status_error_is_runtime_error():
    with pytest.raises(RuntimeError, match="STD_E_NULL"):
        _lib.check("std_gqa_decode", -1)
