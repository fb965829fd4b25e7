"""The split-partial merge in both of its forms: one wave per row (at most 32
splits per KV head; its loads past the last split fall outside a bounded
buffer resource) and one 256-thread block per row (more splits). Decodes and
verifies at key counts whose split plans cover every wave-merge instance
(4, 8, 9, 12 and 16 splits per half-wave) and the block form, against the
fp64 oracle, with NaN past the valid cache rows; the collector verify equals
the plain verify bit for bit in the wave form too."""
import numpy as np
import pytest
import torch

from oracle import attention as ref
from oracle import collector as ref_coll
from std_amd import _lib, ops
from tests.gpu_helpers import announce, assert_close, cache_buffer, dev

pytestmark = pytest.mark.gpu

N_KV, GROUP = 4, 7


def _wave_j(n_split):
    """The wave merge's splits per half-wave (the library's merge_j), None for
    the block form."""
    if n_split <= 1:
        return "unsplit"
    if n_split > 32:
        return None
    return 4 if n_split <= 8 else 8 if n_split <= 16 else 9 if n_split <= 18 else 12 if n_split <= 24 else 16


def _splits(rows, kv, dtype):
    code = {torch.bfloat16: _lib.STD_BF16, torch.float16: _lib.STD_F16, torch.float32: _lib.STD_F32}[dtype]
    return _lib.load_library().std_attn_split_count(N_KV, rows, kv, code)


DECODE_KV = (130, 500, 1000, 1030, 1090, 1500, 2000, 4100, 9000)


def test_decode_lengths_cover_every_merge_form():
    forms = {_wave_j(_splits(GROUP, kv, torch.bfloat16)) for kv in DECODE_KV}
    assert {4, 8, 9, 12, 16, None} <= forms, forms


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("kv", DECODE_KV)
def test_decode_merge_forms_match_oracle(kv, dtype):
    n_split = _splits(GROUP, kv, dtype)
    announce(f"merge decode kv={kv} {dtype} splits={n_split} form={_wave_j(n_split)}")
    g = torch.Generator().manual_seed(9100 + kv)
    q = torch.randn(1, N_KV * GROUP, 1, 128, generator=g).to(dtype)
    k = torch.randn(1, N_KV, kv, 128, generator=g).to(dtype)
    v = torch.randn(1, N_KV, kv, 128, generator=g).to(dtype)
    kc, vc = cache_buffer(k, kv + 40), cache_buffer(v, kv + 40)
    got = ops.gqa_decode(q.to(dev()), kc[:, :, :kv], vc[:, :, :kv])
    assert_close(got, ref.gqa_sdpa(q, k, v), dtype)
    again = ops.gqa_decode(q.to(dev()), kc[:, :, :kv], vc[:, :, :kv])
    assert torch.equal(got, again), "merge not deterministic"


@pytest.mark.parametrize("kv,q_len", [(266, 10), (1034, 10), (2058, 10), (4106, 10)])
def test_verify_merge_forms_match_oracle_and_collector(kv, q_len):
    """Verify (70 rows per KV head) in the wave and block merge forms, and the
    collector verify over the same launch: attention outputs equal bit for bit,
    scores against the oracle."""
    dtype = torch.bfloat16
    n_split = _splits(GROUP * q_len, kv, dtype)
    announce(f"merge verify kv={kv} splits={n_split} form={_wave_j(n_split)}")
    g = torch.Generator().manual_seed(9200 + kv)
    q = torch.randn(1, N_KV * GROUP, q_len, 128, generator=g).to(dtype)
    k = torch.randn(1, N_KV, kv, 128, generator=g).to(dtype)
    v = torch.randn(1, N_KV, kv, 128, generator=g).to(dtype)
    kc, vc = cache_buffer(k, kv + 40), cache_buffer(v, kv + 40)
    got = ops.verify_attention(q.to(dev()), kc[:, :, :kv], vc[:, :, :kv])
    assert_close(got, ref.verify_attention(q, k, v), dtype)
    vis_end = kv - q_len - 16
    out_c, scores = ops.verify_attention_collect(q.to(dev()), kc[:, :, :kv], vc[:, :, :kv], 0, vis_end, kv_len=kv)
    assert torch.equal(out_c, got), "collector verify differs from the plain verify"
    want = ref_coll.verification_scores(q, k, np.arange(vis_end))
    np.testing.assert_allclose(scores.double().cpu().numpy(), want, rtol=2e-4, atol=1e-9)
