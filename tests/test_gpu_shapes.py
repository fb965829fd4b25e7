"""Shape sweep of the attention entry points against the fp64 oracle: key
counts around the 64-key tile and split boundaries (1, 63-65, 127-129,
4095-4097), query rows 1-13, GQA groups 1-16, 1-8 KV heads, both dtypes, the
host-length and the device-length launches."""
import itertools

import numpy as np
import pytest
import torch

from oracle import attention as ref
from std_amd import ops
from tests.gpu_helpers import announce, assert_close, cache_buffer, dev

pytestmark = pytest.mark.gpu

CASES = []
for i, (kv, q_len, group, n_kv) in enumerate(itertools.product((1, 63, 65, 128, 129, 4095, 4097),
                                                                  (1, 2, 13), (1, 7, 16), (1, 4))):
    if q_len > kv or q_len * group > 96:
        continue
    if i % 3:                            # a deterministic third of the grid keeps the sweep short
        continue
    CASES.append((kv, q_len, group, n_kv, torch.bfloat16 if i % 2 else torch.float32))


@pytest.mark.parametrize("kv,q_len,group,n_kv,dtype", CASES)
def test_attention_shapes_match_oracle(kv, q_len, group, n_kv, dtype):
    announce(f"shape kv={kv} q_len={q_len} group={group} n_kv={n_kv} {dtype}")
    g = torch.Generator().manual_seed(kv * 131 + q_len * 17 + group * 5 + n_kv)
    n_q = group * n_kv
    q = torch.randn(1, n_q, q_len, 128, generator=g).to(dtype)
    k = torch.randn(1, n_kv, kv, 128, generator=g).to(dtype)
    v = torch.randn(1, n_kv, kv, 128, generator=g).to(dtype)
    want = ref.verify_attention(q, k, v) if q_len > 1 else ref.gqa_sdpa(q, k, v)
    kc, vc = cache_buffer(k, kv + 40), cache_buffer(v, kv + 40)      # NaN past the valid rows
    got = ops.verify_attention(q.to(dev()), kc[:, :, :kv], vc[:, :, :kv])
    assert_close(got, want, dtype)
    length = torch.tensor([kv - q_len], dtype=torch.int32, device=dev())
    got_dev = ops.attention_devlen(q.to(dev()), kc, vc, length, max_kv_len=kv + 40)
    assert_close(got_dev, want, dtype)
