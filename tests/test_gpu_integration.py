"""The reference-side binding snippets of the repository's integration guide,
run as written: the `hip`
branch of _sparse_aware_attention_forward (section 3, replacing
src/std_repro/std_qwen25vl.py:395-431) and the verify patch of
Qwen2_5_VLSdpaAttention.forward (section 4, replacing
src/specvlm/models/modeling_qwen2_5_vl.py:1057-1132) are read from the
document's code blocks and executed on KVCache objects with CPU lengths (the
reference's cache semantics), for a sequence of draft and verify steps, each
held to the attention oracle over the cache contents."""
import os
import re
import types

import numpy as np
import pytest
import torch

from oracle import attention as ref_attn
from std_amd import ops
from std_amd.kv_cache import KVCache
from tests.gpu_helpers import TOL, announce, dev

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _snippet(section: str, marker: str) -> str:
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    body = text.split("\n## " + section, 1)[1].split("\n## ", 1)[0]
    blocks = re.findall(r"```python\n(.*?)```", body, re.S)
    found = [b for b in blocks if marker in b]
    assert len(found) == 1, f"INTEGRATION.md section {section!r}: no single block with {marker!r}"
    return found[0]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_integration_snippets_on_kvcache_with_cpu_lengths(dtype):
    draft_src = _snippet("3. Draft attention", 'controller.sparse_attn_mode == "hip"')
    verify_src = _snippet("4. Dense verify attention", "verify_attention_append")
    n_q, n_kv, D, P, cap = 28, 4, 128, 2000, 2100
    g = torch.Generator().manual_seed(91)
    data = torch.empty(2, 1, n_kv, cap, D, dtype=dtype, device=dev())
    lengths = torch.zeros(2, dtype=torch.int64)                       # CPU, as kv_cache.py:131-138
    past_key_value = (KVCache(data[0], lengths[0]), KVCache(data[1], lengths[1]))
    k_all = torch.randn(1, n_kv, P, D, generator=g).to(dtype)
    v_all = torch.randn(1, n_kv, P, D, generator=g).to(dtype)
    past_key_value[0].cat(k_all.to(dev()))                             # the prompt prefill
    past_key_value[1].cat(v_all.to(dev()))
    controller = types.SimpleNamespace(sparse_attn_mode="hip")
    steps = [1, 1, 1, 10, 1, 1, 5, 1]                                 # draft steps and verify chunks
    for step, q_len in enumerate(steps):
        q = torch.randn(1, n_q, q_len, D, generator=g).to(dtype)
        kn = torch.randn(1, n_kv, q_len, D, generator=g).to(dtype)
        vn = torch.randn(1, n_kv, q_len, D, generator=g).to(dtype)
        pos = past_key_value[0].length
        announce(f"integration snippet step {step}: q_len={q_len} at length {pos}, {dtype}")
        ns = {"controller": controller, "past_key_value": past_key_value, "query_states": q.to(dev()),
              "key_states": kn.to(dev()), "value_states": vn.to(dev()), "q_len": q_len, "std_ops": ops}
        exec(draft_src if q_len == 1 else verify_src, ns)
        out = ns["attn_output"]
        torch.cuda.synchronize()
        k_all = torch.cat([k_all, kn], 2)
        v_all = torch.cat([v_all, vn], 2)
        assert past_key_value[0].length == past_key_value[1].length == pos + q_len
        assert torch.equal(data[0, :, :, :pos + q_len].cpu(), k_all) and torch.equal(data[1, :, :, :pos + q_len].cpu(),
                                                                                      v_all)
        want = ref_attn.gqa_sdpa(q, k_all, v_all) if q_len == 1 else ref_attn.verify_attention(q, k_all, v_all)
        got = out.float().cpu().numpy()
        assert got.shape == want.shape and np.isfinite(got).all()
        np.testing.assert_allclose(got, want, **TOL[dtype])
