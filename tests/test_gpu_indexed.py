"""Index-addressed sparse KV on the GPU (std_gqa_decode_indexed): the draft
decode reads each head's selected prompt rows straight from the dense cache
through the index list, and its own appended rows from the sparse cache.

It must equal the decode over the physically compacted cache bit for bit
(same keys in the same order, so the same tiles and the same arithmetic),
read nothing of the sparse cache's first n_index rows (they hold NaN here),
match the attention oracle on arbitrary (unsorted) index lists, and clamp
out-of-range indices instead of reading outside the dense cache."""
import numpy as np
import pytest
import torch

from oracle import attention as ref_attn
from std_amd import ops
from tests.gpu_helpers import announce, assert_close, dev

pytestmark = pytest.mark.gpu

D, NQ, NKV = 128, 28, 4


def _dense(P, cap, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(1, NKV, P, D, generator=g).to(torch.bfloat16)
    v = torch.randn(1, NKV, P, D, generator=g).to(torch.bfloat16)
    kd = torch.full((1, NKV, cap, D), float("nan"), dtype=torch.bfloat16, device=dev())
    vd = torch.full_like(kd, float("nan"))
    kd[:, :, :P] = k.to(dev())
    vd[:, :, :P] = v.to(dev())
    return kd, vd


def _sorted_index(P, n, seed):
    g = torch.Generator().manual_seed(seed)
    rows = [torch.sort(torch.randperm(P, generator=g)[:n]).values for _ in range(NKV)]
    return torch.stack(rows).to(torch.int32)


def _caches(kd, vd, index, n_tail, cap, seed):
    """(compacted cache, tail-only cache): both hold the same n_tail appended
    rows after n_index; only the first has the gathered prompt rows."""
    n = index.shape[1]
    g = torch.Generator().manual_seed(seed)
    tail_k = torch.randn(1, NKV, n_tail, D, generator=g).to(torch.bfloat16).to(dev())
    tail_v = torch.randn(1, NKV, n_tail, D, generator=g).to(torch.bfloat16).to(dev())
    ck = torch.full((1, NKV, cap, D), float("nan"), dtype=torch.bfloat16, device=dev())
    cv = torch.full_like(ck, float("nan"))
    ops.compact_kv(kd, vd, ck, cv, index.to(dev()))
    tk, tv = torch.full_like(ck, float("nan")), torch.full_like(cv, float("nan"))
    for c_k, c_v in ((ck, cv), (tk, tv)):
        c_k[:, :, n:n + n_tail] = tail_k
        c_v[:, :, n:n + n_tail] = tail_v
    return (ck, cv), (tk, tv)


@pytest.mark.parametrize("P,n_index,n_tail", [(4096, 1024, 0), (4096, 1024, 9), (16384, 1003, 70), (4096, 17, 3),
                                              (4096, 17, 0), (4096, 16, 0), (4096, 1, 1), (4096, 64, 64),
                                              (131072, 1024, 9), (131072, 20000, 37)])
def test_indexed_equals_compacted_decode(P, n_index, n_tail):
    announce(f"indexed decode P={P} n_index={n_index} tail={n_tail}")
    cap_d, cap_s = P + 64, n_index + n_tail + 40
    kd, vd = _dense(P, cap_d, 31 + n_index)
    index = _sorted_index(P, n_index, 32 + n_tail)
    (ck, cv), (tk, tv) = _caches(kd, vd, index, n_tail, cap_s, 33)
    q = torch.randn(1, NQ, 1, D, generator=torch.Generator().manual_seed(34)).to(torch.bfloat16).to(dev())
    S = n_index + n_tail
    want = ops.gqa_decode(q, ck[:, :, :S], cv[:, :, :S])
    got = ops.gqa_decode_indexed(q, kd, vd, ops.pad_index(index.to(dev())), n_index, tk, tv, kv_len=S)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, want)


def test_indexed_device_length_equals_compacted_devlen():
    """Graph-capturable form: the key count is length[0] + 1, planned for the
    cache capacity, as attention_devlen over the compacted cache."""
    P, n_index, cap_s = 16384, 1024, 1200
    announce(f"indexed decode, device length, P={P} n_index={n_index}")
    kd, vd = _dense(P, P + 64, 41)
    index = _sorted_index(P, n_index, 42)
    padded = ops.pad_index(index.to(dev()))
    for n_tail in (1, 10, 150):
        (ck, cv), (tk, tv) = _caches(kd, vd, index, n_tail, cap_s, 43 + n_tail)
        q = torch.randn(1, NQ, 1, D, generator=torch.Generator().manual_seed(n_tail)).to(torch.bfloat16).to(dev())
        length = torch.tensor([n_index + n_tail - 1], dtype=torch.int32, device=dev())
        want = ops.attention_devlen(q, ck, cv, length, max_kv_len=cap_s)
        got = ops.gqa_decode_indexed(q, kd, vd, padded, n_index, tk, tv, length=length, max_kv_len=cap_s)
        torch.cuda.synchronize()
        assert torch.equal(got, want), n_tail


def test_indexed_unsorted_index_matches_oracle():
    """Any index list, in any order and with repeats, is the key sequence."""
    P, n_index, n_tail = 8192, 700, 12
    announce(f"indexed decode vs oracle, unsorted index, P={P}")
    g = torch.Generator().manual_seed(51)
    k = torch.randn(1, NKV, P, D, generator=g).to(torch.bfloat16)
    v = torch.randn(1, NKV, P, D, generator=g).to(torch.bfloat16)
    index = torch.randint(0, P, (NKV, n_index), generator=g, dtype=torch.int32)
    tail_k = torch.randn(1, NKV, n_tail, D, generator=g).to(torch.bfloat16)
    tail_v = torch.randn(1, NKV, n_tail, D, generator=g).to(torch.bfloat16)
    q = torch.randn(1, NQ, 1, D, generator=g).to(torch.bfloat16)
    kd, vd = k.to(dev()), v.to(dev())
    tk = torch.full((1, NKV, n_index + n_tail + 8, D), float("nan"), dtype=torch.bfloat16, device=dev())
    tv = torch.full_like(tk, float("nan"))
    tk[:, :, n_index:n_index + n_tail] = tail_k.to(dev())
    tv[:, :, n_index:n_index + n_tail] = tail_v.to(dev())
    got = ops.gqa_decode_indexed(q.to(dev()), kd, vd, ops.pad_index(index.to(dev())), n_index, tk, tv,
                                 kv_len=n_index + n_tail)
    ks = torch.stack([torch.cat([k[0, h, index[h].long()], tail_k[0, h]]) for h in range(NKV)])[None]
    vs = torch.stack([torch.cat([v[0, h, index[h].long()], tail_v[0, h]]) for h in range(NKV)])[None]
    assert_close(got, ref_attn.gqa_sdpa(q, ks, vs), torch.bfloat16)


def test_indexed_clamps_out_of_range_indices():
    P, n_index = 2048, 256
    announce("indexed decode with indices outside the dense cache (clamped)")
    kd, vd = _dense(P, P, 61)
    g = torch.Generator().manual_seed(62)
    index = torch.randint(0, P, (NKV, n_index), generator=g, dtype=torch.int32)
    bad = index.clone()
    bad[:, ::7] = P + 1000
    bad[:, 3::11] = -5
    clamped = bad.clamp(0, P - 1)
    tk = torch.full((1, NKV, n_index + 4, D), float("nan"), dtype=torch.bfloat16, device=dev())
    tv = torch.full_like(tk, float("nan"))
    q = torch.randn(1, NQ, 1, D, generator=g).to(torch.bfloat16).to(dev())
    got = ops.gqa_decode_indexed(q, kd, vd, ops.pad_index(bad.to(dev())), n_index, tk, tv, kv_len=n_index)
    want = ops.gqa_decode_indexed(q, kd, vd, ops.pad_index(clamped.to(dev())), n_index, tk, tv, kv_len=n_index)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, want)


def test_indexed_rejects_bad_arguments():
    announce("indexed decode host-side validation")
    kd, vd = _dense(256, 256, 71)
    tk = torch.zeros(1, NKV, 300, D, dtype=torch.bfloat16, device=dev())
    q = torch.zeros(1, NQ, 1, D, dtype=torch.bfloat16, device=dev())
    idx = torch.zeros(NKV, 100, dtype=torch.int32, device=dev())
    with pytest.raises(ValueError):       # rows not padded to a multiple of 16 entries
        ops.gqa_decode_indexed(q, kd, vd, idx, 100, tk, tk, kv_len=120)
    with pytest.raises(ValueError):       # key count below n_index
        ops.gqa_decode_indexed(q, kd, vd, ops.pad_index(idx), 100, tk, tk, kv_len=50)
    with pytest.raises(TypeError):
        ops.gqa_decode_indexed(q.float(), kd, vd, ops.pad_index(idx), 100, tk, tk, kv_len=120)
