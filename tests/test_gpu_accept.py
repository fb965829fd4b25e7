"""GPU parity of greedy acceptance (accepted length, bonus, predictions bit-exact),
device rollback of the cache lengths, and KV append at a device length."""
import numpy as np
import pytest
import torch

from oracle import accept as ref
from std_amd import ops
from std_amd.workloads import WORKLOADS, make_logits
from tests.gpu_helpers import announce, dev

pytestmark = pytest.mark.gpu


def _draft_with_accept(preds, a, vocab, n_draft):
    draft = [int(p) for p in preds[:n_draft]]
    if a < n_draft:
        draft[a] = (preds[a] + 1) % vocab
    return draft


@pytest.mark.parametrize("wname", ["c1", "c2"])
@pytest.mark.parametrize("has_pending", [True, False])
@pytest.mark.parametrize("a", [0, 1, 4, 9])
def test_accept_matches_oracle(wname, has_pending, a):
    w = WORKLOADS[wname]
    n_draft = w.gamma
    rows = n_draft + (1 if has_pending else 0)
    logits = make_logits(w, rows, seed=w.seed_base + 17 + a)
    dense_next = 1234
    preds = ref.verify_predictions(logits, has_pending, dense_next)
    draft = _draft_with_accept(preds, a, w.vocab, n_draft)
    exp_a, exp_bonus, exp_preds = ref.verify_accept(logits, draft, has_pending, dense_next)
    assert exp_a == a
    announce(f"accept {wname} pending={has_pending} a={a}")
    lens = torch.tensor([5000, 1100], dtype=torch.int32, device=dev())
    out = ops.greedy_accept(logits.to(dev()), torch.tensor(draft, dtype=torch.int32, device=dev()), has_pending,
                            torch.tensor([dense_next], dtype=torch.int32, device=dev()), lens)
    torch.cuda.synchronize()
    out = out.cpu().tolist()
    assert out[0] == exp_a and out[1] == exp_bonus and out[2:] == exp_preds
    assert lens.cpu().tolist() == [5000 - (n_draft - a), 1100 - (n_draft - a)]


def test_accept_ties_nan_and_signed_zero():
    vocab = 152064
    logits = torch.randn(4, vocab, generator=torch.Generator().manual_seed(3))
    logits[0, 100] = 50.0
    logits[0, 90000] = 50.0            # duplicated row max at a higher index -> 100
    logits[1, 7] = float("nan")
    logits[1, 3] = float("nan")        # first NaN wins -> 3
    logits[2] = -1.0
    logits[2, 5] = -0.0
    logits[2, 4] = 0.0                 # -0 == +0 -> 4
    logits[3] = float("-inf")          # all equal -> 0
    exp = [ref.argmax_first(logits[r]) for r in range(4)]
    assert exp == [100, 3, 4, 0]
    for dtype in (torch.float32, torch.bfloat16):
        announce(f"accept argmax edge cases {dtype}")
        x = logits.to(dtype)
        exp = [ref.argmax_first(x[r]) for r in range(4)]
        draft = torch.tensor(exp[:3], dtype=torch.int32, device=dev())
        out = ops.greedy_accept(x.to(dev()), draft, True).cpu().tolist()
        torch.cuda.synchronize()
        assert out[2:] == exp and out[0] == 3 and out[1] == exp[3]


def test_accept_small_vocab_and_strided_rows():
    gen = torch.Generator().manual_seed(9)
    base = torch.randn(3, 1000, generator=gen)
    x = base[:, :777]                 # row stride 1000 > vocab 777
    preds = [ref.argmax_first(x[r]) for r in range(3)]
    announce("accept strided rows vocab=777")
    out = ops.greedy_accept(base.to(dev())[:, :777],
                            torch.tensor([preds[0], preds[1]], dtype=torch.int32, device=dev()), True)
    torch.cuda.synchronize()
    assert out.cpu().tolist() == [2, preds[2]] + preds


def test_kv_append_at_device_length_and_len_add():
    w = WORKLOADS["c2"]
    cap, D = 64, w.head_dim
    ck = torch.zeros(1, w.n_kv, cap, D, dtype=w.dtype, device=dev())
    cv = torch.zeros_like(ck)
    gen = torch.Generator().manual_seed(5)
    # projection-shaped new rows: [1, rows, n_kv, D] viewed as [1, n_kv, rows, D]
    proj_k = torch.randn(1, 3, w.n_kv, D, generator=gen).to(w.dtype).to(dev())
    proj_v = torch.randn(1, 3, w.n_kv, D, generator=gen).to(w.dtype).to(dev())
    nk, nv = proj_k.transpose(1, 2), proj_v.transpose(1, 2)
    length = torch.tensor([10, 0], dtype=torch.int32, device=dev())
    announce("kv_append strided new rows at device length 10, then len_add")
    ops.kv_append(ck, cv, nk, nv, length)
    ops.len_add(length[:1], 3)
    ops.kv_append(ck, cv, nk[:, :, :1], nv[:, :, :1], length)
    torch.cuda.synchronize()
    assert length.cpu().tolist() == [13, 0]
    assert torch.equal(ck[:, :, 10:13].cpu(), nk.cpu())
    assert torch.equal(cv[:, :, 10:13].cpu(), nv.cpu())
    assert torch.equal(ck[:, :, 13].cpu(), nk[:, :, 0].cpu())
    assert torch.count_nonzero(ck[:, :, :10]) == 0 and torch.count_nonzero(ck[:, :, 14:]) == 0


def test_kv_append_past_capacity_is_skipped_and_reported():
    """Rows that would land at or past the capacity are not written (the
    memory after the cache is left alone) and mark the device status word;
    an append that fits leaves the word as it was."""
    buf = torch.full((1, 2, 12, 128), -7.0, device=dev())
    buf_v = torch.full_like(buf, -7.0)
    ck, cv = buf[:, :, :8], buf_v[:, :, :8]              # rows 8..11 of the buffers lie past the caches' capacity
    nk = torch.ones(1, 2, 3, 128, device=dev())
    status = torch.zeros(1, dtype=torch.int32, device=dev())
    announce("kv_append past capacity, status word")
    ops.kv_append(ck, cv, nk[:, :, :2], nk[:, :, :2], torch.tensor([0], dtype=torch.int32, device=dev()),
                  status=status)
    torch.cuda.synchronize()
    assert int(status) == 0
    ops.kv_append(ck, cv, nk, nk, torch.tensor([6], dtype=torch.int32, device=dev()), status=status)
    torch.cuda.synchronize()
    assert int(status) == ops.STATUS_CACHE_OVERFLOW
    assert torch.all(ck[:, :, 6:] == 1) and torch.all(ck[:, :, 2:6] == -7) and torch.all(ck[:, :, :2] == 1)
    assert torch.all(buf[:, :, 8:] == -7) and torch.all(buf_v[:, :, 8:] == -7), "an append wrote past the cache"
    status.zero_()
    ops.kv_append(ck, cv, nk, nk, torch.tensor([-2], dtype=torch.int32, device=dev()), status=status)
    torch.cuda.synchronize()
    assert int(status) == ops.STATUS_CACHE_OVERFLOW


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_argmax_rows_matches_oracle_with_ties_and_nan(dtype):
    announce(f"argmax_rows {dtype} 12 x 152064 with planted ties and a NaN")
    g = torch.Generator().manual_seed(31)
    logits = torch.randn(12, 152064, generator=g).to(dtype)
    logits[3, 5000] = logits[3, 140000] = 50.0            # tie: the lower index wins
    logits[7, 100] = float("nan")                           # NaN counts as the maximum
    logits[9] = 0.0
    logits[9, 77] = -0.0                                    # all equal: index 0
    want = [int(p) for p in ref.verify_predictions(logits.float(), True)]
    got = ops.argmax_rows(logits.to(dev()))
    torch.cuda.synchronize()
    assert got.dtype == torch.long and got.cpu().tolist() == want
    assert want[3] == 5000 and want[7] == 100 and want[9] == 0


@pytest.mark.parametrize("hidden", [3584, 100, 4096, 4097, 9000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rms_norm_matches_torch_formula(dtype, hidden):
    """Row widths of one load batch (up to 16 x 256 elements: 3584, 100,
    4096) and of several (4097, 9000)."""
    announce(f"rms_norm {dtype} 33 x {hidden}")
    g = torch.Generator().manual_seed(32)
    x = (torch.randn(1, 33, hidden, generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(dtype)
    got = ops.rms_norm(x.to(dev()), w.to(dev()), 1e-6).cpu()
    xf = x.float()
    want = w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(dtype)   # modeling_qwen2_5_vl.py:192-197
    if dtype == torch.bfloat16:                             # the fp32 sums differ in order only
        diff = (got.float() - want.float()).abs()
        assert (diff <= want.float().abs() * 2 ** -7).all() and (diff == 0).float().mean() > 0.99
    else:
        torch.testing.assert_close(got, want, rtol=2e-6, atol=1e-6)
