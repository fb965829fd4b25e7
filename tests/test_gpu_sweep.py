"""A seeded sweep of shapes against the fp64 oracle, beside the
hand-picked cases of the other GPU tests: decode and verify launches with
random KV-head counts (1-8), group sizes (1-16), query lengths, key counts
drawn near tile (64-key) and split boundaries and far from them, and all
three element types, each through a cache view whose rows past the valid
length are NaN (a read past the range shows up in the output); the batched
decode over random problem counts; the per-KV-head top-k selection over
random visual position sets (with bit-exact duplicated keys); greedy
acceptance over random vocabularies and draft lengths. Every attention and
selection case is run twice and must repeat bit for bit. The case lists are
fixed by their seeds, so a failure names a case that reproduces."""
import random

import numpy as np
import pytest
import torch

from oracle import attention as ref
from std_amd import ops
from tests.gpu_helpers import announce, assert_close, cache_buffer, dev

pytestmark = pytest.mark.gpu

D = 128
DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _kv_len(rng: random.Random, lo: int) -> int:
    """Key counts on and next to tile and split boundaries, and anywhere."""
    pick = rng.random()
    if pick < 0.4:
        base = 64 * rng.randint(1, 160)
        return max(lo, base + rng.choice((-1, 0, 1)))
    if pick < 0.6:
        return max(lo, rng.randint(lo, 96))
    return rng.randint(lo, 12000)


def _cases(seed: int, n: int):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        n_kv = rng.choice((1, 2, 4, 8))
        group = rng.randint(1, 16)
        verify = rng.random() < 0.5
        q_len = rng.randint(2, min(16, 96 // group)) if verify and 96 // group >= 2 else 1
        kv = _kv_len(rng, q_len)
        dtype = rng.choice(DTYPES)
        out.append((n_kv, group, q_len, kv, dtype))
    return out


CASES = _cases(20260, 30)


@pytest.mark.parametrize("n_kv,group,q_len,kv,dtype", CASES,
                         ids=[f"kv{a}-g{b}-q{c}-s{d}-{str(e)[6:]}" for a, b, c, d, e in CASES])
def test_attention_sweep_matches_oracle(n_kv, group, q_len, kv, dtype):
    announce(f"sweep attention n_kv={n_kv} group={group} q_len={q_len} kv={kv} {dtype}")
    g = torch.Generator().manual_seed(n_kv * 100000 + group * 1000 + q_len * 37 + kv)
    n_q = n_kv * group
    q = torch.randn(1, n_q, q_len, D, generator=g).to(dtype)
    k = torch.randn(1, n_kv, kv, D, generator=g).to(dtype)
    v = torch.randn(1, n_kv, kv, D, generator=g).to(dtype)
    kc, vc = cache_buffer(k, kv + 24), cache_buffer(v, kv + 24)
    if q_len == 1:
        got = ops.gqa_decode(q.to(dev()), kc[:, :, :kv], vc[:, :, :kv])
        want = ref.gqa_sdpa(q, k, v)
        again = ops.gqa_decode(q.to(dev()), kc[:, :, :kv], vc[:, :, :kv])
    else:
        got = ops.verify_attention(q.to(dev()), kc[:, :, :kv], vc[:, :, :kv])
        want = ref.verify_attention(q, k, v)
        again = ops.verify_attention(q.to(dev()), kc[:, :, :kv], vc[:, :, :kv])
    assert_close(got, want, dtype)
    torch.cuda.synchronize()
    assert torch.equal(got, again), "repeat call differs"


BATCH_CASES = [(b, n_kv, group, kv, dtype) for (b, (n_kv, group, _, kv, dtype)) in
               zip(random.Random(7).choices(range(1, 41), k=12), _cases(777, 12))]


@pytest.mark.parametrize("n_batch,n_kv,group,kv,dtype", BATCH_CASES,
                         ids=[f"b{a}-kv{b}-g{c}-s{d}-{str(e)[6:]}" for a, b, c, d, e in BATCH_CASES])
def test_batched_decode_sweep_matches_oracle(n_batch, n_kv, group, kv, dtype):
    """n_batch independent decodes in one launch (the problems split or
    streamed whole by the planner), each against the oracle."""
    kv = min(kv, 4000)
    announce(f"sweep batched decode n_batch={n_batch} n_kv={n_kv} group={group} kv={kv} {dtype}")
    g = torch.Generator().manual_seed(n_batch * 7919 + n_kv * 131 + group * 17 + kv)
    n_q = n_kv * group
    q = torch.randn(n_batch, 1, n_q, 1, D, generator=g).to(dtype)
    k = torch.randn(n_batch, 1, n_kv, kv, D, generator=g).to(dtype)
    v = torch.randn(n_batch, 1, n_kv, kv, D, generator=g).to(dtype)
    kb = torch.full((n_batch, 1, n_kv, kv + 16, D), float("nan"), dtype=dtype, device=dev())
    vb = torch.full_like(kb, float("nan"))
    kb[..., :kv, :] = k.to(dev())
    vb[..., :kv, :] = v.to(dev())
    got = ops.gqa_decode_batched(q.to(dev()), kb[..., :kv, :], vb[..., :kv, :])
    again = ops.gqa_decode_batched(q.to(dev()), kb[..., :kv, :], vb[..., :kv, :])
    want = np.stack([ref.gqa_sdpa(q[b], k[b], v[b]) for b in range(n_batch)])
    assert_close(got, want, dtype)
    torch.cuda.synchronize()
    assert torch.equal(got, again), "repeat call differs"


def _select_cases(seed: int, n: int):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        n_kv = rng.choice((1, 2, 4, 8))
        group = rng.randint(1, min(16, 64 // n_kv))
        T = rng.randint(1, 64)
        text_start = rng.randint(1, 6000)
        dup = rng.random() < 0.5
        dtype = rng.choice(DTYPES)
        out.append((n_kv, group, T, text_start, dup, dtype, rng.randint(0, 2 ** 31)))
    return out


SELECT_CASES = _select_cases(4096, 12)


@pytest.mark.parametrize("n_kv,group,T,text_start,dup,dtype,seed", SELECT_CASES,
                         ids=[f"kv{a}-g{b}-T{c}-P{d}-dup{int(e)}-{str(f)[6:]}" for a, b, c, d, e, f, _ in
                              SELECT_CASES])
def test_selection_sweep_matches_oracle(n_kv, group, T, text_start, dup, dtype, seed):
    """Per-KV-head top-k over a random visual position set (gaps anywhere,
    k from 1 to all of them): fp64 column scores to round-off and the
    selected positions bit for bit against the oracle, with bit-exact
    duplicated key rows in half the cases (ties go to the lowest position)."""
    from oracle import selection as sel_ref
    announce(f"sweep selection n_kv={n_kv} group={group} T={T} text_start={text_start} dup={dup} {dtype}")
    rng = np.random.default_rng(seed)
    P = text_start + T
    n_q = n_kv * group
    q = torch.from_numpy(rng.standard_normal((1, n_q, T, D))).to(dtype)
    kf = rng.standard_normal((1, n_kv, P, D)) * rng.lognormal(0.0, 0.5, (1, n_kv, P, 1))
    if dup:                                          # copy some rows onto others, bit for bit
        src = rng.integers(0, P, size=max(1, P // 20))
        dst = rng.integers(0, P, size=src.size)
        kf[:, :, dst] = kf[:, :, src]
    k = torch.from_numpy(kf).to(dtype)
    keep = rng.random(text_start) < rng.uniform(0.3, 1.0)
    keep[rng.integers(0, text_start)] = True         # at least one visual position
    vis = np.flatnonzero(keep).astype(np.int32)
    k_sel = int(rng.integers(1, vis.size + 1))
    kb = cache_buffer(k, P + 24)
    topk, scores = ops.select_topk(q.to(dev()), kb, text_start, torch.from_numpy(vis).to(dev()), k_sel,
                                   return_scores=True)
    again = ops.select_topk(q.to(dev()), kb, text_start, torch.from_numpy(vis).to(dev()), k_sel)
    torch.cuda.synchronize()
    want_scores = sel_ref.selection_scores(q, k, text_start)
    np.testing.assert_allclose(scores.cpu().numpy(), want_scores, rtol=1e-11, atol=1e-300)
    np.testing.assert_array_equal(topk.cpu().numpy(), sel_ref.topk_positions(want_scores, vis, k_sel))
    assert torch.equal(topk, again), "repeat call differs"


def _accept_cases(seed: int, n: int):
    rng = random.Random(seed)
    return [(rng.choice((2, 7, 31, 1000, 4097, 32000, 152064, 151936)), rng.randint(1, 16), rng.random() < 0.5,
             rng.choice(DTYPES), rng.random() < 0.4, rng.randint(0, 2 ** 31)) for _ in range(n)]


ACCEPT_CASES = _accept_cases(99, 16)


@pytest.mark.parametrize("vocab,n_draft,has_pending,dtype,plant,seed", ACCEPT_CASES,
                         ids=[f"V{a}-n{b}-p{int(c)}-{str(d)[6:]}-plant{int(e)}" for a, b, c, d, e, _ in ACCEPT_CASES])
def test_accept_sweep_matches_oracle(vocab, n_draft, has_pending, dtype, plant, seed):
    """Greedy acceptance over random vocabulary sizes and draft lengths, with
    every acceptance length reachable: the accepted length, the bonus token,
    every row's prediction (first maximum; NaN wins; planted exact ties
    between a row's maximum and a later or earlier index) and the rolled-back
    cache lengths, against the oracle."""
    from oracle import accept as acc_ref
    rng = np.random.default_rng(seed)
    rows = n_draft + (1 if has_pending else 0)
    x = rng.standard_normal((rows, vocab)).astype(np.float32)
    if plant:
        for r in range(rows):
            j = int(np.argmax(x[r]))
            x[r, int(rng.integers(0, vocab))] = x[r, j]          # an exact tie with the maximum
        r = int(rng.integers(0, rows))
        x[r, int(rng.integers(0, vocab))] = np.nan               # NaN counts as the maximum
    logits = torch.from_numpy(x).to(dtype)                        # ties survive the rounding
    dense_next = int(rng.integers(0, vocab))
    preds = acc_ref.verify_predictions(logits, has_pending, dense_next)
    a_target = int(rng.integers(0, n_draft + 1))
    draft = [preds[i] for i in range(a_target)]
    if a_target < n_draft:
        draft.append((preds[a_target] + 1) % vocab)               # the first rejection
        draft += [int(t) for t in rng.integers(0, vocab, size=n_draft - a_target - 1)]
    exp_a, exp_bonus, exp_preds = acc_ref.verify_accept(logits, draft, has_pending, dense_next)
    assert exp_a == a_target
    announce(f"sweep accept V={vocab} n_draft={n_draft} pending={has_pending} {dtype} plant={plant} a={exp_a}")
    lens = torch.tensor([70000, 1500], dtype=torch.int32, device=dev())
    out = ops.greedy_accept(logits.to(dev()), torch.tensor(draft, dtype=torch.int32, device=dev()), has_pending,
                            torch.tensor([dense_next], dtype=torch.int32, device=dev()), lens)
    torch.cuda.synchronize()
    out = out.cpu().tolist()
    assert out[0] == exp_a and out[1] == exp_bonus and out[2:] == exp_preds
    assert lens.cpu().tolist() == [70000 - (n_draft - exp_a), 1500 - (n_draft - exp_a)]
