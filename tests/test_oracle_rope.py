"""The rotary-embedding oracle pinned on the CPU: closed forms (position 0 is
the identity), the rotation invariants (pair norms kept, scores depend only
on the relative position) and torch's own CPU evaluation of the reference
formula (modeling_qwen2_5_vl.py:656-671, 690-732) in bf16, fp16 and fp32."""
import numpy as np
import torch

from oracle import rope

D, THETA = 128, 1e6


def _x(n, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, D, generator=g)
    if dtype == "bf16":
        return x.to(torch.bfloat16).float().numpy()
    if dtype == "fp16":
        return x.to(torch.float16).float().numpy()
    return x.numpy()


def test_position_zero_is_identity():
    inv = rope.inv_freq(THETA, D)
    for dtype in ("bf16", "fp16", "fp32"):
        x = _x(5, 1, dtype)
        cos, sin = rope.cos_sin(np.zeros(5, dtype=np.int64), inv, dtype)
        assert (cos == 1).all() and (sin == 0).all()
        np.testing.assert_array_equal(rope.apply_rope(x, cos, sin, dtype), x)


def test_pair_norms_are_kept():
    inv = rope.inv_freq(THETA, D)
    x = _x(64, 2, "fp32")
    pos = np.arange(0, 131072, 2048)
    cos, sin = rope.cos_sin(pos, inv, "fp32")
    y = rope.apply_rope(x, cos, sin, "fp32").astype(np.float64)
    xd = x.astype(np.float64)
    nx = xd[:, :64] ** 2 + xd[:, 64:] ** 2
    ny = y[:, :64] ** 2 + y[:, 64:] ** 2
    np.testing.assert_allclose(ny, nx, rtol=2e-6, atol=1e-9)


def test_scores_depend_on_relative_position_only():
    inv = rope.inv_freq(THETA, D)
    q, k = _x(1, 3, "fp32"), _x(1, 4, "fp32")

    def score(pq, pk):
        cq, sq = rope.cos_sin(np.array([pq]), inv, "fp32")
        ck, sk = rope.cos_sin(np.array([pk]), inv, "fp32")
        a = rope.apply_rope(q, cq, sq, "fp32").astype(np.float64)
        b = rope.apply_rope(k, ck, sk, "fp32").astype(np.float64)
        return float((a * b).sum())

    base = score(37, 5)
    for shift in (1, 100, 4096):
        assert abs(score(37 + shift, 5 + shift) - base) < 2e-3 * max(1.0, abs(base))
    assert abs(score(40, 5) - base) > 1e-3        # a different offset gives a different score


def test_matches_torch_cpu_evaluation():
    """torch's CPU kernels evaluate the reference expression with their own
    cos/sin; the oracle agrees bit for bit except where the two cos/sin
    evaluations round differently: never in bf16 or fp16 for these
    positions; in fp32 torch's cos/sin differ from the correctly rounded value by one ulp
    for ~3 % of angles, which moves a result by at most a few fp32 ulps of
    the products (|x| < 5 here)."""
    inv = rope.inv_freq(THETA, D)
    inv_t = torch.from_numpy(inv)
    pos = np.array([0, 1, 7, 1023, 4096, 32767, 65537, 131071, 131081], dtype=np.int64)
    for dtype, tdt in (("bf16", torch.bfloat16), ("fp16", torch.float16), ("fp32", torch.float32)):
        x = _x(len(pos), 5, dtype)
        cos, sin = rope.cos_sin(pos, inv, dtype)
        got = rope.apply_rope(x, cos, sin, dtype)
        freqs = torch.from_numpy(pos).float()[:, None] * inv_t[None, :]
        emb = torch.cat([freqs, freqs], dim=-1)
        tc, ts = emb.cos().to(tdt), emb.sin().to(tdt)
        xt = torch.from_numpy(x).to(tdt)
        rot = torch.cat([-xt[:, 64:], xt[:, :64]], dim=-1)
        ref = ((xt * tc) + (rot * ts)).float().numpy()
        diff = np.abs(got - ref)
        if dtype in ("bf16", "fp16"):
            np.testing.assert_array_equal(got, ref)
        else:
            assert diff.max() <= 1e-6 and (diff == 0).mean() > 0.9
