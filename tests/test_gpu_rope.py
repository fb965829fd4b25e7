"""Device-length decode-step glue on the GPU: the fused rotary embedding +
K/V append (std_rope_append) against the rope oracle and torch's own
evaluation, and the device-length attention (std_attn_devlen) against the
host-length kernels and the attention oracle."""
import numpy as np
import pytest
import torch

from oracle import attention as ref_attn
from oracle import rope as ref_rope
from std_amd import _lib, ops
from tests.gpu_helpers import announce, assert_close, dev

pytestmark = pytest.mark.gpu

D, NQ, NKV = 128, 28, 4


def _qkv(n, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, n, (NQ + 2 * NKV) * D, generator=g).to(dtype)


def _scalar(v):
    return torch.tensor([v], dtype=torch.int32, device=dev())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_append_matches_oracle(dtype):
    n, cap, length, pos, off = 10, 300, 137, 131000, 3
    announce(f"rope_append {dtype} n={n} len={length} pos={pos}+{off}")
    qkv = _qkv(n, dtype, 11)
    kc = torch.full((1, NKV, cap, D), float("nan"), dtype=dtype, device=dev())
    vc = torch.full_like(kc, float("nan"))
    inv = ref_rope.inv_freq(1e6, D)
    q = ops.rope_append(qkv.to(dev()), NQ, kc, vc, _scalar(length), _scalar(pos), torch.from_numpy(inv).to(dev()),
                        pos_offset=off)
    torch.cuda.synchronize()
    name = "bf16" if dtype == torch.bfloat16 else "fp32"
    x = qkv[0].float().numpy().reshape(n, NQ + 2 * NKV, D)
    cos, sin = ref_rope.cos_sin(pos + off + np.arange(n), inv, name)
    want_q = ref_rope.apply_rope(x[:, :NQ].transpose(1, 0, 2), cos, sin, name)          # [NQ, n, D]
    want_k = ref_rope.apply_rope(x[:, NQ:NQ + NKV].transpose(1, 0, 2), cos, sin, name)  # [NKV, n, D]
    got_q = q[0].float().cpu().numpy()
    got_k = kc[0, :, length:length + n].float().cpu().numpy()
    for got, want in ((got_q, want_q), (got_k, want_k)):
        diff = np.abs(got - want)
        if dtype == torch.bfloat16:   # one bf16 ulp at most, where the two cos/sin round differently
            assert (diff <= np.spacing(np.abs(want)) * 65536).all() and (diff == 0).mean() > 0.995
        else:   # fp32 cos/sin of angles up to 1.3e5 rad: the device's and the oracle's differ by an ulp often
            assert diff.max() <= 1e-6
    np.testing.assert_array_equal(vc[0, :, length:length + n].float().cpu().numpy(),
                                  x[:, NQ + NKV:].transpose(1, 0, 2))
    untouched = torch.cat([kc[0, :, :length], kc[0, :, length + n:], vc[0, :, :length], vc[0, :, length + n:]], 1)
    assert torch.isnan(untouched).all()


def test_rope_append_matches_torch_on_device_and_skips_rows_past_capacity():
    n, cap = 6, 64
    announce("rope_append vs torch formula on the device; capacity edge")
    dtype = torch.bfloat16
    qkv = _qkv(n, dtype, 12).to(dev())
    kc = torch.zeros(1, NKV, cap, D, dtype=dtype, device=dev())
    vc = torch.zeros_like(kc)
    inv = torch.from_numpy(ref_rope.inv_freq(1e6, D)).to(dev())
    length, pos = cap - 4, 77777
    q = ops.rope_append(qkv, NQ, kc, vc, _scalar(length), _scalar(pos), inv)
    freqs = (pos + torch.arange(n, device=dev())).float()[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], -1)
    c, s = emb.cos().to(dtype), emb.sin().to(dtype)
    x = qkv[0].view(n, NQ + 2 * NKV, D).transpose(0, 1)
    rot = torch.cat([-x[..., 64:], x[..., :64]], -1)
    want = (x * c) + (rot * s)
    diff = (q[0].float() - want[:NQ].float()).abs()
    assert (diff == 0).float().mean() > 0.995
    assert (diff <= want[:NQ].float().abs() * 2 ** -7 + 1e-30).all()
    torch.testing.assert_close(kc[0, :, length:], want[NQ:NQ + NKV, :4], rtol=2 ** -7, atol=0)
    assert (kc[0, :, :length] == 0).all()           # rows 4, 5 fall past the capacity: not written


@pytest.mark.parametrize("dtype,q_len,kv,cap", [(torch.bfloat16, 10, 4106, 4500), (torch.float32, 10, 8202, 8400),
                                                 (torch.bfloat16, 1, 131072, 131200)])
def test_attention_devlen_equals_host_length_kernel(dtype, q_len, kv, cap):
    """With >= 64 tiles the split plan is the same at kv and at cap, so the
    device-length launch reproduces the host-length launch bit for bit."""
    announce(f"attention_devlen {dtype} q_len={q_len} kv={kv} cap={cap}")
    g = torch.Generator(device=dev()).manual_seed(21)
    k = torch.randn(1, NKV, cap, D, generator=g, device=dev()).to(dtype)
    v = torch.randn(1, NKV, cap, D, generator=g, device=dev()).to(dtype)
    q = torch.randn(1, NQ, q_len, D, generator=g, device=dev()).to(dtype)
    got = ops.attention_devlen(q, k, v, _scalar(kv - q_len), max_kv_len=cap)
    want = ops.verify_attention(q, k[:, :, :kv], v[:, :, :kv])
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype,cap,kv", [(torch.bfloat16, 1163, 1034), (torch.float32, 1163, 1034),
                                          (torch.bfloat16, 300, 200), (torch.bfloat16, 300, 37)])
def test_attention_devlen_small_cache_matches_oracle(dtype, cap, kv):
    """A decode planned for the cache capacity reads only the device length's
    keys; at cap = 300 (five tiles) the bf16 decode streams unsplit."""
    announce(f"attention_devlen decode {dtype} kv={kv} planned for {cap}")
    g = torch.Generator().manual_seed(22 + kv)
    k = torch.randn(1, NKV, cap, D, generator=g).to(dtype)
    v = torch.randn(1, NKV, cap, D, generator=g).to(dtype)
    q = torch.randn(1, NQ, 1, D, generator=g).to(dtype)
    kd, vd = k.to(dev()), v.to(dev())
    kd[:, :, kv:] = float("nan")                    # rows past the device length must never be read
    vd[:, :, kv:] = float("nan")
    got = ops.attention_devlen(q.to(dev()), kd, vd, _scalar(kv - 1), max_kv_len=cap)
    assert_close(got, ref_attn.gqa_sdpa(q, k[:, :, :kv], v[:, :, :kv]), dtype)
    for q_len in (3, 10):
        qv = torch.randn(1, NQ, q_len, D, generator=g).to(dtype)
        got = ops.attention_devlen(qv.to(dev()), kd, vd, _scalar(kv - q_len), max_kv_len=cap)
        assert_close(got, ref_attn.verify_attention(qv, k[:, :, :kv], v[:, :, :kv]), dtype)


def test_attention_devlen_rejects_length_past_plan_with_nan():
    """A device length outside [0, max_kv_len - q_len] reads nothing, writes NaN
    outputs and marks the status word; a valid one leaves the word alone."""
    announce("attention_devlen with a device length past max_kv_len - q_len")
    k = torch.randn(1, NKV, 512, D, device=dev()).to(torch.bfloat16)
    q = torch.randn(1, NQ, 4, D, device=dev()).to(torch.bfloat16)
    status = torch.zeros(1, dtype=torch.int32, device=dev())
    ops.attention_devlen(q, k, k, _scalar(296), max_kv_len=300, status=status)
    torch.cuda.synchronize()
    assert int(status) == 0
    for bad in (300, -1):
        status.zero_()
        out = ops.attention_devlen(q, k, k, _scalar(bad), max_kv_len=300, status=status)
        torch.cuda.synchronize()
        assert torch.isnan(out.float()).all()
        assert int(status) == ops.STATUS_CACHE_OVERFLOW
    for dt in (torch.float32, torch.float16):          # the fp32 kernel and the fp16 instances report it too
        status.zero_()
        out = ops.attention_devlen(q.to(dt), k.to(dt), k.to(dt), _scalar(-5), max_kv_len=300, status=status)
        torch.cuda.synchronize()
        assert torch.isnan(out.float()).all() and int(status) == ops.STATUS_CACHE_OVERFLOW


@pytest.mark.parametrize("fused", [False, True])
def test_rope_append_past_capacity_is_skipped_and_reported(fused):
    """rope_append / qkv_rope_append with rows at or past the capacity: the
    rows that fit are written, the others are not (memory after the cache is
    untouched), the queries are still produced, and the status word is set."""
    announce(f"rope append past capacity, status word, fused={fused}")
    g = torch.Generator().manual_seed(71)
    cap, n = 20, 3
    buf_k = torch.full((1, NKV, cap + 8, D), -3.0, device=dev()).to(torch.bfloat16)
    buf_v = torch.full((1, NKV, cap + 8, D), -3.0, device=dev()).to(torch.bfloat16)
    kc, vc = buf_k[:, :, :cap], buf_v[:, :, :cap]
    inv = (1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))).float().to(dev())
    status = torch.zeros(1, dtype=torch.int32, device=dev())
    if fused:
        K = 256
        x = torch.randn(1, n, K, generator=g).to(torch.bfloat16).to(dev())
        w = (0.05 * torch.randn((NQ + 2 * NKV) * D, K, generator=g)).to(torch.bfloat16).to(dev())
        q = ops.qkv_rope_append(x, w, None, NQ, kc, vc, _scalar(cap - 1), _scalar(500), inv, status=status)
    else:
        qkv = torch.randn(1, n, (NQ + 2 * NKV) * D, generator=g).to(torch.bfloat16).to(dev())
        q = ops.rope_append(qkv, NQ, kc, vc, _scalar(cap - 1), _scalar(500), inv, status=status)
    torch.cuda.synchronize()
    assert int(status) == ops.STATUS_CACHE_OVERFLOW
    assert torch.isfinite(q.float()).all()
    assert not torch.all(kc[:, :, cap - 1] == -3.0) and torch.all(kc[:, :, :cap - 1] == -3.0)
    assert torch.all(buf_k[:, :, cap:] == -3.0) and torch.all(buf_v[:, :, cap:] == -3.0)


@pytest.mark.parametrize("n,K,n_q,n_kv,length,pos,off,cap",
                         [(1, 3584, 28, 4, 1023, 33000, 0, 1100), (1, 3584, 28, 4, 5, 131000, 7, 64),
                          (3, 896, 7, 1, 40, 900, 2, 44), (4, 1024, 8, 2, 0, 0, 0, 8),
                          (2, 3584, 28, 4, 63, 70, 0, 64)])
def test_qkv_rope_append_equals_projection_then_rope_append(n, K, n_q, n_kv, length, pos, off, cap):
    """The fused projection + rotary + append against the projection (HIP
    GEMV with bias) followed by rope_append, including rows at or past the
    capacity (not written: the last case's second row). At 256 or more
    16-column blocks (the 7B shape) both split K over four waves and the
    results are equal bit for bit; below, the GEMV splits K over two waves, so
    the sums associate differently and elements may differ by one bf16 ulp."""
    announce(f"qkv_rope_append n={n} K={K} heads={n_q}/{n_kv} len={length} pos={pos}+{off} cap={cap}")
    g = torch.Generator(device=dev()).manual_seed(n * 1000 + K + length)
    NW = (n_q + 2 * n_kv) * D
    x = (torch.randn(1, n, K, generator=g, device=dev()) * 2).to(torch.bfloat16)
    w = (torch.randn(NW, K, generator=g, device=dev()) * 0.03).to(torch.bfloat16)
    b = (torch.randn(NW, generator=g, device=dev()) * 0.5).to(torch.bfloat16)
    inv = torch.from_numpy(ref_rope.inv_freq(1e6, D)).to(dev())
    caches = [torch.full((1, n_kv, cap, D), float("nan"), dtype=torch.bfloat16, device=dev()) for _ in range(4)]
    q = ops.qkv_rope_append(x, w, b, n_q, caches[0], caches[1], _scalar(length), _scalar(pos), inv, pos_offset=off)
    want = ops.rope_append(ops.linear(x, w, b), n_q, caches[2], caches[3], _scalar(length), _scalar(pos), inv,
                           pos_offset=off)
    torch.cuda.synchronize()
    assert q.shape == (1, n_q, n, D)
    same_split = NW // 16 >= 256
    pairs = [(q, want), (caches[0].nan_to_num(7.0), caches[2].nan_to_num(7.0)),
             (caches[1].nan_to_num(7.0), caches[3].nan_to_num(7.0))]
    for got, ref in pairs:
        if same_split:
            assert torch.equal(got, ref)
        else:
            _assert_within_one_bf16_ulp(got, ref)


def _assert_within_one_bf16_ulp(a: torch.Tensor, b: torch.Tensor) -> None:
    """|a - b| <= one bf16 ulp of the larger magnitude, elementwise."""
    a32, b32 = a.float(), b.float()
    mag = torch.maximum(a32.abs(), b32.abs()).clamp_min(torch.finfo(torch.bfloat16).tiny)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    assert ((a32 - b32).abs() <= ulp).all()


def test_qkv_rope_append_rejects_bad_arguments():
    announce("qkv_rope_append host-side validation")
    x = torch.zeros(1, 5, 3584, dtype=torch.bfloat16, device=dev())
    w = torch.zeros(36 * D, 3584, dtype=torch.bfloat16, device=dev())
    kc = torch.zeros(1, NKV, 64, D, dtype=torch.bfloat16, device=dev())
    inv = torch.from_numpy(ref_rope.inv_freq(1e6, D)).to(dev())
    with pytest.raises(_lib.StdHipError):            # five rows
        ops.qkv_rope_append(x, w, None, NQ, kc, kc.clone(), _scalar(0), _scalar(0), inv)
    with pytest.raises(ValueError):                 # weight rows do not match the heads
        ops.qkv_rope_append(x[:, :1], w[:-D], None, NQ, kc, kc.clone(), _scalar(0), _scalar(0), inv)
    with pytest.raises(TypeError):
        ops.qkv_rope_append(x[:, :1].float(), w, None, NQ, kc, kc.clone(), _scalar(0), _scalar(0), inv)


@pytest.mark.parametrize("K,n_q,n_kv", [(3584, 28, 4), (896, 7, 1), (1024, 8, 2)])
def test_qkv_rope_append_with_norm_equals_rms_norm_first(K, n_q, n_kv):
    """One row with the layer's input RMSNorm in the same launch: equal, bit
    for bit, to rms_norm followed by the fused projection + rotary + append."""
    announce(f"qkv_rope_append with norm K={K} heads={n_q}/{n_kv}")
    g = torch.Generator(device=dev()).manual_seed(K + n_q)
    NW = (n_q + 2 * n_kv) * D
    x = (torch.randn(1, 1, K, generator=g, device=dev()) * 3).to(torch.bfloat16)
    nw = (1 + 0.2 * torch.randn(K, generator=g, device=dev())).to(torch.bfloat16)
    w = (torch.randn(NW, K, generator=g, device=dev()) * 0.03).to(torch.bfloat16)
    b = (torch.randn(NW, generator=g, device=dev()) * 0.5).to(torch.bfloat16)
    inv = torch.from_numpy(ref_rope.inv_freq(1e6, D)).to(dev())
    caches = [torch.full((1, n_kv, 40, D), float("nan"), dtype=torch.bfloat16, device=dev()) for _ in range(4)]
    q = ops.qkv_rope_append(x, w, b, n_q, caches[0], caches[1], _scalar(17), _scalar(5000), inv,
                            norm_weight=nw, eps=1e-6)
    want = ops.qkv_rope_append(ops.rms_norm(x, nw, 1e-6), w, b, n_q, caches[2], caches[3], _scalar(17),
                               _scalar(5000), inv)
    torch.cuda.synchronize()
    assert torch.equal(q, want)
    for got, ref in ((caches[0], caches[2]), (caches[1], caches[3])):
        assert torch.equal(got.nan_to_num(7.0), ref.nan_to_num(7.0))


def test_qkv_rope_append_norm_limits():
    """The in-launch norm takes one row of at most 3584 elements."""
    announce("qkv_rope_append norm: row and width limits")
    inv = torch.from_numpy(ref_rope.inv_freq(1e6, D)).to(dev())
    kc = torch.zeros(1, NKV, 64, D, dtype=torch.bfloat16, device=dev())
    for n, K in ((2, 3584), (1, 4096)):
        x = torch.zeros(1, n, K, dtype=torch.bfloat16, device=dev())
        w = torch.zeros(36 * D, K, dtype=torch.bfloat16, device=dev())
        with pytest.raises(_lib.StdHipError):
            ops.qkv_rope_append(x, w, None, NQ, kc, kc.clone(), _scalar(0), _scalar(0), inv,
                                norm_weight=torch.ones(K, dtype=torch.bfloat16, device=dev()), eps=1e-6)


def test_qkv_rope_append_misaligned_bias_and_norm_weight():
    """The one-row ring launch DMAs the bias and the norm weight in 16-byte
    pieces; views that start 2 bytes into their buffer take the register
    kernel instead, with the same results bit for bit (7B shape: both split K
    over four waves in the same order)."""
    announce("qkv_rope_append one row, bias and norm weight 2 bytes off 16-byte alignment")
    g = torch.Generator(device=dev()).manual_seed(4242)
    K, n_q, n_kv = 3584, 28, 4
    NW = (n_q + 2 * n_kv) * D
    x = (torch.randn(1, 1, K, generator=g, device=dev()) * 3).to(torch.bfloat16)
    nw_buf = (1 + 0.2 * torch.randn(K + 8, generator=g, device=dev())).to(torch.bfloat16)
    w = (torch.randn(NW, K, generator=g, device=dev()) * 0.03).to(torch.bfloat16)
    b_buf = (torch.randn(NW + 8, generator=g, device=dev()) * 0.5).to(torch.bfloat16)
    inv = torch.from_numpy(ref_rope.inv_freq(1e6, D)).to(dev())
    for off_b, off_n in ((1, 0), (0, 1), (1, 1)):
        b_view, nw_view = b_buf[off_b:off_b + NW], nw_buf[off_n:off_n + K]
        b_al, nw_al = b_view.clone(), nw_view.clone()           # fresh, aligned copies of the same values
        caches = [torch.full((1, n_kv, 40, D), float("nan"), dtype=torch.bfloat16, device=dev()) for _ in range(4)]
        q = ops.qkv_rope_append(x, w, b_view, n_q, caches[0], caches[1], _scalar(17), _scalar(5000), inv,
                                norm_weight=nw_view, eps=1e-6)
        want = ops.qkv_rope_append(x, w, b_al, n_q, caches[2], caches[3], _scalar(17), _scalar(5000), inv,
                                   norm_weight=nw_al, eps=1e-6)
        torch.cuda.synchronize()
        assert torch.equal(q, want), (off_b, off_n)
        for got, ref in ((caches[0], caches[2]), (caches[1], caches[3])):
            assert torch.equal(got.nan_to_num(7.0), ref.nan_to_num(7.0)), (off_b, off_n)
