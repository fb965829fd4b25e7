"""The weight-streaming projection (std_gemv) against a float32 torch
reference of torch.nn.functional.linear, at the 7B decoder's projection
shapes for one decode row and ten verify rows, plus edge shapes; and its
determinism (split-K partials are added in a fixed order)."""
import pytest
import torch
import torch.nn.functional as F

from std_amd import ops
from tests.gpu_helpers import announce, dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K,bias", [(1, 4608, 3584, True), (10, 4608, 3584, True), (1, 3584, 3584, False),
                                         (10, 37888, 3584, False), (1, 3584, 18944, False), (10, 3584, 18944, False),
                                         (1, 152064, 3584, False), (16, 512, 1024, True), (3, 100, 96, True)])
def test_gemv_matches_float32_linear(M, N, K, bias):
    announce(f"gemv M={M} N={N} K={K} bias={bias}")
    g = torch.Generator(device=dev()).manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g, device=dev()).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev()) * 0.02).to(torch.bfloat16)
    b = (torch.randn(N, generator=g, device=dev()) * 0.02).to(torch.bfloat16) if bias else None
    got = ops.linear(x, w, b)
    want = F.linear(x.float(), w.float(), b.float() if bias else None)
    torch.testing.assert_close(got.float(), want, rtol=1e-2, atol=2e-3)
    again = ops.linear(x, w, b)
    torch.cuda.synchronize()
    assert torch.equal(got, again)


def test_gemv_keeps_leading_dims_and_strided_rows():
    announce("gemv on [1, 10, K] views with a row stride")
    x = torch.randn(1, 10, 4096, device=dev()).to(torch.bfloat16)[..., :3584]
    w = (torch.randn(640, 3584, device=dev()) * 0.02).to(torch.bfloat16)
    got = ops.linear(x, w)
    assert got.shape == (1, 10, 640)
    torch.testing.assert_close(got.float(), F.linear(x.float(), w.float()), rtol=1e-2, atol=2e-3)


def _bf16_ulp(t: torch.Tensor) -> torch.Tensor:
    """One bf16 unit in the last place of each element (of its magnitude)."""
    a = t.float().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


@pytest.mark.parametrize("M,I,K,bias", [(1, 18944, 3584, False), (10, 18944, 3584, False), (3, 100, 96, True),
                                         (16, 48, 4128, True)])
def test_gated_linear_equals_torch_activation_of_the_projection(M, I, K, bias):
    """The gate/up epilogue (silu(g) * u with g, u rounded to bf16) against
    torch's own bf16 F.silu(gate) * up of the same projection: the sums are
    the non-gated kernel's, bit for bit, so any difference comes from the
    silu evaluation alone and is held to one bf16 ulp on a tiny fraction."""
    announce(f"gated_linear M={M} I={I} K={K} bias={bias}")
    g = torch.Generator(device=dev()).manual_seed(M + I + K)
    x = torch.randn(M, K, generator=g, device=dev()).to(torch.bfloat16)
    w = (torch.randn(2 * I, K, generator=g, device=dev()) * 0.03).to(torch.bfloat16)
    b = (torch.randn(2 * I, generator=g, device=dev()) * 0.5).to(torch.bfloat16) if bias else None
    got = ops.gated_linear(x, w, b)
    gate, up = ops.linear(x, w, b).chunk(2, dim=-1)
    want = F.silu(gate) * up
    torch.cuda.synchronize()
    assert got.shape == (M, I)
    diff = (got.float() - want.float()).abs()
    assert (diff <= _bf16_ulp(want)).all()
    assert (diff == 0).float().mean() >= 0.999
    ref = F.silu(F.linear(x.float(), w[:I].float(), b[:I].float() if bias else None)) * \
        F.linear(x.float(), w[I:].float(), b[I:].float() if bias else None)
    torch.testing.assert_close(got.float(), ref, rtol=2e-2, atol=2e-3)


@pytest.mark.parametrize("M,N,K", [(1, 3584, 3584), (1, 3584, 18944), (10, 3584, 18944), (5, 72, 160)])
def test_linear_residual_epilogue_equals_torch_add(M, N, K):
    announce(f"linear + residual M={M} N={N} K={K}")
    g = torch.Generator(device=dev()).manual_seed(3 * M + N + K)
    x = torch.randn(1, M, K, generator=g, device=dev()).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev()) * 0.02).to(torch.bfloat16)
    r = (torch.randn(1, M, N, generator=g, device=dev()) * 4).to(torch.bfloat16)
    got = ops.linear(x, w, residual=r)
    want = r + ops.linear(x, w)
    torch.cuda.synchronize()
    assert got.shape == (1, M, N)
    assert torch.equal(got, want)


def test_gated_linear_with_residual_and_validation():
    announce("std_gemv_ex gated + residual; host-side shape checks")
    M, I, K = 4, 160, 256
    g = torch.Generator(device=dev()).manual_seed(5)
    x = torch.randn(M, K, generator=g, device=dev()).to(torch.bfloat16)
    w = (torch.randn(2 * I, K, generator=g, device=dev()) * 0.05).to(torch.bfloat16)
    r = torch.randn(M, I, generator=g, device=dev()).to(torch.bfloat16)
    y = torch.empty(M, I, dtype=torch.bfloat16, device=dev())
    from std_amd import _lib
    _lib.call("std_gemv_ex", x.data_ptr(), K, w.data_ptr(), K, None, r.data_ptr(), I, y.data_ptr(), I, M, I, K, 1,
              _lib.STD_BF16, torch.cuda.current_stream().cuda_stream)
    want = r + ops.gated_linear(x, w)
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    with pytest.raises(ValueError):
        ops.gated_linear(x, w[:-1])                      # odd row count: not a gate/up stack
    with pytest.raises(ValueError):
        ops.linear(x, w, residual=r)                     # residual shaped like a different output


@pytest.mark.parametrize("M,N,K,gated", [(1, 3584, 512, False), (1, 3584, 1024, False), (2, 3584, 1536, False),
                                          (1, 3584, 2560, False), (1, 2048, 1024, True), (3, 2048, 1536, True),
                                          (1, 1024, 768, True), (4, 3000, 2048, False)])
def test_gemv_ring_with_few_steps_per_wave(M, N, K, gated):
    """The register ring when a wave has fewer steps than the ring has slots
    (1-3 steps: the prologue's clamped loads and no full ring iteration) or
    one iteration plus a remainder (5), plain and gated, against a float32
    reference; repeated calls are bit-identical."""
    announce(f"gemv ring few steps M={M} N={N} K={K} gated={gated}")
    g = torch.Generator(device=dev()).manual_seed(M + N + K + int(gated))
    x = torch.randn(M, K, generator=g, device=dev()).to(torch.bfloat16)
    NW = 2 * N if gated else N
    w = (torch.randn(NW, K, generator=g, device=dev()) * 0.02).to(torch.bfloat16)
    if gated:
        got = ops.gated_linear(x, w)
        ref = F.silu(F.linear(x.float(), w[:N].float())) * F.linear(x.float(), w[N:].float())
        again = ops.gated_linear(x, w)
    else:
        got = ops.linear(x, w)
        ref = F.linear(x.float(), w.float())
        again = ops.linear(x, w)
    torch.cuda.synchronize()
    torch.testing.assert_close(got.float(), ref, rtol=2e-2, atol=2e-3)
    assert torch.equal(got, again)


@pytest.mark.parametrize("N,K,gated", [(20000, 3584, False), (9470, 3552, True), (8200, 8224, False),
                                        (3584, 18944, False), (4608, 3584, False), (3584, 3584, False),
                                        (2350, 3616, False)])
def test_gemv_lds_ring_one_row(N, K, gated):
    """One activation row over a weight of 16 MiB or more streams through the
    LDS ring (four waves with 64-k stages, or eight waves with 128-k stages):
    the 7B q/k/v and o shapes, ragged column counts and K ranges that end
    inside a stage, against a float32 reference; the gated sums equal the plain
    projection of the stacked weight bit for bit, with a residual the plain
    result plus it, with a bias the float32 reference plus the bias, and
    repeated calls are bit-identical."""
    announce(f"gemv lds ring N={N} K={K} gated={gated}")
    g = torch.Generator(device=dev()).manual_seed(N + K)
    x = torch.randn(1, K, generator=g, device=dev()).to(torch.bfloat16)
    NW = 2 * N if gated else N
    w = (torch.randn(NW, K, generator=g, device=dev()) * 0.02).to(torch.bfloat16)
    if gated:
        got = ops.gated_linear(x, w)
        gate, up = ops.linear(x, w).chunk(2, dim=-1)
        want = F.silu(gate) * up
        diff = (got.float() - want.float()).abs()
        assert (diff <= _bf16_ulp(want)).all()
        ref = F.silu(F.linear(x.float(), w[:N].float())) * F.linear(x.float(), w[N:].float())
        torch.testing.assert_close(got.float(), ref, rtol=2e-2, atol=2e-3)
    else:
        got = ops.linear(x, w)
        torch.testing.assert_close(got.float(), F.linear(x.float(), w.float()), rtol=1e-2, atol=2e-3)
        r = (torch.randn(1, N, generator=g, device=dev()) * 4).to(torch.bfloat16)
        assert torch.equal(ops.linear(x, w, residual=r), r + got)
        b = torch.randn(N, generator=g, device=dev()).to(torch.bfloat16)
        torch.testing.assert_close(ops.linear(x, w, bias=b).float(), F.linear(x.float(), w.float(), b.float()),
                                   rtol=1e-2, atol=2e-3)
    again = ops.gated_linear(x, w) if gated else ops.linear(x, w)
    torch.cuda.synchronize()
    assert torch.equal(got, again)


def _rms_norm_f32(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen2RMSNorm in float32 with its two bf16 roundings (x * rsqrt(mean(x^2)
    + eps) to bf16, then times the weight to bf16): a reference written
    independently of the HIP kernel's summation order."""
    xf = x.float()
    h = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
    return (w.float() * h.float()).to(torch.bfloat16)


@pytest.mark.parametrize("N,K,gated,residual,bias", [(18944, 3584, True, False, False), (20000, 3584, False, True, True),
                                                     (3584, 3584, False, True, False), (9504, 3584, False, False, True),
                                                     (1000, 896, True, False, True), (700, 1024, False, True, False),
                                                     (3000, 3552, True, False, False)])
def test_gemv_norm_equals_rms_norm_then_gemv(N, K, gated, residual, bias):
    """One row with the input RMSNorm in the projection's launch
    (std_gemv_norm): the gate/up shape with the activation epilogue, plain
    projections with bias and residual at four and eight ring waves, and
    weights under 16 MiB. Where the plain projection also streams through the
    LDS ring (16 MiB and more) the two paths are equal bit for bit; below it
    they split K differently, and both are held to a float32 reference of the
    normalised projection. Two rows take the norm as its own launch."""
    announce(f"gemv norm N={N} K={K} gated={gated} residual={residual} bias={bias}")
    g = torch.Generator(device=dev()).manual_seed(N + K + 17)
    NW = 2 * N if gated else N
    x = (torch.randn(1, 1, K, generator=g, device=dev()) * 3).to(torch.bfloat16)
    nw = (1 + 0.2 * torch.randn(K, generator=g, device=dev())).to(torch.bfloat16)
    w = (torch.randn(NW, K, generator=g, device=dev()) * 0.02).to(torch.bfloat16)
    b = (torch.randn(NW, generator=g, device=dev()) * 0.1).to(torch.bfloat16) if bias else None
    r = (torch.randn(1, 1, N, generator=g, device=dev()) * 2).to(torch.bfloat16) if residual else None
    h = ops.rms_norm(x, nw, 1e-6)
    hr = _rms_norm_f32(x, nw, 1e-6).float()
    if gated:
        got = ops.gated_linear(x, w, b, norm_weight=nw, eps=1e-6)
        want = ops.gated_linear(h, w, b)
        gate, up = F.linear(hr, w.float(), b.float() if bias else None).chunk(2, dim=-1)
        ref = F.silu(gate) * up
    else:
        got = ops.linear(x, w, b, residual=r, norm_weight=nw, eps=1e-6)
        want = ops.linear(h, w, b, residual=r)
        ref = F.linear(hr, w.float(), b.float() if bias else None)
        if residual:
            ref = ref + r.float()
    torch.cuda.synchronize()
    assert got.shape == want.shape
    if NW * K * 2 >= 16 << 20:
        assert torch.equal(got, want)
    # with a residual (|r| up to ~8) the sum's bf16 rounding alone is up to
    # half an ulp of 8 (2^-6), and near cancellations it is all of the
    # relative error
    torch.testing.assert_close(got.float(), ref, rtol=2e-2, atol=2e-2 if residual else 3e-3)
    again = ops.gated_linear(x, w, b, norm_weight=nw, eps=1e-6) if gated else \
        ops.linear(x, w, b, residual=r, norm_weight=nw, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    # two rows: the norm as its own launch, then the projection
    x2 = torch.cat([x, x * 0.5], dim=1)
    two = ops.gated_linear(x2, w, b, norm_weight=nw, eps=1e-6) if gated else ops.linear(x2, w, b, norm_weight=nw,
                                                                                      eps=1e-6)
    h2 = ops.rms_norm(x2, nw, 1e-6)
    assert torch.equal(two, ops.gated_linear(h2, w, b) if gated else ops.linear(h2, w, b))


@pytest.mark.parametrize("M,N,K,gated", [(10, 18944, 3584, True), (10, 3584, 18944, False), (16, 4608, 3584, False),
                                         (2, 20000, 3584, False), (5, 9470, 3552, True), (10, 3584, 3584, False),
                                         (7, 2350, 3616, False)])
def test_gemv_lds_ring_rows(M, N, K, gated):
    """Two to sixteen rows over a weight of 16 MiB or more stream through the
    LDS ring with per-stage activation slabs (four waves, or eight where the
    plain projection has fewer than 256 column blocks): the 7B verify shapes,
    ragged column counts and K ranges that end inside a stage, rows read
    through a row stride, against a float32 reference; the gated output is
    within one bf16 ulp of silu(gate) * up formed from the plain projection
    of the stacked weight (the same four-wave sums; torch's silu rounds
    differently), the residual sum is the plain projection plus the residual
    rounded once, and repeated calls are bit-identical."""
    announce(f"gemv lds ring rows M={M} N={N} K={K} gated={gated}")
    g = torch.Generator(device=dev()).manual_seed(M * 100 + N + K)
    xs = torch.randn(1, M, K + 64, generator=g, device=dev()).to(torch.bfloat16)
    x = xs[..., :K]                                           # row stride K + 64
    NW = 2 * N if gated else N
    w = (torch.randn(NW, K, generator=g, device=dev()) * 0.02).to(torch.bfloat16)
    b = (torch.randn(NW, generator=g, device=dev()) * 0.1).to(torch.bfloat16)
    if gated:
        got = ops.gated_linear(x, w, b)
        gate, up = F.linear(x.float(), w.float(), b.float()).chunk(2, dim=-1)
        torch.testing.assert_close(got.float(), F.silu(gate) * up, rtol=2e-2, atol=2e-3)
        if (2 * N) // 16 >= 256:                          # the stacked plain projection: the same four-wave ring
            pg, pu = ops.linear(x, w, b).chunk(2, dim=-1)
            want = (F.silu(pg.float()).to(torch.bfloat16).float() * pu.float()).to(torch.bfloat16)
            assert ((got.float() - want.float()).abs() <= _bf16_ulp(want.float())).all()
        again = ops.gated_linear(x, w, b)
    else:
        r = (torch.randn(1, M, N, generator=g, device=dev()) * 2).to(torch.bfloat16)
        got = ops.linear(x, w, b, residual=r)
        ref = F.linear(x.float(), w.float(), b.float()) + r.float()
        torch.testing.assert_close(got.float(), ref, rtol=2e-2, atol=2e-2)
        plain = ops.linear(x, w, b)
        torch.testing.assert_close(plain.float(), F.linear(x.float(), w.float(), b.float()), rtol=1e-2, atol=3e-3)
        assert torch.equal(got, (r.float() + plain.float()).to(torch.bfloat16))
        again = ops.linear(x, w, b, residual=r)
    torch.cuda.synchronize()
    assert torch.equal(got, again)
