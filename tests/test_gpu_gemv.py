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
