"""Shared helpers of the GPU parity tests (device placement, cache buffers,
tolerances). Imported by tests/test_gpu_*.py only."""
import sys

import numpy as np
import torch

# Parity bars: bf16 attention rtol 2e-2 / atol 2e-3, fp32 1e-5; fp16 (three
# more mantissa bits than bf16, probabilities and outputs rounded to fp16)
# rtol 5e-3 / atol 5e-4; indices and token ids bit-exact.
TOL = {torch.bfloat16: dict(rtol=2e-2, atol=2e-3), torch.float32: dict(rtol=1e-5, atol=1e-5),
       torch.float16: dict(rtol=5e-3, atol=5e-4)}


def announce(msg: str) -> None:
    """Name the case on stdout before the GPU step runs."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def dev():
    return torch.device("cuda:0")


def cache_buffer(prompt: torch.Tensor, capacity: int, device=None) -> torch.Tensor:
    """A [1, n_kv, capacity, D] cache (head stride capacity*D) holding `prompt`
    [1, n_kv, P, D] in rows [0, P); the rest is filled with NaN so that any
    read past the valid length shows up in the output."""
    device = device or dev()
    _, n_kv, P, D = prompt.shape
    buf = torch.full((1, n_kv, capacity, D), float("nan"), dtype=prompt.dtype, device=device)
    buf[:, :, :P] = prompt.to(device)
    return buf


def assert_close(got: torch.Tensor, ref: np.ndarray, dtype) -> None:
    g = got.detach().float().cpu().numpy().astype(np.float64)
    assert np.isfinite(g).all(), "non-finite output"
    np.testing.assert_allclose(g, ref, **TOL[dtype])
