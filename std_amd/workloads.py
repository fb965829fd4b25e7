"""Seeded synthetic inputs for the STD decode hot path at Qwen2.5-VL-7B
attention shapes (28 query / 4 KV heads, head_dim 128, 128 text rows).

Every tensor of a layer is drawn from one ``torch.Generator`` seeded with
``seed_base + layer`` (``+ 100`` for the tie variant) in the fixed order
  q_text, k, v, q_draft, q_verify, new_k, new_v, (salient / tie positions)
so a test and a benchmark that ask for the same (config, layer) see the same
values on the same device type. Visual positions are [0, V) and text rows
[V, P), as in the synthetic prompts of the configurations.

Workloads (P = prompt length, V = P - 128 visual positions):
  c1  fp32, 1 layer,  P=4096,   K+text=1024; K, V ~ N(0,1)
  c2  bf16, 28 layers, P=16384, K+text=1024; 2% of visual keys get
      +3 * (unit mean of the group's text queries)
  c3  bf16, 28 layers, P=65536, K+text=4096; 1% salient keys in runs of 64
  c4  bf16, 28 layers, P=131072, K+text=1024; key norms log-normal
      (sqrt(D) * exp(0.5 n)); tie variant copies 5% of visual keys bit-exactly
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    dtype: torch.dtype
    n_layers: int
    prompt_len: int
    k_plus_text: int
    seed_base: int
    keys: str                 # "normal" | "salient" | "salient_runs" | "lognormal"
    salient_frac: float = 0.0
    tie_frac: float = 0.0
    n_q: int = 28
    n_kv: int = 4
    head_dim: int = 128
    text_len: int = 128
    gamma: int = 9
    vocab: int = 152064

    @property
    def visual_len(self) -> int:
        return self.prompt_len - self.text_len

    @property
    def text_start(self) -> int:
        return self.visual_len

    @property
    def k(self) -> int:
        """Visual top-k per KV head (std_qwen25vl.py:192-195)."""
        return min(max(1, self.k_plus_text - self.text_len), self.visual_len)

    @property
    def compact_len(self) -> int:
        return self.text_len + self.k

    @property
    def verify_rows(self) -> int:
        return self.gamma + 1


WORKLOADS: Dict[str, Workload] = {
    "c1": Workload("c1", torch.float32, 1, 4096, 1024, 1001, "normal"),
    "c2": Workload("c2", torch.bfloat16, 28, 16384, 1024, 2001, "salient", salient_frac=0.02),
    "c3": Workload("c3", torch.bfloat16, 28, 65536, 4096, 3001, "salient_runs", salient_frac=0.01),
    "c4": Workload("c4", torch.bfloat16, 28, 131072, 1024, 4001, "lognormal", tie_frac=0.05),
}


def _randn(gen, shape, device):
    return torch.randn(*shape, generator=gen, device=device, dtype=torch.float32)


def make_layer(w: Workload, layer: int, tie: bool = False, device: str = "cpu",
               prompt_len: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """Inputs of one layer: q_text [1,n_q,T,D], k/v [1,n_kv,P,D] (prompt KV),
    q_draft [1,n_q,1,D], q_verify [1,n_q,gamma+1,D], new_k/new_v
    [1,n_kv,gamma+1,D] (the verify rows appended to the dense cache).
    ``prompt_len`` overrides the workload's P (same recipe, shorter prompt)."""
    P = prompt_len or w.prompt_len
    V = P - w.text_len
    T, D, Q = w.text_len, w.head_dim, w.verify_rows
    seed = w.seed_base + layer + (100 if tie else 0)
    gen = torch.Generator(device=device).manual_seed(seed)
    q_text = _randn(gen, (1, w.n_q, T, D), device)
    k = _randn(gen, (1, w.n_kv, P, D), device)
    v = _randn(gen, (1, w.n_kv, P, D), device)
    q_draft = _randn(gen, (1, w.n_q, 1, D), device)
    q_verify = _randn(gen, (1, w.n_q, Q, D), device)
    new_k = _randn(gen, (1, w.n_kv, Q, D), device)
    new_v = _randn(gen, (1, w.n_kv, Q, D), device)
    group = w.n_q // w.n_kv
    if w.keys == "lognormal":
        norms = math.sqrt(D) * torch.exp(0.5 * _randn(gen, (1, w.n_kv, P, 1), device))
        k = k / k.norm(dim=-1, keepdim=True) * norms
    elif w.keys in ("salient", "salient_runs"):
        u = q_text.reshape(w.n_kv, group * T, D).mean(dim=1)
        u = u / u.norm(dim=-1, keepdim=True)                      # [n_kv, D]
        n_sal = max(1, int(round(w.salient_frac * V)))
        if w.keys == "salient":
            pos = torch.randperm(V, generator=gen, device=device)[:n_sal]
        else:
            n_runs = max(1, n_sal // 64)
            starts = torch.randperm(V // 64, generator=gen, device=device)[:n_runs] * 64
            pos = (starts[:, None] + torch.arange(64, device=device)[None, :]).reshape(-1)
        k[0, :, pos] += 3.0 * u[:, None, :]
    out = dict(q_text=q_text, k=k, v=v, q_draft=q_draft, q_verify=q_verify, new_k=new_k, new_v=new_v)
    out = {name: t.to(w.dtype) for name, t in out.items()}
    if tie and w.tie_frac > 0:
        n_dup = int(round(w.tie_frac * V))
        perm = torch.randperm(V, generator=gen, device=device)
        dst, src = perm[:n_dup], perm[n_dup:2 * n_dup]
        out["k"][0, :, dst] = out["k"][0, :, src]
    return out


def visual_positions(w: Workload, device: str = "cpu", prompt_len: Optional[int] = None) -> torch.Tensor:
    P = prompt_len or w.prompt_len
    return torch.arange(P - w.text_len, dtype=torch.int32, device=device)


def non_visual_positions(w: Workload, device: str = "cpu", prompt_len: Optional[int] = None) -> torch.Tensor:
    P = prompt_len or w.prompt_len
    return torch.arange(P - w.text_len, P, dtype=torch.int32, device=device)


def make_logits(w: Workload, rows: int, seed: int, device: str = "cpu") -> torch.Tensor:
    gen = torch.Generator(device=device).manual_seed(seed)
    return _randn(gen, (rows, w.vocab), device).to(w.dtype)
