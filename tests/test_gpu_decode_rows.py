"""Single-row decode through the fused bf16 path against an fp32 forward.

A decode step of one bf16 row takes the HIP launches only: RMSNorm folded
into the q/k/v projection with RoPE and the K/V append (qkv_rope_append),
split-K attention over the cache, the o projection and the MLP as GEMVs with
the residual add and the gated activation in their epilogues, and the
lm_head GEMV. The reference is a plain fp32 torch forward of the whole
sequence written here from the model's weights (no std_amd op on it): the
model behind std_qwen25vl.py's decode loop, Qwen2 attention with GQA and
rotary embeddings. Each decode step's logits must match the reference row at
its position to the tolerance below; two planted wiring mistakes in the
reference (the input norm's weight dropped, the decode row's rotary position
off by one) move the reference by several times the measured error, so the
comparison would catch either in the fused path.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from std_amd.decoder import DecoderConfig, RandomDecoder
from std_amd.kv_cache import initialize_past_key_values
from tests.gpu_helpers import announce, dev

# bf16 weights and activations against fp32 arithmetic on the same weights:
# relative L2 error of a logits row.
REL_TOL = 3e-2


def fp32_logits(weights: dict, cfg: DecoderConfig, ids: torch.Tensor, plant: str = "") -> torch.Tensor:
    """Logits [n, vocab] of every position of ids [n] (positions 0..n-1, causal),
    fp32 on the CPU. plant = "no_ln1" drops the input norm's weight; "rope+1"
    gives the last row the rotary position n instead of n-1."""
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps = cfg.rms_norm_eps
    n = ids.shape[0]
    x = weights["embed"][ids]
    pos = torch.arange(n, dtype=torch.float32)
    if plant == "rope+1":
        pos[-1] += 1
    freqs = pos[:, None] * weights["inv_freq"][None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    cos, sin = emb.cos(), emb.sin()

    def norm(v, w):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps) * w

    def rot(t):
        return torch.cat([-t[..., d // 2:], t[..., :d // 2]], dim=-1)

    mask = torch.ones(n, n, dtype=torch.bool).triu(1)
    for p in weights["layers"]:
        h = norm(x, torch.ones_like(p["ln1"]) if plant == "no_ln1" else p["ln1"])
        qkv = h @ p["qkv_w"].t() + p["qkv_b"]
        q = qkv[:, :hq * d].view(n, hq, d).transpose(0, 1)
        k = qkv[:, hq * d:(hq + hkv) * d].view(n, hkv, d).transpose(0, 1)
        v = qkv[:, (hq + hkv) * d:].view(n, hkv, d).transpose(0, 1)
        q = q * cos + rot(q) * sin
        k = k * cos + rot(k) * sin
        k = k.repeat_interleave(hq // hkv, dim=0)
        v = v.repeat_interleave(hq // hkv, dim=0)
        s = (q @ k.transpose(1, 2)) / math.sqrt(d)
        s.masked_fill_(mask, float("-inf"))
        o = torch.softmax(s, dim=-1) @ v                                   # [hq, n, d]
        x = x + o.transpose(0, 1).reshape(n, hq * d) @ p["o_w"].t()
        gate, up = (norm(x, p["ln2"]) @ p["gate_up_w"].t()).chunk(2, dim=-1)
        x = x + (F.silu(gate) * up) @ p["down_w"].t()
    return norm(x, weights["norm"]) @ weights["lm_head"].t()


def host_weights(model: RandomDecoder, ids: torch.Tensor) -> dict:
    """The model's weights as fp32 CPU tensors (embedding rows of ids only)."""
    f = lambda t: t.float().cpu()                                          # noqa: E731
    embed = torch.zeros(model.config.vocab_size, model.config.hidden_size)
    uniq = ids.unique()
    embed[uniq.cpu()] = f(model.embed_tokens[uniq.to(model.device)])
    return {"embed": embed, "inv_freq": f(model.inv_freq), "norm": f(model.norm), "lm_head": f(model.lm_head),
            "layers": [{k: f(v) for k, v in p.items()} for p in model.layers]}


def randomise_norms(model: RandomDecoder, seed: int) -> None:
    """Norm weights ~ 1 + 0.5 N(0, 1), so that a dropped or misplaced norm
    weight shows in the logits (all-ones weights would hide it)."""
    gen = torch.Generator(device=model.device).manual_seed(seed)

    def w():
        return (1 + 0.5 * torch.randn(model.config.hidden_size, generator=gen, device=model.device)).to(model.dtype)
    for p in model.layers:
        p["ln1"], p["ln2"] = w(), w()
    model.norm = w()


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a - b).norm() / b.norm())


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["tiny", "7b"])
def test_single_row_decode_logits_match_fp32_forward(shape):
    cfg = DecoderConfig.tiny(layers=2) if shape == "tiny" else DecoderConfig(num_hidden_layers=2)
    announce(f"single-row fused decode vs fp32 forward, {shape} shape, 2 layers")
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=21)
    randomise_norms(model, 22)
    P, T = 40, 6
    ids = torch.randint(0, cfg.vocab_size, (P + T,), generator=torch.Generator().manual_seed(23))
    assert model.fused_rows(1) and not model.fused_rows(P)       # prefill on the torch path, decode fused
    assert cfg.hidden_size <= 3584                               # the norm folds into the q/k/v launch
    weights = host_weights(model, ids)
    ref = fp32_logits(weights, cfg, ids)

    pkv, _, _ = initialize_past_key_values(cfg, dev(), torch.bfloat16, 128)
    ids_dev = ids.view(1, -1).to(dev())
    with torch.inference_mode():
        got = [model(ids_dev[:, :P], pkv)[0, -1]]
        for t in range(T):
            got.append(model(ids_dev[:, P + t:P + t + 1], pkv)[0, -1])
    assert pkv[0][0].length == P + T
    errs = [rel_err(g.float().cpu(), ref[P - 1 + i]) for i, g in enumerate(got)]
    print(f"[{shape}] prefill rel err {errs[0]:.2e}; decode rel errs "
          + " ".join(f"{e:.2e}" for e in errs[1:]), flush=True)
    assert max(errs) < REL_TOL, errs

    # each planted mistake moves the last row several times further than the
    # fused path's own error
    for plant in ("no_ln1", "rope+1"):
        off = rel_err(fp32_logits(weights, cfg, ids, plant=plant)[-1], ref[-1])
        print(f"[{shape}] planted {plant}: rel diff {off:.2e}", flush=True)
        assert off > 4 * max(errs[1:]), (plant, off)
