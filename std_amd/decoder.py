"""A random-init Qwen2.5-VL-7B-shaped language decoder for the end-to-end
self-speculative decode (the model side of std_qwen25vl.py's loop).

Architecture (Qwen2.5-VL-7B language model, modeling_qwen2_5_vl.py):
RMSNorm -> q/k/v projections with bias -> rotary embedding -> GQA attention
-> o_proj; RMSNorm -> SwiGLU MLP; final RMSNorm -> untied lm_head. With the
reference's position ids (three identical rows, modeling_qwen2_5_vl.py:1368-1384)
the multimodal rotary embedding with mrope_section [16, 24, 24] equals the
1-D rotary embedding (theta 1e6) used here.

Attention on the decode hot path runs in libstdhip.so. For q_len <= 96 / group
(the sparse draft and the dense AR decode at q_len == 1, the dense verify of
gamma + 1 rows) a layer is two launches after the q|k|v projection:
``ops.rope_append`` (rotary embedding of the rows, K/V written into the cache)
and ``ops.attention_devlen`` (offset-causal attention), both reading the cache
length and the position from a device int32 pair (length, position). Eager
calls upload that pair from the host lengths; graph-captured steps pass
``step_state`` and the pair then lives on the device only (advanced by the
step's row count, rolled back by the acceptance kernel), so one captured
graph replays every round. The launches are planned for the cache capacity,
so eager and captured steps run identical kernels. Longer inputs (the prompt
prefill, which is not part of the decode path) use torch's rotary embedding
and chunked fp32 matrix products.

Decode and verify rows (at most 16) run their projections, norms and the
MLP on the HIP GEMV and RMSNorm kernels (std_gemv, std_rms_norm); the prompt
prefill uses torch.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn.functional as F

from . import ops
from .kv_cache import KVCache

MAX_FUSED_ROWS = 96   # query rows per KV head served by one verify launch


@dataclass
class DecoderConfig:
    num_hidden_layers: int = 28
    hidden_size: int = 3584
    num_attention_heads: int = 28
    num_key_value_heads: int = 4
    intermediate_size: int = 18944
    vocab_size: int = 152064
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    max_position_embeddings: int = 128000
    init_std: float = 0.02
    video_token_id: int = 151656     # benchmark_std.py:44
    eos_token_id: int = 151645

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @classmethod
    def qwen25vl_7b(cls) -> "DecoderConfig":
        return cls()

    @classmethod
    def tiny(cls, layers: int = 2, vocab: int = 2048) -> "DecoderConfig":
        """7 query heads / 1 KV head of dim 128 (the GQA group of the 7B model)."""
        return cls(num_hidden_layers=layers, hidden_size=7 * 128, num_attention_heads=7, num_key_value_heads=1,
                   intermediate_size=1536, vocab_size=vocab, video_token_id=vocab - 2, eos_token_id=vocab - 1,
                   max_position_embeddings=8192)


class RandomDecoder:
    """Weights ~ N(0, init_std) (norm weights 1), drawn on the target device
    from one seeded generator in a fixed order."""

    def __init__(self, config: DecoderConfig, device: torch.device, dtype: torch.dtype = torch.bfloat16,
                 seed: int = 5001):
        if config.head_dim != ops.HEAD_DIM:
            raise ValueError(f"head_dim {config.head_dim} unsupported (the HIP path is built for 128)")
        if config.num_attention_heads % config.num_key_value_heads:
            raise ValueError("query heads must be a multiple of KV heads")
        self.config = config
        self.device = torch.device(device)
        self.dtype = dtype
        c = config
        gen = torch.Generator(device=self.device).manual_seed(seed)

        def w(*shape):
            return (torch.randn(*shape, generator=gen, device=self.device, dtype=torch.float32)
                    * c.init_std).to(dtype)

        hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        self.embed_tokens = w(c.vocab_size, c.hidden_size)
        self.layers = []
        for _ in range(c.num_hidden_layers):
            self.layers.append({
                "qkv_w": w((hq + 2 * hkv) * d, c.hidden_size),     # q_proj | k_proj | v_proj rows
                "qkv_b": w((hq + 2 * hkv) * d),
                "o_w": w(c.hidden_size, hq * d),
                "gate_up_w": w(2 * c.intermediate_size, c.hidden_size),
                "down_w": w(c.hidden_size, c.intermediate_size),
                "ln1": torch.ones(c.hidden_size, device=self.device, dtype=dtype),
                "ln2": torch.ones(c.hidden_size, device=self.device, dtype=dtype),
            })
        self.norm = torch.ones(c.hidden_size, device=self.device, dtype=dtype)
        self.lm_head = w(c.vocab_size, c.hidden_size)
        inv = 1.0 / (c.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
        self.inv_freq = inv.to(torch.float32).to(self.device)
        self.sparse_controller = None     # set by SparseDraftController.install()
        self.verify_collector = None      # set by VerificationCollectorV3.install()
        self.capture_text_queries = False
        self.captured_queries: List[Optional[torch.Tensor]] = [None] * c.num_hidden_layers
        # output_attentions of a prompt prefill step: each layer's softmax
        # probabilities [1, n_q, n, past + n] (zero past the causal limit)
        self.output_attentions = False
        self.captured_attentions: List[Optional[torch.Tensor]] = [None] * c.num_hidden_layers
        # Device status word of the decode steps: the appends and attention
        # launches OR ops' cache-overflow bit into it when a device length would
        # place a row, or the attended keys, past a cache's capacity (nothing is
        # written there). The generate loops clear it and read it back with
        # each round.
        self.decode_status = torch.zeros(1, dtype=torch.int32, device=self.device)

    # -- pieces ---------------------------------------------------------------
    def _hip_rows(self, x: torch.Tensor, max_rows: int) -> bool:
        return x.dtype == torch.bfloat16 and x.numel() // x.shape[-1] <= max_rows

    def _linear(self, x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                residual: Optional[torch.Tensor] = None, max_rows: int = 16) -> torch.Tensor:
        """linear(x) (+ residual). bf16 projections of at most max_rows rows
        stream the weights through the HIP GEMV, with the residual add in its
        epilogue; larger ones (prefill) use torch. At the ten verify rows the
        HIP GEMV beats hipBLASLt on every 7B projection (cold weights,
        graph-replayed: q/k/v 11.3 vs 12.5 us, o 8.1 vs 13.0, lm_head 180 vs
        238)."""
        if self._hip_rows(x, max_rows):
            return ops.linear(x, weight, bias, residual=residual)
        y = F.linear(x, weight, bias)
        return y if residual is None else residual + y

    def _rms_norm(self, x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        return ops.rms_norm(x, weight, self.config.rms_norm_eps)

    def _rope(self, position_ids: torch.Tensor):
        freqs = position_ids.to(torch.float32)[:, None] * self.inv_freq[None, :]
        emb = torch.cat([freqs, freqs], dim=-1)
        return emb.cos().to(self.dtype), emb.sin().to(self.dtype)

    @staticmethod
    def _rotate_half(x: torch.Tensor) -> torch.Tensor:
        h = x.shape[-1] // 2
        return torch.cat([-x[..., h:], x[..., :h]], dim=-1)

    def embed(self, input_ids: torch.Tensor, visual_embeds: Optional[torch.Tensor] = None) -> torch.Tensor:
        x = self.embed_tokens[input_ids]                      # [1, n, hidden]
        if visual_embeds is not None:
            vis = input_ids[0] == self.config.video_token_id
            n_vis = int(vis.sum())
            if n_vis:
                if visual_embeds.shape[0] < n_vis:
                    raise ValueError("fewer visual embeddings than video tokens")
                x[0, vis] = visual_embeds[:n_vis].to(x.dtype)
        return x

    def _prefill_attention(self, q, k_new, v_new, kc: KVCache, vc: KVCache, chunk: int = 512,
                           probs: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Causal attention of n prompt rows over the cache (torch, fp32);
        probs (optional, [1, n_q, n, past + n]) receives the probabilities."""
        c = self.config
        g_size = c.num_attention_heads // c.num_key_value_heads
        past = kc.length
        n = q.shape[2]
        kc.cat(k_new)
        vc.cat(v_new)
        out = torch.empty_like(q)
        if probs is not None:
            probs.zero_()
        scale = 1.0 / math.sqrt(c.head_dim)
        for g in range(c.num_key_value_heads):
            for c0 in range(0, n, chunk):
                c1 = min(n, c0 + chunk)
                s_len = past + c1                                           # keys visible to the chunk
                kt = kc.data[0, g, :s_len].float().t().contiguous()          # [D, S]
                vg = vc.data[0, g, :s_len].float()                            # [S, D]
                qg = q[0, g * g_size:(g + 1) * g_size, c0:c1].float()        # [G, m, D]
                s = (qg.reshape(-1, c.head_dim) @ kt).view(g_size, c1 - c0, s_len) * scale
                qpos = past + torch.arange(c0, c1, device=q.device)
                kpos = torch.arange(s_len, device=q.device)
                s.masked_fill_((kpos[None, :] > qpos[:, None])[None], float("-inf"))
                p = torch.softmax(s, dim=-1)
                if probs is not None:
                    probs[0, g * g_size:(g + 1) * g_size, c0:c1, :s_len] = p.to(probs.dtype)
                o = p.reshape(-1, s_len) @ vg
                out[0, g * g_size:(g + 1) * g_size, c0:c1] = o.view(g_size, c1 - c0, c.head_dim).to(q.dtype)
        return out

    def fused_rows(self, n: int) -> bool:
        """Whether n rows per step take the HIP rope/append + attention path
        (never while a prompt prefill step returns its attention
        probabilities, which the torch prefill attention forms)."""
        c = self.config
        return not self.output_attentions and n * (c.num_attention_heads // c.num_key_value_heads) <= MAX_FUSED_ROWS

    def _attention(self, li: int, x: torch.Tensor, cos, sin, kc: KVCache, vc: KVCache,
                   state: Optional[torch.Tensor], host_lengths: bool) -> torch.Tensor:
        """x + self-attention block output of input_layernorm(x) (o_proj included)."""
        c = self.config
        p = self.layers[li]
        n, width = x.shape[1], x.shape[-1]
        residual = x
        hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        controller = self.sparse_controller
        if controller is not None and controller.enabled and n != 1:
            raise RuntimeError("Sparse draft attention currently expects autoregressive q_len=1 calls.")
        qkv = None
        if self.fused_rows(n) and self._hip_rows(x, 1) and width <= ops.QKV_ROPE_NORM_MAX_K:
            # one bf16 row: the norm, projection, rotary embedding and K/V append in one launch
            q = ops.qkv_rope_append(x, p["qkv_w"], p["qkv_b"], hq, kc.data, vc.data, state[0:1], state[1:2],
                                    self.inv_freq, norm_weight=p["ln1"], eps=c.rms_norm_eps, status=self.decode_status)
        else:
            h = self._rms_norm(x, p["ln1"])
            if self.fused_rows(n) and self._hip_rows(h, 1) and width <= ops.QKV_ROPE_MAX_K:
                q = ops.qkv_rope_append(h, p["qkv_w"], p["qkv_b"], hq, kc.data, vc.data, state[0:1], state[1:2],
                                        self.inv_freq, status=self.decode_status)
            else:
                qkv = self._linear(h, p["qkv_w"], p["qkv_b"])                # [1, n, (hq + 2hkv) d]
        if self.fused_rows(n):
            if qkv is not None:
                q = ops.rope_append(qkv, hq, kc.data, vc.data, state[0:1], state[1:2], self.inv_freq,
                                    status=self.decode_status)
            if self.capture_text_queries:
                self.captured_queries[li] = q
            gather = controller.gather_for(li) if controller is not None and controller.enabled else None
            collector = self.verify_collector
            if collector is not None and collector.collecting and n > 1:
                # the verify forward with the visual-attention collector riding its attention pass
                # (planned for the cache capacity, as attention_devlen: the same attention rows)
                out, _ = ops.verify_attention_collect(q, kc.data, vc.data, visual=collector.visual,
                                                      kv_len=kc.capacity, length=state[0:1],
                                                      scores=collector.scores_out(li), status=self.decode_status)
                collector.record(li)
            elif gather is not None:      # index-addressed sparse cache: prompt keys read from the dense cache
                dk, dv, index, n_index = gather
                out = ops.gqa_decode_indexed(q, dk, dv, index, n_index, kc.data, vc.data, length=state[0:1],
                                             max_kv_len=kc.capacity, status=self.decode_status)
            else:
                out = ops.attention_devlen(q, kc.data, vc.data, state[0:1], max_kv_len=kc.capacity,
                                           status=self.decode_status)
            if host_lengths:
                kc.advance(n)
                vc.advance(n)
            return self._linear(out.transpose(1, 2).reshape(1, n, hq * d), p["o_w"], residual=residual)
        q = qkv[..., :hq * d].view(1, n, hq, d).transpose(1, 2)
        k = qkv[..., hq * d:(hq + hkv) * d].view(1, n, hkv, d).transpose(1, 2)
        v = qkv[..., (hq + hkv) * d:].view(1, n, hkv, d).transpose(1, 2)
        q = (q * cos + self._rotate_half(q) * sin).contiguous()
        k = (k * cos + self._rotate_half(k) * sin).contiguous()
        v = v.contiguous()
        if self.capture_text_queries:
            self.captured_queries[li] = q
        if not host_lengths:
            raise ValueError("a device-state step must have at most 96 query rows per KV head")
        probs = None
        if self.output_attentions:
            probs = torch.empty(1, hq, n, kc.length + n, dtype=q.dtype, device=q.device)
            self.captured_attentions[li] = probs
        out = self._prefill_attention(q, k, v, kc, vc, probs=probs)
        collector = self.verify_collector
        if collector is not None and collector.collecting and n > 1 and q.dtype in (torch.bfloat16, torch.float16):
            # a verify longer than the fused launches serve (more than 96 query rows per KV head): the
            # collector's scores from its own launch over the cache these rows were just appended to (in
            # chunks of positions); its attention output is not used
            ops.verify_attention_collect(q, kc.data, vc.data, visual=collector.visual, kv_len=kc.length,
                                         scores=collector.scores_out(li))
            collector.record(li)
        out = out.transpose(1, 2).reshape(1, n, hq * d)
        return residual + F.linear(out, p["o_w"])

    def _mlp(self, li: int, x: torch.Tensor) -> torch.Tensor:
        """x + down(silu(gate(h)) * up(h)) with h = post_attention_layernorm(x);
        up to 16 bf16 rows (decode and verify steps) take HIP launches, the
        activation and the residual add in the GEMV epilogues: at one row two
        (the norm inside the gate/up launch, std_gemv_norm; 7B: 43.1 us against
        46.5 us for the norm launch and the projection), else three."""
        p = self.layers[li]
        if self._hip_rows(x, 1):
            act = ops.gated_linear(x, p["gate_up_w"], norm_weight=p["ln2"], eps=self.config.rms_norm_eps)
            return ops.linear(act, p["down_w"], residual=x)
        h = self._rms_norm(x, p["ln2"])
        if self._hip_rows(h, 16):
            return ops.linear(ops.gated_linear(h, p["gate_up_w"]), p["down_w"], residual=x)
        residual = x
        gate, up = F.linear(h, p["gate_up_w"]).chunk(2, dim=-1)
        return residual + F.linear(F.silu(gate) * up, p["down_w"])

    # -- forward ----------------------------------------------------------------
    @torch.inference_mode()
    def forward(self, input_ids: torch.Tensor, past_key_values: List[List[KVCache]],
                position_ids: Optional[torch.Tensor] = None, visual_embeds: Optional[torch.Tensor] = None,
                all_logits: bool = False, start_position: Optional[int] = None,
                step_state: Optional[torch.Tensor] = None) -> torch.Tensor:
        """input_ids [1, n]; returns logits [1, n, vocab] if all_logits else
        [1, 1, vocab] for the last position. Positions default to
        ``past + arange(n)`` with past = the cache length (the reference's
        cache_position); the sparse draft passes its original positions, as a
        tensor or (without a host-to-device copy) as ``start_position``.

        step_state: a device int32 [2] = (cache length, position of row 0). The
        step then reads both on the device, advances both by n at its end and
        leaves the host lengths alone (graph capture); without it they come
        from the host lengths and start_position, and the host lengths advance."""
        n = input_ids.shape[1]
        x = self.embed(input_ids, visual_embeds)
        host_lengths = step_state is None
        cos = sin = None
        if self.fused_rows(n):
            if host_lengths:
                past = past_key_values[0][0].length
                if start_position is not None:
                    pos0 = int(start_position)
                elif position_ids is not None:
                    pos0 = int(position_ids.reshape(-1)[0])
                else:
                    pos0 = past
                step_state = torch.tensor([past, pos0], dtype=torch.int32).to(self.device)
        else:
            if not host_lengths:
                raise ValueError("a device-state step must have at most 96 query rows per KV head")
            if position_ids is not None:
                position_ids = position_ids.reshape(-1).to(self.device)
            else:
                past = past_key_values[0][0].length if start_position is None else int(start_position)
                position_ids = torch.arange(past, past + n, device=self.device)
            cos, sin = self._rope(position_ids)
        for li in range(self.config.num_hidden_layers):
            kc, vc = past_key_values[li]
            x = self._attention(li, x, cos, sin, kc, vc, step_state, host_lengths)
            x = self._mlp(li, x)
        if not host_lengths:
            ops.len_add(step_state, n)
        if not all_logits:
            x = x[:, -1:]
        if self._hip_rows(x, 1):
            # the final norm in the lm_head launch (std_gemv_norm; 7B: 158.8 us
            # against 163.3 us for the norm launch and the projection)
            return ops.linear(x, self.lm_head, norm_weight=self.norm, eps=self.config.rms_norm_eps)
        return self._linear(self._rms_norm(x, self.norm), self.lm_head)

    __call__ = forward
