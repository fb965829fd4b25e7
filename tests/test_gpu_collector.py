"""GPU parity of the visual-attention collector that rides the verify pass
(std_verify_attn_collect) against the oracle restatement of
VerificationCollectorV3._hook (src/std_repro/dynamic_selection.py:504-519),
and bit-equality of its attention output with the plain verify launch."""
import numpy as np
import pytest
import torch

from oracle import collector as ref_coll
from std_amd import ops
from std_amd.workloads import WORKLOADS, make_layer
from tests.gpu_helpers import announce, cache_buffer, dev

pytestmark = pytest.mark.gpu

# Scores: fp32 sums of exp2 of fp32 logits whose queries carry the fp32 mean
# (bf16 head + bf16 remainder; fp16 head + fp16 remainder for fp16 caches),
# against fp64: relative 2e-4.
RTOL, ATOL = 2e-4, 1e-9


def _layer(wname, layer, prompt_len=None, q_len=None, dtype=torch.bfloat16):
    w = WORKLOADS[wname]
    x = make_layer(w, layer, prompt_len=prompt_len)
    if q_len is not None and q_len != x["q_verify"].shape[2]:
        x = dict(x, q_verify=x["q_verify"][:, :, :q_len].contiguous(), new_k=x["new_k"][:, :, :q_len].contiguous(),
                 new_v=x["new_v"][:, :, :q_len].contiguous())
    if dtype != torch.bfloat16:
        x = {n: x[n].to(dtype) for n in ("q_verify", "k", "v", "new_k", "new_v")}
    k = torch.cat([x["k"], x["new_k"]], 2)
    v = torch.cat([x["v"], x["new_v"]], 2)
    return w, x, k, v


def _check(wname, layer, vis_begin, vis_end, prompt_len=None, q_len=None, append=False, dtype=torch.bfloat16,
           rtol=RTOL):
    w, x, k, v = _layer(wname, layer, prompt_len, q_len, dtype)
    q = x["q_verify"]
    Q, kv_len = q.shape[2], k.shape[2]
    announce(f"collector {wname} layer={layer} kv_len={kv_len} q_len={Q} visual=[{vis_begin},{vis_end}) "
             f"append={append} dtype={dtype}")
    kb = cache_buffer(k, kv_len + 29)
    vb = cache_buffer(v, kv_len + 29)
    qd = q.to(dev())
    want_out = ops.verify_attention(qd, kb[:, :, :kv_len], vb[:, :, :kv_len])
    if append:
        kb2 = cache_buffer(x["k"], kv_len + 29)
        vb2 = cache_buffer(x["v"], kv_len + 29)
        out, scores = ops.verify_attention_collect(qd, kb2, vb2, vis_begin, vis_end, new_key=x["new_k"].to(dev()),
                                                   new_value=x["new_v"].to(dev()), kv_len=kv_len)
        torch.cuda.synchronize()
        assert torch.equal(kb2[:, :, :kv_len], kb[:, :, :kv_len]) and torch.equal(vb2[:, :, :kv_len],
                                                                                    vb[:, :, :kv_len])
    else:
        out, scores = ops.verify_attention_collect(qd, kb, vb, vis_begin, vis_end, kv_len=kv_len)
    torch.cuda.synchronize()
    assert torch.equal(out, want_out), "collector launch changed the verify output"
    want = ref_coll.verification_scores(q, k, np.arange(vis_begin, vis_end))
    got = scores.double().cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, rtol=rtol, atol=ATOL)
    np.testing.assert_allclose(got.sum(axis=1), Q, rtol=1e-4)


def test_collector_c2():
    w = WORKLOADS["c2"]
    _check("c2", 0, 0, w.prompt_len - w.text_len)


def test_collector_c2_append_first_round_rows():
    """Nine verify rows (the first round, no pending token) and the fused append."""
    w = WORKLOADS["c2"]
    _check("c2", 1, 0, w.prompt_len - w.text_len, q_len=9, append=True)


def test_collector_unaligned_visual_range():
    """Visual keys not starting at 0 nor on a 4-key boundary (a system prompt before the video)."""
    _check("c2", 2, 13, 3003, prompt_len=4096)


def test_collector_c4_full_context_lognormal_keys():
    """131082 keys with heavy-tailed key norms, the 128k-context verify."""
    w = WORKLOADS["c4"]
    _check("c4", 0, 0, w.prompt_len - w.text_len, append=True)


@pytest.mark.parametrize("wname", ["c2", "c4"])
def test_collector_fp16(wname):
    """fp16 caches and queries (the dtype the reference loads its model in):
    the same workloads' values converted to fp16, with the fused append. An
    fp16 head + fp16 remainder carries about 22 bits of the mean, so the
    bound is 2e-5 relative (1.9e-6 measured at 131082 keys); a head formed
    twice with different roundings left 4e4 scores beyond 1e-5."""
    w = WORKLOADS[wname]
    _check(wname, 0, 0, w.prompt_len - w.text_len, append=True, dtype=torch.float16, rtol=2e-5)


def test_collector_class_on_a_decoder_verify_forward():
    """VerificationCollectorV3 (the reference's interface) around a bf16 verify
    forward of a two-layer decoder: per-layer scores equal the oracle on that
    forward's rotated queries and cached keys, and the verify logits are the
    same with and without the collector."""
    from std_amd.decoder import DecoderConfig, RandomDecoder
    from std_amd.kv_cache import initialize_past_key_values
    from std_amd.std_qwen25vl import VerificationCollectorV3, prefill_prompt

    announce("collector class on a tiny bf16 decoder verify forward")
    cfg = DecoderConfig.tiny(layers=2)
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=5003)
    gen = torch.Generator().manual_seed(17)
    n_vis, n_text, Q = 1000, 24, 10
    ids = torch.cat([torch.full((n_vis,), cfg.video_token_id),
                     torch.randint(0, cfg.vocab_size - 2, (n_text,), generator=gen)]).view(1, -1).to(dev())
    vis = torch.randn(n_vis, cfg.hidden_size, generator=gen).to(dev(), torch.bfloat16)
    P = n_vis + n_text
    step = torch.randint(0, cfg.vocab_size - 2, (1, Q), generator=gen).to(dev())
    results = []
    for with_collector in (False, True):
        pkv, _, _ = initialize_past_key_values(cfg, dev(), torch.bfloat16, P + 32)
        prefill_prompt(model, {"input_ids": ids, "visual_embeds": vis}, pkv, cfg.video_token_id)
        coll = None
        if with_collector:
            coll = VerificationCollectorV3(model, torch.arange(n_vis))
            coll.install()
            coll.begin_verification(0)
        model.capture_text_queries = True
        logits = model(step, pkv, all_logits=True)
        model.capture_text_queries = False
        if coll is not None:
            coll.end_verification()
            coll.uninstall()
        torch.cuda.synchronize()
        results.append((logits, coll, [q.clone() for q in model.captured_queries], pkv))
    assert torch.equal(results[0][0], results[1][0]), "the collector changed the verify logits"
    _, coll, queries, pkv = results[1]
    scores = coll.latest_scores()
    assert scores.shape == (cfg.num_hidden_layers, cfg.num_key_value_heads, n_vis)
    for li in range(cfg.num_hidden_layers):
        keys = pkv[li][0].data[:, :, :P + Q]
        want = ref_coll.verification_scores(queries[li], keys, np.arange(n_vis))
        np.testing.assert_allclose(scores[li].double().numpy(), want, rtol=RTOL, atol=ATOL)
