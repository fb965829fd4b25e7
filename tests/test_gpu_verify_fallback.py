"""The reference's optional verification paths of std_generate_qwen25vl
(std_qwen25vl.py:780-893) on the tiny decoders: verify_mode="sequential",
the sequential fallbacks and the margin threshold. Sequential verification
runs the same q_len = 1 dense forwards as dense AR decoding over the same
cache rows, so in bf16 -- where the ten-row parallel verify rounds differently
-- it must reproduce dense AR token for token; in fp32 the parallel and
sequential verifies agree, so a replay accepts nothing extra."""
import pytest
import torch

from std_amd.decoder import DecoderConfig, RandomDecoder
from std_amd.std_qwen25vl import ar_generate_qwen25vl, first_divergence, std_generate_qwen25vl
from std_amd.verification_policy import min_prediction_margin
from tests.gpu_helpers import announce, dev

pytestmark = pytest.mark.gpu

N_VISUAL, N_TEXT, TARGET, NEW = 1000, 24, 256, 40


def _inputs(cfg, seed, dtype):
    gen = torch.Generator().manual_seed(seed)
    text = torch.randint(0, cfg.vocab_size - 2, (N_TEXT,), generator=gen)
    ids = torch.cat([torch.full((N_VISUAL,), cfg.video_token_id), text]).view(1, -1)
    vis = torch.randn(N_VISUAL, cfg.hidden_size, generator=gen)
    return {"input_ids": ids.to(dev()), "visual_embeds": vis.to(dev(), dtype)}


@pytest.fixture(scope="module", params=[torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def case(request):
    dtype = request.param
    cfg = DecoderConfig.tiny(layers=2)
    model = RandomDecoder(cfg, dev(), dtype, seed=5011)
    inputs = _inputs(cfg, 41, dtype)
    ar = ar_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=NEW,
                              ignore_eos=True)
    base, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=NEW, gamma=9,
                                    target_k_plus_text=TARGET, ignore_eos=True)
    return dtype, cfg, model, inputs, ar, base


def _std(case, **kw):
    _, cfg, model, inputs, _, _ = case
    res, _ = std_generate_qwen25vl(model, inputs, cfg.video_token_id, cfg.eos_token_id, max_new_tokens=NEW, gamma=9,
                                   target_k_plus_text=TARGET, ignore_eos=True, **kw)
    assert res.generate_len == NEW and res.accepted_draft_tokens == sum(res.accept_lengths)
    assert all(0 <= a <= p for a, p in zip(res.accept_lengths, res.proposed_lengths))
    return res


def test_sequential_verify_mode_reproduces_dense_ar(case):
    dtype, _, _, _, ar, _ = case
    announce(f"verify_mode=sequential, tiny {dtype}")
    res = _std(case, verify_mode="sequential")
    assert first_divergence(res.output_ids, ar.output_ids) is None
    assert res.fallback_count == 0 and res.verify_margin_reruns == 0
    # the pending bonus token is cached before each sequential round
    assert res.pending_lengths == [0] * res.decode_rounds


def test_sequential_guard_replays_every_round_and_reproduces_dense_ar(case):
    dtype, _, _, _, ar, base = case
    announce(f"verify_fallback=sequential_guard, tiny {dtype}")
    res = _std(case, verify_fallback="sequential_guard")
    assert first_divergence(res.output_ids, ar.output_ids) is None
    assert res.fallback_count == res.decode_rounds
    if dtype == torch.float32:
        assert res.fallback_accepted_extra == 0
        assert res.accept_lengths == base.accept_lengths


def test_sequential_on_reject_and_on_low_accept_count_their_rounds(case):
    dtype, _, _, _, ar, base = case
    announce(f"verify_fallback=sequential_on_reject / sequential_on_low_accept, tiny {dtype}")
    res = _std(case, verify_fallback="sequential_on_reject")
    # a round replays exactly when its accepted length (after any replay, which
    # can only lengthen it) stays below the proposal or was below it before
    assert res.fallback_count >= sum(a < p for a, p in zip(res.accept_lengths, res.proposed_lengths))
    assert res.fallback_count <= res.decode_rounds
    low, _ = std_generate_qwen25vl(case[2], case[3], case[1].video_token_id, case[1].eos_token_id,
                                   max_new_tokens=NEW, gamma=9, target_k_plus_text=TARGET, ignore_eos=True,
                                   verify_fallback="sequential_on_low_accept", sequential_fallback_max_accept=0)
    if dtype == torch.float32:
        # (in bf16 a fully accepted round keeps the parallel verify's rows and predictions, so only the
        # modes that replay every round are held to dense AR there)
        assert first_divergence(res.output_ids, ar.output_ids) is None
        assert res.fallback_accepted_extra == 0 and res.accept_lengths == base.accept_lengths
        assert res.fallback_count == sum(a < p for a, p in zip(base.accept_lengths, base.proposed_lengths))
        assert torch.equal(low.output_ids, base.output_ids)
        assert low.fallback_count == sum(a == 0 < p for a, p in zip(base.accept_lengths, base.proposed_lengths))


def test_margin_threshold_counts_reruns_and_reports_the_smallest_margin(case):
    dtype, _, _, _, _, base = case
    announce(f"verify_margin_threshold, tiny {dtype}")
    margins = []

    def hook(r):
        margins.append(min_prediction_margin(r["logits"].unsqueeze(0), range(r["accept_len"] + 1),
                                             has_dense_pending=r["has_pending"]))

    every = _std(case, verify_margin_threshold=1e9, round_hook=hook)
    # every round is below the threshold: one (math) re-verification each, which the exact HIP verify
    # already is, so the tokens are the plain run's
    assert torch.equal(every.output_ids, base.output_ids) and every.accept_lengths == base.accept_lengths
    assert every.verify_margin_reruns == every.decode_rounds and every.fallback_count == 0
    assert len(margins) == every.decode_rounds - 1          # the hook does not run in the final round
    assert 0.0 <= every.min_verify_margin <= min(m for m in margins if m is not None)
    none = _std(case, verify_margin_threshold=0.0)
    assert none.verify_margin_reruns == 0 and none.min_verify_margin == every.min_verify_margin
    seq = _std(case, verify_fallback="sequential_on_low_margin", verify_margin_threshold=1e9)
    assert seq.fallback_count == seq.decode_rounds and seq.verify_margin_reruns == seq.decode_rounds
    assert first_divergence(seq.output_ids, case[4].output_ids) is None
