"""The hot-path ops captured in a HIP graph: every replay, with eager work and
synchronisations in between, reproduces the eager round bit-exactly (the
captured kernels use no memset nodes; workspaces are stream-ordered)."""
import pytest
import torch

from std_amd import ops
from tests.gpu_helpers import announce, dev

pytestmark = pytest.mark.gpu


def _round_inputs(seed):
    gen = torch.Generator(device=dev()).manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device=dev()).to(torch.bfloat16)

    S, P, Q, G = 1034, 2048, 10, 9
    x = dict(
        sparse_k=randn(1, 4, S + 40, 128), sparse_v=randn(1, 4, S + 40, 128),
        dense_k=randn(1, 4, P + Q + 40, 128), dense_v=randn(1, 4, P + Q + 40, 128),
        q_draft=randn(1, 28, 1, 128), nk_draft=randn(1, 4, 1, 128), nv_draft=randn(1, 4, 1, 128),
        q_verify=randn(1, 28, Q, 128), nk_verify=randn(1, 4, Q, 128), nv_verify=randn(1, 4, Q, 128),
        logits=randn(Q, 5000))
    preds = torch.argmax(x["logits"].float(), dim=-1).to(torch.int32)
    draft = preds[:G].clone()
    draft[3] = (draft[3] + 1) % 5000
    x["draft"] = draft
    x["lengths"] = torch.tensor([P + Q, S + 1], dtype=torch.int32, device=dev())
    return x, S, P, Q


def _round(x, S, P, Q):
    d = ops.gqa_decode_append(x["q_draft"], x["sparse_k"], x["sparse_v"], x["nk_draft"], x["nv_draft"], S + 1)
    v = ops.verify_attention_append(x["q_verify"], x["dense_k"], x["dense_v"], x["nk_verify"], x["nv_verify"],
                                    P + Q)
    res = ops.greedy_accept(x["logits"], x["draft"], has_pending=True, rollback_lengths=x["lengths"])
    ops.len_add(x["lengths"][1:], 1)
    return d, v, res


def test_graph_replays_equal_eager_round():
    announce("graph capture of decode_append + verify_append + accept + len_add, 4 replays")
    x, S, P, Q = _round_inputs(31)
    saved = {k: t.clone() for k, t in x.items()}

    def restore():
        for k, t in saved.items():
            x[k].copy_(t)

    d0, v0, r0 = (t.clone() for t in _round(x, S, P, Q))
    state0 = {k: x[k].clone() for k in ("sparse_k", "sparse_v", "dense_k", "dense_v", "lengths")}
    torch.cuda.synchronize()
    assert int(r0[0]) == 3 and x["lengths"].tolist() == [P + Q - 6, S + 1 - 6 + 1]

    restore()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _round(x, S, P, Q)                       # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    restore()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        d, v, r = _round(x, S, P, Q)
    other_q = torch.randn(1, 28, 1, 128, device=dev()).to(torch.bfloat16)
    for rep in range(4):
        restore()
        # unrelated eager work on the same device between replays
        ops.gqa_decode(other_q, x["dense_k"][:, :, :777], x["dense_v"][:, :, :777])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(d, d0) and torch.equal(v, v0) and torch.equal(r, r0), f"replay {rep} differs"
        for k, t in state0.items():
            assert torch.equal(x[k], t), f"replay {rep}: {k} differs"


def test_decoder_step_graph_replays_equal_eager_at_7b_shapes():
    """A 2-layer decoder with the 7B layer and vocabulary shapes: captured AR
    and verify steps replay bit-identically to the eager steps, three times,
    with unrelated eager work between replays. Both read their lengths on the
    device. The AR step is HIP launches only (norm + q/k/v + RoPE + append,
    attention, o/MLP/lm_head GEMVs, argmax); the verify step's q/k/v and
    lm_head projections of several rows are torch GEMMs, the rest HIP."""
    from std_amd.decoder import DecoderConfig, RandomDecoder
    from std_amd.kv_cache import initialize_past_key_values
    from std_amd.std_qwen25vl import _token_argmax, _warm_and_capture

    announce("decoder step graphs vs eager, 7B shapes, 2 layers")
    cfg = DecoderConfig(num_hidden_layers=2)
    model = RandomDecoder(cfg, dev(), torch.bfloat16, seed=3)
    pkv, _, _ = initialize_past_key_values(cfg, dev(), torch.bfloat16, 256)
    gen = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, 150000, (1, 40), generator=gen).to(dev())
    with torch.inference_mode():
        first = _token_argmax(model(prompt, pkv))
        L0 = 40
        state = torch.tensor([L0, L0], dtype=torch.int32, device=dev())
        tok = first.clone()
        draft = torch.randint(0, 150000, (1, 9), generator=gen).to(dev())

        def ar_step():
            logits = model(tok, pkv, step_state=state)
            tok.copy_(_token_argmax(logits))
            return logits

        def verify_step():
            return model(torch.cat([tok, draft], 1), pkv, step_state=state, all_logits=True)

        def run_eager():
            state.copy_(torch.tensor([L0, L0], dtype=torch.int32))
            tok.copy_(first)
            outs = [ar_step().clone() for _ in range(3)]
            outs.append(verify_step().clone())
            torch.cuda.synchronize()
            return outs

        want = run_eager()
        again = run_eager()
        assert all(torch.equal(a, b) for a, b in zip(want, again)), "eager steps are not deterministic"

        def restore():
            state.copy_(torch.tensor([L0, L0], dtype=torch.int32))
            tok.copy_(first)

        (g_ar, out_ar), (g_v, out_v) = _warm_and_capture(lambda: (ar_step(), verify_step()), restore,
                                                          [(ar_step, ()), (verify_step, ())])
        for rep in range(3):
            restore()
            torch.randn(1 << 20, device=dev()).sum()          # unrelated eager work
            torch.cuda.synchronize()
            got = []
            for _ in range(3):
                g_ar.replay()
                got.append(out_ar.clone())
            g_v.replay()
            got.append(out_v.clone())
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(got, want)):
                assert torch.equal(a, b), f"replay {rep}, step {i} differs"
