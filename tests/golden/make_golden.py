"""Write tests/golden/oracle_cases.npz: small seeded cases of every hot-path
function with the oracle's outputs (the fixtures the CPU tests hold the
oracle to and the GPU tests hold the HIP path to).

Run from the repository root:  python tests/golden/make_golden.py
Inputs are drawn with torch.Generator seeds (fixed draw order per case) and
stored next to the outputs, so the fixtures do not depend on the generator.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import accept as ref_accept  # noqa: E402
from oracle import attention as ref_attn  # noqa: E402
from oracle import selection as ref_sel  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_cases.npz")
D = 128


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy()


def main() -> None:
    cases = {}
    # decode: 14 query heads / 2 KV heads, S = 96, fp32 and bf16 inputs
    g = torch.Generator().manual_seed(7001)
    q = torch.randn(1, 14, 1, D, generator=g)
    k = torch.randn(1, 2, 96, D, generator=g)
    v = torch.randn(1, 2, 96, D, generator=g)
    cases["decode_f32_q"], cases["decode_f32_k"], cases["decode_f32_v"] = q.numpy(), k.numpy(), v.numpy()
    cases["decode_f32_out"] = ref_attn.gqa_sdpa(q, k, v)
    qb, kb, vb = (x.to(torch.bfloat16) for x in (q, k, v))
    cases["decode_bf16_q"], cases["decode_bf16_k"], cases["decode_bf16_v"] = bf16_bits(qb), bf16_bits(kb), bf16_bits(vb)
    cases["decode_bf16_out"] = ref_attn.gqa_sdpa(qb, kb, vb)

    # verify: q_len 6 (row i sees keys [0, 100 - 6 + i]), 14/2 heads, kv_len 100, bf16
    g = torch.Generator().manual_seed(7002)
    q = torch.randn(1, 14, 6, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, 100, D, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 2, 100, D, generator=g).to(torch.bfloat16)
    cases["verify_bf16_q"], cases["verify_bf16_k"], cases["verify_bf16_v"] = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    cases["verify_bf16_out"] = ref_attn.verify_attention(q, k, v)

    # selection: 14/2 heads, prompt 160 = 152 visual + 8 text, k = 24, bf16.
    # In each head the rank-k column's key row is copied bit-exactly to a later
    # visual position, so the k-th and (k+1)-th scores tie at the selection
    # boundary and the lower position must win.
    g = torch.Generator().manual_seed(7003)
    P, T, kk = 160, 8, 24
    q_text = torch.randn(1, 14, T, D, generator=g).to(torch.bfloat16)
    key = torch.randn(1, 2, P, D, generator=g).to(torch.bfloat16)
    visual = np.arange(P - T)
    for h in range(2):
        base = ref_sel.selection_scores(q_text, key, P - T)
        order = sorted(visual, key=lambda c: (-base[h, c], c))
        for cand in order[kk - 6:kk + 6]:
            for dst in sorted(set(visual) - set(order[:kk + 1]), reverse=True):
                if dst <= cand:
                    continue
                trial = key.clone()
                trial[:, h, dst] = trial[:, h, cand]
                sc = ref_sel.selection_scores(q_text, trial, P - T)
                top = ref_sel.topk_positions(sc, visual, kk)[h]
                if cand in top and dst not in top and sc[h, cand] == sc[h, dst] and \
                        sc[h, cand] == min(sc[h, c] for c in top):
                    key = trial
                    break
            else:
                continue
            break
        else:
            raise RuntimeError(f"no boundary tie found for head {h}")
    scores = ref_sel.selection_scores(q_text, key, P - T)
    cases["select_q_text"], cases["select_key"] = bf16_bits(q_text), bf16_bits(key)
    cases["select_meta"] = np.array([P, T, kk], dtype=np.int64)
    cases["select_scores"] = scores
    cases["select_topk"] = ref_sel.topk_positions(scores, visual, kk)
    non_visual = np.arange(P - T, P)
    cases["compact_index"] = np.stack([ref_sel.compact_index(non_visual, cases["select_topk"][h]) for h in range(2)])

    # acceptance: 10 rows over a 1000-token vocabulary, accept length 4, with
    # and without a pending token
    g = torch.Generator().manual_seed(7004)
    logits = torch.randn(10, 1000, generator=g)
    preds = ref_accept.verify_predictions(logits, True)
    draft = list(preds[:9])
    draft[4] = (draft[4] + 1) % 1000
    cases["accept_logits"] = logits.numpy()
    cases["accept_draft"] = np.array(draft, dtype=np.int32)
    cases["accept_pending"] = np.array(ref_accept.verify_accept(logits, draft, True)[:2], dtype=np.int64)
    dense_next = preds[0]
    cases["accept_no_pending_logits_rows"] = np.array(9, dtype=np.int64)
    cases["accept_no_pending_dense_next"] = np.array(dense_next, dtype=np.int64)
    cases["accept_no_pending"] = np.array(ref_accept.verify_accept(logits[:9], draft, False, dense_next)[:2],
                                          dtype=np.int64)
    np.savez_compressed(OUT, **cases)
    print(f"wrote {OUT}: {len(cases)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
