"""CPU oracle for the STD decode hot path — TEST INFRASTRUCTURE ONLY.

A numpy (fp64) restatement of the reference's algorithm for each function on
the path, written from the reference files (cited per function), never by
importing them. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
reference results are compared against or as the timed CPU baseline. The
product path (``std_amd``) never imports it and has no CPU fallback.

Modules:
  attention  draft GQA decode (gqa_sdpa) and offset-causal verify (math SDPA)
  selection  causal text-row softmax scores, lowest-index top-K, compaction
  accept     argmax (torch.argmax semantics), greedy prefix, rollback lengths
  collector  the verify pass's visual-attention scores (group-mean query,
             softmax over the visual keys, summed over the positions)
  brute      pure-Python loop versions for tiny inputs (pin the numpy code)

Pinning (each function has at least one independent check in tests/):
  gqa_sdpa / verify_attention   closed-form special cases (uniform keys ->
      mean of V, one dominant key -> its V row), batched == sequential and
      no-future-leakage (reference tests/test_sparse_verify_spike.py:51-80),
      offset mask KAT (:34-49), brute-force loops on tiny shapes.
  selection_scores              invariants (scores >= 0; per KV head the
      scores sum to group * text_len; row sums are 1), brute force on tiny
      shapes, duplicated key columns tie exactly.
  topk_positions                lowest-index tie rule on constructed ties;
      equals a full stable sort.
  compact_index / compact_kv    unique-valued cache fixture of reference
      tests/test_sparse_cache_refresh.py:30-49.
  greedy_prefix / verify_accept KATs of reference tests/test_hsd_spike.py:6-18
      and the pending/no-pending index convention of
      tests/test_verification_fallback.py:45-73.
  rollback_lengths              the closed-form length invariant
      dense_len + |pending| == prompt_len + |generated|.
  verification_scores           brute-force loops on tiny shapes; per KV head
      the scores sum to q_len; mean-query logits equal the mean of the
      group's per-head logits; identical visual keys -> q_len / V each; one
      dominant key takes q_len; keys outside the visual set change nothing.
"""
