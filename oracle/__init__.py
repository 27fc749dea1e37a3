"""CPU oracle for the Qwen3 GRPO rollout-and-loss hot path.

TEST INFRASTRUCTURE ONLY.  This package restates, on the CPU, the semantics of
the reference implementation (qwen3_naive.py / qwen3_grpo_train.py of
qwen3-naive-inference) for the functions on the hot path.  It is the checker:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package never imports, calls or
falls back to anything here.

Modules and what pins each one (the checks live in tests/test_oracle_*.py):
  paged      slot mapping, block tables, chained prefix hash, KV store
             -> closed forms, hand-computed known answers, brute force.
  attention  paged decode / varlen paged causal prefill
             -> torch SDPA (library routine) on gathered pages, single-key and
                equal-key closed forms, chunked == unchunked, GQA mapping.
  grpo       log-softmax gather, group advantages, clipped loss + gradient
             -> torch.log_softmax, closed-form advantages, autograd and
                finite differences, hand-computed loss cases.
  norm_rope  RMSNorm, add+RMSNorm, RoPE cache and rotation
             -> torch rms_norm (library), complex-rotation restatement,
                norm preservation, position-0 identity.
  sampling   temperature softmax draw + log-probability of the drawn token
             (Gumbel-max over Philox4x32-10 uniforms)
             -> Philox known-answer vectors of its authors, chi-square of
                the drawn frequencies against softmax, torch.log_softmax.
  workloads  seeded synthetic inputs for the five benchmark configurations.
"""
