"""CPU oracle for the ALoDLM training step (TEST INFRASTRUCTURE ONLY).

This package restates, on the CPU in plain PyTorch eager (float32 or float64),
the reference training step of amazon-science/ALoDLM: the dual-stream batch
builder, the Qwen3 decoder layer, the recurrent rollout with the halting gate,
the NELBO objective with sequence-level credit, the autoregressive auxiliary
loss, gradient clipping and AdamW.  Every function cites the reference
file:line it follows.

Only the test-suite, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker.  The product package
``alodlm_amd`` never imports it and has no CPU fallback.

Pinning (each function is checked by tests/test_oracle.py):
  * build_batch / attention_mask / sparse_plan: golden vectors written by
    tests/golden/make_golden.py from the reference, the reference's own
    known-answer tests (test_objective.py:88-105) and the closed-form density.
  * outcome_loss: the reference's analytic restatement (test_objective.py:32-74)
    and golden vectors.
  * sequence_score_function: the reference's known answer (test_objective.py:22-30).
  * autoregressive_loss: the reference's known answer (test_objective.py:76-86).
  * decoder layer / rollout / full step: golden vectors of the integrated step
    (loss, metrics, gates, exits and every gradient) written by
    tests/golden/make_golden.py, plus torch SDPA / brute-force attention.
  * gate init: the uniform-mass known answer (test_gate.py:18-30).
  * AdamW / cosine schedule / clip: closed form of the first step and
    torch.optim.AdamW.
  * masking draws on a Philox device generator (draws.py): the Random123
    known-answer vectors, and torch's own device draws on a GPU.
"""

from .step import *  # noqa: F401,F403
