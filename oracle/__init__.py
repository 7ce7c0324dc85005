"""CPU oracle for the RoseRLHF hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker (or, in the bench, as the
timed CPU restatement).  The product package ``rosellm_amd`` never imports it
and has no CPU fallback.

Modules:
  * ``roserlhf_oracle`` — PyTorch-CPU restatement of every function on the
    path (rosellm/roserlhf/losses.py, advantages.py), differentiable through
    autograd like the reference's own composition.
  * ``brute`` — float64 scalar-loop forms written from the mathematical
    definitions and the closed-form gradients, used to pin the restatement.
"""
