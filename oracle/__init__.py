"""CPU oracle of the self-speculative decode step — TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithms on the CPU (numpy for integer / selection work,
torch fp32 on the CPU for the floating-point layers) so the GPU kernels can be checked against it.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only as the
checker or the timed CPU baseline. The product (trida_stack_amd) never imports it and has no CPU
fallback.

Modules and what pins them (the reference ships no golden vectors for this path):
  accept     greedy + rejection-sampling acceptance   pinned by brute force on tiny vocabularies,
                                                      closed forms and hand-computed cases
  gdn        gated-delta rule, conv, prep, rollback   pinned by transformers' torch GDR fixtures
                                                      (tests/golden), recurrent == chunked,
                                                      split-carry and snapshot invariants
  attention  canvas attention with draft/verify masks pinned by torch SDPA on explicit masks and
                                                      a per-query brute-force softmax
  model      CPU hybrid decoder + decode loops        pinned by canvas-clean-rows == AR logits,
                                                      commit == AR state, greedy self-spec == AR
"""
