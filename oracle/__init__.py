"""CPU oracle for the attention hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline), never as the product path. The product path
(``llm_infer_rust_amd``) runs the HIP library and raises if it is missing.

Each function restates the reference's (MabinogiX/llm_infer_rust) algorithm
in numpy (float64 / float32) or torch-CPU fp32 and cites the file:line it
follows. How each function is pinned (reference fixtures, closed forms,
library routines, brute force):

  bf16.round_bf16 / round_f16     torch's own casts (bit-exact), special values
  kv_store.write_kv               reference fixtures base.rs:232-285, 336-365
  plan.decode_page_metadata       two independent routes (host loop,
                                  masked-select) + hand-computed cases
  plan.prefill_page_metadata      same rules, prefix + extend lengths
  plan.check_work_list            the split-KV partition is this build's own
                                  design (no reference counterpart); checked by
                                  coverage invariants only
  norms.*                         ops.rs:455-479 exact residual fixture,
                                  torch.nn.functional.rms_norm, closed forms
  attention.*                     torch scaled_dot_product_attention (float64),
                                  pure-Python brute force on tiny shapes,
                                  closed forms (one key, identical keys),
                                  reference's eager-vs-padded agreement tests
"""
