"""MI355X (gfx950) attention hot path of the Rust mini-sglang server.

Host-side mirror of the reference's attention-backend seam over the C ABI of
``libmi355x_attn.so`` (declared in ``include/mi355x_attn.h``):

* ``backend``  — ``Attention`` / ``AttentionBatch`` / decode plans (the new
  ``--attention-backend mi355x`` value);
* ``prefill``  — ragged and paged causal prefill plans;
* ``kv_cache`` — KV-pool layout and ``BaseAttention.write_kv``;
* ``ops``      — RMSNorm, residual-RMSNorm, QK-norm.

The HIP library is the only compute path; importing the ops without it built
raises on first use.
"""

__all__ = ["backend", "kv_cache", "ops", "prefill"]
