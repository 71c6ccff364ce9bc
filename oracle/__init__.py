"""Oracle: CPU restatement of the reference Wan DiT block.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only to check the
HIP results against it (or, for cpu_baseline, as the timed CPU path that is
reported beside the GPU number).  The product path (wam_ops) never imports it and has no CPU fallback.

Modules:
  block   - WanTransformerBlock.forward / WanAttention.forward (fp32 or an
            emulation of the reference's bf16 rounding points), incl. the
            original-mode KV cache and candidate verification.
  kvcache - allocate_slots / update_cache / restore_cache / clear_pred_cache.
  rope    - get_mesh_id grid ids and WanRotaryPosEmbed frequencies.
  metrics - max-abs / cosine / rel-L2 / finiteness (tools/metrics.py:11-47).

Pinning (what checks each function; see tests/test_oracle.py):
  layer_norm, rms_norm, gelu_tanh, sdpa, rope - brute-force float64 loops and
      closed forms (zero-mean/unit-variance, norm preservation of the rotation,
      relative-position invariance of RoPE, softmax of a one-hot score row).
  block_forward composition and the KV cache protocol - golden vectors written
      by tests/golden/make_reference_vectors.py from the reference model.py.
  rope frequencies - closed-form base frequencies and grid ids.
"""
