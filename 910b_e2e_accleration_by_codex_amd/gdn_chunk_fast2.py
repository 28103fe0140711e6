"""The ``--gdn-v2`` name of the chunked prefill (src/gdn_chunk_fast2.py:11-62).

In the reference v2 differs from v1 only in how the torch ops are batched; both compute the same
recurrence.  Here both names run the single fused HIP kernel of gdn_chunk_fast.py.
"""
from .gdn_chunk_fast import chunk_gated_delta_rule


def fast_chunk_gated_delta_rule_v2(query, key, value, g, beta, chunk_size=64, initial_state=None,
                                   output_final_state=False, use_qk_l2norm_in_kernel=False, **kwargs):
    """Signature of src/gdn_chunk_fast2.py:11-12 (plus ``cu_seqlens`` through kwargs)."""
    return chunk_gated_delta_rule(query, key, value, g, beta, chunk_size, initial_state,
                                  output_final_state, use_qk_l2norm_in_kernel, **kwargs)
