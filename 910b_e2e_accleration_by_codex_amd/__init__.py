"""MI355X-native (gfx950 HIP) Gated DeltaNet hot path with the reference's Python interface.

Public functions keep the reference's names and signatures:
  fast_chunk_gated_delta_rule     (src/gdn_chunk_fast.py:65)   chunked prefill, v1 name
  fast_chunk_gated_delta_rule_v2  (src/gdn_chunk_fast2.py:11)  chunked prefill, v2 name
  recurrent_single_step           (src/recurrent_single_step.py:8)
  elem_conv_update, patch_model   (src/cb_engine.py:43, :54)
plus the fused layer cores (gdn_decode_core, gdn_prefill_core), the conv prefill, the gated norm
and the slot-state / graph helpers of the engine.  All compute runs in libgdn_mi355x.so; there is
no CPU fallback.
"""
from ._lib import GDNError, LIB_PATH
from .recurrent_single_step import recurrent_single_step
from .cb_engine import (ELEM_CONV, GDNDecodeGraph, GDNSlots, causal_conv1d_update, elem_conv_update,
                        fused_gated_rmsnorm, fused_rmsnorm, gated_rmsnorm, gdn_decode_core, gdn_decode_layer,
                        patch_model)
from .gdn_chunk_fast import (Rows, Varlen, _unit_lower_inv, causal_conv1d_prefill, chunk_gated_delta_rule,
                             chunk_inverse_records, fast_chunk_gated_delta_rule, gdn_gating, gdn_prefill_core)
from .gdn_chunk_fast2 import fast_chunk_gated_delta_rule_v2

__all__ = [
    "GDNError", "LIB_PATH", "recurrent_single_step", "ELEM_CONV", "GDNDecodeGraph", "GDNSlots",
    "causal_conv1d_update", "elem_conv_update", "fused_gated_rmsnorm", "fused_rmsnorm", "gated_rmsnorm",
    "gdn_decode_core", "gdn_decode_layer", "patch_model", "_unit_lower_inv",
    "causal_conv1d_prefill", "chunk_gated_delta_rule", "fast_chunk_gated_delta_rule", "gdn_gating",
    "gdn_prefill_core", "Varlen", "Rows", "chunk_inverse_records",
    "fast_chunk_gated_delta_rule_v2",
]
