"""MI355X (gfx950) kernels for the Gated DeltaNet path.

Same import surface as the reference's ``engine.kernels``
(engine/kernels/__init__.py:15-28) for the GDN path, plus the decode,
conv and spec-verify entry points that the reference reached through
third-party packages (fla, causal-conv1d) via HF:

- ``chunk_gated_delta_rule``            chunk-64 prefill (delta_rule.py)
- ``install_delta_rule_monkeypatch``    point HF / fla at these kernels
- ``fused_recurrent_gated_delta_rule``  decode / spec-verify recurrence
- ``recurrent_gated_delta_rule``        HF-signature adapter of the above
- ``causal_conv1d_fn``, ``causal_conv1d_update``
- ``gdn_state_commit``, ``LinearAttentionSlotPool``

All of them run hand-written HIP kernels from ``libgdn_mi355x.so`` through
a C ABI (include/gdn_capi.h); there is no CPU or Triton fallback.
"""
from .causal_conv1d import causal_conv1d_fn, causal_conv1d_update
from .delta_rule import chunk_gated_delta_rule, install_delta_rule_monkeypatch
from .fused_recurrent import fused_recurrent_gated_delta_rule, recurrent_gated_delta_rule
from .state_pool import LinearAttentionSlotPool, gdn_state_commit

__all__ = [
    "chunk_gated_delta_rule",
    "install_delta_rule_monkeypatch",
    "fused_recurrent_gated_delta_rule",
    "recurrent_gated_delta_rule",
    "causal_conv1d_fn",
    "causal_conv1d_update",
    "gdn_state_commit",
    "LinearAttentionSlotPool",
]
