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
- ``gdn_state_commit``, ``gdn_conv_state_commit``
- ``chunk_gated_delta_rule_from_projections``,
  ``fused_recurrent_gated_delta_rule_from_projections``  gates computed in
  the kernels from the layer's raw a / b projections
- ``rms_norm_gated``                    the GDN output norm in one pass
- ``gdn_in_proj_decode``                a decode step's four input projections
  and the conv update in one kernel (in_proj.py)
- ``gdn_out_proj_decode``               a decode step's output projection,
  K split over workgroups (in_proj.py)
- ``gated_delta_net_forward``, ``install_gdn_layer_patch``  HF's GDN layer
  forward on these kernels (native GQA, fused gates and norm)

The engine side (slot-indexed pools in place of the reference cache's
gather/scatter, and the speculative-verify rollback) is
:mod:`engine.runtime.slot_pools`.

All of them run hand-written HIP kernels from ``libgdn_mi355x.so`` through
a C ABI (include/gdn_capi.h); there is no CPU or Triton fallback.
"""
from .causal_conv1d import causal_conv1d_fn, causal_conv1d_update
from .delta_rule import (chunk_gated_delta_rule, chunk_gated_delta_rule_from_projections,
                         install_delta_rule_monkeypatch)
from .fused_recurrent import (fused_recurrent_gated_delta_rule, fused_recurrent_gated_delta_rule_from_projections,
                              recurrent_gated_delta_rule)
from .gdn_layer import gated_delta_net_forward, install_gdn_layer_patch, rms_norm_gated
from .in_proj import gdn_in_proj_decode, gdn_out_proj_decode
from .state_pool import gdn_conv_state_commit, gdn_state_commit

__all__ = [
    "chunk_gated_delta_rule",
    "install_delta_rule_monkeypatch",
    "fused_recurrent_gated_delta_rule",
    "recurrent_gated_delta_rule",
    "causal_conv1d_fn",
    "causal_conv1d_update",
    "gdn_state_commit",
    "gdn_conv_state_commit",
    "chunk_gated_delta_rule_from_projections",
    "fused_recurrent_gated_delta_rule_from_projections",
    "rms_norm_gated",
    "gdn_in_proj_decode",
    "gdn_out_proj_decode",
    "gated_delta_net_forward",
    "install_gdn_layer_patch",
]
