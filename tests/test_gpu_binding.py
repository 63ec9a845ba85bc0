"""The reference's own binding on the MI355X: ``install_delta_rule_monkeypatch``.

The reference installs its delta-rule kernel by rebinding module-level
functions before the model is built (engine/model/qwen3_next.py:104-115 ->
engine/kernels/delta_rule.py:446-480), and HF's GDN layer then calls them
with its own argument forms (transformers modeling_qwen3_5_moe.py:430-541):
keyword ``g=`` / ``beta=``, q and k repeated to the 32 v-heads
(``repeat_interleave``), ``cu_seqlens=None``, ``**kwargs``, the conv input as
a ``[B, C, T]`` transposed view, and the ``DynamicCache``'s own conv and
recurrent state tensors (the conv window updated in place by
``causal_conv1d_update``).

This test runs transformers' unmodified ``Qwen3_5MoeGatedDeltaNet.forward``
on the GPU in bf16 after the installer, checks that the module functions it
resolves are the HIP entry points, and compares a prefill and three cached
decode steps with the fixture of HF's fp32 forward (the same values the
fused layer forward is checked against in test_gpu_layer).  The module's
attributes are restored afterwards.

Tolerances as in test_gpu_layer: outputs max abs error <= 3e-2 * max|ref|,
states relative error <= 1e-2, conv windows max abs error <= 2e-2.
"""
import numpy as np
import pytest
import torch

from oracle import gdn

import layer_cases as lc

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

DEV = "cuda"
PATCHED = ("torch_chunk_gated_delta_rule", "torch_recurrent_gated_delta_rule", "causal_conv1d_fn",
           "causal_conv1d_update", "chunk_gated_delta_rule", "fused_recurrent_gated_delta_rule",
           "is_fast_path_available")


@pytest.fixture
def patched_hf(monkeypatch):
    """Run the installer with every attribute it may touch saved first;
    monkeypatch restores them when the test ends."""
    import importlib
    monkeypatch.delenv("PARIS_DISABLE_HELION_DELTA", raising=False)
    mods = []
    for name in ("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe",
                 "transformers.models.qwen3_5.modeling_qwen3_5",
                 "transformers.models.qwen3_next.modeling_qwen3_next"):
        try:
            mods.append(importlib.import_module(name))
        except Exception:
            continue
    for mod in mods:
        for attr in PATCHED:
            if hasattr(mod, attr):
                monkeypatch.setattr(mod, attr, getattr(mod, attr))
    from engine.kernels import install_delta_rule_monkeypatch
    assert install_delta_rule_monkeypatch() is True
    return mods[0]


def test_installer_binds_hf_gdn_functions_to_the_hip_entry_points(patched_hf):
    from engine import kernels
    hf = patched_hf
    assert hf.torch_chunk_gated_delta_rule is kernels.chunk_gated_delta_rule
    assert hf.torch_recurrent_gated_delta_rule is kernels.recurrent_gated_delta_rule
    assert hf.causal_conv1d_fn is kernels.causal_conv1d_fn
    assert hf.causal_conv1d_update is kernels.causal_conv1d_update
    # the layer forward itself stays HF's (only its module functions are rebound)
    assert hf.Qwen3_5MoeGatedDeltaNet.forward is not kernels.gated_delta_net_forward


def test_hf_forward_through_the_installed_kernels_matches_hf(patched_hf):
    from transformers.cache_utils import DynamicCache
    from engine.kernels import _lib
    hf = patched_hf
    golden = lc.load_golden()
    cfg, layer = lc.gpu_layer("tiny", golden)
    assert type(layer).forward is hf.Qwen3_5MoeGatedDeltaNet.forward
    _lib.load()  # the HIP library, not a fallback
    cache = DynamicCache(config=cfg)
    with torch.no_grad():
        for i in range(4):
            x = torch.from_numpy(golden[f"cache.x{i}"]).to(DEV, torch.bfloat16)
            y = layer(x, cache_params=cache)  # HF's own forward: prefill (B=2, T=70), then 3 decode steps
            print(f"HF forward through the installed kernels, step {i}", flush=True)
            assert lc.layer_close(y, golden[f"cache.y{i}"]), i
    s_gpu = cache.layers[0].recurrent_states[0].float().cpu().numpy().astype(np.float64)
    assert gdn.state_rel_err(s_gpu, golden["cache.state"].astype(np.float64)) < 1e-2
    conv = cache.layers[0].conv_states[0]
    assert conv.dtype == torch.bfloat16  # the cache's own tensor, updated in place by the kernel
    assert lc.conv_close(conv[0], golden["cache.conv"][:1]) and lc.conv_close(conv[1], golden["cache.conv"][1:])
