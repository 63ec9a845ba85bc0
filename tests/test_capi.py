"""C ABI: the library loads, exports every function include/gdn_capi.h
declares, and rejects bad arguments before touching the GPU (no kernel is
launched in these tests, so they run without one)."""
import ctypes
import os
import re

import pytest
import torch

from conftest import REPO
from engine.kernels import _lib

HEADER = os.path.join(REPO, "include", "gdn_capi.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|size_t|const char \*)\s*\*?\s*(\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: run __graft_entry__.build() first")
    return _lib.load()


def test_header_lists_the_entry_points():
    assert header_functions() == sorted([
        "causal_conv1d_fwd", "causal_conv1d_update", "gdn_abi_version", "gdn_chunk_fwd",
        "gdn_chunk_fwd_gated", "gdn_chunk_workspace_bytes", "gdn_last_error_string", "gdn_recurrent_fwd",
        "gdn_recurrent_fwd_gated", "gdn_rmsnorm_gated_fwd", "gdn_state_commit", "gdn_conv_state_commit", "gdn_in_proj_decode",
        "gdn_out_proj_decode", "gdn_out_proj_workspace_bytes", "gdn_out_proj_decode_noalloc"])


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in header_functions():
        assert hasattr(raw, name), name
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_abi_version(lib):
    assert lib.gdn_abi_version() == _lib.ABI_VERSION == 8


def _rec_call(lib, **over):
    args = dict(q=1, k=1, v=1, qkv_dtype=1, qs=4096, ks=4096, vs=4096, g=1, beta=1, beta_dtype=0,
                sin=None, sin_idx=None, sin_rows=0, sout=None, sout_idx=None, sout_rows=0, o=1, o_dtype=1,
                snap=None, cu=None, n=2, t=1, hk=32, hv=32, kd=128, vd=128, scale=0.1, l2=1, stream=None)
    args.update(over)
    return lib.gdn_recurrent_fwd(*args.values())


def test_recurrent_rejects_unsupported_head_dim(lib):
    # built: K in {64, 128, 256}, V a positive multiple of 32 (valid sizes are
    # not called here: they would launch)
    assert _rec_call(lib, kd=96, vd=128) == 2
    assert "K=96" in lib.gdn_last_error_string().decode()
    assert _rec_call(lib, kd=64, vd=48) == 2
    assert _rec_call(lib, kd=128, vd=0) == 2
    assert _rec_call(lib, kd=512, vd=128) == 2


def test_recurrent_rejects_bad_gqa_and_nulls(lib):
    assert _rec_call(lib, hk=12) == 1
    assert _rec_call(lib, q=None) == 1
    assert _rec_call(lib, snap=1, cu=1) == 1       # snapshots need equal lengths
    assert _rec_call(lib, qs=100) == 1             # stride smaller than a row
    assert _rec_call(lib, n=0) == 0                # empty batch: nothing to do
    assert lib.gdn_last_error_string().decode() == ""


def test_state_rows_must_cover_the_sequences_without_ids(lib):
    # one state row per sequence unless ids select rows; ids outside the rows
    # are handled on the device (no row), so any row count is accepted with ids
    assert _rec_call(lib, sin=256, sin_rows=1) == 1          # 2 sequences, 1 row, no ids
    assert "do not cover" in lib.gdn_last_error_string().decode()
    assert _rec_call(lib, sout=256, sout_rows=-1, sout_idx=256) == 1  # negative row count
    assert _rec_call(lib, sin=256, sin_rows=2, n=0) == 0
    assert lib.causal_conv1d_update(16, 64, 256, None, 1, 1, None, 16, 64, 2, 1, 64, 4, 4, 1, 1, None) == 1


def test_conv_rejects_bad_shapes(lib):
    def call(**over):
        args = dict(x=16, xs=64, w=1, b=None, y=16, ys=64, si=None, sii=None, sir=0, so=None, soi=None, sor=0,
                    cu=None, n=1, t=4, c=64, width=4, sl=4, silu=1, dt=1, stream=None)
        args.update(over)
        return lib.causal_conv1d_fwd(*args.values())
    assert call(c=12, xs=12, ys=12) == 1          # C % 8
    assert call(width=5) == 2
    assert call(sl=5) == 2
    assert call(x=8) == 1                          # misaligned
    assert call(dt=3) == 2                         # no such dtype (0 fp32, 1 bf16, 2 fp16)
    assert call(so=256, sor=0) == 1                # final-state rows do not cover the sequence


def test_commit_rejects_bad_sizes(lib):
    assert lib.gdn_state_commit(1, 1, 4, 1, 1, 2, 0, 32, 128, 128, None) == 1
    assert lib.gdn_state_commit(None, 1, 4, 1, 1, 2, 4, 32, 128, 128, None) == 1
    assert lib.gdn_state_commit(1, 1, -1, 1, 1, 2, 4, 32, 128, 128, None) == 1  # negative pool_rows
    assert lib.gdn_conv_state_commit(1, 1, 4, 1, 1, 2, 8192, 4, 4, 1, None) == 1   # L must exceed S
    assert lib.gdn_conv_state_commit(None, 1, 4, 1, 1, 2, 8192, 4, 8, 1, None) == 1
    assert lib.gdn_conv_state_commit(1, 1, 4, 1, 1, 2, 8192, 4, 8, 3, None) == 2   # dtype
    assert lib.gdn_conv_state_commit(None, None, 0, None, None, 0, 8192, 4, 8, 1, None) == 0  # nothing to do


def test_chunk_workspace_is_host_arithmetic(lib):
    a = lib.gdn_chunk_workspace_bytes(1, 4096, 32, 128, 128)
    b = lib.gdn_chunk_workspace_bytes(4, 4096, 32, 128, 128)
    assert a > 0 and b >= a
    # a batch of 256+ (sequence, v-head) pairs runs one workgroup per pair
    # with all its operands in LDS: no workspace
    assert lib.gdn_chunk_workspace_bytes(8, 4096, 32, 128, 128) == 0
    assert lib.gdn_chunk_workspace_bytes(16, 16 * 1038, 32, 128, 128) == 0


def test_wrappers_refuse_cpu_tensors():
    from engine.kernels import causal_conv1d_fn, chunk_gated_delta_rule, fused_recurrent_gated_delta_rule
    q = torch.zeros(1, 2, 2, 128)
    g = torch.zeros(1, 2, 2)
    with pytest.raises(ValueError, match="GPU"):
        fused_recurrent_gated_delta_rule(q, q, q, g, g)
    with pytest.raises(ValueError, match="GPU"):
        chunk_gated_delta_rule(q, q, q, g, g)
    with pytest.raises(ValueError, match="GPU"):
        causal_conv1d_fn(torch.zeros(1, 8, 4), torch.zeros(8, 4))


def test_monkeypatch_opt_out(monkeypatch):
    from engine.kernels import install_delta_rule_monkeypatch
    monkeypatch.setenv("PARIS_DISABLE_HELION_DELTA", "1")
    assert install_delta_rule_monkeypatch() is False


def test_product_path_never_imports_the_oracle():
    pkg = os.path.join(REPO, "paris-hackathon-2026-inference_amd")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(root, f)).read()
                assert "import oracle" not in src and "from oracle" not in src, f


def _rec_gated_call(lib, **over):
    args = dict(q=1, k=1, v=1, qkv_dtype=1, qs=4096, ks=4096, vs=4096, a=1, b=1, ab_dtype=1, ab_stride=32,
                A_log=1, dt_bias=1, sin=None, sin_idx=None, sin_rows=0, sout=None, sout_idx=None, sout_rows=0,
                o=1, o_dtype=1, snap=None, cu=None, n=2, t=1, hk=32, hv=32, kd=128, vd=128, scale=0.1, l2=1,
                stream=None)
    args.update(over)
    return lib.gdn_recurrent_fwd_gated(*args.values())


def test_gated_entry_points_check_their_gate_arguments(lib):
    assert _rec_gated_call(lib, A_log=None) == 1
    assert "A_log" in lib.gdn_last_error_string().decode()
    assert _rec_gated_call(lib, dt_bias=None) == 1
    assert _rec_gated_call(lib, ab_stride=16) == 1         # stride below Hv
    assert _rec_gated_call(lib, ab_dtype=7) == 1
    assert _rec_gated_call(lib, kd=96, vd=64) == 2          # K not built
    # chunk variant: same gate checks ahead of its own (A_log, then workspace)
    chunk = dict(q=256, k=256, v=256, qkv_dtype=1, qs=4096, ks=4096, vs=4096, a=1, b=1, ab_dtype=1, ab_stride=32,
                 A_log=None, dt_bias=1, h0=None, h0_idx=None, h0_rows=0, hT=None, hT_idx=None, hT_rows=0,
                 o=1, o_dtype=1,
                 cu=None, n=1, t=128, hk=16, hv=32, kd=128, vd=128, scale=0.1, l2=1,  # 2 chunks, 32 pairs: prep + scan
                 ws=None, ws_bytes=0, stream=None)
    assert lib.gdn_chunk_fwd_gated(*chunk.values()) == 1
    chunk.update(A_log=1)
    assert lib.gdn_chunk_fwd_gated(*chunk.values()) == 3   # workspace missing


def test_rmsnorm_gated_rejects_bad_arguments(lib):
    def call(**over):
        args = dict(x=256, xdt=1, xs=4096, z=256, zdt=1, zs=4096, w=256, wdt=1, y=256, ydt=1, ys=4096,
                    n=4, h=32, d=128, eps=1e-6, stream=None)
        args.update(over)
        return lib.gdn_rmsnorm_gated_fwd(*args.values())
    assert call(d=64) == 2
    assert call(x=None) == 1
    assert call(xs=100) == 1                               # stride below H*D
    assert call(x=8) == 1                                  # misaligned rows
    assert call(eps=-1.0) == 1
    assert call(n=0) == 0                                  # nothing to do


def _inproj_call(lib, **over):
    args = dict(x=16, xs=2048, wq=16, wz=16, wb=16, wa=16, m=4, k=2048, nq=8192, nz=4096, nb=32, na=32,
                cw=16, cb=None, pool=16, idx=None, rows=4, y=16, z=16, b=16, a=16, silu=1, stream=None)
    args.update(over)
    return lib.gdn_in_proj_decode(*args.values())


def test_in_proj_decode_rejects_bad_arguments(lib):
    assert _inproj_call(lib, k=1000, xs=1000) == 2
    assert "K=1000" in lib.gdn_last_error_string().decode()
    assert _inproj_call(lib, nq=8190) == 2   # qkv columns not a multiple of 64
    assert _inproj_call(lib, nb=40) == 2     # b wider than 32
    assert _inproj_call(lib, na=6) == 2      # a not a multiple of 4
    assert _inproj_call(lib, xs=1024) == 1   # row stride below K
    assert _inproj_call(lib, pool=None) == 1
    assert _inproj_call(lib, wb=None) == 1   # n_b > 0 needs its weight
    assert _inproj_call(lib, x=24) == 1      # misaligned
    assert _inproj_call(lib, rows=3) == 1    # the pool does not cover row m without ids
    assert "pool rows" in lib.gdn_last_error_string().decode()
    assert _inproj_call(lib, m=0) == 0       # nothing to do, nothing launched



def test_in_proj_python_gate_matches_the_built_hidden_sizes(lib):
    """The layer takes the fused decode input side only for hidden sizes the
    kernel is instantiated for; every other size is refused by the C side."""
    from engine.kernels.in_proj import SUPPORTED_K, fused_in_proj_supported
    for k in (1024, 2048, 3072, 4096):
        gated = fused_in_proj_supported(k, 8192, 4096, 32, 32, 4)
        assert gated == (k in SUPPORTED_K)
        if not gated:
            assert _inproj_call(lib, k=k, xs=k) == 2
    assert not fused_in_proj_supported(2048, 8192, 4096, 32, 32, 3)


def _outproj_call(lib, **over):
    args = dict(x=256, xs=4096, w=256, m=64, k=4096, n=2048, y=256, ys=2048, ws=256, ws_bytes=1 << 30,
                stream=None)
    args.update(over)
    return lib.gdn_out_proj_decode(*args.values())


def test_out_proj_workspace_is_host_arithmetic(lib):
    # the partial sums [splits][row blocks][64 rows][N] fp32, one split per
    # 1024 of K when K is a multiple of 1024, else per 512
    assert lib.gdn_out_proj_workspace_bytes(64, 4096, 2048) == 4 * 64 * 2048 * 4
    assert lib.gdn_out_proj_workspace_bytes(64, 2048, 1024) == 2 * 64 * 1024 * 4
    assert lib.gdn_out_proj_workspace_bytes(64, 3072, 2048) == 3 * 64 * 2048 * 4
    assert lib.gdn_out_proj_workspace_bytes(65, 8192, 2048) == 8 * 2 * 64 * 2048 * 4
    assert lib.gdn_out_proj_workspace_bytes(7, 1536, 128) == 3 * 64 * 128 * 4
    assert lib.gdn_out_proj_workspace_bytes(0, 4096, 2048) == 0


def test_out_proj_decode_rejects_bad_arguments(lib):
    assert _outproj_call(lib, k=4000, xs=4000) == 2        # K not a multiple of 512
    assert "K=4000" in lib.gdn_last_error_string().decode()
    assert _outproj_call(lib, k=16384, xs=16384) == 2      # more than 16 splits
    assert _outproj_call(lib, n=2000, ys=2000) == 2        # N not a multiple of 64
    assert _outproj_call(lib, xs=2048) == 1                # row stride below K
    assert _outproj_call(lib, ys=1024) == 1
    assert _outproj_call(lib, x=24) == 1                   # misaligned
    assert _outproj_call(lib, ws=24) == 1                  # workspace not 16-byte aligned
    assert _outproj_call(lib, ws=None) == 1
    assert _outproj_call(lib, k=3072, xs=3072, ws_bytes=1 << 20) == 1  # too small for 64 rows' partials
    assert "workspace" in lib.gdn_last_error_string().decode()
    assert _outproj_call(lib, m=0) == 0                    # nothing to do, nothing launched


def test_out_proj_python_gate():
    from engine.kernels.in_proj import fused_out_proj_supported
    assert fused_out_proj_supported(4096, 2048) and fused_out_proj_supported(2048, 1024)
    assert not fused_out_proj_supported(4000, 2048) and not fused_out_proj_supported(4096, 2000)
    assert not fused_out_proj_supported(16384, 2048)


def test_out_proj_noalloc_rejects_sizes_beyond_its_scratch(lib):
    """Host-side check, no launch: 512 rows at K = 3072, N = 2048 need 12 MiB
    of partial sums, past the 8 MiB built-in scratch."""
    st = lib.gdn_out_proj_decode_noalloc(16, 3072, 16, 512, 3072, 2048, 16, 2048, None)
    assert st == 2  # GDN_ERR_UNSUPPORTED
    assert b"scratch" in lib.gdn_last_error_string()
