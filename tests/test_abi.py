"""The C-ABI library loads and exports every symbol include/flashgrpo_amd.h declares (no GPU calls)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashgrpo_amd.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(fg_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from flashgrpo_amd import _lib

    assert _declared() == _lib.exported_symbols()


def test_library_exports_every_declared_symbol():
    from flashgrpo_amd import _lib

    path = _lib.library_path()
    if not os.path.exists(path):
        pytest.skip("native library not built (run __graft_entry__.build())")
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (fg_[a-z0-9_]+)", out))
    missing = [s for s in _declared() if s not in exported]
    assert not missing, missing


def test_library_loads_and_reports_errors_without_gpu_work():
    from flashgrpo_amd import _lib

    if not os.path.exists(_lib.library_path()):
        pytest.skip("native library not built")
    lib = _lib.load()
    assert lib.fg_version() == 1
    # A shape error is caught on the host before any launch.
    rc = lib.fg_kv_path_gather(None, 0, 0, 0, 0, 2, 0, 0, 0, 0, None, None, None, 0, None, 0, None, None)
    assert rc != 0 and b"null pointer" in lib.fg_last_error()
    rc = lib.fg_sample_tokens(ctypes.c_void_p(64), 1, 8, 1, 0, None, None, None, 0, 0, 0, 0, None, 0, 1.0, 0, 0, 0,
                              ctypes.c_void_p(64), None, 0, None)
    assert rc != 0 and b"vocab" in lib.fg_last_error()
    assert lib.fg_sample_workspace(64) >= 64 * 16 * 20 and lib.fg_sample_workspace(0) == 0
    # the fused MLP GEMM: K (hidden) must be a multiple of 64, tile heights 64 / 128 / 192 / 256 only
    p = ctypes.c_void_p(256)
    rc = lib.fg_gate_up_swiglu(p, 96, p, 96, p, 8, 4, 8, 96, 0, None)
    assert rc != 0 and b"multiple of 64" in lib.fg_last_error()
    rc = lib.fg_gate_up_swiglu(p, 64, p, 64, p, 8, 4, 8, 64, 96, None)
    assert rc != 0 and b"tile_rows" in lib.fg_last_error()
    # the split-K projection: K a multiple of 64, every split non-empty, 2-4 ring stages
    rc = lib.fg_linear_parts(p, 96, p, 96, p, 8, 16, 96, 1, 64, 64, 0, None)
    assert rc != 0 and b"multiple of 64" in lib.fg_last_error()
    rc = lib.fg_linear_parts(p, 192, p, 192, p, 8, 16, 192, 4, 64, 64, 0, None)
    assert rc != 0 and b"splits" in lib.fg_last_error()
    rc = lib.fg_linear_parts(p, 192, p, 192, p, 8, 16, 192, 3, 64, 64, 5, None)
    assert rc != 0 and b"stages" in lib.fg_last_error()
    rc = lib.fg_linear_parts(p, 192, p, 192, p, 8, 16, 192, 3, 256, 64, 0, None)
    assert rc != 0 and b"tile_m" in lib.fg_last_error()
    # the q/k/v projection with its rotary epilogue: rows = batch * num_nodes, tiles of 64 / 128
    args = [p, 128, p, 128, None, 8, 128, 64, 64, 0, 2, 4, 4, 1, 64, p, p, p, p, p, 64 * 16, 64 * 16, 16,
            None, None, None]
    assert lib.fg_linear_rope_kv_write(*args[:5], 7, *args[6:]) != 0 and b"batch * num_nodes" in lib.fg_last_error()
    assert lib.fg_linear_rope_kv_write(*args[:7], 96, *args[8:]) != 0 and b"tile_m" in lib.fg_last_error()
    assert lib.fg_linear_rope_kv_write(*args[:14], 12, *args[15:]) != 0 and b"head_dim" in lib.fg_last_error()
    assert lib.fg_rope_cos_sin(p, p, 0, p, 2, 4, 63, p, None) != 0 and b"bad shape" in lib.fg_last_error()
    rc = lib.fg_residual_rmsnorm_parts(p, 1, 4, 12, p, 12, p, 1e-6, p, 12, None)
    assert rc != 0 and b"multiple of 8" in lib.fg_last_error()
    rc = lib.fg_gate_up_swiglu(None, 64, p, 64, p, 8, 4, 8, 64, 0, None)
    assert rc != 0 and b"null pointer" in lib.fg_last_error()
    rc = lib.fg_chain_cell_norm(p, 12, p, 12, 1, 4, 12, p, p, p, p, 1e-5, p, None)
    assert rc != 0 and b"multiple of 8" in lib.fg_last_error()


def test_tree_attention_split_policy():
    """Key split only when sequences x kv heads leave the chip idle (host-side sizing)."""
    from flashgrpo_amd import _lib

    lib = _lib.load()
    assert lib.fg_tree_attention_workspace(64, 29, 28, 4, 128, 2640) == 0      # 7B rounds: 256 workgroups
    small = lib.fg_tree_attention_workspace(16, 29, 28, 4, 128, 2640)          # 16 sequences, 2k keys: 64 workgroups
    assert small > 16 * 29 * 28 * 128 * 4                                        # at least two parts of fp32 O
    assert lib.fg_tree_attention_workspace(32, 13, 12, 2, 128, 900) == 0       # parts would be under 8 tiles
    assert lib.fg_tree_attention_workspace(2, 13, 12, 2, 64, 900) == 0         # fp32-only head dim


def test_rope_pair_rows_interleaves_each_q_and_k_head():
    import torch

    from flashgrpo_amd import kernels as K

    Hq, Hkv, d = 2, 1, 8
    rows = torch.arange((Hq + 2 * Hkv) * d)
    got = K.rope_pair_rows(rows, Hq, Hkv, d).tolist()
    pairs = lambda h: [h * d + (j // 2 if j % 2 == 0 else d // 2 + j // 2) for j in range(d)]
    assert got == pairs(0) + pairs(1) + pairs(2) + list(range(3 * d, 4 * d))  # v head in order
    w = torch.randn((Hq + 2 * Hkv) * d, 5)
    assert torch.equal(K.rope_pair_rows(w, Hq, Hkv, d)[1], w[4])
