"""C ABI checks that need no GPU: the library loads, exports every function
include/msst_hip.h declares, and rejects bad arguments on the host before
any launch (the reference only asserts, and its asserts vanish under
-DNDEBUG, ops_attention.cu:525-534 / CMakeLists.txt:28)."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "msst_hip.h")

OK, INVALID, UNSUPPORTED, ALIGN, LAUNCH, WORKSPACE = 0, -1, -2, -3, -4, -5


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(msst_\w+)\s*\(", text)))


def test_library_exports_every_declared_function(msst):
    lib = msst.lib()
    names = declared_functions()
    assert len(names) >= 18
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares a signature for each of them
    assert sorted(msst.EXPORTED) == names


def test_status_strings(msst):
    lib = msst.lib()
    assert lib.msst_abi_version() == 1
    assert lib.msst_status_string(OK) == b"ok"
    assert lib.msst_status_string(WORKSPACE) == b"workspace too small"


def test_host_rope_table_matches_oracle_bit_exact(msst, oracle):
    for n in (1, 62, 801):
        c, s = msst.rope_table(n, 64)
        oc, os_ = oracle.rope_table(n, 64)
        np.testing.assert_array_equal(c, oc)
        np.testing.assert_array_equal(s, os_)


def _last(msst):
    return msst.lib().msst_last_error().decode()


def test_linear_rejects_bad_arguments(msst):
    lib = msst.lib()
    p = ctypes.c_void_p(0x1000)
    rc = lib.msst_linear(None, 0, p, 0, None, None, p, 0, 4, 4, 4, 0, None)
    assert rc == INVALID and "null" in _last(msst)
    rc = lib.msst_linear(p, 7, p, 0, None, None, p, 0, 4, 4, 4, 0, None)
    assert rc == INVALID
    rc = lib.msst_linear(p, 0, p, 0, None, None, p, 0, 4, 0, 4, 0, None)
    assert rc == INVALID
    rc = lib.msst_linear(p, 0, p, 0, None, None, p, 0, 4, 4, 4, 9, None)
    assert rc == INVALID and "activation" in _last(msst)
    odd = ctypes.c_void_p(0x1002)
    rc = lib.msst_linear(odd, 0, p, 0, None, None, p, 0, 4, 4, 4, 0, None)
    assert rc == ALIGN
    # M == 0 is a no-op, not an error
    assert lib.msst_linear(p, 0, p, 0, None, None, p, 0, 0, 4, 4, 0, None) == OK


def test_attention_rejects_unsupported_head_dim(msst):
    lib = msst.lib()
    p = ctypes.c_void_p(0x1000)
    for D in (0, 257, 300):
        rc = lib.msst_attention(p, p, p, p, 0, 1, 1, 8, 8, D, 0.0, None)
        assert rc == UNSUPPORTED and "256" in _last(msst)
    # D = 64 (MFMA kernels) needs 16-byte alignment; other D element alignment.
    rc = lib.msst_attention(p, p, p, ctypes.c_void_p(0x1008), 0, 1, 1, 8, 8, 64, 0.0, None)
    assert rc == ALIGN
    rc = lib.msst_attention(p, p, p, ctypes.c_void_p(0x1002), 0, 1, 1, 8, 8, 32, 0.0, None)
    assert rc == ALIGN
    rc = lib.msst_attention(p, p, p, ctypes.c_void_p(0x1001), 1, 1, 1, 8, 8, 32, 0.0, None)
    assert rc == ALIGN


def test_gated_attention_rejects_short_rows(msst):
    lib = msst.lib()
    p = ctypes.c_void_p(0x1000)
    L = msst.seq_layout(1, 1, 8, 8, 0, 1)
    rc = lib.msst_gated_rope_attention(p, 1, 3 * 8 * 64 - 8, None, None, None, p, 512,
                                       ctypes.byref(L), 8, 64, 0.0, None)
    assert rc == INVALID
    rc = lib.msst_gated_rope_attention(p, 1, 3 * 8 * 64, p, None, None, p, 512, ctypes.byref(L),
                                       8, 64, 0.0, None)
    assert rc == INVALID and "cos" in _last(msst)


def test_norm_gate_rejects_too_many_gates(msst):
    lib = msst.lib()
    p = ctypes.c_void_p(0x1000)
    rc = lib.msst_rms_norm_gate(p, 0, p, 1.0, p, 0, p, 0, p, p, 4, 64, 17, None)
    assert rc == UNSUPPORTED


def test_stack_workspace_and_validation(msst):
    lib = msst.lib()
    d = msst.StackDesc(1, 801, 62, 512, 8, 64, 2048, 12, msst.F16)
    ws = lib.msst_roformer_stack_workspace(ctypes.byref(d))
    M = 801 * 62
    # xn + max(qkv, hidden) + merged (fp16) + gates, plus tables (x is worked on in place)
    assert ws >= M * 512 * 2 + M * 2048 * 2 + M * 512 * 2 + M * 8 * 4
    assert ws < 1.1 * (M * 512 * 2 + M * 2048 * 2 + M * 512 * 2 + M * 8 * 4) + 2**20
    bad = msst.StackDesc(1, 801, 62, 512, 8, 32, 2048, 12, msst.F16)
    assert lib.msst_roformer_stack_workspace(ctypes.byref(bad)) < 0
    p = ctypes.c_void_p(0x1000)
    rc = lib.msst_roformer_stack(p, ctypes.byref(d), None, None, p, ws, None)
    assert rc == INVALID  # depth 12 needs layer weights
    d0 = msst.StackDesc(1, 801, 62, 512, 8, 64, 2048, 0, msst.F16)
    ws0 = lib.msst_roformer_stack_workspace(ctypes.byref(d0))
    rc = lib.msst_roformer_stack(p, ctypes.byref(d0), None, None, p, ws0 - 256, None)
    assert rc == WORKSPACE
    rc = lib.msst_roformer_stack(p, ctypes.byref(d0), None, None, ctypes.c_void_p(0x1010), ws0,
                                 None)
    assert rc == ALIGN


def test_product_does_not_reference_oracle():
    """The shipped sources never include, link or load the oracle."""
    pkg = os.path.join(ROOT, "cuda-msst-infer_amd")
    for dirpath, _, files in os.walk(pkg):
        if "_build" in dirpath:
            continue
        for f in files:
            if f.endswith((".hip", ".cpp", ".hpp", ".h", ".py", "Makefile")):
                text = open(os.path.join(dirpath, f), errors="ignore").read().lower()
                for needle in ("msst_oracle", "import oracle", "from oracle", "orc_"):
                    assert needle not in text, (f, needle)


def _band_cfg(msst, dims, dim=64, hidden=128, L=2):
    arr = (ctypes.c_int * len(dims))(*dims)
    return msst.BandConfig(len(dims), arr, dim, hidden, L, 0, 0, None), arr


def test_band_config_validation(msst):
    lib = msst.lib()
    cfg, _keep = _band_cfg(msst, [4, 8, 130])
    # header 256-aligned + dim * sum(ceil64(dims)) halves
    n = lib.msst_band_plan_bytes(ctypes.byref(cfg))
    assert n > 0 and n % 2 == 0 and n >= 64 * (64 + 64 + 192) * 2
    assert lib.msst_band_split_workspace(ctypes.byref(cfg), 10) >= 10 * 320 * 2
    for dims, dim, hid, L in (([3], 64, 128, 2),          # odd band dim
                              ([2] * 65, 64, 128, 2),     # too many bands
                              ([4], 60, 128, 2),          # dim not a multiple of 64
                              ([4], 64, 100, 2),          # hidden not a multiple of 64
                              ([4], 64, 128, 9),          # too many linears
                              ([2048], 64, 128, 2)):      # band wider than 1024
        cfg, _k = _band_cfg(msst, dims, dim, hid, L)
        assert lib.msst_band_plan_bytes(ctypes.byref(cfg)) == -1
        rc = lib.msst_band_split(ctypes.byref(cfg), ctypes.c_void_p(256), ctypes.c_void_p(256), 4,
                                 ctypes.c_void_p(256), ctypes.c_void_p(256), 1 << 20, None)
        assert rc == UNSUPPORTED, _last(msst)


def test_band_calls_reject_before_launch(msst):
    lib = msst.lib()
    cfg, _keep = _band_cfg(msst, [4, 8])
    p = ctypes.c_void_p(4096)
    assert lib.msst_band_split(ctypes.byref(cfg), None, p, 4, p, p, 1 << 20, None) == INVALID
    assert lib.msst_band_split(ctypes.byref(cfg), p, p, 4, p, p, 8, None) == WORKSPACE
    assert lib.msst_mask_estimator(ctypes.byref(cfg), p, p, 7, 4, p, p, 1 << 20, None) == INVALID
    assert lib.msst_mask_estimator(ctypes.byref(cfg), p, p, 0, 4, p, p, 8, None) == WORKSPACE
    assert lib.msst_mask_estimator(ctypes.byref(cfg), p, ctypes.c_void_p(4098), 0, 4, p, p,
                                   1 << 20, None) == ALIGN
    # plan init: misaligned plan, too-small plan (no device memory is touched)
    assert lib.msst_band_plan_init(ctypes.byref(cfg), None, None, None, None, None,
                                   ctypes.c_void_p(4100), 1 << 20, None) == ALIGN
    assert lib.msst_band_plan_init(ctypes.byref(cfg), None, None, None, None, None,
                                   p, 16, None) == WORKSPACE
