"""The C-ABI library loads and exports every symbol include/kat.h declares
(CPU only: nothing here launches a kernel)."""

import ctypes
import os
import re
import subprocess

import pytest

from fastalgebraictransformer_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kat.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(kat_[a-z0-9_]+)\s*\(", src)))


def test_library_is_built():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"


def test_exports_match_header():
    declared = _declared()
    assert declared, "no entry points parsed from include/kat.h"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted(set(re.findall(r"\bT (kat_[a-z0-9_]+)\b", out)))
    assert exported == declared
    assert sorted(_lib.EXPORTED) == declared


def test_load_and_version():
    lib = _lib.load()
    assert lib.kat_version() >= 100
    for name in _declared():
        assert hasattr(lib, name)


def test_workspace_sizes():
    lib = _lib.load()
    assert lib.kat_attn_bwd_workspace_size(4, 16, 4096, 128, 1) >= 4 * 16 * 4096 * 4
    # bf16 / fp16 with an MFMA head dim: per-row stats (8 B), the fp16 copy of
    # Q and the fp16 dS tiles (the causal half of T x T per head: 64 x 64
    # tiles of 8 KB); fp32 only needs Delta and cinv
    rows = 4 * 16 * 4096
    tiles = 64 * 65 // 2
    assert lib.kat_attn_bwd_workspace_size(4, 16, 4096, 128, 1) >= rows * 8 + rows * 128 * 2 + 64 * tiles * 8192
    assert lib.kat_attn_bwd_workspace_size(4, 16, 4096, 64, 2) >= rows * 8 + rows * 64 * 2 + 64 * tiles * 8192
    assert lib.kat_attn_bwd_workspace_size(4, 16, 4096, 128, 0) < rows * 16
    assert lib.kat_attn_bwd_workspace_size(0, 16, 4096, 128, 1) == 0
    # decode partials: B*H*splits rows of (layout width + 1) floats; a head
    # dim between the widths takes its width's layout, others are unsupported
    assert lib.kat_attn_decode_workspace_size(2, 3, 1000, 96, 1) == \
        lib.kat_attn_decode_workspace_size(2, 3, 1000, 128, 1) > 0
    assert lib.kat_attn_decode_workspace_size(2, 3, 1000, 20, 0) == \
        lib.kat_attn_decode_workspace_size(2, 3, 1000, 32, 0) > 0
    for D, dt in ((100, 1), (264, 1), (256 + 8, 2), (132, 0), (18, 0)):
        assert lib.kat_attn_decode_workspace_size(2, 3, 1000, D, dt) == 0, (D, dt)
    n = lib.kat_men_bwd_workspace_size(16384, 4096, 1)
    assert n > 0 and n % (4096 * 4) == 0
    assert lib.kat_men_bwd_workspace_size(8, 96, 3) % (96 * 8) == 0


def test_backward_workspace_is_bounded_by_the_cap(monkeypatch):
    # the dS tiles are sized by the call's mode (causal: the lower triangle of
    # each head's tiles) and capped: a head whose tiles exceed the cap runs in
    # bands of its keys, so the workspace stays within the cap plus O(T D)
    # (stats, the fp16 copy of Q, per-tile values, fp32 dQ partial sums)
    lib = _lib.load()
    monkeypatch.delenv("KAT_ATTN_DS_CAP_BYTES", raising=False)
    causal = lib.kat_attn_bwd_workspace_size(4, 16, 4096, 128, 1)
    assert causal == lib.kat_attn_bwd_masked_workspace_size(4, 16, 4096, 128, 1, 1)
    # 64 heads x 2304 tiles of 8 KB (the causal runs of 8 dQ blocks)
    rows, tri = 4 * 16 * 4096, 64 * 2304 * 8192
    assert causal < rows * (8 + 256) + tri + (1 << 20)
    assert lib.kat_attn_bwd_masked_workspace_size(4, 16, 4096, 128, 1, 0) > causal + tri // 2
    T, D = 65536, 128
    linear = T * (8 + 2 * D) + T * D * 4 + (1 << 20)
    # 4.3 GB of causal tiles per head: banded under the default 4 GiB cap
    assert lib.kat_attn_bwd_workspace_size(1, 1, T, D, 1) <= (4 << 30) + linear
    for cap in (1 << 30, 256 << 20):
        monkeypatch.setenv("KAT_ATTN_DS_CAP_BYTES", str(cap))
        for c in (1, 0):
            n = lib.kat_attn_bwd_masked_workspace_size(1, 1, T, D, 1, c)
            assert cap // 4 < n <= cap + linear, (cap, c, n)
    # a cap below one band of 512 keys still sizes that band: at T = 4096 its
    # causal runs hold 8 + 7 x 8 key tiles x 8 query tiles (4 MiB), plus the
    # fp32 dQ partial sums
    monkeypatch.setenv("KAT_ATTN_DS_CAP_BYTES", "1")
    n = lib.kat_attn_bwd_workspace_size(1, 1, 4096, 128, 1)
    assert 512 * 8192 < n < 4096 * (8 + 256 + 512) + 512 * 8192 + (1 << 20)


def _msg(lib):
    return lib.kat_last_error().decode()


def test_argument_errors_are_reported_without_launching():
    lib = _lib.load()
    rc = lib.kat_rswiglu_fwd(None, None, None, -1, 4, 4, 4, 4, 1, None)
    assert rc == 1 and "negative" in _msg(lib)
    rc = lib.kat_rsoftmax_fwd(ctypes.c_void_p(16), None, 2, 8, 8, 8, 1e-6, 0, None)
    assert rc == 1 and "null" in _msg(lib)
    rc = lib.kat_rsoftmax_fwd(ctypes.c_void_p(16), ctypes.c_void_p(16), 2, 8, 4, 8, 1e-6, 0, None)
    assert rc == 1 and "leading dimension" in _msg(lib)
    # empty inputs are a no-op success
    assert lib.kat_rswiglu_fwd(None, None, None, 0, 8, 8, 8, 8, 1, None) == 0
    strides = _lib.i64_array([0] * 12)
    lstr = _lib.i64_array([0] * 3)
    rc = lib.kat_attn_fwd(None, None, None, None, None, None, 1, 1, 8, 1040, strides, lstr, 1.0,
                          1e-6, 1, 1, None)
    assert rc == 2 and "head dim 1040 > 1024" in _msg(lib)
    rc = lib.kat_attn_fwd(None, None, None, None, None, None, 1, 1, 8, 64, strides, lstr, 1.0,
                          1e-6, 1, 1, None)
    assert rc == 1 and "null" in _msg(lib)
    rc = lib.kat_attn_bwd(*([None] * 11), 0, 1, 1, 8, 64, _lib.i64_array([0] * 24), lstr, 1.0, 1e-6,
                          1, 1, None)
    assert rc == 1
    rc = lib.kat_men_fwd(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                         ctypes.c_void_p(16), 2, 8, 8, 8, 1e-6, 3, 1, None)
    assert rc == 2 and "weight dtype" in _msg(lib)


def test_python_side_raises_on_bad_status():
    with pytest.raises(RuntimeError, match="kat_rswiglu_fwd"):
        lib = _lib.load()
        _lib.check(lib.kat_rswiglu_fwd(None, None, None, -1, 4, 4, 4, 4, 1, None),
                   "kat_rswiglu_fwd")
