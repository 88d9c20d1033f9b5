"""The C-ABI library loads on a machine without a GPU and exports every entry
point include/pagedkv.h declares. Only host-side calls are made here
(argument validation and workspace sizing); no kernel is launched."""
import ctypes
import os
import re

import pytest

from serving import _native

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "pagedkv.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pkv_[a-z_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert set(names) == set(_native.EXPORTED), names


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    # and nm agrees that they are exported C symbols (no C++ mangling)
    raw = ctypes.CDLL(_native.LIB_PATH)
    for name in declared_functions():
        getattr(raw, name)


def test_version_matches_header():
    m = re.search(r"#define PKV_VERSION (\d+)", open(HEADER).read())
    assert _native.lib().pkv_version() == int(m.group(1))


def test_validation_errors_without_gpu():
    L = _native.lib()
    # bad dtype, non-power-of-two block size, head dim not a multiple of 8,
    # hq not a multiple of hkv: all rejected on the host
    rc = L.pkv_paged_attention(1, None, 1, 1, 1, 10, 16, 1, 1, 1, None, 1, 1, 1, 0,
                               8, 1, 64, 0.0, 1, 0, 9, None, 0, None, None)
    assert rc == -1 and b"dtype" in L.pkv_last_error()
    rc = L.pkv_paged_attention(1, None, 1, 1, 1, 10, 12, 1, 1, 1, None, 1, 1, 1, 0,
                               8, 1, 64, 0.0, 1, 0, 2, None, 0, None, None)
    assert rc == -1 and b"power of two" in L.pkv_last_error()
    rc = L.pkv_paged_attention(1, None, 1, 1, 1, 10, 16, 1, 1, 1, None, 1, 1, 1, 0,
                               8, 1, 60, 0.0, 1, 0, 2, None, 0, None, None)
    assert rc == -1 and b"multiple of 8" in L.pkv_last_error()
    rc = L.pkv_paged_attention(1, None, 1, 1, 1, 10, 16, 1, 1, 1, None, 1, 1, 1, 0,
                               6, 4, 64, 0.0, 1, 0, 2, None, 0, None, None)
    assert rc == -1 and b"multiple of Hkv" in L.pkv_last_error()
    rc = L.pkv_paged_attention(1, None, 1, 1, 1, 10, 16, 1, 1, 1, None, 1, 1, 1, 0,
                               8, 1, 264, 0.0, 1, 0, 2, None, 0, None, None)
    assert rc == -2
    # q_len > 1 needs query_start_loc
    rc = L.pkv_paged_attention(1, None, 1, 1, 1, 10, 16, 1, 1, 1, None, 1, 1, 4, 0,
                               8, 1, 64, 0.0, 1, 0, 2, None, 0, None, None)
    assert rc == -1 and b"query_start_loc" in L.pkv_last_error()
    rc = L.pkv_append(1, 1, 10, 1, 1, 1, 5, 64, 7, None, None)
    assert rc == -1
    rc = L.pkv_gather(1, 1, 1, 1, 10, 16, 1, 1, 17, 64, 2, None, None)
    assert rc == -1 and b"capacity" in L.pkv_last_error()
    # nothing to do: succeeds without touching the device
    assert L.pkv_append(None, None, 10, None, None, None, 0, 64, 2, None, None) == 0


def test_workspace_sizing():
    L = _native.lib()
    # a single partition needs no workspace
    assert L.pkv_attention_workspace_bytes(4, 1, 8, 1, 64, 2, 16, 32, 4096, 2) == 0
    # split: bytes grow with the number of partitions
    a = L.pkv_attention_workspace_bytes(32, 1, 8, 1, 32, 16, 16, 256, 64, 0)
    b = L.pkv_attention_workspace_bytes(32, 1, 8, 1, 32, 16, 16, 256, 128, 0)
    assert a > b > 0
    with pytest.raises(ValueError):
        _native.check(-1, "x")


def test_linear_validation_without_gpu():
    """Host-side rejections of the projection entry points (no launch)."""
    L = _native.lib()
    # an unknown dtype is not taken, k must be a multiple of 32
    assert L.pkv_linear(16, 16, 16, None, 4, 8, 64, 64, 5, None) == -2
    assert L.pkv_linear(16, 16, 16, None, 4, 8, 40, 40, 2, None) == -2
    assert L.pkv_linear(None, 16, 16, None, 4, 8, 64, 64, 2, None) == -1
    assert L.pkv_linear(16, 16, 16, None, 4, 8, 64, 32, 2, None) == -1  # x_stride < k
    assert L.pkv_linear_swiglu(16, 16, 16, None, 4, 8, 48, 48, 1, None) == -2
    assert L.pkv_linear_residual(16, 16, 16, None, 4, 8, 64, 64, 5, None) == -2
    assert L.pkv_linear_residual(16, 16, 16, None, 4, 8, 64, 32, 2, None) == -1
    # the fused norm: k above 1024 refused before any launch, norm weight checked
    assert L.pkv_linear_swiglu_rmsnorm(16, 16, 16, 1e-5, 16, None, 4, 8, 1056, 1056, 2,
                                       None) == -2
    assert L.pkv_linear_swiglu_rmsnorm(16, 16, None, 1e-5, 16, None, 4, 8, 64, 64, 2,
                                       None) == -1
    assert L.pkv_linear_rope_qkv_rmsnorm(16, 16, 16, 16, 8, 1e-5, 16, None, 4, 64, 64, 16, 16,
                                         16, 8, 4, 1, 8, 2, None, None) == -1
    # odd head dim, missing tables
    assert L.pkv_linear_rope_qkv(16, 16, 16, 16, 16, None, 4, 64, 64, 16, 16, 16, 8, 4, 1, 7,
                                 2, None, None) == -1
    assert L.pkv_linear_rope_qkv(16, 16, 16, 16, 16, None, 4, 64, 64, 16, None, 16, 8, 4, 1, 8,
                                 2, None, None) == -1
