"""The C-ABI library loads and exports every entry point include/starkv_hip.h declares;
argument validation fails loudly without touching the GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "starkv_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(starkv_\w+)\s*\(", text)))


def test_header_declares_the_api():
    names = declared()
    for n in ("starkv_lowrank_decode", "starkv_quant_decode", "starkv_pack_kv", "starkv_write_codes",
              "starkv_fold_q", "starkv_decode_grid", "starkv_decode_workspace_bytes", "starkv_last_error",
              "starkv_abi_version"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from starkv_serve import _hip
    assert os.path.exists(_hip.LIB_PATH), "build the library first (__graft_entry__.build())"
    raw = ctypes.CDLL(_hip.LIB_PATH)
    for n in declared():
        assert hasattr(raw, n), n
    assert set(declared()) == set(_hip.SIGNATURES)
    assert _hip.lib().starkv_abi_version() == _hip.ABI_VERSION


def test_bad_arguments_return_errors():
    from starkv_serve import _hip
    L = _hip.lib()
    rc = L.starkv_pack_kv(None, None, 0, None, 0, 2, None, 0, 0, 16, 1, None, 64, 1, 32, None, None, None, 1280, 64, 999)
    assert rc != 0 and b"row_bytes" in L.starkv_last_error()
    rc = L.starkv_write_codes(None, None, 0, None, 0, 2, None, 0, 0, 2, 16, 1, None, 48, 1, 16, 16)
    assert rc != 0 and b"int32 or int64" in L.starkv_last_error()
    with pytest.raises(RuntimeError, match="row_bytes"):
        _hip.check(L.starkv_pack_kv(None, None, 0, None, 0, 2, None, 0, 0, 16, 1, None, 64, 1, 32, None, None,
                                    None, 1280, 64, 999), "pack_kv")


def test_workspace_size_is_a_host_function():
    from starkv_serve import _hip
    L = _hip.lib()
    a = L.starkv_decode_workspace_bytes(64, 32, 80, 64, 256)
    b = L.starkv_decode_workspace_bytes(64, 32, 80, 64, 128)
    assert a > b > 64 * 80 * 4096
