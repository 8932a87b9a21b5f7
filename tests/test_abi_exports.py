"""The C-ABI library loads and exports every symbol its header declares (no GPU calls)."""
import ctypes
import os
import re

import pytest

from shardcompute_amd import _lib
from shardcompute_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "shardcompute_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sc_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert _declared() == sorted(_lib.EXPORTS)


@pytest.mark.skipif(not os.path.exists(LIB_PATH), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name


@pytest.mark.skipif(not os.path.exists(LIB_PATH), reason="library not built")
def test_abi_version_and_error_channel():
    lib = _lib.load()
    assert lib.sc_abi_version() == _lib.ABI_VERSION
    # argument checks run before any HIP call, so these are safe without a GPU
    rc = lib.sc_qmm_bf16(None, None, None, None, None, None, 1, 1, 64, 4, 64, None)
    assert rc == -1 and b"null pointer" in lib.sc_last_error()
    rc = lib.sc_qmm_bf16_path(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              None, ctypes.c_void_p(16), 1, 1, 64, 3, 64, 0, None)
    assert rc == -2 and b"bits=3" in lib.sc_last_error()
    rc = lib.sc_qmm_bf16_path(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              None, ctypes.c_void_p(16), 1, 1, 100, 4, 64, 0, None)
    assert rc == -1 and b"multiple of group_size" in lib.sc_last_error()
    rc = lib.sc_vocab_gather_bf16(None, 0, 0, None, 4, 4, 0, None, None)
    assert rc == 0  # empty input is a no-op
    rc = lib.sc_quantize_affine(None, 2, 64, 5, 64, None, None, None, None)
    assert rc == -2
