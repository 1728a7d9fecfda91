"""C-ABI checks that need no GPU: the library loads, exports every entry point the header
declares, and reports errors through return codes and bb_last_error()."""
import ctypes
import subprocess

import numpy as np

from bebelm_amd import _lib


def test_library_exports_every_header_symbol():
    names = _lib.header_symbols()
    assert len(names) >= 30
    L = _lib.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) <= set(_lib._SIGS), "binding lacks a header symbol"


def test_dynamic_symbol_table_matches_header():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    for n in _lib.header_symbols():
        assert n in exported, n


def test_null_arguments_return_error_codes():
    L = _lib.lib()
    assert L.bb_ctx_create(0, None) == _lib.BB_ERR_ARG
    assert b"null" in L.bb_last_error()
    assert L.bb_moe_forward(None, None, None, 1, None, 0, None) == _lib.BB_ERR_ARG
    assert L.bb_ctx_synchronize(None) == _lib.BB_ERR_ARG
    assert L.bb_tensor_upload(None, 12, None, 0, None, 0, None) == _lib.BB_ERR_ARG
    assert L.bb_ctx_destroy(None) == _lib.BB_OK
    assert L.bb_version().startswith(b"bebelm_moe")


def test_header_documents_reference_counterparts():
    text = open(_lib.HEADER).read()
    for ref in ("matmul.rs:850", "matmul.rs:908", "matmul.rs:141", "matmul.rs:1015", "model.rs:473-555",
                "model.rs:286-371", "rmsnorm.rs:10", "activation.rs:16", "elementwise.rs:12", "tensor.rs:99-105"):
        assert ref in text, ref
