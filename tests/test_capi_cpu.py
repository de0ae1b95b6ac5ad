"""The C-ABI library loads and exports every symbol include/qimm.h declares
(no compute calls: this runs without a GPU), and its error paths are codes."""
import ctypes as C
import os
import re
import subprocess

import pytest

import qimm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qimm.h")


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(qimm_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_entry_points():
    names = header_functions()
    for must in ("qimm_ctx_create", "qimm_weight_upload", "qimm_dequant", "qimm_qmatmul",
                 "qimm_attention", "qimm_block_create", "qimm_block_forward", "qimm_kv_create"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = qimm.load()
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", qimm.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (qimm_[a-z0-9_]+)", out))
    assert set(header_functions()) <= exported


def test_python_binding_covers_the_header():
    assert sorted(n for n, _, _ in qimm.SIGNATURES) == header_functions()


def test_abi_version_and_status_strings():
    lib = qimm.load()
    assert lib.qimm_abi_version() == 1
    assert lib.qimm_status_string(0) == b"ok"
    assert lib.qimm_status_string(3) == b"unsupported GGML type"


def test_null_arguments_return_codes():
    lib = qimm.load()
    assert lib.qimm_ctx_create(0, None) == 1
    assert lib.qimm_ctx_destroy(None) == 1
    assert lib.qimm_weight_free(None) == 1
    assert lib.qimm_kv_destroy(None) == 1
    assert lib.qimm_block_destroy(None) == 1
    assert lib.qimm_last_error(None) == b"null context"


def test_ctx_create_without_gpu_fails_cleanly():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    rc = qimm.load().qimm_ctx_create(0, C.byref(h))
    assert rc != 0 and not h.value
