"""CPU tests of the C-ABI boundary (include/qw_linear.h): the library loads
without a GPU, exports every declared entry point, and its host-side argument
checks return status codes (no compute call is made here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qw_linear.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:qw_status|size_t|const char\*|int)\s+(qw_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def L(qw):
    return qw.lib()


def test_header_declares_the_boundary():
    fns = header_functions()
    for name in ["qw_init", "qw_destroy", "qw_workspace_query", "qw_weight_pack", "qw_weight_free", "qw_linear",
                 "qw_mlp_fused", "qw_lmhead_argmax", "qw_graph_begin", "qw_graph_end", "qw_graph_launch",
                 "qw_last_error"]:
        assert name in fns, name


def test_library_exports_every_declared_symbol(L, qw):
    fns = header_functions()
    missing = [f for f in fns if not hasattr(L, f)]
    assert not missing, missing
    assert sorted(qw.EXPORTS) == fns  # the Python binding covers the same set


def test_version_and_status_strings(L, qw):
    assert L.qw_abi_version() == 1
    seen = set()
    for s in range(10):
        txt = L.qw_status_string(s).decode()
        assert txt and txt not in seen
        seen.add(txt)


def test_workspace_query_monotone(L):
    a = L.qw_workspace_query(1, 1024, 1024)
    b = L.qw_workspace_query(4096, 8224, 4096)
    c = L.qw_workspace_query(16384, 8224, 4096)
    assert 0 < a <= b <= c and a % 4096 == 0 and b % 4096 == 0


def test_null_arguments_rejected(L, qw):
    p = ctypes.c_void_p()
    assert L.qw_init(None, 0, 0) == qw.ERR_NULL
    assert L.qw_destroy(None) in (qw.OK, qw.ERR_NULL)
    assert L.qw_weight_free(None) in (qw.OK, qw.ERR_NULL)
    assert L.qw_weight_pack(None, None, qw.F32, qw.WFMT_BF16, 64, 64, None, ctypes.byref(p)) == qw.ERR_NULL
    assert L.qw_linear(None, None, None, qw.BF16, 0, 1, None, qw.BF16, 0, None, None) == qw.ERR_NULL
    assert L.qw_lmhead_argmax(None, None, None, qw.BF16, 1, None, None, None) == qw.ERR_NULL
    assert L.qw_mlp_fused(None, None, None, None, qw.BF16, None, 1e-6, None, qw.BF16, None, qw.BF16, 1,
                          None) == qw.ERR_NULL
    assert L.qw_graph_launch(None, None) == qw.ERR_NULL
    assert L.qw_last_error(None) is not None


def test_init_without_gpu_fails_cleanly(L, qw):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    p = ctypes.c_void_p()
    assert L.qw_init(ctypes.byref(p), 0, 0) == qw.ERR_HIP
    assert not p.value


def test_missing_library_fails_loudly(qw, monkeypatch):
    monkeypatch.setattr(qw, "_LIB", None)
    monkeypatch.setattr(qw, "LIB_PATH", os.path.join(ROOT, "no_such_dir", "libqw_linear.so"))
    with pytest.raises(ImportError):
        qw.lib()
