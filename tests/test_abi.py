"""The C ABI library loads and exports every declared symbol (no GPU calls)."""
import ctypes

import pytest

import qe_moe


def test_library_exports_every_header_symbol():
    lib = qe_moe.load()
    names = qe_moe.header_symbols()
    assert "qe_moe_forward" in names and "qe_moe_forward_normed" in names
    for n in names:
        assert hasattr(lib, n), n


def test_expert_bytes_and_argument_errors():
    lib = qe_moe.load()
    assert lib.qe_moe_expert_bytes() == 1769472
    h = ctypes.c_void_p()
    assert lib.qe_moe_create(0, 0, 8, ctypes.byref(h)) == qe_moe.QE_ERR_ARG
    assert b"bad argument" in lib.qe_moe_last_error()
    assert lib.qe_moe_create(0, 1, 0, ctypes.byref(h)) == qe_moe.QE_ERR_ARG
    assert lib.qe_moe_forward(None, 0, None, None, 1, None) == qe_moe.QE_ERR_ARG
    assert lib.qe_moe_forward_norm(None, 0, None, None, 1, None, None, None) == qe_moe.QE_ERR_ARG
    assert lib.qe_moe_load_pack(None, b"x.pack", 0, 0, 1, None) == qe_moe.QE_ERR_ARG
    assert lib.qe_moe_destroy(None) == 0
    # converter argument checks return before any device call
    assert lib.qe_moe_nl4_quantize_rows(None, 8, 1, 2048, None, None) == qe_moe.QE_ERR_ARG
    assert lib.qe_moe_nl4_quantize_rows(16, 8, 1, 100, 32, None) == qe_moe.QE_ERR_ARG
    assert lib.qe_moe_nl4_quantize_rows(16, 8, 1, 2048, 40, None) == qe_moe.QE_ERR_ARG
    assert lib.qe_moe_nl4_quantize_rows(16, 2, 1, 2048, 32, None) == qe_moe.QE_ERR_ARG
    assert b"unsupported source type 2" in lib.qe_moe_last_error()
    assert lib.qe_moe_nl4_quantize_rows(16, 8, 1 << 26, 2048, 32, None) == qe_moe.QE_ERR_ARG
    assert lib.qe_moe_convert_experts(None, 0, 16, 32, 48, 8, None) == qe_moe.QE_ERR_ARG


def test_python_constants_match_the_header():
    import os
    import re
    hdr = open(qe_moe.HEADER).read()
    for name in ("QE_MOE_T_MAX", "QE_MOE_DISPATCH_NOALLOC_T_MAX"):
        assert int(re.search(r"#define %s (\d+)" % name, hdr).group(1)) == getattr(qe_moe, name), name
    assert os.path.exists(qe_moe.HEADER)


def test_missing_library_fails_loudly(tmp_path):
    saved = qe_moe._lib
    qe_moe._lib = None
    try:
        with pytest.raises(qe_moe.LibraryMissing):
            qe_moe.load(str(tmp_path / "nope.so"))
    finally:
        qe_moe._lib = saved
