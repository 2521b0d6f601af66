"""The C ABI library (CPU): it loads, exports every symbol include/biq.h declares, and its
host-only helpers follow the reference's storage contract.  No compute call needs a GPU here."""
import ctypes
import os
import re

import pytest

from conftest import ROOT


def header_functions():
    text = open(os.path.join(ROOT, "include", "biq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(biq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    from burn_image_amd import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = header_functions()
    assert len(names) >= 8
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures must mirror the header"


def test_version_and_error_state():
    from burn_image_amd import _lib
    assert "gfx950" in _lib.version()
    lib = _lib.load()
    # an argument error sets the thread-local message and touches no GPU
    rc = lib.biq_q4_linear(None, None, 0, 1, 8, 8, None, None, 1, 8, 8, None, None, 0)
    assert rc == _lib.ERR_INVALID_ARG
    assert b"null pointer" in lib.biq_last_error()


def test_storage_contract_matches_reference():
    """artifacts.rs:513-536 and boogu_import.rs:1693-1719."""
    from burn_image_amd import q4
    assert q4.q4s_storage_block_and_axis(q4.QWEN3_VL, [256, 128]) == (128, 0)
    assert q4.q4s_stored_dtype(q4.QWEN3_VL, [256, 128]) == "q4s-block128-f32-packed-axis0"
    assert q4.q4s_stored_dtype(q4.BOOGU_DENOISER, [64, 3360]) == "q4s-block64x1-f32-packed-axis1"
    assert q4.q4s_storage_block_and_axis(q4.BOOGU_DENOISER, [3360, 840]) == (32, 1)
    assert q4.q4s_storage_block_and_axis(q4.BOOGU_DENOISER, [13568, 3360]) == (128, 1)
    assert q4.q4s_storage_block_and_axis(q4.BOOGU_DENOISER, [12, 16]) is None
    assert q4.q4s_storage_block_and_axis(q4.QWEN3_VL, [256, 100]) is None
    assert q4.q4s_stored_dtype(q4.FLUX_VAE, [256, 128]) is None


@pytest.mark.parametrize("args,needle", [
    # biq_attention: GQA heads not divisible (native_flash.rs:2828-2841 fails closed)
    (dict(Hq=4, Hkv=3), b"divisible"),
    (dict(Sq=0), b"non-empty"),
    (dict(Skv=0), b"non-empty"),
    (dict(D=136), b"head width"),
    (dict(causal=1, Skv=7), b"Sq == Skv"),
])
def test_attention_validation_fails_closed(args, needle):
    from burn_image_amd import _lib
    lib = _lib.load()
    p = dict(B=1, Hq=4, Hkv=2, Sq=8, Skv=8, D=64, causal=0)
    p.update(args)
    st = _lib.strides3((1, 1, 64))
    dummy = ctypes.c_void_p(256)
    rc = lib.biq_attention(None, dummy, dummy, dummy, dummy, _lib.DTYPE_BF16, _lib.DTYPE_F32,
                           p["B"], p["Hq"], p["Hkv"], p["Sq"], p["Skv"], p["D"], st, st, st, st,
                           0.0, p["causal"], None, 0)
    assert rc != _lib.OK
    assert needle in lib.biq_last_error()


def test_q4_linear_validation_fails_closed():
    from burn_image_amd import _lib
    lib = _lib.load()
    d = ctypes.c_void_p(256)
    # block not supported by the packed route (qtensor.rs:311-317)
    assert lib.biq_q4_linear(None, d, 0, 4, 96, 96, d, d, 1, 48, 8, None, d, 0) == _lib.ERR_UNSUPPORTED
    # K not divisible by the block
    assert lib.biq_q4_linear(None, d, 0, 4, 96, 96, d, d, 1, 64, 8, None, d, 0) == _lib.ERR_INVALID_ARG
    # N not divisible by 8
    assert lib.biq_q4_linear(None, d, 0, 4, 128, 128, d, d, 1, 128, 12, None, d, 0) == _lib.ERR_INVALID_ARG
    # empty M, K or N fails closed with a message, on the small-M route and the GEMM route alike
    for m, k, n in ((0, 128, 8), (0, 128, 4096), (4, 0, 8), (64, 128, 0)):
        for y_dtype in (_lib.DTYPE_F32, _lib.DTYPE_BF16):
            assert lib.biq_q4_linear(None, d, _lib.DTYPE_BF16, m, k, max(k, 1), d, d, 1, 128, n, None,
                                     d, y_dtype) == _lib.ERR_INVALID_ARG
            assert b"non-empty" in lib.biq_last_error()
