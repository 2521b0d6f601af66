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
                           0.0, p["causal"], None, 0, None, 0, 0)
    assert rc != _lib.OK
    assert needle in lib.biq_last_error()


def test_burn_attention_op_rejects_bias_softcap_and_general_masks():
    """ModuleOps::attention (patches/burn-cubecl-0.21.0/src/ops/module.rs:342-367): the flash
    kernel takes no additive bias, no softcap and no mask other than key padding; each returns
    BIQ_ERR_UNSUPPORTED before any GPU work (the reference routes them to a dense fallback)."""
    from burn_image_amd import _lib
    lib = _lib.load()
    st = _lib.strides3((1, 1, 64))
    d = ctypes.c_void_p(256)
    I4 = ctypes.c_int64 * 4

    def call(mask=None, mstr=None, bias=None, softcap=None, scale=None):
        return lib.biq_attention_burn(None, d, d, d, d, _lib.DTYPE_F16, 2, 4, 4, 8, 8, 64, st, st, st, st,
                                      mask, mstr, bias, 0, int(scale is not None), float(scale or 0.0),
                                      int(softcap is not None), float(softcap or 0.0))

    assert call(bias=d) == _lib.ERR_UNSUPPORTED and b"attn_bias" in lib.biq_last_error()
    assert call(softcap=30.0) == _lib.ERR_UNSUPPORTED and b"softcap" in lib.biq_last_error()
    # a full [B, H, Sq, Skv] mask, a per-head mask and a per-query mask cannot run
    for strides in ((256, 64, 8, 1), (8, 8, 0, 1), (64, 0, 8, 1)):
        assert call(mask=d, mstr=I4(*strides)) == _lib.ERR_UNSUPPORTED
        assert b"key-padding" in lib.biq_last_error()
    assert call(scale=-1.0) == _lib.ERR_INVALID_ARG


def test_attention_key_mask_mode_validation():
    from burn_image_amd import _lib
    lib = _lib.load()
    st = _lib.strides3((1, 1, 64))
    d = ctypes.c_void_p(256)
    rc = lib.biq_attention(None, d, d, d, d, _lib.DTYPE_BF16, _lib.DTYPE_F32, 1, 4, 2, 8, 8, 64, st, st, st,
                           st, 0.0, 0, None, 0, d, 8, 7)
    assert rc == _lib.ERR_INVALID_ARG and b"key mask mode" in lib.biq_last_error()


@pytest.mark.parametrize("cu,S,ok", [
    ([0, 4, 8], 8, True),
    ([0, 8], 8, True),
    ([1, 4, 8], 8, False),      # does not start at 0
    ([0, 4, 4, 8], 8, False),   # empty segment
    ([0, 6, 4, 8], 8, False),   # descending
    ([0, 4, 7], 8, False),      # does not end at S
    ([0, -4, 8], 8, False),     # negative bound
    ([0, 4, 9], 8, False),      # past the sequence
])
def test_cu_seqlens_host_validator(cu, S, ok):
    """Host-side segment table check (a malformed table never reaches the kernel through the
    Python API; the reference holds its frame ranges on the host, vision.rs:53-78,344-345)."""
    import burn_image_amd as B
    if ok:
        B.check_cu_seqlens(cu, S)
    else:
        with pytest.raises(B.InvalidArgument):
            B.check_cu_seqlens(cu, S)


def test_frame_ranges_to_cu_seqlens():
    """vision.rs:319-386 frame ranges -> segment table, and the contract's failures."""
    import burn_image_amd as B
    assert list(B.frame_ranges_to_cu_seqlens([(0, 3), (3, 10), (10, 16)], 16)) == [0, 3, 10, 16]
    for bad in ([(0, 3), (4, 16)], [(0, 3), (3, 3), (3, 16)], [(0, 3), (3, 12)], [(1, 16)], [(0, 17)]):
        with pytest.raises(B.InvalidArgument):
            B.frame_ranges_to_cu_seqlens(bad, 16)


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


@pytest.mark.parametrize("owner,shape", [("boogu", (3360, 840)), ("boogu", (64, 3360)), ("boogu", (13568, 256)),
                                         ("qwen", (256, 128)), ("qwen", (1024, 4096))])
def test_q4s_payload_split_matches_oracle_quantizer(oracle, owner, shape):
    """The importer's single payload (words then f32 scales, artifacts.rs:7364-7377 / 7276-7283)
    built from the oracle's byte-exact quantizers splits back into exactly those words and scales,
    as views of the payload (no copy), under the stored-dtype contract (artifacts.rs:527-536) and
    the importer's size contract (boogu_import.rs:1693-1719, e.g. 256 x 128 Qwen: 256*128/2 +
    256*4 bytes)."""
    import numpy as np
    import torch
    from burn_image_amd import q4
    rng = np.random.default_rng(sum(shape))
    w = (rng.standard_normal(shape) * 0.05).astype(np.float32)
    if owner == "boogu":
        words, scales, _blk = oracle.q4_quantize_kn(w)
        dtype = q4.q4s_stored_dtype(q4.BOOGU_DENOISER, shape)
    else:
        words, scales = oracle.q4_quantize_nk(w)
        dtype = q4.q4s_stored_dtype(q4.QWEN3_VL, shape)
    payload_np = np.frombuffer(words.astype("<u4").tobytes() + scales.astype("<f4").tobytes(), np.uint8).copy()
    if shape == (256, 128):
        assert payload_np.size == 256 * 128 // 2 + 256 * 4
    payload = torch.from_numpy(payload_np)
    wv, sv, lay, blk = q4.split_payload(payload, dtype, shape)
    assert np.array_equal(wv.numpy().view(np.uint32), words) and np.array_equal(sv.numpy(), scales)
    assert wv.data_ptr() == payload.data_ptr()            # views, not copies
    assert sv.data_ptr() == payload.data_ptr() + words.nbytes
    assert lay == (1 if owner == "boogu" else 0)
    # contract failures: wrong size, wrong block string, wrong layout, shape without a contract
    from burn_image_amd import InvalidArgument
    with pytest.raises(InvalidArgument):
        q4.split_payload(payload[:-4], dtype, shape)
    with pytest.raises(InvalidArgument):
        q4.payload_layout(dtype.replace("block", "block1"), shape, payload_np.size)
    with pytest.raises(InvalidArgument):
        other = dtype.replace("axis1", "axisX") if "axis1" in dtype else dtype.replace("axis0", "axis1")
        q4.payload_layout(other, shape, payload_np.size)
    with pytest.raises(InvalidArgument):
        q4.payload_layout(dtype, (shape[0], shape[1] + 4), payload_np.size)


def test_q4_linear_scale_grid_beyond_2gb_fails_closed():
    """Block 8 with K * N = 2^32 makes a 2 GiB scale grid: the 32-bit scale descriptor cannot
    address it, so the call returns BIQ_ERR_UNSUPPORTED instead of reading zeros past 2 GiB."""
    from burn_image_amd import _lib
    lib = _lib.load()
    d = ctypes.c_void_p(256)
    K = N = 1 << 16
    rc = lib.biq_q4_linear(None, d, _lib.DTYPE_BF16, 4096, K, K, d, d, 1, 8, N, None, d, _lib.DTYPE_BF16)
    assert rc == _lib.ERR_UNSUPPORTED and b"scale grid" in lib.biq_last_error()
    # one block size up the grid halves and passes the check (it would then launch: not called here)
