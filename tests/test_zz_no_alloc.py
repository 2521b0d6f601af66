"""biq_q4_linear_noalloc (through the C ABI) against biq_q4_linear: the same kernels and work
split on a static scratch array, so the outputs must be bitwise equal.  Each case makes two calls
in a row, the second with a smaller input (the array keeps the first call's contents)."""
import ctypes
import os

import numpy as np
import pytest
import torch

from gpu_util import dev, dev_words

pytestmark = pytest.mark.gpu

from burn_image_amd import _lib  # noqa: E402
from burn_image_amd import workloads as W  # noqa: E402

_DT = {"f32": (_lib.DTYPE_F32, torch.float32), "f16": (_lib.DTYPE_F16, torch.float16),
       "bf16": (_lib.DTYPE_BF16, torch.bfloat16)}


def _inputs(gpu, seed, M, K, N, layout, block, xdt):
    words, scales = W.q4_weight(7, seed, K, N, layout=layout, block=block)
    x = W.activations(7, 100 + seed, M, K, xdt)
    return dev(x, _DT[xdt][1], gpu), dev_words(words, gpu), torch.from_numpy(scales).to(gpu)


def _call(fn, x, xdt, M, K, w, s, layout, block, N, ydt, bias=None):
    y = torch.full((M, N), float("nan"), dtype=_DT[ydt][1], device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = fn(stream, x.data_ptr(), _DT[xdt][0], M, K, K, w.data_ptr(), s.data_ptr(), layout, block, N,
            None if bias is None else bias.data_ptr(), y.data_ptr(), _DT[ydt][0])
    return rc, y


# (M, K, N, layout, block, activation dtype, output dtype): first call, then a smaller second one
CASES = [
    # K-split tail tiles: 4608 x 3072 x 9216 (96 partial tiles, 12 MiB), then 300 x 1024 x 1000
    ((4608, 3072, 9216, 1, 128, "bf16", "f32"), (300, 1024, 1000, 1, 32, "f16", "bf16")),
    # Qwen layout, 1024 x 4096 x 4096 (256 partial tiles: the whole 32 MiB), then 256 x 768 x 512
    ((1024, 4096, 4096, 0, 128, "bf16", "f32"), (256, 768, 512, 0, 128, "f32", "f32")),
    # small-M route: 16 x 3072 x 9216 partial rows, then the modulation row 1 x 3360 x 13440
    ((16, 3072, 9216, 1, 128, "bf16", "f32"), (1, 3360, 13440, 1, 32, "f32", "f32")),
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_q4_linear_twice(gpu, first, second):
    lib = _lib.load()
    for i, (M, K, N, layout, block, xdt, ydt) in enumerate((first, second)):
        print(f"[noalloc] call {i}: M{M} K{K} N{N} layout {layout} block {block} {xdt}->{ydt}", flush=True)
        x, w, s = _inputs(gpu, i, M, K, N, layout, block, xdt)
        bias = torch.linspace(-1, 1, N, device=gpu) if i == 1 else None
        rc_ref, ref = _call(lib.biq_q4_linear, x, xdt, M, K, w, s, layout, block, N, ydt, bias)
        rc, out = _call(lib.biq_q4_linear_noalloc, x, xdt, M, K, w, s, layout, block, N, ydt, bias)
        torch.cuda.synchronize()
        assert rc_ref == _lib.OK and rc == _lib.OK, lib.biq_last_error()
        assert torch.equal(out, ref), f"call {i}: max diff {(out.float() - ref.float()).abs().max().item()}"


def test_noalloc_rejects_splits_beyond_its_scratch(gpu, monkeypatch):
    """Forcing 16 K parts on 432 tiles (176 tail tiles -> 2816 partial tiles, 352 MiB) exceeds the
    32 MiB array: the call fails closed before any GPU work and names both sizes."""
    lib = _lib.load()
    M, K, N = 4608, 12288, 3072
    x, w, s = _inputs(gpu, 5, M, K, N, 1, 128, "bf16")
    monkeypatch.setenv("BIQ_GEMM_STREAMK", "16")
    rc, y = _call(lib.biq_q4_linear_noalloc, x, "bf16", M, K, w, s, 1, 128, N, "f32")
    torch.cuda.synchronize()
    assert rc == _lib.ERR_UNSUPPORTED
    msg = lib.biq_last_error()
    assert b"static scratch" in msg and str(32 << 20).encode() in msg, msg
    assert torch.isnan(y).all()  # nothing was written
    monkeypatch.delenv("BIQ_GEMM_STREAMK")
    rc, y = _call(lib.biq_q4_linear_noalloc, x, "bf16", M, K, w, s, 1, 128, N, "f32")
    rc_ref, ref = _call(lib.biq_q4_linear, x, "bf16", M, K, w, s, 1, 128, N, "f32")
    torch.cuda.synchronize()
    assert rc == _lib.OK and rc_ref == _lib.OK and torch.equal(y, ref)
