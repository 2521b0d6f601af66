"""GPU parity of the Q4S format kernels and the packed-Q4 GEMM (through the C ABI) against the
oracle.  Gate: dequantised weights and quantised bytes bit-exact; GEMM outputs max-abs <= 2e-3
and mean|a-b|/mean|b| <= 1e-3 against the float64 oracle rounded to f32."""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import assert_parity, dev, dev_words, host

pytestmark = pytest.mark.gpu

import burn_image_amd as B  # noqa: E402
from burn_image_amd import workloads as W  # noqa: E402

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def weight(words, scales, layout, block, K, N, device):
    shape = (K, N) if layout == 1 else (N, K)
    return B.from_packed(dev_words(words, device), dev(scales, device=device), layout, block, shape)


@pytest.mark.parametrize("K,N", [(128, 128), (3360, 64), (24, 16), (13568, 24), (64, 3360)])
def test_gpu_row_layout_quantizer_bit_exact(gpu, oracle, K, N):
    rng = np.random.default_rng(K + N)
    w = (rng.standard_normal((K, N)) * rng.uniform(0.01, 2.0, (1, N))).astype(np.float32)
    w[:, 1] = 0.0
    w[: min(K, 8), 2] = np.array([7.0, 3.5, -3.5, 2.5, -2.5, 0.5, -0.5, 0.0], np.float32)[: min(K, 8)]
    q = B.quantize_row_layout_q4s_block_up_to128_f32(dev(w, device=gpu))
    words, scales, blk = oracle.q4_quantize_kn(w)
    assert q.block == blk
    assert np.array_equal(host_words(q.words), words)
    assert host(q.scales).tobytes() == scales.tobytes()


def host_words(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("N,K", [(128, 128), (6144, 256), (3, 4096)])
def test_gpu_qwen_quantizer_bit_exact(gpu, oracle, N, K):
    rng = np.random.default_rng(N * 7 + K)
    v = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    v[0, :128] = 0.0
    q = B.quantize_q4s_block128_f32(dev(v, device=gpu))
    words, scales = oracle.q4_quantize_nk(v)
    assert np.array_equal(host_words(q.words), words)
    assert host(q.scales).tobytes() == scales.tobytes()


def test_gpu_quantizer_rejects_non_finite_and_bad_shapes(gpu):
    w = torch.zeros((16, 8), device=gpu)
    w[3, 2] = float("nan")
    with pytest.raises(B.InvalidArgument, match="non-finite"):
        B.quantize_row_layout_q4s_block_up_to128_f32(w)
    with pytest.raises(B.InvalidArgument, match="no supported exact block"):
        B.quantize_row_layout_q4s_block_up_to128_f32(torch.zeros((12, 8), device=gpu))
    with pytest.raises(B.InvalidArgument, match="not divisible by 8"):
        B.quantize_row_layout_q4s_block_up_to128_f32(torch.zeros((16, 12), device=gpu))
    with pytest.raises(B.InvalidArgument, match="not divisible by 128"):
        B.quantize_q4s_block128_f32(torch.zeros((2, 127), device=gpu))


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("block", [8, 16, 32, 64, 128])
def test_gpu_dequant_bit_exact(gpu, oracle, layout, block):
    K, N = 384, 200
    words, scales = W.q4_weight(11, block * 2 + layout, K, N, layout=layout, block=block)
    q = weight(words, scales, layout, block, K, N, gpu)
    assert host(q.dequantize()).tobytes() == oracle.q4_dequant(words, scales, layout, block, K, N).tobytes()


def test_gpu_kat_probe_reference(gpu):
    """Browser probe KAT (runtime.rs:4737-4781): GPU-quantised exactly-representable weights,
    f32 lhs; the reference gates max_abs <= 5e-4 against the f32 product."""
    g = np.load(os.path.join(GOLDEN, "kat_probe.npz"), allow_pickle=False)
    q = B.quantize_row_layout_q4s_block_up_to128_f32(dev(g["weight"], device=gpu))
    assert np.array_equal(host_words(q.words), g["words"])
    y = host(B.linear_forward(B.Linear(q), dev(g["lhs"], device=gpu)))
    assert np.max(np.abs(y - g["expected"])) <= 5e-4
    assert_parity(y, g["expected"].astype(np.float32), "kat_probe")


@pytest.mark.parametrize("layout", [1, 0])
def test_gpu_c1_linear_golden(gpu, layout):
    g = np.load(os.path.join(GOLDEN, "c1_linear.npz"), allow_pickle=False)
    tag = "kn" if layout == 1 else "nk"
    q = weight(g[f"words_{tag}"], g[f"scales_{tag}"], layout, 128, 512, 512, gpu)
    y = host(B.q_matmul(dev(g["x"], device=gpu), q))
    assert_parity(y, g[f"y_{tag}"], f"c1_linear_{tag}")


@pytest.mark.parametrize("layout", [1, 0])
@pytest.mark.parametrize("block", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("xdt", ["bf16", "f32", "f16"])
def test_gpu_q4_linear_blocks_dtypes_tails(gpu, oracle, layout, block, xdt):
    M, K, N = 77, 640 if block != 8 else 648, 200
    if layout == 0 and block != 128:
        K = 640 if block != 8 else 648
    x = W.activations(12, 1, M, K, xdt)
    words, scales = W.q4_weight(12, 2 + block + layout, K, N, layout=layout, block=block)
    q = weight(words, scales, layout, block, K, N, gpu)
    y = host(B.q_matmul(dev(x, TORCH_DT[xdt], gpu), q))
    ref = oracle.q4_linear_f64(x, words, scales, layout, block, N).astype(np.float32)
    assert_parity(y, ref, f"blk{block}_l{layout}_{xdt}")


@pytest.mark.parametrize("K", [128, 384, 1152])
@pytest.mark.parametrize("xdt", ["bf16", "f16"])
@pytest.mark.parametrize("glu", [False, True])
def test_gpu_q4_linear_odd_tile_counts(gpu, oracle, K, xdt, glu):
    """The [K/8, N] block-128 path streams K tiles in pairs: an odd tile count (1, 3, 9 tiles of
    128) runs one extra tile past K whose loads read zeros, with and without the tail split."""
    M, N = 150, 520
    x = W.activations(21, K, M, K, xdt)
    w1, s1 = W.q4_weight(21, K + 1, K, N, layout=1)
    q1 = weight(w1, s1, 1, 128, K, N, gpu)
    xd = dev(x, TORCH_DT[xdt], gpu)
    ref = oracle.q4_linear_f64(x, w1, s1, 1, 128, N)
    if glu:
        w3, s3 = W.q4_weight(21, K + 2, K, N, layout=1)
        y = host(B.q_matmul_swiglu(xd, q1, weight(w3, s3, 1, 128, K, N, gpu)))
        ref = silu_gate_ref(ref, oracle.q4_linear_f64(x, w3, s3, 1, 128, N))
    else:
        y = host(B.q_matmul(xd, q1))
    assert_parity(y, ref.astype(np.float32), f"odd_tiles_K{K}_{xdt}_glu{int(glu)}")


def test_gpu_q4_linear_bias_and_output_dtypes(gpu, oracle):
    M, K, N = 130, 256, 136
    x = W.activations(13, 1, M, K, "bf16")
    words, scales = W.q4_weight(13, 2, K, N, layout=1)
    bias = np.linspace(-2, 2, N).astype(np.float32)
    q = weight(words, scales, 1, 128, K, N, gpu)
    ref = oracle.q4_linear_f64(x, words, scales, 1, 128, N, bias=bias).astype(np.float32)
    lin = B.Linear(q, dev(bias, device=gpu))
    xd = dev(x, torch.bfloat16, gpu)
    assert_parity(host(B.linear_forward(lin, xd)), ref, "bias_f32")
    y16 = host(B.linear_forward(lin, xd, out_dtype=torch.float16))
    assert np.max(np.abs(y16 - ref)) <= np.max(np.abs(ref)) * 2.0 ** -10
    yb = host(B.linear_forward(lin, xd, out_dtype=torch.bfloat16))
    assert np.max(np.abs(yb - ref)) <= np.max(np.abs(ref)) * 2.0 ** -7
    # 16-bit outputs are the f32 result rounded once to nearest even, bit for bit
    yf = host(B.linear_forward(lin, xd))
    assert np.array_equal(yb.view(np.uint32), W.round_to_bf16(yf).view(np.uint32))
    assert np.array_equal(y16, yf.astype(np.float16).astype(np.float32))
    # rank-3 input keeps its leading shape
    y3 = B.linear_forward(lin, xd[:128].reshape(2, 64, K))
    assert tuple(y3.shape) == (2, 64, N)


def sample_rows(M, n=40, seed=0):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, n)]))


@pytest.mark.parametrize("name", list(W.C3_SHAPES))
def test_gpu_c3_projection_full_shape(gpu, oracle, name, monkeypatch):
    """C3 at M = 4608: sampled rows against the float64 oracle; every element against an fp32
    product of the (bit-exact) dequantised weight; row-permutation equivariance.  Rows of a tail
    tile whose K is split between workgroups are summed in another order than rows of a tile one
    workgroup owns, so under a row permutation the output is equal within the parity gate; with
    the split switched off (every tile owned) it is bit-exact."""
    K, N = W.C3_SHAPES[name]
    M = 4608
    idx = list(W.C3_SHAPES).index(name)
    x = W.activations(3, 2 * idx, M, K, "bf16")
    words, scales = W.q4_weight(3, 2 * idx + 1, K, N, layout=1)
    q = weight(words, scales, 1, 128, K, N, gpu)
    xd = dev(x, torch.bfloat16, gpu)
    y = B.q_matmul(xd, q)
    rows = sample_rows(M, seed=idx)
    ref = oracle.q4_linear_f64(x, words, scales, 1, 128, N, rows=rows).astype(np.float32)
    assert_parity(host(y[torch.from_numpy(rows).to(gpu)]), ref, f"c3_{name}_sampled")
    with torch.no_grad():
        full_ref = torch.matmul(xd.float(), q.dequantize())
    assert_parity(host(y), host(full_ref), f"c3_{name}_full_vs_fp32")
    perm = torch.randperm(M, generator=torch.Generator().manual_seed(idx)).to(gpu)
    y_perm = B.q_matmul(xd[perm].contiguous(), q)
    assert_parity(host(y_perm), host(y[perm]), f"c3_{name}_row_permutation", max_abs=1e-4, mean_rel=1e-6)
    monkeypatch.setenv("BIQ_GEMM_STREAMK", "0")
    y_owned = B.q_matmul(xd, q)
    assert_parity(host(y_owned), host(y), f"c3_{name}_owned_tiles", max_abs=1e-4, mean_rel=1e-6)
    assert torch.equal(B.q_matmul(xd[perm].contiguous(), q), y_owned[perm])


@pytest.mark.parametrize("name", list(W.C5_SHAPES))
def test_gpu_c5_qwen_projection(gpu, oracle, name):
    K, N = W.C5_SHAPES[name]
    M = 1024
    idx = list(W.C5_SHAPES).index(name)
    x = W.activations(5, 4 + 2 * idx, M, K, "bf16")
    words, scales = W.q4_weight(5, 5 + 2 * idx, K, N, layout=0)
    q = weight(words, scales, 0, 128, K, N, gpu)
    lin = B.Linear(q)
    y = B.qwen_linear_forward(lin, dev(x, torch.bfloat16, gpu))
    rows = sample_rows(M, seed=10 + idx)
    ref = oracle.q4_linear_f64(x, words, scales, 0, 128, N, rows=rows).astype(np.float32)
    assert_parity(host(y)[rows], ref, f"c5_{name}")


def test_gpu_real_checkpoint_shapes(gpu, oracle):
    """Released Boogu widths: K = 3360 (block 32) to N = 840 and 13568 -> 3360 (block 128)."""
    for (K, N, seed) in ((3360, 840, 1), (13568, 3360, 2)):
        blk = oracle.q4_kn_block(K, N)
        M = 45
        x = W.activations(14, seed, M, K, "f32")
        words, scales = W.q4_weight(14, 10 + seed, K, N, layout=1, block=blk)
        q = weight(words, scales, 1, blk, K, N, gpu)
        y = host(B.q_matmul(dev(x, device=gpu), q))
        ref = oracle.q4_linear_f64(x, words, scales, 1, blk, N).astype(np.float32)
        assert_parity(y, ref, f"real_{K}x{N}_blk{blk}")


@pytest.mark.parametrize("layout", [1, 0])
@pytest.mark.parametrize("block", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("xdt", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("M", [1, 7, 16])
def test_gpu_q4_linear_small_m(gpu, oracle, layout, block, xdt, M):
    """Rows <= 16 with an f32 output take the split-K streaming route: column tail (N = 200),
    a K that is a multiple of 8 but not of 32 (block 8), and several K chunks per column group."""
    K, N = (1048 if block == 8 else 1024), 200
    x = W.activations(15, M + block, M, K, xdt)
    words, scales = W.q4_weight(15, 3 + block + layout, K, N, layout=layout, block=block)
    q = weight(words, scales, layout, block, K, N, gpu)
    y = host(B.q_matmul(dev(x, TORCH_DT[xdt], gpu), q))
    ref = oracle.q4_linear_f64(x, words, scales, layout, block, N).astype(np.float32)
    assert_parity(y, ref, f"smallm_M{M}_blk{block}_l{layout}_{xdt}")


@pytest.mark.parametrize("xdt", ["f32", "bf16"])
@pytest.mark.parametrize("M, K, block", [(8, 1024, 128), (2, 256, 32), (5, 1048, 8), (8, 3360, 32)])
def test_gpu_q4_linear_small_m_staged_edges(gpu, oracle, xdt, M, K, block):
    """The [K/8, N] small-M kernel for M <= 8 stages the activations in LDS (f32 as hi parts in
    MFMA rows 0..7 and lo parts in rows 8..15): M = 8 fills both halves; K = 256 gives fewer K
    units than waves (idle waves still join the reduction); K = 3360 ends in a partial unit.  The
    activations are a row-strided view (row stride > K) and N = 200 leaves a column tail."""
    N = 200
    x = W.activations(19, M + K, M, K, xdt)
    words, scales = W.q4_weight(19, block + K, K, N, layout=1, block=block)
    wide = torch.zeros((M, K + 40), dtype=TORCH_DT[xdt], device=gpu)
    wide[:, 8:8 + K] = dev(x, TORCH_DT[xdt], gpu)
    xv = wide[:, 8:8 + K]
    assert xv.stride(0) == K + 40
    y = host(B.q_matmul(xv, weight(words, scales, 1, block, K, N, gpu)))
    ref = oracle.q4_linear_f64(x, words, scales, 1, block, N).astype(np.float32)
    assert_parity(y, ref, f"smallm_staged_M{M}_K{K}_blk{block}_{xdt}")


def test_gpu_q4_linear_small_m_bias_and_boundary(gpu, oracle):
    """Bias on the streaming route; M = 16 (streaming) and M = 17 (tiled MFMA route) agree with
    the oracle on the same rows; a second call overwrites the output (the route writes partial
    rows per K chunk and an ordered reduction adds them and the bias into y)."""
    K, N = 3360, 840
    blk = oracle.q4_kn_block(K, N)
    x = W.activations(16, 1, 17, K, "bf16")
    words, scales = W.q4_weight(16, 2, K, N, layout=1, block=blk)
    bias = np.linspace(-1, 1, N).astype(np.float32)
    lin = B.Linear(weight(words, scales, 1, blk, K, N, gpu), dev(bias, device=gpu))
    ref = oracle.q4_linear_f64(x, words, scales, 1, blk, N, bias=bias).astype(np.float32)
    xd = dev(x, torch.bfloat16, gpu)
    out = torch.full((16, N), 123.0, device=gpu)
    for _ in range(2):
        B.q_matmul(xd[:16], lin.weight, out=out, bias=lin.bias)
        assert_parity(host(out), ref[:16], "smallm_bias_M16")
    assert_parity(host(B.linear_forward(lin, xd)), ref, "tiled_bias_M17")


def test_gpu_q4_linear_modulation_row(gpu, oracle):
    """One conditioning row through the released Boogu modulation width (3360 -> 4 x 3360)."""
    K, N = 3360, 13440
    blk = oracle.q4_kn_block(K, N)
    x = W.activations(17, 1, 1, K, "f32")
    words, scales = W.q4_weight(17, 2, K, N, layout=1, block=blk)
    y = host(B.q_matmul(dev(x, device=gpu), weight(words, scales, 1, blk, K, N, gpu)))
    ref = oracle.q4_linear_f64(x, words, scales, 1, blk, N).astype(np.float32)
    assert_parity(y, ref, f"modulation_1x{K}x{N}_blk{blk}")


def test_gpu_q4_linear_small_m_deterministic_and_graph_replay(gpu, oracle):
    """Split-K partials are added in a fixed order: repeated calls are bitwise equal.  After one
    eager call has sized the stream's workspace, the call can be captured in a HIP graph; every
    replay (with eager work in between) matches the eager result bitwise."""
    K, N, M = 3072, 1024, 3
    x = W.activations(18, 1, M, K, "bf16")
    words, scales = W.q4_weight(18, 2, K, N, layout=1)
    q = weight(words, scales, 1, 128, K, N, gpu)
    xd = dev(x, torch.bfloat16, gpu)
    y0 = B.q_matmul(xd, q)
    ref = oracle.q4_linear_f64(x, words, scales, 1, 128, N).astype(np.float32)
    assert_parity(host(y0), ref, "smallm_det")
    for _ in range(3):
        assert torch.equal(B.q_matmul(xd, q), y0)
    stream = torch.cuda.Stream()
    out = torch.zeros((M, N), device=gpu)
    with torch.cuda.stream(stream):
        B.q_matmul(xd, q, out=out)  # sizes this stream's workspace outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        B.q_matmul(xd, q, out=out)
    for i in range(4):
        out.fill_(float(i))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y0), f"replay {i}"
        B.q_matmul(xd[:1], q)  # unrelated eager work between replays


@pytest.mark.parametrize("M,K,N,block,xdt,glu", [
    (4608, 3072, 9216, 128, "bf16", False),  # 1296 tiles: a tail of 16 tiles in 6 K parts
    (4608, 1024, 12288, 128, "bf16", True),  # SwiGLU, 3456 tiles: a tail of 128 in 2 parts
    (300, 1024, 1000, 32, "f16", False),     # 12 ragged tiles, block 32
    (300, 2048, 1000, 64, "bf16", True),     # SwiGLU, 24 ragged tiles, block 64
    (256, 768, 512, 128, "f32", False),      # f32 activations: one K unit is two staged tiles
    (200, 512, 256, 8, "bf16", False),       # block 8 (masked MFMA path)
])
def test_gpu_q4_linear_split_tail(gpu, oracle, monkeypatch, M, K, N, block, xdt, glu):
    """Tail tiles split along K between workgroups: sampled rows against the float64 oracle, the
    whole output against the every-tile-owned launch (same gate as any two summation orders),
    repeated calls and graph replays (GEMM + tail reduction kernels) bitwise equal."""
    x = W.activations(19, M + K, M, K, xdt)
    words, scales = W.q4_weight(19, N, K, N, layout=1, block=block)
    q = weight(words, scales, 1, block, K, N, gpu)
    xd = dev(x, TORCH_DT[xdt], gpu)
    rows = sample_rows(M, seed=M)
    ref = oracle.q4_linear_f64(x, words, scales, 1, block, N, rows=rows).astype(np.float32)
    if glu:
        w3, s3 = W.q4_weight(19, N + 1, K, N, layout=1, block=block)
        q3 = weight(w3, s3, 1, block, K, N, gpu)
        ref = silu_gate_ref(ref, oracle.q4_linear_f64(x, w3, s3, 1, block, N, rows=rows).astype(np.float32))
        call = lambda out=None: B.q_matmul_swiglu(xd, q, q3, out=out)  # noqa: E731
    else:
        call = lambda out=None: B.q_matmul(xd, q, out=out)  # noqa: E731
    y = call()
    assert_parity(host(y[torch.from_numpy(rows).to(gpu)]), ref, f"split_tail_{M}x{K}x{N}_blk{block}_{xdt}")
    for _ in range(3):
        assert torch.equal(call(), y)
    stream = torch.cuda.Stream()
    out = torch.zeros_like(y)
    with torch.cuda.stream(stream):
        call(out)  # sizes this stream's scratch outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        call(out)
    for i in range(3):
        out.fill_(float(i))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y), f"replay {i}"
        call()  # eager work on the default stream between replays
    monkeypatch.setenv("BIQ_GEMM_STREAMK", "0")
    assert_parity(host(call()), host(y), "split_tail_vs_owned", max_abs=1e-4, mean_rel=1e-6)


def silu_gate_ref(y1, y3):
    """silu(a) * b in float64 (feed_forward.rs:32-36)."""
    y1 = y1.astype(np.float64)
    return (y1 / (1.0 + np.exp(-y1)) * y3.astype(np.float64)).astype(np.float32)


@pytest.mark.parametrize("layout", [1, 0])
@pytest.mark.parametrize("block", [8, 32, 128])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_gpu_q4_swiglu_blocks_dtypes_tails(gpu, oracle, layout, block, xdt):
    """Fused silu(x.W1) * (x.W3): column tail (N = 200, not a multiple of the 128-column tile),
    row tail (M = 77), both layouts, small and large blocks, 16- and 32-bit activations."""
    M, K, N = 77, (648 if block == 8 else 640), 200
    x = W.activations(19, block + layout, M, K, xdt)
    w1, s1 = W.q4_weight(19, 1 + block + layout, K, N, layout=layout, block=block)
    w3, s3 = W.q4_weight(19, 2 + block + layout, K, N, layout=layout, block=block)
    q1, q3 = weight(w1, s1, layout, block, K, N, gpu), weight(w3, s3, layout, block, K, N, gpu)
    y = host(B.q_matmul_swiglu(dev(x, TORCH_DT[xdt], gpu), q1, q3))
    ref = silu_gate_ref(oracle.q4_linear_f64(x, w1, s1, layout, block, N),
                        oracle.q4_linear_f64(x, w3, s3, layout, block, N))
    assert_parity(y, ref, f"swiglu_blk{block}_l{layout}_{xdt}")


def test_gpu_q4_swiglu_feed_forward_and_dtypes(gpu, oracle):
    """LuminaFeedForward: linear_2(silu(linear_1 x) * linear_3 x) against the oracle's three
    f64 GEMMs with the f32-rounded gated state in between; bf16 / f16 gated outputs within their
    rounding of the f32 gate."""
    M, width, inner = 130, 256, 384
    x = W.activations(20, 1, M, width, "bf16")
    w1, s1 = W.q4_weight(20, 2, width, inner, layout=1)
    w3, s3 = W.q4_weight(20, 3, width, inner, layout=1)
    w2, s2 = W.q4_weight(20, 4, inner, width, layout=1)
    lin = [B.Linear(weight(w, s, 1, 128, k, n, gpu)) for (w, s, k, n) in
           ((w1, s1, width, inner), (w2, s2, inner, width), (w3, s3, width, inner))]
    ffn = B.LuminaFeedForward(*lin)
    xd = dev(x, torch.bfloat16, gpu)
    gated = silu_gate_ref(oracle.q4_linear_f64(x, w1, s1, 1, 128, inner),
                          oracle.q4_linear_f64(x, w3, s3, 1, 128, inner))
    ref = oracle.q4_linear_f64(gated, w2, s2, 1, 128, width).astype(np.float32)
    assert_parity(host(ffn.forward(xd)), ref, "lumina_ffn")
    g16 = host(B.q_matmul_swiglu(xd, lin[0].weight, lin[2].weight, out_dtype=torch.float16))
    assert np.max(np.abs(g16 - gated)) <= np.max(np.abs(gated)) * 2.0 ** -10
    gb = host(B.q_matmul_swiglu(xd, lin[0].weight, lin[2].weight, out_dtype=torch.bfloat16))
    assert np.max(np.abs(gb - gated)) <= np.max(np.abs(gated)) * 2.0 ** -7
    gf = host(B.q_matmul_swiglu(xd, lin[0].weight, lin[2].weight, out_dtype=torch.float32))
    assert np.array_equal(gb.view(np.uint32), W.round_to_bf16(gf).view(np.uint32))
    assert np.array_equal(g16, gf.astype(np.float16).astype(np.float32))
    with pytest.raises(B.InvalidArgument, match="share layout"):
        B.q_matmul_swiglu(xd, lin[0].weight, lin[1].weight)


def test_gpu_q4_swiglu_released_width(gpu, oracle):
    """Released Boogu FFN width: 3360 -> 13568 with block-32 scales, sampled rows."""
    K, N, M = 3360, 13568, 256
    blk = oracle.q4_kn_block(K, N)
    x = W.activations(21, 1, M, K, "f32")
    w1, s1 = W.q4_weight(21, 2, K, N, layout=1, block=blk)
    w3, s3 = W.q4_weight(21, 3, K, N, layout=1, block=blk)
    y = host(B.q_matmul_swiglu(dev(x, device=gpu), weight(w1, s1, 1, blk, K, N, gpu),
                               weight(w3, s3, 1, blk, K, N, gpu)))
    rows = sample_rows(M, n=24, seed=21)
    ref = silu_gate_ref(oracle.q4_linear_f64(x, w1, s1, 1, blk, N, rows=rows),
                        oracle.q4_linear_f64(x, w3, s3, 1, blk, N, rows=rows))
    assert_parity(y[rows], ref, f"swiglu_released_{K}x{N}_blk{blk}")


@pytest.mark.parametrize("layout", [1, 0])
def test_gpu_q4_linear_on_loaded_payload(gpu, oracle, layout):
    """An importer payload (words then scales, artifacts.rs:7364-7377) copied to the GPU as one
    uint8 buffer runs the GEMM through zero-copy views, against the f64 oracle."""
    rng = np.random.default_rng(95 + layout)
    if layout == 1:
        K, N = 3360, 840
        w = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
        words, scales, blk = oracle.q4_quantize_kn(w)
        shape, dtype = (K, N), B.q4s_stored_dtype(B.BOOGU_DENOISER, (K, N))
    else:
        N, K = 1024, 4096
        w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        words, scales = oracle.q4_quantize_nk(w)
        blk = 128
        shape, dtype = (N, K), B.q4s_stored_dtype(B.QWEN3_VL, (N, K))
    payload = torch.from_numpy(np.frombuffer(words.astype("<u4").tobytes() + scales.astype("<f4").tobytes(),
                                             np.uint8).copy()).to(gpu)
    q = B.from_payload(payload, dtype, shape)
    assert q.words.data_ptr() == payload.data_ptr() and q.block == blk and q.layout == layout
    x = W.activations(15, layout, 200, K, "bf16")
    y = B.q_matmul(dev(x, torch.bfloat16, gpu), q)
    ref = oracle.q4_linear_f64(x, words, scales, layout, blk, N).astype(np.float32)
    assert_parity(host(y), ref, f"payload_layout{layout}")


def test_gpu_release_stream_workspace(gpu, oracle):
    """biq_release_stream_workspace frees the scratch of a stream (after waiting for it); the next
    call on that stream allocates again and gives the same bits."""
    K, N, M = 3072, 1024, 5
    x = W.activations(19, 1, M, K, "bf16")
    words, scales = W.q4_weight(19, 2, K, N, layout=1)
    q = weight(words, scales, 1, 128, K, N, gpu)
    xd = dev(x, torch.bfloat16, gpu)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        y0 = B.q_matmul(xd, q)
        B._lib.check(B._lib.load().biq_release_stream_workspace(stream.cuda_stream))
        y1 = B.q_matmul(xd, q)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    with torch.cuda.stream(stream):
        B._lib.check(B._lib.load().biq_release_stream_workspace(stream.cuda_stream))
    B._lib.check(B._lib.load().biq_release_stream_workspace(stream.cuda_stream))  # nothing left: fine
