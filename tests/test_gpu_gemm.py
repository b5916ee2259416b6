"""GPU parity for aten.mm / aten.addmm / aten.bmm through the C-ABI.

Reference behaviour: src/shaders/mm/index.ts:32-93, src/shaders/bmm/
index.ts:27-96; addmm is the reference's mm + broadcast add composition.
"""
import numpy as np
import pytest

from gpu_util import assert_parity, normwise, round_in, sample_rows

pytestmark = pytest.mark.gpu


def _arr(t):
    return np.asarray(t["data"], np.float32).reshape(t["shape"])


def run_mm(ctx, A, B, dtype, bias=None, trans_b=False, alpha=1.0, beta=1.0):
    ta, tb = ctx.from_numpy(A, dtype), ctx.from_numpy(B, dtype)
    M, N = A.shape[0], (B.shape[0] if trans_b else B.shape[1])
    to = ctx.tensor(dtype, [M, N])
    tbias = ctx.from_numpy(bias, dtype) if bias is not None else None
    ctx.reset()
    ctx.mm(ta, tb, to, bias=tbias, alpha=alpha, beta=beta, trans_b=trans_b)
    kernel = ctx.last_kernel
    ctx.submit()
    ctx.sync()
    return to.get_f32(), kernel


def test_reference_kats_mm_bmm(gpu_ctx, kats):
    for c in kats:
        if c["op"] not in ("aten.mm.default", "aten.bmm.default"):
            continue
        a, b = round_in(_arr(c["a"]), c["dtype"]), round_in(_arr(c["b"]), c["dtype"])
        ta, tb = gpu_ctx.from_numpy(a, c["dtype"]), gpu_ctx.from_numpy(b, c["dtype"])
        shape = list(a.shape[:-1]) + [b.shape[-1]]
        to = gpu_ctx.tensor(c["dtype"], shape)
        gpu_ctx.reset()
        if c["op"] == "aten.mm.default":
            gpu_ctx.mm(ta, tb, to)
        else:
            gpu_ctx.bmm(ta, tb, to)
        gpu_ctx.submit()
        gpu_ctx.sync()
        got = to.get_f32()
        exp = np.matmul(a.astype(np.float64), b.astype(np.float64))
        if c["expected"] is not None:
            assert np.max(np.abs(got.ravel() - np.asarray(c["expected"]))) <= c["tol"], c["source"]
        assert np.max(np.abs(got - exp)) <= c["tol"], c["source"]


def test_config1_mm_fp32_512(gpu_ctx, orc, pkg):
    I = pkg.inputs
    A = I.uniform(0, (512, 512), -1, 1)
    B = I.uniform(1, (512, 512), -1, 1)
    got, kernel = run_mm(gpu_ctx, A, B, "float32")
    ref, refa = orc.gemm_f64(A, B)
    assert_parity(got, ref, refa, "float32", 512, "config1 " + kernel)
    emu = orc.emu_gemm(0, A, B)
    assert normwise(got, emu) < 1e-6


@pytest.mark.parametrize("trans_b", [False, True])
def test_config4_addmm_fp16(gpu_ctx, orc, pkg, trans_b):
    I = pkg.inputs
    X = I.as_f16(I.normal(10, (4096, 768)))
    W = I.as_f16(I.normal(11, (768, 3072), 0.0, 0.02))
    bias = I.as_f16(I.uniform(12, (3072,), -0.1, 0.1))
    Wop = np.ascontiguousarray(W.T) if trans_b else W
    got, kernel = run_mm(gpu_ctx, X, Wop, "float16", bias=bias, trans_b=trans_b)
    # every one of the 4096 x 3072 outputs against the fp64 brute force
    ref, refa = orc.gemm_f64(X, W, bias)
    assert ref.shape == (4096, 3072)
    assert_parity(got, ref, refa, "float16", 768, "config4 addmm " + kernel)
    rows = sample_rows(4096)
    emu = orc.emu_addmm(1, X, W, bias, rows=rows[:64])
    assert normwise(got[rows[:64]], emu) < 2e-2


def test_config4_addmm_nn_equals_nt_bitwise(gpu_ctx, pkg):
    """Both weight layouts feed identical k-ordered fragments to the MFMA."""
    I = pkg.inputs
    X = I.as_f16(I.normal(20, (512, 768)))
    W = I.as_f16(I.normal(21, (768, 384), 0.0, 0.02))
    bias = I.as_f16(I.uniform(22, (384,), -0.1, 0.1))
    nn, _ = run_mm(gpu_ctx, X, W, "float16", bias=bias)
    nt, _ = run_mm(gpu_ctx, X, np.ascontiguousarray(W.T), "float16", bias=bias, trans_b=True)
    assert np.array_equal(nn.view(np.uint32), nt.view(np.uint32))


@pytest.mark.parametrize("trans_b", [False, True])
def test_config4_bmm_fp16(gpu_ctx, orc, pkg, trans_b):
    """The config-4 bmm in both layouts of the right operand ([K, N] as given,
    and its [N, K] transpose with trans_b), every element against fp64; both
    take the short-K kernel (K = 64, a 16 Mi-element output)."""
    I = pkg.inputs
    A = I.as_f16(I.normal(30, (16, 1024, 64)))
    B = I.as_f16(I.normal(31, (16, 64, 1024)))
    Bop = np.ascontiguousarray(B.transpose(0, 2, 1)) if trans_b else B
    ta, tb = gpu_ctx.from_numpy(A, "float16"), gpu_ctx.from_numpy(Bop, "float16")
    to = gpu_ctx.tensor("float16", [16, 1024, 1024])
    gpu_ctx.reset()
    gpu_ctx.bmm(ta, tb, to, trans_b=trans_b)
    kernel = gpu_ctx.last_kernel
    gpu_ctx.submit()
    gpu_ctx.sync()
    got = to.get_f32()
    ref, refa = orc.gemm_f64(A, B)
    assert kernel.endswith(("_nk_sk" if trans_b else "_kn_sk")), kernel
    assert_parity(got, ref, refa, "float16", 64, "bmm " + kernel)


SK_SHAPES = [(45, 40, 8), (130, 264, 24), (257, 136, 64), (128, 128, 16), (300, 200, 56), (1, 1000, 40)]


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("trans_b", [False, True])
def test_short_k_kernel_edges(gpu_ctx, orc, pkg, monkeypatch, dtype, trans_b):
    """The short-K kernel forced (WGX_SK=1) onto ragged shapes: partial 128 x
    128 tiles in M and N, K from 8 to 64 (zero-padded to whole k-steps), a
    batch of 3 and a single row; mm with a column bias, alpha and beta, and
    bmm; both dtypes and both layouts of B."""
    monkeypatch.setenv("WGX_SK", "1")
    I = pkg.inputs
    for i, (M, N, K) in enumerate(SK_SHAPES):
        A = round_in(I.uniform(3100 + i, (M, K), -1, 1), dtype)
        B = round_in(I.uniform(3200 + i, (K, N), -1, 1), dtype)
        bias = round_in(I.uniform(3300 + i, (N,), -0.5, 0.5), dtype)
        alpha, beta = (0.5, 2.0) if i % 2 else (1.0, 1.0)
        Bop = np.ascontiguousarray(B.T) if trans_b else B
        got, kernel = run_mm(gpu_ctx, A, Bop, dtype, bias=bias, trans_b=trans_b, alpha=alpha, beta=beta)
        assert kernel.endswith("_sk"), kernel
        ref, refa = orc.gemm_f64(A, B)
        ref = alpha * ref + beta * bias
        refa = abs(alpha) * refa + abs(beta) * np.abs(bias)
        assert_parity(got, ref, refa, dtype, K, f"sk mm {dtype} {M}x{N}x{K} tb={trans_b} {kernel}")
        Ab = round_in(I.uniform(3400 + i, (3, M, K), -1, 1), dtype)
        Bb = round_in(I.uniform(3500 + i, (3, K, N), -1, 1), dtype)
        Bbop = np.ascontiguousarray(Bb.transpose(0, 2, 1)) if trans_b else Bb
        ta, tb = gpu_ctx.from_numpy(Ab, dtype), gpu_ctx.from_numpy(Bbop, dtype)
        to = gpu_ctx.tensor(dtype, [3, M, N])
        gpu_ctx.reset()
        gpu_ctx.bmm(ta, tb, to, trans_b=trans_b)
        kernel = gpu_ctx.last_kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        assert kernel.endswith("_sk"), kernel
        ref, refa = orc.gemm_f64(Ab, Bb)
        assert_parity(to.get_f32(), ref, refa, dtype, K, f"sk bmm {dtype} {M}x{N}x{K} tb={trans_b} {kernel}")


SHAPES = [(5, 3, 7), (1, 1, 1), (33, 65, 17), (64, 64, 64), (100, 37, 129), (130, 260, 72),
          (257, 129, 200), (96, 1000, 8), (7, 300, 513)]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("trans_b", [False, True])
def test_mm_shapes_sweep(gpu_ctx, orc, pkg, dtype, trans_b):
    I = pkg.inputs
    for i, (M, N, K) in enumerate(SHAPES):
        A = round_in(I.uniform(100 + i, (M, K), -1, 1), dtype)
        B = round_in(I.uniform(200 + i, (K, N), -1, 1), dtype)
        bias = round_in(I.uniform(300 + i, (N,), -0.5, 0.5), dtype)
        Bop = np.ascontiguousarray(B.T) if trans_b else B
        alpha, beta = (0.5, 2.0) if i % 2 else (1.0, 1.0)
        got, kernel = run_mm(gpu_ctx, A, Bop, dtype, bias=bias, trans_b=trans_b, alpha=alpha, beta=beta)
        ref, refa = orc.gemm_f64(A, B)
        ref = alpha * ref + beta * bias
        refa = abs(alpha) * refa + abs(beta) * np.abs(bias)
        assert_parity(got, ref, refa, dtype, K, f"mm {dtype} {M}x{N}x{K} tb={trans_b} {kernel}")


def test_bmm_trans_and_ragged(gpu_ctx, orc, pkg):
    I = pkg.inputs
    for dtype in ("float32", "float16"):
        A = round_in(I.uniform(400, (3, 45, 70), -1, 1), dtype)
        B = round_in(I.uniform(401, (3, 70, 33), -1, 1), dtype)
        for tb in (False, True):
            Bop = np.ascontiguousarray(B.transpose(0, 2, 1)) if tb else B
            ta, tbb = gpu_ctx.from_numpy(A, dtype), gpu_ctx.from_numpy(Bop, dtype)
            to = gpu_ctx.tensor(dtype, [3, 45, 33])
            gpu_ctx.reset()
            gpu_ctx.bmm(ta, tbb, to, trans_b=tb)
            gpu_ctx.submit()
            gpu_ctx.sync()
            ref, refa = orc.gemm_f64(A, B)
            assert_parity(to.get_f32(), ref, refa, dtype, 70, f"bmm {dtype} tb={tb}")


@pytest.mark.parametrize("tile", ["256x192b", "192x256b"])
def test_large_tile_kernel_edges(gpu_ctx, orc, pkg, tile, monkeypatch):
    """The large-tile [N, K] kernel forced onto ragged shapes: partial tiles
    in M and N, K with a partial last slice (K % 32 != 0), several tiles per
    block, a batch of transposed-B products, alpha/beta and both dtypes."""
    I = pkg.inputs
    monkeypatch.setenv("WGX_MFMA_TILE", tile)
    for i, (M, N, K) in enumerate([(300, 200, 104), (513, 385, 136), (256, 192, 32), (1024, 768, 2056),
                                   (40, 24, 64)]):
        for dtype in ("float16", "bfloat16"):
            A = round_in(I.uniform(1400 + i, (M, K), -1, 1), dtype)
            B = round_in(I.uniform(1500 + i, (K, N), -1, 1), dtype)
            bias = round_in(I.uniform(1600 + i, (N,), -0.5, 0.5), dtype)
            alpha, beta = (0.5, 2.0) if i % 2 else (1.0, 1.0)
            got, kernel = run_mm(gpu_ctx, A, np.ascontiguousarray(B.T), dtype, bias=bias, trans_b=True,
                                 alpha=alpha, beta=beta)
            assert kernel.endswith("_nk_big") and tile[:-1] in kernel, kernel
            ref, refa = orc.gemm_f64(A, B)
            ref = alpha * ref + beta * bias
            refa = abs(alpha) * refa + abs(beta) * np.abs(bias)
            assert_parity(got, ref, refa, dtype, K, f"big {tile} {dtype} {M}x{N}x{K} {kernel}")
    A = round_in(I.uniform(1700, (3, 260, 72), -1, 1), "float16")
    B = round_in(I.uniform(1701, (3, 72, 200), -1, 1), "float16")
    ta = gpu_ctx.from_numpy(A, "float16")
    tbb = gpu_ctx.from_numpy(np.ascontiguousarray(B.transpose(0, 2, 1)), "float16")
    to = gpu_ctx.tensor("float16", [3, 260, 200])
    gpu_ctx.reset()
    gpu_ctx.bmm(ta, tbb, to, trans_b=True)
    kernel = gpu_ctx.last_kernel
    gpu_ctx.submit()
    gpu_ctx.sync()
    assert kernel.endswith("_nk_big"), kernel
    ref, refa = orc.gemm_f64(A, B)
    assert_parity(to.get_f32(), ref, refa, "float16", 72, f"big bmm {tile} {kernel}")


@pytest.mark.parametrize("tile", ["256x192b", "192x256b"])
def test_kn_operand_staged_for_large_tile_kernel(gpu_ctx, orc, pkg, tile, monkeypatch):
    """A [K, N] B on the large-tile kernel: rewritten as [N, K] by the staging
    pass, then multiplied by the [N, K] kernel.  Ragged tiles in M, N and K
    (partial 64 x 64 staging tiles), a batch, alpha / beta, both 16-bit
    types; the result must carry the same bits as the [N, K] form of the
    same product and be within the fp16 bound of the fp64 oracle."""
    I = pkg.inputs
    monkeypatch.setenv("WGX_MFMA_TILE", tile)
    for i, (M, N, K) in enumerate([(300, 200, 104), (513, 392, 136), (256, 192, 32), (70, 8, 2056)]):
        for dtype in ("float16", "bfloat16"):
            A = round_in(I.uniform(2400 + i, (M, K), -1, 1), dtype)
            B = round_in(I.uniform(2500 + i, (K, N), -1, 1), dtype)
            bias = round_in(I.uniform(2600 + i, (N,), -0.5, 0.5), dtype)
            alpha, beta = (0.5, 2.0) if i % 2 else (1.0, 1.0)
            nn, k_nn = run_mm(gpu_ctx, A, B, dtype, bias=bias, alpha=alpha, beta=beta)
            nt, k_nt = run_mm(gpu_ctx, A, np.ascontiguousarray(B.T), dtype, bias=bias, trans_b=True,
                              alpha=alpha, beta=beta)
            assert k_nn.endswith("_kn2nk_big") and tile[:-1] in k_nn, k_nn
            assert k_nt.endswith("_nk_big") and not k_nt.endswith("kn2nk_big"), k_nt
            ref, refa = orc.gemm_f64(A, B)
            ref = alpha * ref + beta * bias
            refa = abs(alpha) * refa + abs(beta) * np.abs(bias)
            assert_parity(nn, ref, refa, dtype, K, f"staged {tile} {dtype} {M}x{N}x{K} {k_nn}")
            assert np.array_equal(nn, nt), f"staged {tile} {dtype} {M}x{N}x{K}: [K,N] != [N,K] bits"
    # a batch of [K, N] right operands
    A = round_in(I.uniform(2700, (3, 260, 72), -1, 1), "float16")
    B = round_in(I.uniform(2701, (3, 72, 200), -1, 1), "float16")
    ta, tbb = gpu_ctx.from_numpy(A, "float16"), gpu_ctx.from_numpy(B, "float16")
    to = gpu_ctx.tensor("float16", [3, 260, 200])
    gpu_ctx.reset()
    gpu_ctx.bmm(ta, tbb, to)
    kernel = gpu_ctx.last_kernel
    gpu_ctx.submit()
    gpu_ctx.sync()
    assert kernel.endswith("_kn2nk_big"), kernel
    ref, refa = orc.gemm_f64(A, B)
    assert_parity(to.get_f32(), ref, refa, "float16", 72, f"staged bmm {tile} {kernel}")


def test_config4_addmm_nn_takes_staged_large_tiles(gpu_ctx, orc, pkg):
    """The config-4 addmm in aten.mm's own [K, N] weight layout runs the
    staging pass and the large-tile kernel by default, and replays of the
    recorded pair agree with its [N, K] form bit for bit."""
    I = pkg.inputs
    M, K, N = 4096, 768, 3072
    X = round_in(I.normal(2800, (M, K)), "float16")
    W = round_in(I.normal(2801, (K, N), 0, 0.02), "float16")
    b = round_in(I.uniform(2802, (N,), -0.1, 0.1), "float16")
    nn, k_nn = run_mm(gpu_ctx, X, W, "float16", bias=b)
    assert k_nn.endswith("_kn2nk_big"), k_nn
    nt, _ = run_mm(gpu_ctx, X, np.ascontiguousarray(W.T), "float16", bias=b, trans_b=True)
    assert np.array_equal(nn, nt)
    rows = sample_rows(M, 64)
    ref, refa = orc.gemm_f64(X, W, b, rows=rows)
    assert_parity(nn[rows], ref, refa, "float16", K, f"config4 NN {k_nn}")


@pytest.mark.parametrize("cfg", ["1x1w4", "1x1w8", "2x1w4", "2x1w8", "1x2w4"])
def test_wave_split_f32_gemm(gpu_ctx, orc, pkg, monkeypatch, cfg):
    """fp32 GEMMs with few tiles on every wave-split configuration: both B
    layouts (the same bits either way), ragged edges, alpha / beta / bias."""
    monkeypatch.setenv("WGX_WS", cfg)
    I = pkg.inputs
    for i, (M, K, N) in enumerate([(512, 512, 512), (100, 72, 130), (33, 256, 65)]):
        A = I.uniform(900 + i, (M, K), -1, 1).astype(np.float32)
        B = I.uniform(910 + i, (K, N), -1, 1).astype(np.float32)
        bias = I.uniform(920 + i, (N,), -0.5, 0.5).astype(np.float32)
        alpha, beta = (1.0, 1.0) if i == 0 else (0.75, -1.5)
        nn, k_nn = run_mm(gpu_ctx, A, B, "float32", bias=bias, alpha=alpha, beta=beta)
        nt, k_nt = run_mm(gpu_ctx, A, np.ascontiguousarray(B.T), "float32", bias=bias, alpha=alpha,
                          beta=beta, trans_b=True)
        assert k_nn.endswith("_kn_ws") and k_nt.endswith("_nk_ws"), (k_nn, k_nt)
        ref, refa = orc.gemm_f64(A, B, None)
        ref = alpha * ref + beta * bias.astype(np.float64)
        refa = abs(alpha) * refa + abs(beta) * np.abs(bias.astype(np.float64))
        assert_parity(nn, ref, refa, "float32", K, f"ws {cfg} mm {M}x{K}x{N} {k_nn}")
        assert np.array_equal(nn.view(np.uint32), nt.view(np.uint32)), f"ws {cfg} {M}x{K}x{N}: NN != NT"
