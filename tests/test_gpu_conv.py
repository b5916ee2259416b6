"""GPU parity for aten.convolution (implicit-im2col GEMM, 1x1, depthwise,
grouped and transposed fallbacks) and the conv_with_clamp epilogue, through
the C-ABI.  Reference behaviour: src/shaders/convolution/index.ts:58-310.
"""
import numpy as np
import pytest

from gpu_util import assert_parity, normwise, round_in

pytestmark = pytest.mark.gpu


def _arr(t):
    return np.asarray(t["data"], np.float32).reshape(t["shape"])


def run_conv(ctx, x, w, b, dtype, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1,
             transposed=False, output_padding=(0, 0), out_shape=None, clamp=None):
    tx, tw = ctx.from_numpy(x, dtype), ctx.from_numpy(w, dtype)
    tb = ctx.from_numpy(b, dtype) if b is not None else None
    ty = ctx.tensor(dtype, out_shape)
    ctx.reset()
    ctx.convolution(tx, tw, tb, list(stride), list(padding), list(dilation), transposed,
                    list(output_padding), groups, ty, clamp=clamp)
    kernel = ctx.last_kernel
    ctx.submit()
    ctx.sync()
    return ty.get_f32(), kernel


def test_reference_kats_conv(gpu_ctx, kats):
    for c in kats:
        if c["op"] != "aten.convolution.default":
            continue
        dt = c["dtype"]
        x, w = round_in(_arr(c["input"]), dt), round_in(_arr(c["weight"]), dt)
        b = round_in(_arr(c["bias"]), dt) if c["bias"] else None
        got, kernel = run_conv(gpu_ctx, x, w, b, dt, c["stride"], c["padding"], c["dilation"],
                               c["groups"], c["transposed"], c["output_padding"], c["out_shape"])
        if c["expected"] is not None:
            err = np.max(np.abs(got.ravel() - np.asarray(c["expected"])))
            assert err <= max(c["tol"], 2e-5), f"{c['source']} via {kernel}: {err}"
        else:  # element-0 checks of the 1x1 tile tests
            e0 = float(np.dot(x.reshape(x.shape[1], -1)[:, 0].astype(np.float64),
                              w.reshape(w.shape[0], -1)[0].astype(np.float64)))
            assert abs(got.ravel()[0] - e0) <= c["tol"], c["source"]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("variant", ["2a", "2b"])
def test_config2_conv(gpu_ctx, orc, pkg, dtype, variant):
    I = pkg.inputs
    if variant == "2a":
        xs, ws, s, os_ = (1, 64, 80, 80), (128, 64, 3, 3), (1, 1), [1, 128, 80, 80]
    else:
        xs, ws, s, os_ = (1, 128, 80, 80), (256, 128, 3, 3), (2, 2), [1, 256, 40, 40]
    x = round_in(I.uniform(40, xs, -1, 1), dtype)
    w = round_in(I.kaiming_uniform(41, ws), dtype)
    b = round_in(I.uniform(42, (ws[0],), -0.1, 0.1), dtype)
    got, kernel = run_conv(gpu_ctx, x, w, b, dtype, s, (1, 1), out_shape=os_)
    ref, refa = orc.conv2d_f64(x, w, b, s, (1, 1))
    K = ws[1] * ws[2] * ws[3]
    assert_parity(got, ref, refa, dtype, K, f"config{variant} {dtype} {kernel}")
    if dtype == "float16":
        emu = orc.emu_conv2d(1, x, w, b, s, (1, 1))
        assert normwise(got, emu) < 2e-2


@pytest.mark.parametrize("case", ["A", "B"])
def test_config3_depthwise_fp16(gpu_ctx, orc, pkg, case):
    I = pkg.inputs
    if case == "A":
        xs, ws, s, p, os_ = (1, 256, 40, 40), (256, 1, 3, 3), (1, 1), (1, 1), [1, 256, 40, 40]
    else:
        xs, ws, s, p, os_ = (1, 512, 20, 20), (512, 1, 5, 5), (2, 2), (2, 2), [1, 512, 10, 10]
    x = I.as_f16(I.normal(50, xs))
    w = I.as_f16(I.uniform(51, ws, -0.5, 0.5))
    b = np.zeros(ws[0], np.float32)
    got, kernel = run_conv(gpu_ctx, x, w, b, "float16", s, p, groups=ws[0], out_shape=os_)
    assert kernel.startswith("depthwise"), kernel
    ref, refa = orc.conv2d_f64(x, w, b, s, p, groups=ws[0])
    assert_parity(got, ref, refa, "float16", ws[2] * ws[3], f"config3{case} {kernel}")
    emu = orc.emu_conv2d(1, x, w, b, s, p, groups=ws[0])
    assert normwise(got, emu) < 1e-2


DW_SWEEP = [
    # x shape, kernel, stride, clamp -- "same" padding (k // 2), dilation 1
    ((2, 24, 40, 40), 3, 1, False),      # 8-wide segments, 16-byte rows
    ((1, 8, 20, 20), 5, 2, False),       # 4-wide segments, rows straddle chunks
    ((1, 6, 13, 17), 3, 1, True),        # odd width, clamp epilogue
    ((1, 4, 15, 15), 3, 2, False),       # stride 2, odd size
    ((1, 5, 9, 22), 5, 1, False),        # 5x5 stride 1
    ((1, 3, 300, 300), 3, 1, False),     # bands of one large plane (last band short)
    ((1, 2, 129, 131), 5, 2, True),      # bands, stride 2, odd sizes
    ((1, 1537, 8, 8), 3, 1, False),      # several planes per block, partial last block
    ((3, 7, 1, 1), 3, 1, False),         # 1x1 image: every tap but the centre is padding
    ((1, 4, 8, 256), 3, 1, False),       # 32 segments per row
    ((1, 3, 10, 512), 3, 1, True),       # 64 segments: one plane per wave
    ((40, 256, 40, 40), 3, 1, False),    # enough waves for 8-row bands
    ((84, 512, 20, 20), 5, 2, False),    # 8-row bands, stride 2, masked last segment
]


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_depthwise_sweep(gpu_ctx, orc, pkg, dtype):
    """Depthwise fast family (K x K, stride 1/2, same padding) against the fp64
    oracle, including bands of large planes, several planes per block and the
    clamp epilogue."""
    I = pkg.inputs
    for i, (xs, k, s, clamp) in enumerate(DW_SWEEP):
        c = xs[1]
        x = round_in(I.normal(1000 + i, xs), dtype)
        w = round_in(I.uniform(1100 + i, (c, 1, k, k), -0.5, 0.5), dtype)
        b = round_in(I.uniform(1200 + i, (c,), -0.5, 0.5), dtype)
        p = (k // 2, k // 2)
        ref, refa = orc.conv2d_f64(x, w, b, (s, s), p, groups=c)
        cl = (-0.5, 0.75) if clamp else None
        got, kernel = run_conv(gpu_ctx, x, w, b, dtype, (s, s), p, groups=c,
                               out_shape=list(ref.shape), clamp=cl)
        if cl:
            ref = np.clip(ref, *cl)
        assert kernel.startswith(f"depthwise_{ {'float16': 'f16', 'float32': 'f32'}[dtype] }"
                                 f"_{k}x{k}s{s}"), kernel
        assert_parity(got, ref, refa, dtype, k * k, f"dw {i} {dtype} {xs} k{k} s{s} {kernel}")


def _reg_kernel_applies(iw, ow, k, s):
    """Widths the fp16 register kernel takes: even input and output widths,
    at most 64 segments of 4 or 8 outputs per row."""
    ov = 4 if (ow + 3) // 4 * 4 < (ow + 7) // 8 * 8 or (s == 2 and k == 5) else 8
    return iw % 2 == 0 and ow % 2 == 0 and (ow + ov - 1) // ov <= 64


def test_depthwise_register_kernel_forced(gpu_ctx, orc, pkg, monkeypatch):
    """The fp16 register kernel on every sweep shape it accepts (even widths),
    including the small ones the automatic choice gives to the LDS-tiled
    kernel, plain and with the SiLU + residual epilogue."""
    W, I = pkg.wgx, pkg.inputs
    monkeypatch.setenv("WGX_DW_KERNEL", "reg")
    dtype = "float16"
    for i, (xs, k, s, clamp) in enumerate(DW_SWEEP):
        c = xs[1]
        x = round_in(I.normal(1000 + i, xs), dtype)
        w = round_in(I.uniform(1100 + i, (c, 1, k, k), -0.5, 0.5), dtype)
        b = round_in(I.uniform(1200 + i, (c,), -0.5, 0.5), dtype)
        p = (k // 2, k // 2)
        ref, refa = orc.conv2d_f64(x, w, b, (s, s), p, groups=c)
        cl = (-0.5, 0.75) if clamp else None
        got, kernel = run_conv(gpu_ctx, x, w, b, dtype, (s, s), p, groups=c,
                               out_shape=list(ref.shape), clamp=cl)
        if cl:
            ref = np.clip(ref, *cl)
        if _reg_kernel_applies(xs[3], ref.shape[3], k, s):
            assert "_r" in kernel, (xs, kernel)
        assert_parity(got, ref, refa, dtype, k * k, f"dw reg {i} {xs} k{k} s{s} {kernel}")
    for i, (xs, ws, s, p, d, (cs, rs), inplace) in enumerate(RESIDUAL_CASES):
        if d != (1, 1):
            continue
        g = xs[1]
        x = round_in(I.uniform(1900 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(1910 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(1920 + i, (ws[0],), -0.5, 0.5), dtype)
        ref, refa = orc.conv2d_f64(x, w, b, s, p, d, g)
        r = round_in(I.uniform(1930 + i, ref.shape, -2, 2), dtype)
        tx, tw, tb = gpu_ctx.from_numpy(x, dtype), gpu_ctx.from_numpy(w, dtype), gpu_ctx.from_numpy(b, dtype)
        tr = gpu_ctx.from_numpy(r, dtype)
        ty = tr if inplace else gpu_ctx.tensor(dtype, list(ref.shape))
        gpu_ctx.reset()
        gpu_ctx.convolution(tx, tw, tb, list(s), list(p), list(d), False, [0, 0], g, ty,
                            activation=W.ACT_SILU, residual=tr, conv_scale=cs, residual_scale=rs)
        kernel = gpu_ctx.last_kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        if _reg_kernel_applies(xs[3], ref.shape[3], ws[2], s[1]):
            assert "_r" in kernel, (xs, kernel)
        want = cs * (ref / (1.0 + np.exp(-ref))) + rs * r.astype(np.float64)
        bound = 1.1 * abs(cs) * refa + abs(rs) * np.abs(r.astype(np.float64))
        assert_parity(ty.get_f32(), want, bound, dtype, ws[1] * ws[2] * ws[3],
                      f"residual reg {i} {xs}x{ws} {kernel}")


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_depthwise_unaligned_views(gpu_ctx, orc, pkg, dtype):
    """Input and output views that start off a 16-byte boundary (program
    memory-plan offsets can): the staging reads aligned chunks around the view
    and the tail chunk of the input element-wise, stores fall back to scalar."""
    I = pkg.inputs
    es = 2 if dtype == "float16" else 4
    xs, k = (1, 16, 24, 24), 3
    x = round_in(I.normal(1300, xs), dtype)
    w = round_in(I.uniform(1301, (16, 1, k, k), -0.5, 0.5), dtype)
    ref, refa = orc.conv2d_f64(x, w, None, (1, 1), (1, 1), groups=16)
    nx = int(np.prod(xs))
    bx = gpu_ctx.storage_buffer(nx * es + 64)
    by = gpu_ctx.storage_buffer(nx * es + 64)
    for ox, oy in ((es, 3 * es), (7 * es, 0), (64 - 0, es)):
        # the input view ends exactly at the end of its buffer when ox == 64
        tx = gpu_ctx.tensor(dtype, list(xs), bx + ox)
        tx.set_data(x.astype(np.float16) if dtype == "float16" else x.astype(np.float32))
        tw = gpu_ctx.from_numpy(w, dtype)
        ty = gpu_ctx.tensor(dtype, list(xs), by + oy)
        gpu_ctx.reset()
        gpu_ctx.convolution(tx, tw, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 16, ty)
        kernel = gpu_ctx.last_kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        assert_parity(ty.get_f32(), ref, refa, dtype, 9, f"unaligned x+{ox} y+{oy} {kernel}")
    gpu_ctx.reset()
    gpu_ctx.free(bx)
    gpu_ctx.free(by)


SILU_CASES = [
    # x shape, w shape, stride, pad, groups -- one per kernel family
    ((1, 16, 20, 20), (32, 16, 3, 3), (1, 1), (1, 1), 1),        # implicit-im2col GEMM
    ((1, 3, 32, 32), (16, 3, 3, 3), (2, 2), (1, 1), 1),          # small-tap direct kernel (stem)
    ((1, 32, 12, 12), (48, 32, 1, 1), (1, 1), (0, 0), 1),        # 1x1, few tiles: one-tap im2col
    ((1, 16, 160, 160), (32, 16, 1, 1), (1, 1), (0, 0), 1),      # 1x1, many tiles: plain GEMM
    ((1, 128, 40, 40), (256, 128, 3, 3), (2, 2), (1, 1), 1),     # split-K GEMM + reduction
    ((1, 24, 16, 16), (24, 1, 3, 3), (1, 1), (1, 1), 24),        # depthwise, register kernel (fp16)
    ((1, 6, 13, 17), (6, 1, 5, 5), (2, 2), (2, 2), 6),           # depthwise, LDS kernel
    ((1, 8, 12, 12), (8, 1, 3, 3), (1, 1), (2, 2), 8),           # depthwise, generic (dilation 2 below)
    ((1, 8, 10, 10), (12, 4, 3, 3), (1, 1), (1, 1), 2),          # grouped direct
]


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_conv_silu_epilogue(gpu_ctx, orc, pkg, dtype):
    """The SiLU epilogue (bias, then x * sigmoid(x), one rounding) on every
    convolution kernel family, against the fp64 oracle's convolution followed
    by SiLU in fp64."""
    W, I = pkg.wgx, pkg.inputs
    for i, (xs, ws, s, p, g) in enumerate(SILU_CASES):
        d = (2, 2) if i == 7 else (1, 1)
        x = round_in(I.uniform(1800 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(1810 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(1820 + i, (ws[0],), -0.5, 0.5), dtype)
        ref, refa = orc.conv2d_f64(x, w, b, s, p, d, g)
        tx, tw, tb = gpu_ctx.from_numpy(x, dtype), gpu_ctx.from_numpy(w, dtype), gpu_ctx.from_numpy(b, dtype)
        ty = gpu_ctx.tensor(dtype, list(ref.shape))
        gpu_ctx.reset()
        gpu_ctx.convolution(tx, tw, tb, list(s), list(p), list(d), False, [0, 0], g, ty, activation=W.ACT_SILU)
        kernel = gpu_ctx.last_kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        silu = ref / (1.0 + np.exp(-ref))
        # |d silu / dx| <= 1.1: the convolution's error bound, scaled
        assert_parity(ty.get_f32(), silu, 1.1 * refa, dtype, ws[1] * ws[2] * ws[3],
                      f"silu {i} {dtype} {xs}x{ws} {kernel}")


CONV_SWEEP = [
    # x shape, w shape, stride, pad, dilation, groups
    ((1, 3, 64, 64), (16, 3, 3, 3), (2, 2), (1, 1), (1, 1), 1),      # stem: K = 27
    ((1, 32, 20, 20), (64, 32, 1, 1), (1, 1), (0, 0), (1, 1), 1),    # pointwise, few tiles: one-tap im2col
    ((1, 16, 160, 160), (32, 16, 1, 1), (1, 1), (0, 0), (1, 1), 1),  # pointwise, 400 tiles: [IC, H*W] GEMM
    ((2, 32, 17, 19), (48, 32, 1, 1), (1, 1), (0, 0), (1, 1), 1),    # pointwise, batch 2, ragged
    ((1, 16, 21, 13), (24, 16, 1, 1), (2, 2), (0, 0), (1, 1), 1),    # strided 1x1 -> im2col path
    ((2, 24, 15, 15), (40, 24, 3, 3), (1, 1), (2, 2), (2, 2), 1),    # dilation 2
    ((1, 16, 33, 31), (72, 16, 5, 5), (2, 1), (2, 1), (1, 1), 1),    # 5x5, mixed stride/pad
    ((1, 8, 9, 9), (8, 8, 7, 7), (1, 1), (3, 3), (1, 1), 1),         # 7x7 (49 taps)
    ((1, 64, 8, 8), (300, 64, 3, 3), (1, 1), (1, 1), (1, 1), 1),     # OC not a tile multiple
    ((2, 16, 12, 12), (16, 1, 3, 3), (1, 1), (1, 1), (1, 1), 16),    # depthwise, batch 2
    ((1, 12, 19, 23), (12, 1, 7, 7), (2, 3), (3, 2), (1, 2), 12),    # depthwise generic
    ((1, 8, 10, 10), (12, 4, 3, 3), (1, 1), (1, 1), (1, 1), 2),      # grouped fallback
    ((1, 3, 70, 70), (8, 3, 4, 4), (3, 3), (0, 0), (1, 1), 1),       # no padding, K = 48
    ((1, 3, 40, 36), (48, 3, 3, 3), (1, 1), (1, 1), (1, 1), 1),      # small-tap kernel, 48 of 64 channels
    ((2, 1, 17, 19), (20, 1, 5, 5), (2, 1), (2, 1), (1, 1), 1),      # small-tap, 25 taps, batch 2, ragged
    ((1, 2, 15, 15), (5, 2, 3, 3), (1, 2), (2, 1), (2, 2), 1),       # small-tap, dilation 2
    ((1, 16, 160, 160), (16, 16, 3, 3), (1, 1), (1, 1), (1, 1), 1),  # <= 32 channels, 400 tiles: 32x32 wave-split (fp16)
    ((1, 8, 129, 131), (24, 8, 3, 3), (1, 1), (1, 1), (1, 1), 1),    # the same, ragged: 24 channels, 265 tiles
]


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_conv_sweep(gpu_ctx, orc, pkg, dtype):
    I = pkg.inputs
    for i, (xs, ws, s, p, d, g) in enumerate(CONV_SWEEP):
        x = round_in(I.uniform(500 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(600 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(700 + i, (ws[0],), -0.5, 0.5), dtype) if i % 3 else None
        ref, refa = orc.conv2d_f64(x, w, b, s, p, d, g)
        got, kernel = run_conv(gpu_ctx, x, w, b, dtype, s, p, d, g, out_shape=list(ref.shape))
        K = ws[1] * ws[2] * ws[3]
        assert_parity(got, ref, refa, dtype, K, f"sweep {i} {dtype} {xs}x{ws} s{s} p{p} d{d} g{g} {kernel}")


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_conv_transpose(gpu_ctx, orc, pkg, dtype):
    I = pkg.inputs
    for i, (xs, ws, s, p, d, g, op) in enumerate([
        ((1, 4, 7, 6), (4, 3, 3, 3), (2, 2), (1, 1), (1, 1), 1, (1, 1)),
        ((2, 6, 5, 5), (6, 2, 2, 3), (2, 1), (0, 1), (1, 2), 3, (1, 0)),
    ]):
        x = round_in(I.uniform(800 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(810 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(820 + i, (ws[1] * g,), -0.5, 0.5), dtype)
        ref, refa = orc.conv_transpose2d_f64(x, w, b, s, p, d, g, op)
        got, kernel = run_conv(gpu_ctx, x, w, b, dtype, s, p, d, g, True, op, list(ref.shape))
        assert_parity(got, ref, refa, dtype, xs[1] // g * ws[2] * ws[3], f"convT {i} {dtype} {kernel}")


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_conv_with_clamp_epilogue(gpu_ctx, orc, pkg, dtype):
    """et_vk.conv_with_clamp: bias, then clamp, then one rounding."""
    I = pkg.inputs
    for xs, ws, g in (((1, 16, 12, 12), (32, 16, 3, 3), 1), ((1, 16, 12, 12), (16, 1, 3, 3), 16)):
        x = round_in(I.uniform(900, xs, -1, 1), dtype)
        w = round_in(I.uniform(901, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(902, (ws[0],), -0.5, 0.5), dtype)
        ref, refa = orc.conv2d_f64(x, w, b, (1, 1), (1, 1), groups=g)
        got, kernel = run_conv(gpu_ctx, x, w, b, dtype, (1, 1), (1, 1), groups=g,
                               out_shape=list(ref.shape), clamp=(0.0, 6.0))
        assert got.min() >= 0.0 and got.max() <= 6.0
        assert_parity(got, np.clip(ref, 0.0, 6.0), refa, dtype, ws[1] * 9, f"clamp {kernel}")


WS_CONFIGS = ["1x1w4", "1x1w8", "2x1w4", "2x1w8", "1x2w4"]
WS_CASES = [
    # x shape, w shape, stride, pad, dilation: ragged M and N, batch 2,
    # dilation, 5x5, a K range that is not a multiple of the 64-wide slice
    ((1, 16, 21, 13), (24, 16, 3, 3), (1, 1), (1, 1), (1, 1)),
    ((2, 24, 15, 15), (40, 24, 3, 3), (1, 1), (2, 2), (2, 2)),
    ((1, 16, 33, 31), (72, 16, 5, 5), (2, 1), (2, 1), (1, 1)),
    ((1, 64, 20, 20), (64, 64, 3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 128, 10, 10), (100, 128, 3, 3), (2, 2), (1, 1), (1, 1)),
]


@pytest.mark.parametrize("cfg", WS_CONFIGS)
@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_wave_split_configurations(gpu_ctx, orc, pkg, monkeypatch, dtype, cfg):
    """Every instantiated wave-split configuration (forced through WGX_WS)
    against the float64 convolution, including batch 2 and ragged tiles."""
    monkeypatch.setenv("WGX_WS", cfg)
    monkeypatch.setenv("WGX_CONV_LDS", "off")  # the 3x3 cases would take the LDS-patch kernel
    I = pkg.inputs
    for i, (xs, ws, s, p, d) in enumerate(WS_CASES):
        x = round_in(I.uniform(800 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(810 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(820 + i, (ws[0],), -0.5, 0.5), dtype) if i % 2 else None
        ref, refa = orc.conv2d_f64(x, w, b, s, p, d, 1)
        got, kernel = run_conv(gpu_ctx, x, w, b, dtype, s, p, d, 1, out_shape=list(ref.shape))
        tm, tn = cfg.split("w")[0].split("x")
        assert kernel.endswith(f"_{32 * int(tm)}x{32 * int(tn)}w{cfg.split('w')[1]}_conv_ws"), kernel
        K = ws[1] * ws[2] * ws[3]
        assert_parity(got, ref, refa, dtype, K, f"ws {cfg} case {i} {dtype} {xs}x{ws} {kernel}")


RESIDUAL_CASES = [
    # x shape, w shape, stride, pad, dilation, (conv scale, residual scale), in place
    ((1, 24, 16, 16), (24, 1, 3, 3), (1, 1), (1, 1), (1, 1), (1.0, 1.0), False),   # register kernel (fp16)
    ((2, 16, 20, 20), (16, 1, 5, 5), (2, 2), (2, 2), (1, 1), (0.5, 1.0), False),   # register kernel, stride 2
    ((1, 6, 13, 17), (6, 1, 3, 3), (1, 1), (1, 1), (1, 1), (1.0, -2.0), False),    # LDS kernel (odd width)
    ((1, 8, 12, 12), (8, 1, 3, 3), (1, 1), (2, 2), (2, 2), (1.0, 1.0), False),     # generic (dilation 2)
    ((1, 32, 10, 10), (32, 1, 3, 3), (1, 1), (1, 1), (1, 1), (1.0, 1.0), True),    # residual is the output
]


DENSE_RESIDUAL_CASES = [
    # x shape, w shape, stride, pad, (conv scale, residual scale), in place, forced configuration
    ((1, 32, 20, 24), (48, 32, 3, 3), 1, 1, (1.0, 1.0), False, None),
    ((2, 64, 16, 16), (40, 64, 3, 3), 2, 1, (0.5, -1.0), False, None),
    ((1, 64, 24, 24), (64, 64, 3, 3), 1, 1, (1.0, 1.0), True, None),      # residual is the output
    ((1, 32, 17, 13), (24, 32, 3, 3), 1, 1, (1.0, 2.0), False, "2x2w4"),  # W > 1, ragged edges
    ((2, 32, 16, 32), (64, 32, 3, 3), 1, 1, (1.0, 1.0), True, "2x4w1"),   # the 64 x 128 tile, in place
    ((1, 32, 12, 20), (40, 32, 3, 3), 1, 1, (1.0, -0.5), False, None),    # width 20: 8-byte row pieces
    ((2, 32, 16, 16), (64, 32, 3, 3), 1, 1, (0.5, 1.0), False, "2x2w1"),  # 64 x 64 tile (pre-ordered, 16-bit)
    ((2, 32, 18, 16), (64, 32, 3, 3), 2, 1, (1.0, 1.0), False, "2x2w1"),  # the same at stride 2
]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_dense_conv_silu_residual_epilogue(gpu_ctx, orc, pkg, monkeypatch, dtype):
    """Dense 3x3 convolution + SiLU + an output-shaped residual in one launch
    of the LDS-patch kernel (channel-major float32, channel-last 16-bit),
    out = cs * silu(conv) + rs * residual, including a residual that is the
    output itself, against the fp64 oracle."""
    W, I = pkg.wgx, pkg.inputs
    for i, (xs, ws, s, p, (cs, rs), inplace, cfg) in enumerate(DENSE_RESIDUAL_CASES):
        if cfg is not None:
            if dtype == "float32" and cfg == "2x4w1":
                continue  # the 64 x 128 tile is 16-bit only
            monkeypatch.setenv("WGX_CONV_LDS", cfg)
        else:
            monkeypatch.delenv("WGX_CONV_LDS", raising=False)
        x = round_in(I.uniform(2400 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(2410 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(2420 + i, (ws[0],), -0.5, 0.5), dtype)
        ref, refa = orc.conv2d_f64(x, w, b, (s, s), (p, p), (1, 1), 1)
        r = round_in(I.uniform(2430 + i, ref.shape, -2, 2), dtype)
        tx, tw, tb = gpu_ctx.from_numpy(x, dtype), gpu_ctx.from_numpy(w, dtype), gpu_ctx.from_numpy(b, dtype)
        tr = gpu_ctx.from_numpy(r, dtype)
        ty = tr if inplace else gpu_ctx.tensor(dtype, list(ref.shape))
        gpu_ctx.reset()
        gpu_ctx.convolution(tx, tw, tb, [s, s], [p, p], [1, 1], False, [0, 0], 1, ty,
                            activation=W.ACT_SILU, residual=tr, conv_scale=cs, residual_scale=rs)
        kernel = gpu_ctx.last_kernel
        assert kernel.startswith("conv_lds_" if dtype == "float32" else "conv_cl_"), kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        want = cs * (ref / (1.0 + np.exp(-ref))) + rs * r.astype(np.float64)
        bound = 1.1 * abs(cs) * refa + abs(rs) * np.abs(r.astype(np.float64))
        assert_parity(ty.get_f32(), want, bound, dtype, ws[1] * 9,
                      f"dense residual {i} {dtype} {xs}x{ws} s{s} {kernel}")


def test_paired_convolution_launches(gpu_ctx, orc, pkg, monkeypatch):
    """Two adjacent independent float32 batch-1 convolutions run as one paired
    launch (both strides, with and without row segments, a bias, SiLU and a
    residual); a second convolution that reads the first one's output is not
    paired; WGX_MERGE=0 keeps every launch apart.  Every output against the
    float64 convolution."""
    W, I = pkg.wgx, pkg.inputs
    monkeypatch.delenv("WGX_CONV_LDS", raising=False)
    # (the part with more input channels runs 32 x 32 tiles: pairs 1 and 2
    # the second part, pair 3 the first; pair 4, equal: both on 32 x 64)
    shapes = [((1, 32, 20, 24), (48, 32, 3, 3), 1, 1), ((1, 64, 16, 16), (40, 64, 3, 3), 2, 1),
              ((1, 16, 13, 10), (24, 16, 3, 3), 1, 1), ((1, 24, 21, 19), (16, 24, 3, 3), 2, 0),
              ((1, 64, 12, 16), (32, 64, 3, 3), 1, 1), ((1, 32, 18, 20), (48, 32, 3, 3), 2, 1),
              ((1, 32, 14, 18), (24, 32, 3, 3), 1, 1), ((1, 32, 16, 12), (40, 32, 3, 3), 2, 1)]

    def record(i, xs, ws, s, p, res=False):
        x = I.uniform(3400 + i, xs, -1, 1)
        w = I.uniform(3410 + i, ws, -0.5, 0.5)
        b = I.uniform(3420 + i, (ws[0],), -0.5, 0.5)
        ref, refa = orc.conv2d_f64(x, w, b, (s, s), (p, p), (1, 1), 1)
        tx, tw, tb = gpu_ctx.from_numpy(x, "float32"), gpu_ctx.from_numpy(w, "float32"), gpu_ctx.from_numpy(b, "float32")
        ty = gpu_ctx.tensor("float32", list(ref.shape))
        if res:
            r = I.uniform(3430 + i, ref.shape, -2, 2)
            tr = gpu_ctx.from_numpy(r, "float32")
            gpu_ctx.convolution(tx, tw, tb, [s, s], [p, p], [1, 1], False, [0, 0], 1, ty,
                                activation=W.ACT_SILU, residual=tr, conv_scale=1.0, residual_scale=0.5)
            want = ref / (1.0 + np.exp(-ref)) + 0.5 * r
            bound = 1.1 * refa + 0.5 * np.abs(r)
        else:
            gpu_ctx.convolution(tx, tw, tb, [s, s], [p, p], [1, 1], False, [0, 0], 1, ty)
            want, bound = ref, refa
        assert gpu_ctx.last_kernel.startswith("conv_lds_f32_"), gpu_ctx.last_kernel
        return ty, want, bound, ws[1] * 9

    for merge, expect in (("1", 4), ("0", 0)):
        monkeypatch.setenv("WGX_MERGE", merge)
        gpu_ctx.reset()
        outs = [record(i, *sh, res=(i == 3)) for i, sh in enumerate(shapes)]
        gpu_ctx.submit()
        gpu_ctx.sync()
        assert gpu_ctx.paired_launches == expect
        for i, (ty, want, bound, K) in enumerate(outs):
            assert_parity(ty.get_f32(), want, bound, "float32", K, f"paired {merge} conv {i} {shapes[i]}")
    # b reads a's output: not independent, two launches
    monkeypatch.setenv("WGX_MERGE", "1")
    gpu_ctx.reset()
    x = I.uniform(3500, (1, 16, 12, 12), -1, 1)
    w1 = I.uniform(3501, (16, 16, 3, 3), -0.5, 0.5)
    w2 = I.uniform(3502, (8, 16, 3, 3), -0.5, 0.5)
    tx, t1, t2 = gpu_ctx.from_numpy(x, "float32"), gpu_ctx.from_numpy(w1, "float32"), gpu_ctx.from_numpy(w2, "float32")
    ty1 = gpu_ctx.tensor("float32", [1, 16, 12, 12])
    ty2 = gpu_ctx.tensor("float32", [1, 8, 12, 12])
    gpu_ctx.convolution(tx, t1, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 1, ty1)
    gpu_ctx.convolution(ty1, t2, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 1, ty2)
    gpu_ctx.submit()
    gpu_ctx.sync()
    assert gpu_ctx.paired_launches == 0
    y1 = ty1.get_f32()
    ref2, refa2 = orc.conv2d_f64(y1, w2, None, (1, 1), (1, 1), (1, 1), 1)
    assert_parity(ty2.get_f32(), ref2, refa2, "float32", 16 * 9, "dependent pair")


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_depthwise_silu_residual_epilogue(gpu_ctx, orc, pkg, dtype):
    """Depthwise convolution + SiLU + an output-shaped residual in one launch,
    out = cs * silu(conv) + rs * residual, against the fp64 oracle."""
    W, I = pkg.wgx, pkg.inputs
    for i, (xs, ws, s, p, d, (cs, rs), inplace) in enumerate(RESIDUAL_CASES):
        g = xs[1]
        x = round_in(I.uniform(1900 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(1910 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(1920 + i, (ws[0],), -0.5, 0.5), dtype)
        ref, refa = orc.conv2d_f64(x, w, b, s, p, d, g)
        r = round_in(I.uniform(1930 + i, ref.shape, -2, 2), dtype)
        tx, tw, tb = gpu_ctx.from_numpy(x, dtype), gpu_ctx.from_numpy(w, dtype), gpu_ctx.from_numpy(b, dtype)
        tr = gpu_ctx.from_numpy(r, dtype)
        ty = tr if inplace else gpu_ctx.tensor(dtype, list(ref.shape))
        gpu_ctx.reset()
        gpu_ctx.convolution(tx, tw, tb, list(s), list(p), list(d), False, [0, 0], g, ty,
                            activation=W.ACT_SILU, residual=tr, conv_scale=cs, residual_scale=rs)
        kernel = gpu_ctx.last_kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        want = cs * (ref / (1.0 + np.exp(-ref))) + rs * r.astype(np.float64)
        bound = 1.1 * abs(cs) * refa + abs(rs) * np.abs(r.astype(np.float64))
        assert_parity(ty.get_f32(), want, bound, dtype, ws[1] * ws[2] * ws[3],
                      f"residual {i} {dtype} {xs}x{ws} {kernel}")


LDS_CASES = [
    # x shape, w shape, stride, pad: ragged output channels, widths that are
    # not a multiple of the 8-pixel region, batch 2, stride 2, padding 0 and 2,
    # and maps smaller than one region
    ((1, 16, 21, 13), (24, 16, 3, 3), 1, 1),
    ((2, 32, 15, 17), (40, 32, 3, 3), 1, 1),
    ((1, 64, 20, 20), (64, 64, 3, 3), 1, 1),
    ((1, 128, 10, 10), (100, 128, 3, 3), 2, 1),
    ((2, 48, 33, 31), (72, 48, 3, 3), 2, 1),
    ((1, 16, 9, 9), (16, 16, 3, 3), 1, 0),
    ((1, 32, 12, 11), (8, 32, 3, 3), 2, 2),
    ((1, 16, 3, 5), (33, 16, 3, 3), 1, 1),
]
LDS_CONFIGS = ["2x2w1", "2x2w4", "2x1w2", "1x2w8", "2x1w1"]
# float32 chunks are 8 input channels: counts that are not a multiple of 16
# (the widths that are a multiple of 4 take the row-segment patch loads)
LDS_CASES_F32 = [
    ((1, 8, 13, 13), (16, 8, 3, 3), 1, 1),
    ((2, 24, 10, 9), (40, 24, 3, 3), 2, 1),
    ((1, 40, 17, 16), (72, 40, 3, 3), 1, 1),
    ((1, 16, 12, 12), (24, 16, 3, 3), 1, 0),
    ((2, 8, 9, 16), (32, 8, 3, 3), 2, 1),
    ((1, 24, 7, 28), (40, 24, 3, 3), 1, 2),
    ((1, 32, 21, 36), (33, 32, 3, 3), 2, 2),
]


@pytest.mark.parametrize("cfg", LDS_CONFIGS)
@pytest.mark.parametrize("dtype,form", [("float32", "lds"), ("float16", "cl"), ("bfloat16", "cl"),
                                        ("float16", "lds"), ("bfloat16", "lds")])
def test_lds_patch_configurations(gpu_ctx, orc, pkg, monkeypatch, dtype, form, cfg):
    """Every configuration of the LDS-patch 3x3 kernels (forced through
    WGX_CONV_LDS; 16-bit data in both patch forms, channel-last and
    channel-major, WGX_CONV_CL) against the float64 convolution; every second
    case with a bias, with SiLU or with a clamp in the epilogue."""
    W = pkg.wgx
    monkeypatch.setenv("WGX_CONV_LDS", cfg)
    monkeypatch.setenv("WGX_CONV_CL", "1" if form == "cl" else "0")
    I = pkg.inputs
    for i, (xs, ws, s, p) in enumerate(LDS_CASES):
        x = round_in(I.uniform(900 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(910 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(920 + i, (ws[0],), -0.5, 0.5), dtype) if i % 2 else None
        ref, refa = orc.conv2d_f64(x, w, b, (s, s), (p, p), (1, 1), 1)
        tx, tw = gpu_ctx.from_numpy(x, dtype), gpu_ctx.from_numpy(w, dtype)
        tb = gpu_ctx.from_numpy(b, dtype) if b is not None else None
        ty = gpu_ctx.tensor(dtype, list(ref.shape))
        mode = i % 3  # 0 plain, 1 SiLU, 2 clamp
        gpu_ctx.reset()
        gpu_ctx.convolution(tx, tw, tb, [s, s], [p, p], [1, 1], False, [0, 0], 1, ty,
                            clamp=(-0.25, 0.5) if mode == 2 else None,
                            activation=W.ACT_SILU if mode == 1 else W.ACT_NONE)
        kernel = gpu_ctx.last_kernel
        pre = form == "cl" and cfg == "2x2w1"  # pre-ordered weights
        assert kernel.startswith(f"conv_{form}_") and kernel.endswith(
            f"_{32 * int(cfg[0])}x{32 * int(cfg[2])}w{cfg.split('w')[1]}" + ("_pre" if pre else "")), kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        got = ty.get_f32()
        if mode == 1:
            # the reference applies SiLU to the rounded-in-fp64 conv output; the
            # bound carries the conv's error through SiLU (|d silu| <= 1.1)
            ref = ref / (1.0 + np.exp(-ref))
            refa = 1.1 * refa
        elif mode == 2:
            ref = np.clip(ref, -0.25, 0.5)
        assert_parity(got, ref, refa, dtype, ws[1] * 9, f"lds {cfg} case {i} {dtype} {xs}x{ws} s{s} p{p} {kernel}")


# 16-bit images whose width is a multiple of 8 columns (the channel-last
# kernel's row-segment patch loads): every patch offset within a segment
# (padding 0, 1, 2 at both strides), maps narrower than a segment row,
# ragged output channels and batch 2
CL_SEG_CASES = [
    ((1, 16, 16, 16), (24, 16, 3, 3), 1, 1),
    ((2, 32, 15, 24), (40, 32, 3, 3), 1, 1),
    ((1, 64, 20, 40), (64, 64, 3, 3), 1, 0),
    ((1, 32, 10, 16), (100, 32, 3, 3), 2, 1),
    ((2, 48, 33, 32), (72, 48, 3, 3), 2, 1),
    ((1, 16, 9, 8), (16, 16, 3, 3), 1, 2),
    ((1, 32, 12, 24), (8, 32, 3, 3), 2, 2),
    ((1, 16, 3, 8), (33, 16, 3, 3), 1, 1),
    ((1, 32, 17, 40), (64, 32, 3, 3), 2, 0),
    ((1, 32, 12, 16), (200, 32, 3, 3), 1, 1),   # pre-ordered: 4 output-channel tiles share a patch
    ((2, 16, 14, 24), (150, 16, 3, 3), 2, 1),   # 3 share, stride 2
]


@pytest.mark.parametrize("rv", ["1", "0"])
@pytest.mark.parametrize("cfg", ["2x4w1", "2x2w1", "2x2w1c16", "2x2w4", "2x1w4", "1x2w8", "1x1w1"])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_channel_last_row_segments(gpu_ctx, orc, pkg, monkeypatch, dtype, cfg, rv):
    """The channel-last 16-bit kernel with its patch loaded as 16-byte row
    segments turned channel-last in registers (WGX_CONV_RV=1) and as element
    loads (WGX_CONV_RV=0), forced into each configuration, against the
    float64 convolution; a bias and SiLU on every second case.  The 64 x 128
    tile (2x4) is built for stride 1 only."""
    W, I = pkg.wgx, pkg.inputs
    monkeypatch.setenv("WGX_CONV_LDS", cfg)
    monkeypatch.setenv("WGX_CONV_CL", "1")
    monkeypatch.setenv("WGX_CONV_RV", rv)
    for i, (xs, ws, s, p) in enumerate(CL_SEG_CASES):
        if cfg == "2x4w1" and s != 1:
            continue
        x = round_in(I.uniform(1900 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(1910 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(1920 + i, (ws[0],), -0.5, 0.5), dtype) if i % 2 else None
        ref, refa = orc.conv2d_f64(x, w, b, (s, s), (p, p), (1, 1), 1)
        tx, tw = gpu_ctx.from_numpy(x, dtype), gpu_ctx.from_numpy(w, dtype)
        tb = gpu_ctx.from_numpy(b, dtype) if b is not None else None
        ty = gpu_ctx.tensor(dtype, list(ref.shape))
        gpu_ctx.reset()
        gpu_ctx.convolution(tx, tw, tb, [s, s], [p, p], [1, 1], False, [0, 0], 1, ty,
                            activation=W.ACT_SILU if i % 2 else W.ACT_NONE)
        kernel = gpu_ctx.last_kernel
        tile = f"_{32 * int(cfg[0])}x{32 * int(cfg[2])}w{cfg.split('w')[1]}"
        if rv == "0":
            tile = tile.replace("c16", "")  # 16-column regions take row segments only
        # the one-wave 64 x 64 tile (either stride) and 64 x 128 tile (stride
        # 1) run on pre-ordered weights (a reorder pass first)
        pre = cfg in ("2x4w1", "2x2w1", "2x2w1c16")
        assert kernel.startswith("conv_cl_") and kernel.endswith(tile + ("_pre" if pre else "")), kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        if i % 2:
            ref = ref / (1.0 + np.exp(-ref))
            refa = 1.1 * refa
        assert_parity(ty.get_f32(), ref, refa, dtype, ws[1] * 9,
                      f"cl seg rv={rv} {cfg} case {i} {dtype} {xs}x{ws} s{s} p{p} {kernel}")


@pytest.mark.parametrize("pre", ["1", "0"])
def test_batched_16bit_convolution_default_choice(gpu_ctx, orc, pkg, monkeypatch, pre):
    """Batched 16-bit 3x3 convolutions through the automatic kernel choice:
    enough tiles for the many-tile rule, which takes the channel-last kernel:
    the 64 x 64 one-wave tile on pre-ordered weights (a reorder pass into a
    workspace first) at either stride or, with WGX_CONV_PRE=0, the 64 x 128
    tile on the raw weights at stride 1 and the GEMM at stride 2; every
    output element against the float64 convolution."""
    I = pkg.inputs
    monkeypatch.setenv("WGX_CONV_PRE", pre)
    # (16-column regions at stride 1 where the width is a multiple of 16)
    want16 = "conv_cl_f16_3x3s1_64x64w1c16_pre" if pre == "1" else "conv_cl_f16_3x3s1_64x128w1"
    want = "conv_cl_f16_3x3s1_64x64w1_pre" if pre == "1" else "conv_cl_f16_3x3s1_64x128w1"
    want2 = "conv_cl_f16_3x3s2_64x64w1_pre" if pre == "1" else "gemm_mfma_f16"
    cases = [((128, 32, 32, 32), (64, 32, 3, 3), 1, 1, want16), ((256, 32, 20, 24), (40, 32, 3, 3), 1, 1, want),
             ((512, 32, 20, 24), (40, 32, 3, 3), 2, 1, want2)]
    for i, (xs, ws, s, p, want) in enumerate(cases):
        x = round_in(I.uniform(2900 + i, xs, -1, 1), "float16")
        w = round_in(I.uniform(2910 + i, ws, -0.5, 0.5), "float16")
        b = round_in(I.uniform(2920 + i, (ws[0],), -0.5, 0.5), "float16")
        ref, refa = orc.conv2d_f64(x, w, b, (s, s), (p, p), (1, 1), 1)
        got, kernel = run_conv(gpu_ctx, x, w, b, "float16", (s, s), (p, p), out_shape=list(ref.shape))
        assert kernel.startswith(want), kernel
        assert_parity(got, ref, refa, "float16", ws[1] * 9, f"batched {i} {xs}x{ws} s{s} {kernel}")


@pytest.mark.parametrize("rv", ["1", "0"])
@pytest.mark.parametrize("cfg", ["1x2w4", "2x1w2", "1x1w1", "2x2w8"])
def test_lds_patch_float32_eight_channel_chunks(gpu_ctx, orc, pkg, monkeypatch, cfg, rv):
    """The float32 LDS-patch kernel on input channel counts that are a
    multiple of 8 but not of 16 (its chunks are 8 channels), widths with and
    without the row-segment patch loads (WGX_CONV_RV=0 forces element
    loads), padding 0 to 2, against the float64 convolution, with a bias and
    SiLU on every second case."""
    W, I = pkg.wgx, pkg.inputs
    monkeypatch.setenv("WGX_CONV_LDS", cfg)
    monkeypatch.setenv("WGX_CONV_RV", rv)
    for i, (xs, ws, s, p) in enumerate(LDS_CASES_F32):
        x = I.uniform(960 + i, xs, -1, 1)
        w = I.uniform(970 + i, ws, -0.5, 0.5)
        b = I.uniform(980 + i, (ws[0],), -0.5, 0.5) if i % 2 else None
        ref, refa = orc.conv2d_f64(x, w, b, (s, s), (p, p), (1, 1), 1)
        tx, tw = gpu_ctx.from_numpy(x, "float32"), gpu_ctx.from_numpy(w, "float32")
        tb = gpu_ctx.from_numpy(b, "float32") if b is not None else None
        ty = gpu_ctx.tensor("float32", list(ref.shape))
        gpu_ctx.reset()
        gpu_ctx.convolution(tx, tw, tb, [s, s], [p, p], [1, 1], False, [0, 0], 1, ty,
                            activation=W.ACT_SILU if i % 2 else W.ACT_NONE)
        kernel = gpu_ctx.last_kernel
        assert kernel.startswith("conv_lds_f32_"), kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        if i % 2:
            ref = ref / (1.0 + np.exp(-ref))
            refa = 1.1 * refa
        assert_parity(ty.get_f32(), ref, refa, "float32", ws[1] * 9, f"lds f32 {cfg} case {i} {xs}x{ws} s{s} {kernel}")


# bfloat16 dense convolutions on every route (the GEMM's im2col mode is built
# for float32 and float16 only): the direct kernel for spatial kernels the
# LDS-patch kernel does not take, the plain GEMM for 1x1 convolutions with
# few tiles, and the 64 x 64 LDS-patch tile where float16 would take the
# GEMM (widths not a multiple of 8, stride 2 without pre-ordered weights)
BF16_ROUTE_CASES = [
    ((1, 8, 20, 20), (16, 8, 5, 5), 1, 2, {}, "conv_grouped_direct"),
    ((2, 24, 20, 20), (16, 24, 3, 3), 1, 1, {}, "conv_grouped_direct"),
    ((1, 32, 40, 40), (64, 32, 1, 1), 1, 0, {}, "gemm_mfma_bf16_"),
    ((2, 48, 12, 12), (24, 48, 1, 1), 2, 0, {}, "conv_grouped_direct"),
    ((64, 32, 40, 41), (64, 32, 3, 3), 1, 1, {}, "conv_cl_bf16_3x3s1_64x64w1_pre"),
    ((512, 32, 20, 24), (40, 32, 3, 3), 2, 1, {"WGX_CONV_PRE": "0"}, "conv_cl_bf16_3x3s2_64x64w1"),
]


@pytest.mark.parametrize("case", range(len(BF16_ROUTE_CASES)))
def test_bfloat16_convolution_routes(gpu_ctx, orc, pkg, monkeypatch, case):
    """Each bfloat16 route records (no set-up failure), names the expected
    kernel and matches the float64 convolution on every element."""
    I = pkg.inputs
    xs, ws, s, p, env, want = BF16_ROUTE_CASES[case]
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    x = round_in(I.uniform(3900 + case, xs, -1, 1), "bfloat16")
    w = round_in(I.uniform(3910 + case, ws, -0.5, 0.5), "bfloat16")
    b = round_in(I.uniform(3920 + case, (ws[0],), -0.5, 0.5), "bfloat16")
    ref, refa = orc.conv2d_f64(x, w, b, (s, s), (p, p), (1, 1), 1)
    got, kernel = run_conv(gpu_ctx, x, w, b, "bfloat16", (s, s), (p, p), out_shape=list(ref.shape))
    assert kernel.startswith(want), kernel
    assert_parity(got, ref, refa, "bfloat16", ws[1] * ws[2] * ws[3], f"bf16 route {case} {xs}x{ws} s{s} {kernel}")


# clamp and residual in one launch (the epilogues are instantiated per clamp /
# residual pair): out = cs * clamp(silu(conv)) + rs * residual, on the dense
# LDS-patch kernels (8-byte row pieces at width 20, the pre-ordered 64 x 64
# tile at both strides, W > 1 with ragged edges) and the depthwise kernels
CLAMP_RES_CASES = [
    ((1, 32, 12, 20), (40, 32, 3, 3), 1, 1, 1, None),
    ((2, 32, 16, 16), (256, 32, 3, 3), 1, 1, 1, "2x2w1"),
    ((2, 32, 18, 16), (128, 32, 3, 3), 2, 1, 1, "2x2w1"),
    ((1, 32, 17, 13), (24, 32, 3, 3), 1, 1, 1, "2x2w4"),
    ((2, 32, 16, 24), (128, 32, 3, 3), 1, 1, 1, "2x2w1c16"),   # 16-column regions, ragged last
    ((1, 32, 22, 40), (256, 32, 3, 3), 2, 1, 1, "2x2w1c16"),   # the same at stride 2
    ((2, 48, 20, 20), (48, 1, 3, 3), 1, 1, 48, None),
    ((2, 64, 20, 20), (64, 1, 5, 5), 2, 2, 64, None),
]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_conv_clamp_and_residual(gpu_ctx, orc, pkg, monkeypatch, dtype):
    """SiLU, a clamp and a residual together against the float64 convolution
    (the clamp is 1-Lipschitz, so the SiLU bound carries through it)."""
    W, I = pkg.wgx, pkg.inputs
    cs, rs, lo, hi = 0.5, -1.0, -0.25, 0.5
    for i, (xs, ws, s, p, g, cfg) in enumerate(CLAMP_RES_CASES):
        if cfg is not None:
            monkeypatch.setenv("WGX_CONV_LDS", cfg)
        else:
            monkeypatch.delenv("WGX_CONV_LDS", raising=False)
        x = round_in(I.uniform(4400 + i, xs, -1, 1), dtype)
        w = round_in(I.uniform(4410 + i, ws, -0.5, 0.5), dtype)
        b = round_in(I.uniform(4420 + i, (ws[0],), -0.5, 0.5), dtype)
        ref, refa = orc.conv2d_f64(x, w, b, (s, s), (p, p), (1, 1), g)
        r = round_in(I.uniform(4430 + i, ref.shape, -2, 2), dtype)
        tx, tw, tb = gpu_ctx.from_numpy(x, dtype), gpu_ctx.from_numpy(w, dtype), gpu_ctx.from_numpy(b, dtype)
        tr = gpu_ctx.from_numpy(r, dtype)
        ty = gpu_ctx.tensor(dtype, list(ref.shape))
        gpu_ctx.reset()
        gpu_ctx.convolution(tx, tw, tb, [s, s], [p, p], [1, 1], False, [0, 0], g, ty, clamp=(lo, hi),
                            activation=W.ACT_SILU, residual=tr, conv_scale=cs, residual_scale=rs)
        kernel = gpu_ctx.last_kernel
        if cfg in ("2x2w1", "2x2w1c16") and dtype != "float32":
            assert kernel.endswith(("c16_pre" if cfg.endswith("c16") else "w1_pre")), kernel
        gpu_ctx.submit()
        gpu_ctx.sync()
        want = cs * np.clip(ref / (1.0 + np.exp(-ref)), lo, hi) + rs * r.astype(np.float64)
        bound = 1.1 * abs(cs) * refa + abs(rs) * np.abs(r.astype(np.float64))
        assert_parity(ty.get_f32(), want, bound, dtype, ws[1] * ws[2] * ws[3],
                      f"clamp+residual case {i} {dtype} {xs}x{ws} s{s} g{g} {kernel}")
