"""CPU tests of the C-ABI boundary: libwgx.so loads and exports every symbol
include/wgx.h declares, and the host-only validation context reproduces the
reference's accept/reject behaviour and integer shape logic without a GPU.
"""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "wgx.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wgx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(pkg):
    L = pkg.wgx.lib()
    names = declared_symbols()
    assert len(names) >= 25
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(pkg.wgx.SIGNATURES), set(names) ^ set(pkg.wgx.SIGNATURES)


def test_struct_layouts_match_header(pkg):
    W = pkg.wgx
    assert ctypes.sizeof(W.CTensor) == 8 + 4 + 4 + 8 * 8
    assert ctypes.sizeof(W.CConvArgs) == 4 * 14  # 13 words of conv arguments + activation


@pytest.fixture()
def hctx(pkg):
    c = pkg.wgx.Context(-1)
    yield c
    c.destroy()


def test_host_context_buffers(hctx):
    assert not hctx.has_device and hctx.arch == "host"
    p = hctx.storage_buffer(1)
    assert hctx.buffer_size(p) == 4  # max(4, round_up(size, 4)), src/context.ts:86-92
    t = hctx.tensor("float32", [2, 3])
    assert t.byte_length == 24 and t.numel == 6
    t.set_data(np.arange(6, dtype=np.float32))
    t.set_data(np.array([7, 8], np.float32))
    assert t.get_data().ravel().tolist() == [7, 8, 2, 3, 4, 5]
    with pytest.raises(ValueError, match="pass a view"):
        t.set_data(np.zeros(8, np.float32))
    with pytest.raises(ValueError, match="exceeds maximum rank"):
        hctx.tensor("float32", [1] * 9)
    with pytest.raises(ValueError, match="positive integers"):
        hctx.tensor("float32", [0, 3])
    with pytest.raises(ValueError, match="< required"):
        hctx.tensor("float32", [4, 4], buffer=hctx.storage_buffer(16))


def test_submit_without_device_fails_loudly(hctx, pkg):
    a, b, o = hctx.tensor("float32", [4, 4]), hctx.tensor("float32", [4, 4]), hctx.tensor("float32", [4, 4])
    hctx.mm(a, b, o)
    with pytest.raises(pkg.wgx.WgxError, match="no device"):
        hctx.submit()


def test_mm_validation(hctx, pkg):
    E = pkg.wgx.WgxError
    a = hctx.tensor("float32", [4, 8])
    b = hctx.tensor("float32", [8, 5])
    o = hctx.tensor("float32", [4, 5])
    hctx.mm(a, b, o)  # K = 8: 16-byte rows, so float32 runs on the matrix cores
    assert hctx.last_kernel.startswith("gemm_mfma_f32")
    hctx.mm(hctx.tensor("float32", [4, 7]), hctx.tensor("float32", [7, 5]), o)
    assert hctx.last_kernel.startswith("gemm_f32")  # K = 7: the vector-FMA kernel
    with pytest.raises(E, match="inner dimensions must match"):
        hctx.mm(a, a, o)
    with pytest.raises(E, match="Output shape|output shape"):
        hctx.mm(a, b, hctx.tensor("float32", [5, 4]))
    with pytest.raises(E, match="2D"):
        hctx.mm(hctx.tensor("float32", [1, 4, 8]), b, o)
    with pytest.raises(E, match="matching"):
        hctx.mm(hctx.tensor("float16", [4, 8]), b, o)
    h = [hctx.tensor("float16", s) for s in ([64, 96], [96, 80], [64, 80])]
    hctx.mm(*h)
    assert hctx.last_kernel.startswith("gemm_mfma_f16") and "_kn" in hctx.last_kernel
    hctx.mm(h[0], hctx.tensor("float16", [80, 96]), h[2], trans_b=True)
    assert hctx.last_kernel.endswith("nk")
    # the config-4 addmm shape: large tiles in both weight layouts, a [K, N]
    # weight through the [N, K] staging pass
    big = [hctx.tensor("float16", s) for s in ([4096, 768], [768, 3072], [4096, 3072])]
    hctx.mm(*big)
    assert hctx.last_kernel == "gemm_mfma_f16_256x192w8_kn2nk_big", hctx.last_kernel
    hctx.mm(big[0], hctx.tensor("float16", [3072, 768]), big[2], trans_b=True)
    assert hctx.last_kernel == "gemm_mfma_f16_256x192w8_nk_big", hctx.last_kernel
    with pytest.raises(E, match="bias"):
        hctx.mm(*h, bias=hctx.tensor("float16", [7]))


def test_buffer_bounds_are_enforced(hctx, pkg):
    """A view larger than its buffer never reaches a launch record."""
    W = pkg.wgx
    small = hctx.storage_buffer(64)
    t = W.Tensor(hctx, "float32", [16], small, 64)
    big = W.Tensor.__new__(W.Tensor)
    big.ctx, big.dtype, big.shape, big.ptr = hctx, "float32", [32], small
    big.numel, big.byte_length = 32, 128
    with pytest.raises(W.WgxError, match="not inside a buffer"):
        hctx.mm(big.__class__.__new__(W.Tensor) if False else big, t, t)


def test_conv_validation_and_variants(hctx, pkg, monkeypatch):
    E = pkg.wgx.WgxError
    T = hctx.tensor

    def conv(xs, ws, os_, stride=(1, 1), pad=(0, 0), dil=(1, 1), groups=1, transposed=False,
             op=(0, 0), dtype="float16", bias=True):
        x, w, y = T(dtype, xs), T(dtype, ws), T(dtype, os_)
        b = T(dtype, [os_[1]]) if bias else None
        hctx.convolution(x, w, b, stride, pad, dil, transposed, op, groups, y)
        return hctx.last_kernel

    # dense 3x3 over a multiple of 16 channels: the LDS-patch kernel at batch
    # 1 (32 x 64 tiles, 64 x 32 for 16-bit data at stride 2, W waves up to
    # the 16-channel chunk count), 64 x 64 one-wave tiles for batched float32,
    # for batched 16-bit data the 64 x 64 channel-last tile on pre-ordered
    # weights while it gives every SIMD a wave (WGX_CONV_PRE=0: the 64 x 128
    # tile at stride 1), else the GEMM kernels
    assert conv([1, 64, 80, 80], [128, 64, 3, 3], [1, 128, 80, 80], pad=(1, 1)) == "conv_cl_f16_3x3s1_32x64w4"
    assert conv([1, 128, 80, 80], [256, 128, 3, 3], [1, 256, 40, 40], (2, 2), (1, 1)) == "conv_cl_f16_3x3s2_64x32w8"
    assert conv([1, 64, 80, 80], [128, 64, 3, 3], [1, 128, 80, 80], pad=(1, 1), dtype="float32") == "conv_lds_f32_3x3s1_32x64w4"
    assert conv([1, 128, 80, 80], [256, 128, 3, 3], [1, 256, 40, 40], (2, 2), (1, 1), dtype="float32") == "conv_lds_f32_3x3s2_32x64w8"
    assert conv([1, 64, 80, 80], [128, 64, 3, 3], [1, 128, 80, 80], pad=(1, 1), dtype="bfloat16") == "conv_cl_bf16_3x3s1_32x64w4"
    assert conv([16, 64, 80, 80], [128, 64, 3, 3], [16, 128, 80, 80], pad=(1, 1), dtype="float32") == "conv_lds_f32_3x3s1_64x64w1"
    assert conv([16, 64, 80, 80], [128, 64, 3, 3], [16, 128, 80, 80], pad=(1, 1)) == "conv_cl_f16_3x3s1_64x64w1c16_pre"
    assert conv([64, 64, 80, 80], [128, 64, 3, 3], [64, 128, 80, 80], pad=(1, 1)) == "conv_cl_f16_3x3s1_64x64w1c16_pre"
    assert conv([8, 32, 160, 160], [64, 32, 3, 3], [8, 64, 160, 160], pad=(1, 1)) == "conv_cl_f16_3x3s1_64x64w1c16_pre"
    assert conv([16, 128, 40, 40], [256, 128, 3, 3], [16, 256, 40, 40], pad=(1, 1)) == "conv_cl_f16_3x3s1_64x64w1_pre"
    assert conv([64, 128, 80, 80], [256, 128, 3, 3], [64, 256, 40, 40], (2, 2), (1, 1)) == "conv_cl_f16_3x3s2_64x64w1_pre"
    assert conv([2, 128, 40, 40], [256, 128, 3, 3], [2, 256, 40, 40], pad=(1, 1)) == "conv_cl_f16_3x3s1_32x64w8"
    # bfloat16 has no im2col GEMM: 1x1 convolutions take the plain GEMM, other
    # spatial kernels outside the LDS-patch kernel the direct one, and the
    # many-tile rule keeps the 64 x 64 LDS-patch tile
    assert conv([1, 8, 20, 20], [16, 8, 5, 5], [1, 16, 16, 16], dtype="bfloat16") == "conv_grouped_direct"
    assert conv([1, 32, 40, 40], [64, 32, 1, 1], [1, 64, 40, 40], dtype="bfloat16").startswith("gemm_mfma_bf16_")
    assert conv([64, 32, 40, 41], [64, 32, 3, 3], [64, 64, 40, 41], pad=(1, 1), dtype="bfloat16") == "conv_cl_bf16_3x3s1_64x64w1_pre"
    monkeypatch.setenv("WGX_CONV_PRE", "0")
    assert conv([64, 128, 80, 80], [256, 128, 3, 3], [64, 256, 40, 40], (2, 2), (1, 1), dtype="bfloat16") == "conv_cl_bf16_3x3s2_64x64w1"
    assert conv([64, 64, 80, 80], [128, 64, 3, 3], [64, 128, 80, 80], pad=(1, 1)) == "conv_cl_f16_3x3s1_64x128w1"
    assert conv([16, 128, 40, 40], [256, 128, 3, 3], [16, 256, 40, 40], pad=(1, 1)).startswith("gemm_mfma_f16")
    assert conv([64, 128, 80, 80], [256, 128, 3, 3], [64, 256, 40, 40], (2, 2), (1, 1)).startswith("gemm_mfma_f16")
    monkeypatch.delenv("WGX_CONV_PRE")
    assert conv([4, 64, 80, 80], [128, 64, 3, 3], [4, 128, 80, 80], pad=(1, 1)) == "conv_cl_f16_3x3s1_32x64w2"
    monkeypatch.setenv("WGX_CONV_LDS", "2x1w2")
    assert conv([16, 64, 80, 80], [128, 64, 3, 3], [16, 128, 80, 80], pad=(1, 1)) == "conv_cl_f16_3x3s1_64x32w2"
    monkeypatch.setenv("WGX_CONV_LDS", "off")
    # fewer 64 x 64 tiles than CUs: the wave-split kernel, 64 x 32 tiles with
    # 4 waves (400 of them) or 8 waves (200)
    assert conv([1, 64, 80, 80], [128, 64, 3, 3], [1, 128, 80, 80], pad=(1, 1)) == "gemm_mfma_f16_64x32w4_conv_ws"
    assert conv([1, 128, 80, 80], [256, 128, 3, 3], [1, 256, 40, 40], (2, 2), (1, 1)) == "gemm_mfma_f16_64x32w8_conv_ws"
    assert conv([1, 64, 20, 20], [64, 64, 3, 3], [1, 64, 20, 20], pad=(1, 1), dtype="float32") == "gemm_mfma_f32_32x32w8_conv_ws"
    assert conv([1, 64, 160, 160], [64, 64, 3, 3], [1, 64, 160, 160], pad=(1, 1)) == "gemm_mfma_f16_64x64w4_conv"
    # at most 32 output channels: 32 x 32 wave-split tiles however many there are
    assert conv([1, 16, 160, 160], [16, 16, 3, 3], [1, 16, 160, 160], pad=(1, 1)) == "gemm_mfma_f16_32x32w4_conv_ws"
    assert conv([1, 16, 320, 320], [32, 16, 3, 3], [1, 32, 160, 160], (2, 2), (1, 1)) == "gemm_mfma_f16_32x32w4_conv_ws"
    assert conv([1, 8, 129, 131], [24, 8, 3, 3], [1, 24, 129, 131], pad=(1, 1)) == "gemm_mfma_f16_32x32w4_conv_ws"
    assert conv([1, 16, 160, 160], [16, 16, 3, 3], [1, 16, 160, 160], pad=(1, 1), dtype="float32") == "gemm_mfma_f32_64x64w4_conv"
    # without it, 100 output tiles for 256 CUs split K = 1152 into ranges (suffix _k<ranges>)
    monkeypatch.setenv("WGX_WS", "off")
    assert "_conv_k" in conv([1, 128, 80, 80], [256, 128, 3, 3], [1, 256, 40, 40], (2, 2), (1, 1))
    monkeypatch.setenv("WGX_WS", "1x2w4")
    assert conv([1, 128, 80, 80], [256, 128, 3, 3], [1, 256, 40, 40], (2, 2), (1, 1)) == "gemm_mfma_f16_32x64w4_conv_ws"
    monkeypatch.delenv("WGX_WS")
    # 1x1: a plain GEMM over the [IC, H*W] plane when its 64 x 64 tiles fill the CUs,
    # else the one-tap im2col form on the wave-split kernel
    assert conv([1, 64, 8, 8], [64, 64, 1, 1], [1, 64, 8, 8]).endswith("_conv_ws")
    # one K slice of 64 channels: the 4-wave form (8 waves would leave 7 without a slice)
    assert conv([1, 64, 40, 40], [64, 64, 1, 1], [1, 64, 40, 40]) == "gemm_mfma_f16_32x32w4_conv_ws"
    assert conv([1, 512, 20, 20], [64, 512, 1, 1], [1, 64, 20, 20]) == "gemm_mfma_f16_32x32w8_conv_ws"
    assert "_kn" in conv([1, 16, 160, 160], [32, 16, 1, 1], [1, 32, 160, 160])
    # batch 1: fewer register-kernel waves than two per CU, the LDS-tiled kernel
    assert conv([1, 256, 40, 40], [256, 1, 3, 3], [1, 256, 40, 40], pad=(1, 1), groups=256) == "depthwise_f16_3x3s1_v8"
    assert conv([1, 512, 20, 20], [512, 1, 5, 5], [1, 512, 10, 10], (2, 2), (2, 2), groups=512) == "depthwise_f16_5x5s2_v4"
    # enough planes: the register kernel (8- and 5-row bands)
    assert conv([40, 256, 40, 40], [256, 1, 3, 3], [40, 256, 40, 40], pad=(1, 1), groups=256) == "depthwise_f16_3x3s1_r8v8"
    assert conv([84, 512, 20, 20], [512, 1, 5, 5], [84, 512, 10, 10], (2, 2), (2, 2), groups=512) == "depthwise_f16_5x5s2_r5v4"
    monkeypatch.setenv("WGX_DW_KERNEL", "reg")
    assert conv([1, 256, 40, 40], [256, 1, 3, 3], [1, 256, 40, 40], pad=(1, 1), groups=256) == "depthwise_f16_3x3s1_r4v8"
    monkeypatch.delenv("WGX_DW_KERNEL")
    # odd widths (and float32) take the LDS-tiled kernel of the same family
    assert conv([1, 6, 13, 17], [6, 1, 3, 3], [1, 6, 13, 17], pad=(1, 1), groups=6) == "depthwise_f16_3x3s1_v4"
    assert conv([1, 256, 40, 40], [256, 1, 3, 3], [1, 256, 40, 40], pad=(1, 1), groups=256,
                dtype="float32") == "depthwise_f32_3x3s1_v8"
    # dilation 2 is outside the fast family: the general depthwise kernel
    assert conv([1, 8, 12, 12], [8, 1, 3, 3], [1, 8, 12, 12], pad=(2, 2), dil=(2, 2), groups=8) == "depthwise_f16_3x3"
    assert conv([1, 8, 10, 10], [12, 4, 3, 3], [1, 12, 10, 10], pad=(1, 1), groups=2) == "conv_grouped_direct"
    assert conv([1, 2, 3, 3], [2, 2, 3, 3], [1, 2, 6, 6], (2, 2), (1, 1), transposed=True, op=(1, 1)) == "conv_transpose_direct"
    # a stem (K = IC*KH*KW = 27 taps, 16 output channels): the direct small-tap kernel
    assert conv([1, 3, 64, 64], [16, 3, 3, 3], [1, 16, 32, 32], (2, 2), (1, 1), dtype="float32") == "conv_small_taps_oc16"
    assert conv([1, 3, 64, 64], [16, 3, 3, 3], [1, 16, 32, 32], (2, 2), (1, 1)) == "conv_small_taps_oc16"
    assert conv([1, 3, 64, 64], [48, 3, 3, 3], [1, 48, 64, 64], (1, 1), (1, 1)) == "conv_small_taps_oc64"
    assert conv([1, 4, 64, 64], [16, 4, 3, 3], [1, 16, 64, 64], (1, 1), (1, 1)).startswith("gemm_mfma_f16")  # 36 taps
    # the reference's output-size rule, floor((I + 2p - d(K-1) - 1) / s) + 1
    with pytest.raises(E, match=r"expected output spatial \[3, 3\]"):
        conv([1, 2, 5, 5], [3, 2, 3, 3], [1, 3, 2, 2], (2, 2), (1, 1))
    with pytest.raises(E, match=r"expected output spatial \[6, 6\]"):
        conv([1, 2, 3, 3], [2, 2, 3, 3], [1, 2, 5, 5], (2, 2), (1, 1), transposed=True, op=(1, 1))
    with pytest.raises(E, match="weight in-ch"):
        conv([1, 4, 8, 8], [8, 3, 3, 3], [1, 8, 6, 6])
    with pytest.raises(E, match="output_padding"):
        conv([1, 4, 8, 8], [8, 4, 3, 3], [1, 8, 6, 6], op=(1, 0))
    with pytest.raises(E, match="kernel larger than input"):
        conv([1, 4, 2, 2], [8, 4, 5, 5], [1, 8, 1, 1])
    with pytest.raises(E, match="output_padding >= stride"):
        conv([1, 2, 3, 3], [2, 2, 3, 3], [1, 2, 7, 7], (2, 2), (1, 1), transposed=True, op=(2, 2))
    with pytest.raises(E, match="4D"):
        conv([1, 4, 8], [8, 4, 3, 3], [1, 8, 6, 6])
    with pytest.raises(E, match="matching float32, float16 or bfloat16"):
        hctx.convolution(T("bfloat16", [1, 4, 8, 8]), T("float16", [8, 4, 3, 3]), None, (1, 1), (0, 0),
                         (1, 1), False, (0, 0), 1, T("bfloat16", [1, 8, 6, 6]))


def test_im2col_table_matches_oracle_indexing(pkg, orc):
    """The k -> (offset, tap) rule the conv kernels use reproduces im2col
    exactly (gathered on the CPU here and multiplied in float64)."""
    I = pkg.inputs
    x = I.uniform(1, (1, 5, 9, 11), -1, 1)
    w = I.uniform(2, (4, 5, 3, 2), -1, 1)
    s, p, d = (2, 1), (1, 2), (2, 1)
    y, _ = orc.conv2d_f64(x, w, None, s, p, d)
    IC, IH, IW, KH, KW = 5, 9, 11, 3, 2
    OH, OW = y.shape[2:]
    K = IC * KH * KW
    cols = np.zeros((K, OH * OW))
    for k in range(K):
        ic, tap = divmod(k, KH * KW)
        kh, kw = divmod(tap, KW)
        off = ic * IH * IW + kh * d[0] * IW + kw * d[1]
        for n in range(OH * OW):
            oh, ow = divmod(n, OW)
            ih0, iw0 = oh * s[0] - p[0], ow * s[1] - p[1]
            ih, iw = ih0 + kh * d[0], iw0 + kw * d[1]
            if 0 <= ih < IH and 0 <= iw < IW:
                cols[k, n] = x.ravel()[ih0 * IW + iw0 + off]
    got = w.reshape(4, K).astype(np.float64) @ cols
    assert np.max(np.abs(got - y.reshape(4, -1))) < 1e-12


def test_conv_residual_validation(hctx, pkg):
    """The residual epilogue's checks: depthwise convolutions and the dense
    3x3 ones the LDS-patch kernel takes, the output's shape and dtype, the
    output itself or no overlap at all."""
    E = pkg.wgx.WgxError
    T = hctx.tensor
    x, w, b = T("float16", [1, 8, 10, 10]), T("float16", [8, 1, 3, 3]), T("float16", [8])
    y, r = T("float16", [1, 8, 10, 10]), T("float16", [1, 8, 10, 10])
    hctx.convolution(x, w, b, 1, 1, 1, False, 0, 8, y, residual=r, residual_scale=0.5)
    assert hctx.last_kernel.startswith("depthwise_f16_3x3s1")
    hctx.convolution(x, w, b, 1, 1, 1, False, 0, 8, y, residual=y)  # in place
    # a dense 3x3 convolution over 8 input channels: no LDS-patch kernel (16-bit
    # chunks are 16 channels), so no residual epilogue
    with pytest.raises(E, match="the LDS-patch kernel takes"):
        hctx.convolution(x, T("float16", [8, 8, 3, 3]), b, 1, 1, 1, False, 0, 1, y, residual=r)
    # over 16: the channel-last LDS-patch kernel adds it
    x16 = T("float16", [1, 16, 10, 10])
    hctx.convolution(x16, T("float16", [8, 16, 3, 3]), b, 1, 1, 1, False, 0, 1, y, residual=r)
    assert hctx.last_kernel.startswith("conv_cl_f16_3x3s1")
    with pytest.raises(E, match="the LDS-patch kernel takes"):
        hctx.convolution(x16, T("float16", [8, 16, 1, 1]), b, 1, 0, 1, False, 0, 1, y, residual=r)
    with pytest.raises(E, match="match the output"):
        hctx.convolution(x, w, b, 1, 1, 1, False, 0, 8, y, residual=T("float16", [1, 8, 10, 11]))
    with pytest.raises(E, match="match the output"):
        hctx.convolution(x, w, b, 1, 1, 1, False, 0, 8, y, residual=T("float32", [1, 8, 10, 10]))
    buf = hctx.storage_buffer(2 * 800 + 64)
    W = pkg.wgx
    y2 = W.Tensor(hctx, "float16", [1, 8, 10, 10], buf, 2 * 800 + 64)
    r2 = W.Tensor(hctx, "float16", [1, 8, 10, 10], buf + 32, 2 * 800 + 32)
    with pytest.raises(E, match="partly overlaps"):
        hctx.convolution(x, w, b, 1, 1, 1, False, 0, 8, y2, residual=r2)
