"""CPU oracle for the GEMM-shaped hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
(``wgpu-executorch_amd/``) never imports it.

Thin ctypes/numpy wrappers over ``liboracle.so`` (built from ``oracle.c`` by
``oracle/Makefile``).  See ``oracle.c`` for what each function restates and
which reference file:line it follows.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

DT_F32, DT_F16, DT_BF16 = 0, 1, 2

_f = ctypes.POINTER(ctypes.c_float)
_d = ctypes.POINTER(ctypes.c_double)
_u16 = ctypes.POINTER(ctypes.c_uint16)
_i = ctypes.POINTER(ctypes.c_int)
_i64 = ctypes.c_int64


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)
    return os.path.join(_HERE, "liboracle.so")


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        L.orc_f32_to_f16_n.argtypes = [_f, _u16, _i64]
        L.orc_f16_to_f32_n.argtypes = [_u16, _f, _i64]
        L.orc_f32_to_bf16_n.argtypes = [_f, _u16, _i64]
        L.orc_bf16_to_f32_n.argtypes = [_u16, _f, _i64]
        L.orc_num_threads.restype = ctypes.c_int
        L.orc_gemm_f64.argtypes = [ctypes.c_int] * 4 + [_f, _i64, _f, _i64, ctypes.c_int, _f,
                                                         ctypes.c_int, _d, _d, _i, ctypes.c_int]
        L.orc_conv2d_f64.argtypes = [_i, _f, _f, _f, _d, _d]
        L.orc_conv_transpose2d_f64.argtypes = [_i, _f, _f, _f, _d, _d]
        L.orc_emu_gemm.argtypes = [ctypes.c_int] * 5 + [_f, _i64, _f, _i64, ctypes.c_int, _f,
                                                        _i, ctypes.c_int]
        L.orc_emu_addmm.argtypes = [ctypes.c_int] * 4 + [_f, _f, ctypes.c_int, _f, _f, _i,
                                                         ctypes.c_int]
        L.orc_emu_conv2d.argtypes = [ctypes.c_int, _i, ctypes.c_int, _f, _f, _f, _f]
        _LIB = L
    return _LIB


def _fp(a):
    return a.ctypes.data_as(_f)


def _dp(a):
    return a.ctypes.data_as(_d)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def num_threads() -> int:
    return lib().orc_num_threads()


# ---------------------------------------------------------------- formats
def f32_to_f16_bits(x) -> np.ndarray:
    x = _c32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_fp(x), out.ctypes.data_as(_u16), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_n(h.ctypes.data_as(_u16), _fp(out), h.size)
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    x = _c32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_fp(x), out.ctypes.data_as(_u16), x.size)
    return out


def bf16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_f32_n(h.ctypes.data_as(_u16), _fp(out), h.size)
    return out


def round_to(dt: int, x) -> np.ndarray:
    """Round float32 values to the storage dtype and back to float32."""
    if dt == DT_F16:
        return f16_bits_to_f32(f32_to_f16_bits(x))
    if dt == DT_BF16:
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    return _c32(x)


# ---------------------------------------------------------------- fp64 brute force
def gemm_f64(A, B, bias=None, *, b_trans=False, bias_mode=None, rows=None):
    """fp64 C = A @ B (+bias), returns (C, Cabs) as float64 arrays.

    A: [M,K] or [batch,M,K] (a 2-D A is shared across a 3-D B's batch).
    B: [K,N] / [N,K] (b_trans) or batched.  bias: [N] (addmm) by default.
    rows: optional list of row indices to compute (then C has len(rows) rows).
    """
    A = _c32(A)
    B = _c32(B)
    batch = B.shape[0] if B.ndim == 3 else (A.shape[0] if A.ndim == 3 else 1)
    M, K = A.shape[-2], A.shape[-1]
    N = B.shape[-2] if b_trans else B.shape[-1]
    sA = M * K if A.ndim == 3 else 0
    sB = B.shape[-1] * B.shape[-2] if B.ndim == 3 else 0
    if bias_mode is None:
        bias_mode = 0 if bias is None else 1
    bias_arr = _c32(bias) if bias is not None else np.zeros(1, np.float32)
    if rows is not None:
        rows_arr = np.ascontiguousarray(rows, dtype=np.int32)
        nrows = rows_arr.size
        rp = rows_arr.ctypes.data_as(_i)
    else:
        rows_arr, nrows, rp = None, M, None
    C = np.empty((batch, nrows, N), np.float64)
    Ca = np.empty((batch, nrows, N), np.float64)
    lib().orc_gemm_f64(batch, M, N, K, _fp(A), sA, _fp(B), sB, int(b_trans), _fp(bias_arr),
                       bias_mode, _dp(C), _dp(Ca), rp, nrows)
    if A.ndim == 2 and B.ndim == 2:
        return C[0], Ca[0]
    return C, Ca


def conv_params(x_shape, w_shape, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1,
                has_bias=False, transposed=False, output_padding=(0, 0)):
    """The 17-word ConvParams block (src/shaders/convolution/index.ts:151-162)."""
    B, IC, IH, IW = x_shape
    sH, sW = stride
    pH, pW = padding
    dH, dW = dilation
    KH, KW = w_shape[2], w_shape[3]
    if transposed:
        OC = w_shape[1] * groups
        OH = (IH - 1) * sH - 2 * pH + dH * (KH - 1) + output_padding[0] + 1
        OW = (IW - 1) * sW - 2 * pW + dW * (KW - 1) + output_padding[1] + 1
    else:
        OC = w_shape[0]
        OH = (IH + 2 * pH - dH * (KH - 1) - 1) // sH + 1
        OW = (IW + 2 * pW - dW * (KW - 1) - 1) // sW + 1
    return np.array([B, IC, IH, IW, OC, OH, OW, KH, KW, sH, sW, pH, pW, dH, dW, groups,
                     int(has_bias)], dtype=np.int32)


def conv2d_f64(x, w, bias=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1):
    x, w = _c32(x), _c32(w)
    p = conv_params(x.shape, w.shape, stride, padding, dilation, groups, bias is not None)
    B, OC, OH, OW = p[0], p[4], p[5], p[6]
    y = np.empty((B, OC, OH, OW), np.float64)
    ya = np.empty_like(y)
    b = _c32(bias) if bias is not None else np.zeros(1, np.float32)
    lib().orc_conv2d_f64(p.ctypes.data_as(_i), _fp(x), _fp(w), _fp(b), _dp(y), _dp(ya))
    return y, ya


def conv_transpose2d_f64(x, w, bias=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1),
                         groups=1, output_padding=(0, 0)):
    x, w = _c32(x), _c32(w)
    p = conv_params(x.shape, w.shape, stride, padding, dilation, groups, bias is not None,
                    transposed=True, output_padding=output_padding)
    B, OC, OH, OW = p[0], p[4], p[5], p[6]
    y = np.empty((B, OC, OH, OW), np.float64)
    ya = np.empty_like(y)
    b = _c32(bias) if bias is not None else np.zeros(1, np.float32)
    lib().orc_conv_transpose2d_f64(p.ctypes.data_as(_i), _fp(x), _fp(w), _fp(b), _dp(y),
                                   _dp(ya))
    return y, ya


# ---------------------------------------------------------------- wgsl-emu
def emu_gemm(dt, A, B, *, b_trans=False, rows=None):
    A = _c32(A)
    B = _c32(B)
    batch = B.shape[0] if B.ndim == 3 else (A.shape[0] if A.ndim == 3 else 1)
    M, K = A.shape[-2], A.shape[-1]
    N = B.shape[-2] if b_trans else B.shape[-1]
    sA = M * K if A.ndim == 3 else 0
    sB = B.shape[-1] * B.shape[-2] if B.ndim == 3 else 0
    if rows is not None:
        rows_arr = np.ascontiguousarray(rows, dtype=np.int32)
        nrows, rp = rows_arr.size, rows_arr.ctypes.data_as(_i)
    else:
        rows_arr, nrows, rp = None, M, None
    C = np.empty((batch, nrows, N), np.float32)
    lib().orc_emu_gemm(dt, batch, M, N, K, _fp(A), sA, _fp(B), sB, int(b_trans), _fp(C), rp,
                       nrows)
    if A.ndim == 2 and B.ndim == 2:
        return C[0]
    return C


def emu_addmm(dt, X, W, bias, *, w_trans=False, rows=None):
    X, W, bias = _c32(X), _c32(W), _c32(bias)
    M, K = X.shape
    N = W.shape[0] if w_trans else W.shape[1]
    if rows is not None:
        rows_arr = np.ascontiguousarray(rows, dtype=np.int32)
        nrows, rp = rows_arr.size, rows_arr.ctypes.data_as(_i)
    else:
        rows_arr, nrows, rp = None, M, None
    out = np.empty((nrows, N), np.float32)
    lib().orc_emu_addmm(dt, M, N, K, _fp(X), _fp(W), int(w_trans), _fp(bias), _fp(out), rp,
                        nrows)
    return out


def emu_conv2d(dt, x, w, bias=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1,
               transposed=False, output_padding=(0, 0)):
    x, w = _c32(x), _c32(w)
    p = conv_params(x.shape, w.shape, stride, padding, dilation, groups, bias is not None,
                    transposed=transposed, output_padding=output_padding)
    B, OC, OH, OW = p[0], p[4], p[5], p[6]
    y = np.empty((B, OC, OH, OW), np.float32)
    b = _c32(bias) if bias is not None else np.zeros(1, np.float32)
    lib().orc_emu_conv2d(dt, p.ctypes.data_as(_i), int(transposed), _fp(x), _fp(w), _fp(b),
                         _fp(y))
    return y
