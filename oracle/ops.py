"""numpy restatements of the non-GEMM operators a program chain needs --
TEST INFRASTRUCTURE ONLY (tests/, smoke() and bench.py's cpu_baseline leg may
use it, as the checker; the product never imports it).

  max_pool2d_with_indices  src/shaders/max-pool-2d/index.ts:41-106 and
                           max-pool-2d-spatial.wgsl.ts:42-79: per window, the
                           first strictly greatest element in row-major (kh
                           outer, kw inner) order over the cells inside the
                           image; the initial value is -65504 (f16 kernels) or
                           -3.4e38 (f32 kernels) with index 0; the index is the
                           flat position ih * IW + iw in the plane.  Output
                           size floor/ceil((I + 2p - d(K-1) - 1) / s) + 1, at
                           least 0 (index.ts:73-78).
  softmax_f64              src/shaders/softmax/index.ts:62-125: exp(x - max)
                           / sum exp(x - max) along dim, in float64.
  permute                  src/shaders/permute/index.ts:33-99: out dim k is
                           input dim dims[k] (a pure index map).
"""
from __future__ import annotations

import math

import numpy as np


def pool_out_size(i: int, k: int, s: int, p: int, d: int, ceil_mode: bool) -> int:
    """max-pool-2d/index.ts:73-78."""
    num = i + 2 * p - (d * (k - 1) + 1)
    q = math.ceil(num / s) if ceil_mode else math.floor(num / s)
    return max(0, q + 1)


def max_pool2d_with_indices(x, kernel, stride, padding, dilation, ceil_mode=False, dtype="float32"):
    """Returns (values float64, indices int32) of an NCHW float array."""
    x = np.asarray(x, np.float64)
    B, C, IH, IW = x.shape
    (kH, kW), (sH, sW), (pH, pW), (dH, dW) = kernel, stride, padding, dilation
    OH = pool_out_size(IH, kH, sH, pH, dH, ceil_mode)
    OW = pool_out_size(IW, kW, sW, pW, dW, ceil_mode)
    floor = -65504.0 if dtype == "float16" else -3.4e38
    best = np.full((B, C, OH, OW), floor)
    idx = np.zeros((B, C, OH, OW), np.int32)
    oh = np.arange(OH)[:, None]
    ow = np.arange(OW)[None, :]
    for kh in range(kH):
        ih = oh * sH - pH + kh * dH                       # [OH, 1]
        for kw in range(kW):
            iw = ow * sW - pW + kw * dW                   # [1, OW]
            inside = (ih >= 0) & (ih < IH) & (iw >= 0) & (iw < IW)   # [OH, OW]
            v = x[:, :, np.clip(ih, 0, IH - 1), np.clip(iw, 0, IW - 1)]
            take = inside & (v > best)                    # NaN and -inf never win
            best = np.where(take, v, best)
            idx = np.where(take, (ih * IW + iw).astype(np.int32), idx)
    return best, idx


def softmax_f64(x, dim: int):
    x = np.asarray(x, np.float64)
    m = np.max(x, axis=dim, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=dim, keepdims=True)


def permute(x, dims):
    rank = np.ndim(x)
    perm = [d + rank if d < 0 else d for d in dims]
    if sorted(perm) != list(range(rank)):
        raise ValueError("invalid permute dims")
    return np.ascontiguousarray(np.transpose(x, perm))
