"""CPU evaluation of a wgpu-executorch program.json -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg may use this module, as the
checker.  It restates what WgpuExecutionContext.recordProgram does
(src/context.ts:219-317): values are resolved the way resolveArgs resolves them
(src/program.ts:188-224), constants come from weights.bin at their offsets, and
the chain runs in order.  Each operator is computed in float64 and its output
is rounded to the tensor's storage dtype, which is where the device kernels
round too (one rounding per op).  Convolutions use the oracle's fp64 brute
force (orc_conv2d_f64); the other operators follow the PyTorch definitions of
the ops the reference registers:

  aten.mm / aten.bmm           float64 matmul      (src/shaders/mm, src/shaders/bmm)
  aten.sigmoid.default         1 / (1 + exp(-x))   (src/shaders/sigmoid)
  aten.mul.Tensor              a * b, broadcast     (src/shaders/mul)
  aten.add.Tensor / sub.Tensor a +- alpha * b       (src/shaders/add/index.ts:33-129)
  aten.cat.default             concatenation        (src/shaders/cat)
  aten.split_with_sizes_copy   split along dim      (src/shaders/split-with-sizes)
  aten.upsample_nearest2d.vec  out[i] = in[floor(i * in / out)]  (src/shaders/upsample-nearest-2d)
  aten.max_pool2d_with_indices values and int32 indices (oracle/ops.py, src/shaders/max-pool-2d)
  aten.permute_copy.default    transpose by dims   (oracle/ops.py, src/shaders/permute)
  aten._softmax.default        exp(x-max)/sum      (oracle/ops.py, src/shaders/softmax)
  view / clone / squeeze / unsqueeze / prepack   byte copies

Memory-plan pools are not modelled: values live in their own arrays, which is
what the pool plan must be equivalent to when lifetimes do not overlap.
"""
from __future__ import annotations

from typing import Dict, List

import numpy as np

from . import conv2d_f64, ops

_NP = {"float16": np.float16, "float32": np.float32, "int32": np.int32, "int64": np.int64}


def _round(x: np.ndarray, dtype: str) -> np.ndarray:
    return np.asarray(x).astype(_NP[dtype]).astype(np.float64)


def evaluate(program: dict, weights: bytes, inputs: List[np.ndarray]) -> List[np.ndarray]:
    """Runs the chain; returns the output tensors as float64 arrays."""
    vals = program["values"]
    env: Dict[int, np.ndarray] = {}
    for i, v in enumerate(vals):
        if v["type"] == "tensor" and "weightsOffset" in v:
            a = np.frombuffer(weights, dtype=_NP[v["dtype"]], count=int(np.prod(v["shape"])) if v["shape"] else 1,
                              offset=v["weightsOffset"])
            env[i] = a.astype(np.float64).reshape(v["shape"])
    for idx, arr in zip(program["inputIds"], inputs):
        env[idx] = _round(np.asarray(arr, np.float64).reshape(vals[idx]["shape"]), vals[idx]["dtype"])

    def arg(j):
        v = vals[j]
        t = v["type"]
        if t == "tensor":
            return env.get(j)
        if t == "scalar":
            return v["value"]
        if t == "list":
            return list(v["items"])
        if t == "tensorlist":
            return [env.get(k) for k in v["items"]]
        return None

    def put(j, x):
        v = vals[j]
        env[j] = _round(np.asarray(x, np.float64).reshape(v["shape"]), v["dtype"])

    for op in program["chain"]:
        name, a = op["name"], op["args"]
        if name == "aten.convolution.default":
            x, w, b = arg(a[0]), arg(a[1]), arg(a[2])
            stride, pad, dil, transposed, groups = arg(a[3]), arg(a[4]), arg(a[5]), arg(a[6]), arg(a[8])
            if transposed:
                raise NotImplementedError("transposed convolution in a program")
            y, _ = conv2d_f64(x.astype(np.float32), w.astype(np.float32),
                              None if b is None else b.astype(np.float32),
                              tuple(stride), tuple(pad), tuple(dil), int(groups))
            put(a[-1], y)
        elif name in ("aten.mm.default", "aten.bmm.default"):
            put(a[-1], np.matmul(arg(a[0]), arg(a[1])))
        elif name == "aten.sigmoid.default":
            put(a[-1], 1.0 / (1.0 + np.exp(-arg(a[0]))))
        elif name == "aten.mul.Tensor":
            put(a[-1], arg(a[0]) * arg(a[1]))
        elif name in ("aten.add.Tensor", "aten.sub.Tensor"):
            alpha = arg(a[2]) if len(a) == 4 else 1
            sgn = 1.0 if name == "aten.add.Tensor" else -1.0
            put(a[-1], arg(a[0]) + sgn * float(alpha) * arg(a[1]))
        elif name == "aten.cat.default":
            xs, dim = arg(a[0]), int(arg(a[1]))
            put(a[-1], np.concatenate(xs, axis=dim))
        elif name == "aten.split_with_sizes_copy.default":
            x, sizes, dim = arg(a[0]), arg(a[1]), int(arg(a[2]))
            outs = vals[a[3]]["items"]
            cuts = np.cumsum(sizes)[:-1]
            for j, part in zip(outs, np.split(x, cuts, axis=dim)):
                put(j, part)
        elif name == "aten.upsample_nearest2d.vec":
            x = arg(a[0])
            oh, ow = vals[a[-1]]["shape"][2:]
            ih, iw = x.shape[2:]
            ri = (np.arange(oh) * ih) // oh
            ci = (np.arange(ow) * iw) // ow
            put(a[-1], x[:, :, ri][:, :, :, ci])
        elif name == "aten.max_pool2d_with_indices.default":
            x = arg(a[0])
            hw = lambda v: (v[0], v[0]) if len(v) == 1 else tuple(v)
            k, s, p, d = hw(arg(a[1])), hw(arg(a[2])), hw(arg(a[3])), hw(arg(a[4]))
            outs = vals[a[6]]["items"]
            y, ix = ops.max_pool2d_with_indices(x, k, s, p, d, bool(arg(a[5])), vals[outs[0]]["dtype"])
            put(outs[0], y)
            if len(outs) > 1:
                env[outs[1]] = ix.astype(np.float64)
        elif name == "aten.permute_copy.default":
            put(a[-1], ops.permute(arg(a[0]), arg(a[1])))
        elif name == "aten._softmax.default":
            put(a[-1], ops.softmax_f64(arg(a[0]), int(arg(a[1]))))
        elif name in ("aten.view_copy.default", "aten.clone.default", "aten.squeeze_copy.dims",
                      "aten.unsqueeze_copy.default", "et_vk.prepack.default"):
            put(a[-1], arg(a[0]).reshape(vals[a[-1]]["shape"]))
        else:
            raise NotImplementedError(name)
    return [env.get(i) for i in program["outputIds"]]
