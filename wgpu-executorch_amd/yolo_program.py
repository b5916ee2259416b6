"""Synthetic YOLO-N-style fp16 detector, emitted as a wgpu-executorch program.

The output is the reference's on-disk program format (src/program.ts:26-165):
a ``program.json`` dict (values table, op chain, input / output ids, memory
plan) plus a ``weights.bin`` byte string.  The graph is a random-init
detector of the YOLO-N family at batch 1, input [1, 3, 640, 640]:

* stem: 3x3 conv 3->16, stride 2, SiLU;
* backbone: 3x3 stride-2 convs to 32/64/128/256 channels (strides 4..32),
  each followed by a CSP block (1x1 conv, split in two halves, bottlenecks of
  3x3 conv + depthwise 3x3 + residual add on one half, concat, 1x1 conv) and,
  at stride 32, an SPPF block (1x1 conv, three 5x5 max-pools, concat, 1x1);
* neck: FPN (nearest 2x upsample + concat + CSP) then PAN (3x3 stride-2
  conv + concat + CSP);
* heads at 80x80, 40x40 and 20x20: a box branch (two 3x3 convs, 1x1 to 4)
  and a class branch (two depthwise 3x3 + 1x1 pairs, 1x1 to 80 classes),
  concatenated to 84 channels, flattened and joined into [1, 84, 8400].

SiLU is written the way ExecuTorch exports it, sigmoid then mul (the shipped
yolo26n program has 88 sigmoid and 90 mul ops).  Weights are Kaiming-uniform,
biases U(+-1/sqrt(fan_in)), both from the seeded SplitMix64 generator in
``inputs``.  Intermediate tensors get memory-plan pools from a lifetime-based
greedy planner, and pool sizes follow the converter's rule: the largest tensor
assigned to a pool (utils/pte_to_program.py:386-413).  Constants are packed
into weights.bin at 4-byte alignment, as utils/convert_model_to_fp16.mjs:61-66
does, so a loader has to realign them.
"""
from __future__ import annotations

import json
from typing import Dict, List, Tuple

import numpy as np

from . import inputs as I

DTYPE = "float16"
ES = 2  # bytes per element


class _Builder:
    def __init__(self, seed_base: int = 1000):
        self.values: List[dict] = []
        self.chain: List[dict] = []
        self.weights = bytearray()
        self.seed = seed_base
        self.params = 0
        self.conv_flops = 0.0
        self.shapes: Dict[int, Tuple[int, ...]] = {}

    # ---------------------------------------------------------------- values
    def _add(self, v: dict) -> int:
        self.values.append(v)
        return len(self.values) - 1

    def tensor(self, shape, dtype: str = DTYPE) -> int:
        i = self._add({"type": "tensor", "shape": list(shape), "dtype": dtype})
        self.shapes[i] = tuple(shape)
        return i

    def const(self, arr: np.ndarray) -> int:
        data = arr.astype(np.float16).tobytes()
        while len(self.weights) % 4:
            self.weights.append(0)
        off = len(self.weights)
        self.weights += data
        i = self._add({"type": "tensor", "shape": list(arr.shape), "dtype": DTYPE,
                       "weightsOffset": off, "weightsLength": len(data)})
        self.shapes[i] = tuple(arr.shape)
        self.params += arr.size
        return i

    def lst(self, items) -> int:
        return self._add({"type": "list", "items": [int(x) for x in items]})

    def scalar(self, v) -> int:
        return self._add({"type": "scalar", "value": v})

    def tlist(self, items) -> int:
        return self._add({"type": "tensorlist", "items": list(items)})

    def op(self, name: str, args: List[int]):
        self.chain.append({"name": name, "args": args})

    # ---------------------------------------------------------------- layers
    def conv(self, x: int, oc: int, k: int, s: int = 1, groups: int = 1, act: bool = True) -> int:
        b, ic, h, w = self.shapes[x]
        p = k // 2
        oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
        wshape = (oc, ic // groups, k, k)
        wt = I.kaiming_uniform(self.seed, wshape)
        fan_in = (ic // groups) * k * k
        bias = I.uniform(self.seed + 1, (oc,), -1.0 / np.sqrt(fan_in), 1.0 / np.sqrt(fan_in))
        self.seed += 2
        wi, bi = self.const(wt), self.const(bias)
        y = self.tensor((b, oc, oh, ow))
        self.op("aten.convolution.default",
                [x, wi, bi, self.lst([s, s]), self.lst([p, p]), self.lst([1, 1]), self.scalar(False),
                 self.lst([0, 0]), self.scalar(groups), y])
        self.conv_flops += 2.0 * b * oc * oh * ow * (ic // groups) * k * k
        return self.silu(y) if act else y

    def silu(self, x: int) -> int:
        sig = self.tensor(self.shapes[x])
        self.op("aten.sigmoid.default", [x, sig])
        y = self.tensor(self.shapes[x])
        self.op("aten.mul.Tensor", [x, sig, y])
        return y

    def add(self, a: int, b: int) -> int:
        y = self.tensor(self.shapes[a])
        self.op("aten.add.Tensor", [a, b, self.scalar(1), y])
        return y

    def split2(self, x: int) -> Tuple[int, int]:
        b, c, h, w = self.shapes[x]
        h0, h1 = self.tensor((b, c // 2, h, w)), self.tensor((b, c - c // 2, h, w))
        self.op("aten.split_with_sizes_copy.default",
                [x, self.lst([c // 2, c - c // 2]), self.scalar(1), self.tlist([h0, h1])])
        return h0, h1

    def cat(self, xs: List[int], dim: int = 1) -> int:
        shp = list(self.shapes[xs[0]])
        shp[dim] = sum(self.shapes[x][dim] for x in xs)
        y = self.tensor(shp)
        self.op("aten.cat.default", [self.tlist(xs), self.scalar(dim), y])
        return y

    def upsample2(self, x: int) -> int:
        b, c, h, w = self.shapes[x]
        y = self.tensor((b, c, 2 * h, 2 * w))
        self.op("aten.upsample_nearest2d.vec", [x, self._add({"type": "null"}), self.lst([2, 2]), y])
        return y

    def maxpool5(self, x: int) -> int:
        y = self.tensor(self.shapes[x])
        idx = self.tensor(self.shapes[x], "int32")  # indices: written by no kernel here
        self.op("aten.max_pool2d_with_indices.default",
                [x, self.lst([5, 5]), self.lst([1, 1]), self.lst([2, 2]), self.lst([1, 1]),
                 self.scalar(False), self.tlist([y, idx])])
        return y

    def view(self, x: int, shape) -> int:
        y = self.tensor(shape)
        self.op("aten.view_copy.default", [x, self.lst(shape), y])
        return y

    # ---------------------------------------------------------------- blocks
    def bottleneck(self, x: int) -> int:
        c = self.shapes[x][1]
        y = self.conv(x, c, 3)
        y = self.conv(y, c, 3, groups=c)  # depthwise 3x3
        return self.add(x, y)

    def csp(self, x: int, oc: int, n: int) -> int:
        y = self.conv(x, oc, 1)
        a, b = self.split2(y)
        parts = [a, b]
        for _ in range(n):
            b = self.bottleneck(b)
            parts.append(b)
        return self.conv(self.cat(parts), oc, 1)

    def sppf(self, x: int) -> int:
        c = self.shapes[x][1]
        y = self.conv(x, c // 2, 1)
        p1 = self.maxpool5(y)
        p2 = self.maxpool5(p1)
        p3 = self.maxpool5(p2)
        return self.conv(self.cat([y, p1, p2, p3]), c, 1)

    def head(self, x: int, ncls: int = 80) -> int:
        b, c, h, w = self.shapes[x]
        cb = max(64, c // 4)
        box = self.conv(self.conv(x, cb, 3), cb, 3)
        box = self.conv(box, 4, 1, act=False)
        cc = max(80, c)
        cls = self.conv(self.conv(x, c, 3, groups=c), cc, 1)
        cls = self.conv(self.conv(cls, cc, 3, groups=cc), cc, 1)
        cls = self.conv(cls, ncls, 1, act=False)
        out = self.cat([box, cls])
        return self.view(out, (b, 4 + ncls, h * w))


def _plan_pools(b: _Builder, inputs: List[int], outputs: List[int]) -> List[dict]:
    """Greedy lifetime-based pool assignment for the non-constant tensors.

    A tensor's lifetime runs from the op that writes it to the last op that
    reads it; a pool is reused only once its previous tenant is dead, so no op
    ever reads and writes the same pool.  Graph inputs and outputs get pools
    too (the converter plans them as well)."""
    first: Dict[int, int] = {i: -1 for i in inputs}
    last: Dict[int, int] = {}

    def tensors_of(arg: int) -> List[int]:
        v = b.values[arg]
        if v["type"] == "tensor":
            return [arg]
        if v["type"] == "tensorlist":
            return list(v["items"])
        return []

    for k, op in enumerate(b.chain):
        for a in op["args"]:
            for t in tensors_of(a):
                if "weightsOffset" in b.values[t]:
                    continue
                first.setdefault(t, k)
                last[t] = k
    end = len(b.chain)
    for t in outputs:
        last[t] = end
    order = sorted(first, key=lambda t: (first[t], t))
    pools: List[int] = []      # pool id -> size
    free_at: List[int] = []    # pool id -> op index after which it is free
    for t in order:
        nbytes = int(np.prod(b.shapes[t])) * (4 if b.values[t]["dtype"] == "int32" else ES)
        start = first[t]
        pid = -1
        best = None
        for p in range(len(pools)):
            if free_at[p] < start:
                waste = abs(pools[p] - nbytes)
                if best is None or waste < best:
                    best, pid = waste, p
        if pid < 0:
            pools.append(0)
            free_at.append(-2)
            pid = len(pools) - 1
        pools[pid] = max(pools[pid], nbytes)
        free_at[pid] = last.get(t, start)
        b.values[t]["memObjId"] = pid
    return [{"id": p, "size": s} for p, s in enumerate(pools)]


def build(img: int = 640, width=(16, 32, 64, 128, 256), depth=(1, 2, 2, 1), ncls: int = 80):
    """Returns (program dict, weights bytes, info dict)."""
    b = _Builder()
    x = b.tensor((1, 3, img, img))
    c0, c1, c2, c3, c4 = width
    y = b.conv(x, c0, 3, 2)                          # /2
    y = b.csp(b.conv(y, c1, 3, 2), c1, depth[0])     # /4
    p3 = b.csp(b.conv(y, c2, 3, 2), c2, depth[1])    # /8
    p4 = b.csp(b.conv(p3, c3, 3, 2), c3, depth[2])   # /16
    p5 = b.sppf(b.csp(b.conv(p4, c4, 3, 2), c4, depth[3]))  # /32
    # FPN
    n4 = b.csp(b.cat([b.upsample2(p5), p4]), c3, 1)
    n3 = b.csp(b.cat([b.upsample2(n4), p3]), c2, 1)
    # PAN
    o4 = b.csp(b.cat([b.conv(n3, c2, 3, 2), n4]), c3, 1)
    o5 = b.csp(b.cat([b.conv(o4, c3, 3, 2), p5]), c4, 1)
    heads = [b.head(t, ncls) for t in (n3, o4, o5)]
    out = b.cat(heads, dim=2)
    pools = _plan_pools(b, [x], [out])
    program = {"version": "1", "chain": b.chain, "values": b.values, "inputIds": [x],
               "outputIds": [out], "memoryPlan": {"pools": pools}}
    info = {"params": int(b.params), "conv_flops": b.conv_flops, "ops": len(b.chain),
            "convs": sum(1 for o in b.chain if o["name"] == "aten.convolution.default"),
            "pool_bytes": int(sum(p["size"] for p in pools)), "input_shape": [1, 3, img, img],
            "output_shape": list(b.shapes[out])}
    return program, bytes(b.weights), info


def make_input(img: int = 640) -> np.ndarray:
    """Input frame: U(0, 1), rounded to float16, as float32."""
    return I.as_f16(I.uniform(77, (1, 3, img, img), 0.0, 1.0))


def write(dirpath: str, img: int = 640, **kw) -> dict:
    """Writes program.json, weights.bin and input.bin (float16) into dirpath."""
    import os

    program, weights, info = build(img, **kw)
    os.makedirs(dirpath, exist_ok=True)
    with open(os.path.join(dirpath, "program.json"), "w") as f:
        json.dump(program, f)
    with open(os.path.join(dirpath, "weights.bin"), "wb") as f:
        f.write(weights)
    make_input(img).astype(np.float16).tofile(os.path.join(dirpath, "input.bin"))
    with open(os.path.join(dirpath, "info.json"), "w") as f:
        json.dump(info, f)
    return info
