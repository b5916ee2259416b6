"""The YOLO-N-style fp16 program (recordProgram end to end).

CPU: the generator emits a valid program in the reference's format (pool
rule, lifetimes, alignment, sizes); the JS host layer records it on a
host-only device (every driver's validation runs); the program evaluator the
GPU runs are checked against is pinned against torch on each operator and
against the reference's own program KAT.
GPU: the program runs through Node -> N-API -> libwgx on GPU 0 and its output
is compared with the CPU evaluation of the same program, at 160x160 and at
the full 640x640 configuration.
"""
import importlib
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUNNER = os.path.join(ROOT, "wgpu-executorch_amd", "js", "run_program.js")
NODE = shutil.which("node")
needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


@pytest.fixture(scope="module")
def Y(pkg):
    return importlib.import_module("wgpu_executorch_amd.yolo_program")


def _tensor_ids(prog, arg):
    v = prog["values"][arg]
    if v["type"] == "tensor":
        return [arg]
    if v["type"] == "tensorlist":
        return list(v["items"])
    return []


def test_generator_matches_the_configuration(Y):
    prog, weights, info = Y.build()
    assert info["input_shape"] == [1, 3, 640, 640]
    assert info["output_shape"] == [1, 84, 8400]  # three heads: 6400 + 1600 + 400 anchors
    assert 2.2e6 <= info["params"] <= 2.8e6      # "about 2.5M parameters"
    names = {op["name"] for op in prog["chain"]}
    assert {"aten.convolution.default", "aten.sigmoid.default", "aten.mul.Tensor", "aten.cat.default",
            "aten.upsample_nearest2d.vec", "aten.split_with_sizes_copy.default"} <= names
    convs = [op for op in prog["chain"] if op["name"] == "aten.convolution.default"]
    groups = [prog["values"][op["args"][8]]["value"] for op in convs]
    assert any(g > 1 for g in groups)  # depthwise blocks present
    # channel progression 16/32/64/128/256 at strides 2..32
    outs = [prog["values"][op["args"][-1]]["shape"] for op in convs]
    seen = {(s[1], 640 // s[2]) for s in outs}
    for c, s in [(16, 2), (32, 4), (64, 8), (128, 16), (256, 32)]:
        assert (c, s) in seen


def test_generator_pool_plan_follows_converter_rule(Y):
    prog, weights, _ = Y.build(img=160)
    vals = prog["values"]
    es = {"float16": 2, "float32": 4, "int32": 4}
    sizes = {}
    for v in vals:
        if v["type"] == "tensor" and "memObjId" in v:
            nb = int(np.prod(v["shape"])) * es[v["dtype"]]
            sizes[v["memObjId"]] = max(sizes.get(v["memObjId"], 0), nb)
    # utils/pte_to_program.py:386-413: pool size = largest tensor in the pool
    assert {p["id"]: p["size"] for p in prog["memoryPlan"]["pools"]} == sizes
    # constants: 4-byte aligned inside weights.bin, as the fp16 converter writes them
    for v in vals:
        if v["type"] == "tensor" and "weightsOffset" in v:
            assert "memObjId" not in v and v["weightsOffset"] % 4 == 0
            assert v["weightsOffset"] + v["weightsLength"] <= len(weights)
    # no op reads a pool another live tensor occupies: check lifetimes per pool
    first, last = {}, {}
    for k, op in enumerate(prog["chain"]):
        for a in op["args"]:
            for t in _tensor_ids(prog, a):
                if "memObjId" in vals[t]:
                    first.setdefault(t, k)
                    last[t] = k
    for t in prog["inputIds"]:
        first[t] = -1
    for t in prog["outputIds"]:
        last[t] = len(prog["chain"])
    by_pool = {}
    for t in first:
        by_pool.setdefault(vals[t]["memObjId"], []).append((first[t], last[t]))
    for spans in by_pool.values():
        spans.sort()
        for (s0, e0), (s1, e1) in zip(spans, spans[1:]):
            assert e0 < s1, "two live tensors share a pool"


def _expected_silu_fusions(prog):
    """conv -> sigmoid -> mul triples recordProgram folds: the two
    intermediates read by nothing else (a product that shares memory with the
    convolution's input is moved, not left unfused).  Returns (triples, adds):
    adds counts the triples whose next op is an add of the product (read by
    nothing else) on a depthwise convolution, which join the launch too."""
    vals, chain = prog["values"], prog["chain"]
    uses = {}
    for op in chain:
        for a in op["args"]:
            for t in _tensor_ids(prog, a):
                uses[t] = uses.get(t, 0) + 1
    for t in prog["outputIds"]:
        uses[t] = uses.get(t, 0) + 1
    n, adds, k = 0, 0, 0
    while k + 2 < len(chain):
        conv, sig, mul = chain[k:k + 3]
        c = conv["args"][-1]
        ok = (conv["name"] == "aten.convolution.default" and sig["name"] == "aten.sigmoid.default"
              and mul["name"] == "aten.mul.Tensor" and sig["args"][0] == c)
        if ok:
            s = sig["args"][1]
            ok = sorted(mul["args"][:2]) == sorted([c, s]) and uses.get(c) == 3 and uses.get(s) == 2
        if not ok:
            k += 1
            continue
        n += 1
        y, w = mul["args"][2], vals[conv["args"][1]]["shape"]
        groups = vals[conv["args"][8]]["value"]
        nxt = chain[k + 3] if k + 3 < len(chain) else None
        if (nxt is not None and nxt["name"] == "aten.add.Tensor" and uses.get(y) == 2
                and (nxt["args"][0] == y) != (nxt["args"][1] == y)
                and w[1] == 1 and w[0] == groups == vals[conv["args"][0]]["shape"][1]):
            adds += 1
            k += 4
        else:
            k += 3
    return n, adds


def _expected_view_copies(prog):
    """Copies that zero-copy views take out of this graph: one per piece of
    every split and of every cat along a dimension that only size-1
    dimensions precede, and every view_copy.  No tensor of this graph is a
    piece of two such ops and none is a program input or output, so each of
    them becomes a view."""
    vals = prog["values"]
    n = 0
    for op in prog["chain"]:
        a = op["args"]
        if op["name"] == "aten.split_with_sizes_copy.default":
            n += len(vals[a[3]]["items"])
        elif op["name"] == "aten.cat.default":
            shape = vals[a[2]]["shape"]
            d = vals[a[1]]["value"] % len(shape)
            if all(x == 1 for x in shape[:d]):
                n += len(vals[a[0]]["items"])
        elif op["name"] == "aten.view_copy.default":
            n += 1
    return n


def _pool_chain_launches_saved(prog, views):
    """Launches the runtime saves by folding the SPPF block's chained same-size
    max-pools (pool k+1 reads pool k's values) into one: a pool joins only if
    its values and indices outputs are disjoint from the chain's input and
    from every earlier output (indices may repeat one region exactly).  Pool
    tensors overlap when they share a memory-plan pool; with views, the
    values of the block (pieces of the channel concatenation that follows)
    live in the view slab, apart from every pool."""
    vals, chain = prog["values"], prog["chain"]
    ks = [k for k, op in enumerate(chain) if op["name"] == "aten.max_pool2d_with_indices.default"]
    saved, k = 0, 0
    while k < len(ks):
        x = chain[ks[k]]["args"][0]
        region = lambda t: ("view", t) if views and vals[t]["dtype"] != "int32" else ("pool", vals[t]["memObjId"])
        ys, ids = [], []
        j = k
        while j < len(ks) and ks[j] == ks[k] + (j - k) and len(ys) < 3:
            y, ix = vals[chain[ks[j]]["args"][-1]]["items"]
            if ys and chain[ks[j]]["args"][0] != ys[-1]:
                break
            taken = {region(x)} | {region(t) for t in ys} | {region(t) for t in ids}
            if ys and (region(y) in taken or (region(ix) in taken and region(ix) not in {region(t) for t in ids})):
                break
            if not ys and len({region(x), region(y), region(ix)}) < 3:
                break
            ys.append(y)
            ids.append(ix)
            j += 1
        saved += max(0, len(ys) - 1)
        k = max(j, k + 1)
    return saved


@needs_node
def test_js_host_records_the_program(Y, tmp_path):
    Y.write(str(tmp_path), img=160)
    prog = json.load(open(tmp_path / "program.json"))
    res = {}
    for flags in ((), ("--no-fuse",), ("--no-views",), ("--no-fuse", "--no-views")):
        cmd = [NODE, RUNNER, str(tmp_path), "--device", "-1", "--record-only", *flags]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        res[flags] = json.loads(r.stdout.strip().splitlines()[-1])
        assert res[flags]["ops"] == len(prog["chain"])
    base = res[("--no-fuse", "--no-views")]["commands"]
    assert base >= len(prog["chain"])
    # every conv -> sigmoid -> mul the rule allows is one launch instead of
    # three, and a residual add after a depthwise one joins it
    n, adds = _expected_silu_fusions(prog)
    v = _expected_view_copies(prog)
    assert n > 0 and adds > 0 and v > 0
    # the SPPF pools fold as far as their memory allows in each layout
    pv, pn = _pool_chain_launches_saved(prog, True), _pool_chain_launches_saved(prog, False)
    assert pv == 2
    assert base - res[("--no-views",)]["commands"] == 2 * n + adds
    assert base - res[("--no-fuse",)]["commands"] == v + pv - pn
    assert base - res[()]["commands"] == 2 * n + adds + v + pv - pn
    # the caller's input and output tensors bound in place: two copies fewer
    cmd = [NODE, RUNNER, str(tmp_path), "--device", "-1", "--record-only", "--no-bind-io"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert json.loads(r.stdout.strip().splitlines()[-1])["commands"] == res[()]["commands"] + 2


# ------------------------------------------------------------ evaluator pins
def test_evaluator_reference_program_kat(orc):
    """The reference's 2-op add+mm program KAT (tests/api/program.test.ts:54-68)."""
    from oracle import program_eval

    prog = {"version": "1",
            "chain": [{"name": "aten.add.Tensor", "args": [0, 1, 2, 3]},
                      {"name": "aten.mm.default", "args": [3, 4, 5]}],
            "values": [{"type": "tensor", "shape": [2, 2], "dtype": "float32", "memObjId": 0},
                       {"type": "tensor", "shape": [2, 2], "dtype": "float32", "memObjId": 1},
                       {"type": "scalar", "value": 1.5},
                       {"type": "tensor", "shape": [2, 2], "dtype": "float32", "memObjId": 2},
                       {"type": "tensor", "shape": [2, 2], "dtype": "float32", "memObjId": 3},
                       {"type": "tensor", "shape": [2, 2], "dtype": "float32", "memObjId": 0}],
            "inputIds": [0, 1, 4], "outputIds": [5],
            "memoryPlan": {"pools": [{"id": i, "size": 16} for i in range(4)]}}
    ins = [np.array([1, 2, 3, 4.0]), np.array([10, 20, 30, 40.0]), np.array([1, 2, 3, 4.0])]
    out = program_eval.evaluate(prog, b"", ins)[0]
    assert out.ravel().tolist() == [112, 160, 240, 352]


def test_evaluator_ops_match_torch(orc):
    """Each non-conv operator of the evaluator against torch on the CPU."""
    import torch
    import torch.nn.functional as F

    from oracle import program_eval

    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 6, 9, 7)).astype(np.float16).astype(np.float64)

    def run(name, args_vals, out_shapes, out_dtype="float16"):
        values, args = [], []
        for a in args_vals:
            if isinstance(a, np.ndarray):
                values.append({"type": "tensor", "shape": list(a.shape), "dtype": "float16"})
            elif isinstance(a, list):
                values.append({"type": "list", "items": a})
            else:
                values.append({"type": "scalar", "value": a})
            args.append(len(values) - 1)
        outs = []
        for s in out_shapes:
            values.append({"type": "tensor", "shape": list(s), "dtype": out_dtype})
            outs.append(len(values) - 1)
        if len(outs) > 1:
            values.append({"type": "tensorlist", "items": outs})
            args.append(len(values) - 1)
        else:
            args.append(outs[0])
        prog = {"version": "1", "chain": [{"name": name, "args": args}], "values": values,
                "inputIds": [i for i, a in enumerate(args_vals) if isinstance(a, np.ndarray)],
                "outputIds": outs, "memoryPlan": {"pools": []}}
        return program_eval.evaluate(prog, b"", [a for a in args_vals if isinstance(a, np.ndarray)])

    tx = torch.from_numpy(x)
    f16 = lambda t: t.to(torch.float16).to(torch.float64).numpy()
    assert np.array_equal(run("aten.sigmoid.default", [x], [x.shape])[0], f16(torch.sigmoid(tx)))
    up = run("aten.upsample_nearest2d.vec", [x, [2, 2]], [(1, 6, 18, 14)])[0]
    assert np.array_equal(up, F.interpolate(tx, scale_factor=2, mode="nearest").numpy())
    mp = run("aten.max_pool2d_with_indices.default", [x, [5, 5], [1, 1], [2, 2], [1, 1], False],
             [x.shape, x.shape])[0]
    assert np.array_equal(mp, F.max_pool2d(tx, 5, 1, 2).numpy())
    mp2 = run("aten.max_pool2d_with_indices.default", [x, [3, 3], [2, 2], [1, 1], [1, 1], False],
              [(1, 6, 5, 4), (1, 6, 5, 4)])[0]
    assert np.array_equal(mp2, F.max_pool2d(tx, 3, 2, 1).numpy())
    sp = run("aten.split_with_sizes_copy.default", [x, [2, 4], 1], [(1, 2, 9, 7), (1, 4, 9, 7)])
    assert np.array_equal(sp[0], x[:, :2]) and np.array_equal(sp[1], x[:, 2:])


# ------------------------------------------------------------ GPU runs
def _gpu_vs_cpu(Y, tmp_path, img, flags=()):
    from oracle import program_eval

    Y.write(str(tmp_path), img=img)
    out = tmp_path / "out.bin"
    print(f"[yolo program] img={img} flags={list(flags)}: running on GPU 0 through Node", flush=True)
    r = subprocess.run([NODE, RUNNER, str(tmp_path), "--device", "0", "--warmup", "1", "--reps", "3",
                        "--out", str(out), *flags],
                       capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-3000:]
    gpu = np.fromfile(out, dtype=np.float16).astype(np.float64)
    prog = json.load(open(tmp_path / "program.json"))
    weights = open(tmp_path / "weights.bin", "rb").read()
    x = np.fromfile(tmp_path / "input.bin", dtype=np.float16).astype(np.float64)
    ref = program_eval.evaluate(prog, weights, [x])[0].ravel()
    assert gpu.shape == ref.shape and np.all(np.isfinite(gpu))
    d = np.abs(gpu - ref)
    # One rounding per op on both sides; the difference is accumulation order
    # (fp32 on the GPU, fp64 here) propagated through ~30 layers of fp16.
    rel = np.linalg.norm(gpu - ref) / np.linalg.norm(ref)
    frac = np.mean(d > 0.02 + 0.02 * np.abs(ref))
    print(f"[yolo program] img={img}: normwise rel err {rel:.2e}, max abs {d.max():.3e}, "
          f"fraction outside 0.02+0.02|ref|: {frac:.2e}", flush=True)
    # measured: rel ~6e-4, max abs ~6e-4 on outputs of magnitude ~0.5
    assert rel < 3e-3
    assert frac == 0.0 and d.max() < 1e-2


@needs_node
@pytest.mark.gpu
def test_yolo_program_gpu_matches_cpu_160(Y, orc, tmp_path):
    _gpu_vs_cpu(Y, tmp_path, 160)


@needs_node
@pytest.mark.gpu
@pytest.mark.parametrize("flags", [("--no-fuse",), ("--no-views",), ("--no-fuse", "--no-views"),
                                   ("--no-bind-io",)],
                         ids=["views", "fused", "op_by_op", "copied_io"])
def test_yolo_program_gpu_matches_cpu_160_variants(Y, orc, tmp_path, flags):
    _gpu_vs_cpu(Y, tmp_path, 160, flags)


@needs_node
@pytest.mark.gpu
def test_yolo_program_gpu_matches_cpu_640(Y, orc, tmp_path):
    _gpu_vs_cpu(Y, tmp_path, 640)
