"""The reference's real yolo26n program end to end (tests/program/yolo26n.test.ts).

Fixtures (tests/golden/yolo26n/, reference data only): program.json and
weights.bin (float32, example/public/assets/yolo26n/), program-fp16.json and
weights-fp16.bin (the reference's float16 conversion, with its 4-byte
constant alignment), and reference-output.f32, the PyTorch float32 output
[1, 84, 8400] for the input value[i] = (i % 251) / 250 - 0.5
(yolo26n.test.ts:17-25).

CPU: the converter's consistency rules hold for both programs; the JS host
records every one of the 397 ops on a host-only device, with and without the
graph passes; the oracle's program evaluator (float64 per op, one rounding
per op to the storage type) reproduces the PyTorch fixture within the
reference's own tolerances, which pins the evaluator, including permute,
softmax, bmm and the max-pool indices, on the real graph.
GPU: the program runs through Node -> N-API -> libwgx on GPU 0 and must meet
the reference's tolerances against the fixture: float32 within 0.01
absolute everywhere (yolo26n.test.ts:76-98), float16 within 0.5 absolute
except at most 5 % of the outputs (yolo26n.test.ts:120-131).
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden", "yolo26n")
RUNNER = os.path.join(ROOT, "wgpu-executorch_amd", "js", "run_program.js")
NODE = shutil.which("node")
needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")
N_IN = 3 * 640 * 640

VARIANTS = {"float32": ("program.json", "weights.bin", np.float32),
            "float16": ("program-fp16.json", "weights-fp16.bin", np.float16)}


def make_input(dtype):
    i = np.arange(N_IN)
    return ((i % 251) / 250 - 0.5).astype(dtype)


def reference_output():
    return np.fromfile(os.path.join(GOLD, "reference-output.f32"), dtype=np.float32).astype(np.float64)


def stage(tmp_path, dtype):
    """A run_program.js directory: program.json, weights.bin, input.bin."""
    prog, weights, npdt = VARIANTS[dtype]
    d = tmp_path / dtype
    d.mkdir(exist_ok=True)
    shutil.copy(os.path.join(GOLD, prog), d / "program.json")
    os.symlink(os.path.join(GOLD, weights), d / "weights.bin")
    make_input(npdt).tofile(d / "input.bin")
    return d


def check_fp32(out, ref):
    d = np.abs(out - ref)
    assert out.shape == ref.shape and np.all(np.isfinite(out))
    bad = int((d > 0.01).sum())
    assert bad == 0 and d.max() <= 0.01, f"{bad}/{d.size} beyond 0.01, max {d.max():.3e} at {int(np.argmax(d))}"
    return float(d.max())


def check_fp16(out, ref):
    d = np.abs(out - ref)
    assert out.shape == ref.shape
    beyond = int((d > 0.5).sum())
    assert beyond <= 0.05 * d.size, f"{beyond}/{d.size} beyond 0.5"
    return beyond


# ------------------------------------------------------------ CPU
def test_fixture_files_are_the_converted_pair():
    for dtype, (prog, weights, _) in VARIANTS.items():
        p = json.load(open(os.path.join(GOLD, prog)))
        assert len(p["chain"]) == 397
        assert p["values"][p["inputIds"][0]]["shape"] == [1, 3, 640, 640]
        assert p["values"][p["outputIds"][0]]["shape"] == [1, 84, 8400]
        assert p["values"][p["inputIds"][0]]["dtype"] == dtype
    assert os.path.getsize(os.path.join(GOLD, "reference-output.f32")) == 4 * 84 * 8400
    # the float16 conversion pads constants to 4-byte offsets only: some sit
    # at offsets that are not 16-byte aligned (utils/convert_model_to_fp16.mjs:61-66)
    p = json.load(open(os.path.join(GOLD, "program-fp16.json")))
    offs = [v["weightsOffset"] % 16 for v in p["values"] if v["type"] == "tensor" and "weightsOffset" in v]
    assert any(o != 0 for o in offs)


@needs_node
@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_js_host_records_every_op(tmp_path, dtype):
    d = stage(tmp_path, dtype)
    res = {}
    for flags in ((), ("--no-fuse", "--no-views", "--no-bind-io")):
        r = subprocess.run([NODE, RUNNER, str(d), "--device", "-1", "--record-only", *flags],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr[-2000:]
        res[flags] = json.loads(r.stdout.strip().splitlines()[-1])
        assert res[flags]["ops"] == 397
    # the graph passes fold SiLU triples and elide view copies; the three
    # chained 5x5 max-pools of the SPPF block fold into one launch
    assert res[()]["commands"] < res[("--no-fuse", "--no-views", "--no-bind-io")]["commands"]


def _validate(prog, nbytes):
    js = ("const W=require(process.argv[1]);const fs=require('fs');"
          "W.validateProgram(JSON.parse(fs.readFileSync(0,'utf8')), Number(process.argv[2]));")
    return subprocess.run([NODE, "-e", js, os.path.join(ROOT, "wgpu-executorch_amd", "js"), str(nbytes)],
                          input=json.dumps(prog), capture_output=True, text=True, timeout=60)


@needs_node
def test_converter_rules_accept_the_programs_and_reject_broken_ones():
    """utils/pte_to_program.py:421-475, as validateProgram applies them."""
    for dtype, (prog, weights, _) in VARIANTS.items():
        p = json.load(open(os.path.join(GOLD, prog)))
        n = os.path.getsize(os.path.join(GOLD, weights))
        assert _validate(p, n).returncode == 0, _validate(p, n).stderr
    p = json.load(open(os.path.join(GOLD, "program.json")))
    n = os.path.getsize(os.path.join(GOLD, "weights.bin"))
    cases = []
    q = json.loads(json.dumps(p)); q["chain"][5]["args"][0] = len(q["values"]) + 3
    cases.append((q, n, r"chain\[5\] '.*' references values\[\d+\] but only \d+ values exist"))
    q = json.loads(json.dumps(p)); q["outputIds"] = [10**6]
    cases.append((q, n, r"outputIds references values\[1000000\] out of range"))
    q = json.loads(json.dumps(p))
    sc = next(i for i, v in enumerate(q["values"]) if v["type"] == "scalar")
    q["inputIds"] = [sc]
    cases.append((q, n, r"inputIds references values\[\d+\] of type 'scalar', expected 'tensor'"))
    q = json.loads(json.dumps(p)); q["memoryPlan"]["pools"] = q["memoryPlan"]["pools"][:-1]
    cases.append((q, n, r"has memObjId=\d+ but no matching pool in memoryPlan"))
    cases.append((p, n - 4, r"Weights size mismatch: declared \d+ bytes, actual \d+ bytes"))
    q = json.loads(json.dumps(p))
    last = max((i for i, v in enumerate(q["values"]) if "weightsOffset" in v), key=lambda i: q["values"][i]["weightsOffset"])
    q["values"][last]["weightsOffset"] += 8
    cases.append((q, n, r"weights \[\d+:\d+\] exceeds weights.bin size"))
    import re
    for q, nb, pat in cases:
        r = _validate(q, nb)
        assert r.returncode != 0 and re.search(pat, r.stderr), (pat, r.stderr[-500:])


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_oracle_program_evaluator_matches_the_pytorch_fixture(orc, dtype):
    from oracle import program_eval

    prog, weights, npdt = VARIANTS[dtype]
    p = json.load(open(os.path.join(GOLD, prog)))
    w = open(os.path.join(GOLD, weights), "rb").read()
    out = program_eval.evaluate(p, w, [make_input(npdt)])[0].ravel()
    ref = reference_output()
    if dtype == "float32":
        err = check_fp32(out, ref)
        assert err < 5e-3  # measured 1.9e-3
    else:
        beyond = check_fp16(out, ref)
        assert beyond < 0.002 * ref.size  # measured 244 of 705600


# ------------------------------------------------------------ GPU
def _run_gpu(tmp_path, dtype, flags=()):
    d = stage(tmp_path, dtype)
    out = tmp_path / f"out_{dtype}.bin"
    print(f"[yolo26n] {dtype} flags={list(flags)}: running on GPU 0 through Node", flush=True)
    r = subprocess.run([NODE, RUNNER, str(d), "--device", "0", "--warmup", "1", "--reps", "3",
                        "--out", str(out), *flags], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-3000:]
    info = json.loads(r.stdout.strip().splitlines()[-1])
    gpu = np.fromfile(out, dtype=VARIANTS[dtype][2]).astype(np.float64)
    return gpu, info


@needs_node
@pytest.mark.gpu
def test_yolo26n_float32_matches_pytorch(tmp_path, pkg):
    gpu, info = _run_gpu(tmp_path, "float32")
    err = check_fp32(gpu, reference_output())
    print(f"[yolo26n] float32: max abs err {err:.3e}, {info['commands']} launches, "
          f"{info['frame_ms_device']:.3f} ms/frame device", flush=True)


@needs_node
@pytest.mark.gpu
@pytest.mark.parametrize("flags", [(), ("--no-fuse", "--no-views", "--no-bind-io")], ids=["passes", "op_by_op"])
def test_yolo26n_float16_matches_pytorch(tmp_path, pkg, orc, flags):
    from oracle import program_eval

    gpu, info = _run_gpu(tmp_path, "float16", flags)
    ref = reference_output()
    beyond = check_fp16(gpu, ref)
    # and against the oracle's evaluation of the same float16 program, whose
    # difference is accumulation order (fp32 on the GPU, fp64 on the CPU)
    p = json.load(open(os.path.join(GOLD, "program-fp16.json")))
    w = open(os.path.join(GOLD, "weights-fp16.bin"), "rb").read()
    cpu = program_eval.evaluate(p, w, [make_input(np.float16)])[0].ravel()
    rel = np.linalg.norm(gpu - cpu) / np.linalg.norm(cpu)
    print(f"[yolo26n] float16 {list(flags)}: {beyond} of {ref.size} beyond 0.5 of PyTorch; "
          f"normwise vs the oracle's fp16 evaluation {rel:.2e}; {info['commands']} launches, "
          f"{info['frame_ms_device']:.3f} ms/frame device", flush=True)
    assert rel < 5e-3
