"""Benchmark of the GEMM-shaped hot path on one MI355X.

Default workload (the configuration the headline metric is quoted on):
aten.convolution as implicit-im2col GEMM, float32 NCHW, batch 1 --
  2a: x[1,64,80,80]  * w[128,64,3,3]  s1 p1 -> y[1,128,80,80]
  2b: x[1,128,80,80] * w[256,128,3,3] s2 p1 -> y[1,256,40,40]
One step = both convolutions, recorded once and replayed with one submit per
step (one captured HIP graph).  Inputs are resident in HBM before timing.

Printed: ONE JSON line on stdout (the contract).  Per-configuration numbers
for every other configuration (mm 512^3 fp32, the conv pair in fp16 on MFMA,
depthwise fp16, addmm fp16 NN/NT, bmm fp16, the synthetic YOLO-N and the
reference's yolo26n fp16 programs) go to stderr and, with --detail
PATH, to a JSON file.  Each is measured at shape (single launch per sample)
and amortised (a graph of many instances rotating over >= 300 MB of distinct
buffers, so the 256 MB MALL cannot hold the working set); roofline fractions
quote the amortised number.

The CPU baseline is the oracle's order-faithful C restatement of the
reference WGSL kernels (Dawn + SwiftShader cannot run offline), timed on this
host's cores on a bounded sample of the same workload.
"""
import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {  # MI355X published dense peaks
    "hbm_GBps": 8000.0,
    "fp16_TFLOPs": 2500.0,
    "bf16_TFLOPs": 2500.0,
    "fp32_TFLOPs": 157.3,
}
CONV2 = {
    "2a": dict(x=(1, 64, 80, 80), w=(128, 64, 3, 3), s=(1, 1), p=(1, 1), y=(1, 128, 80, 80)),
    "2b": dict(x=(1, 128, 80, 80), w=(256, 128, 3, 3), s=(2, 2), p=(1, 1), y=(1, 256, 40, 40)),
}


def conv_flops(c):
    _, oc, oh, ow = c["y"]
    _, icg, kh, kw = c["w"]
    return 2.0 * oc * oh * ow * icg * kh * kw * c["y"][0]


def conv_bytes(c, es):
    n = int(np.prod(c["x"])) + int(np.prod(c["w"])) + c["w"][0] + int(np.prod(c["y"]))
    return n * es


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- builders
def build_conv(ctx, I, c, dtype, seed, bias=True, batch=1, repeat=1):
    xs = (batch,) + tuple(c["x"][1:])
    ys = [batch] + list(c["y"][1:])
    x = I.uniform(seed, xs, -1, 1)
    w = I.kaiming_uniform(seed + 1, c["w"])
    tx, tw = ctx.from_numpy(x, dtype), ctx.from_numpy(w, dtype)
    tb = ctx.from_numpy(I.uniform(seed + 2, (c["w"][0],), -0.1, 0.1), dtype) if bias else None
    ty = ctx.tensor(dtype, ys)
    groups = c.get("groups", 1)
    for _ in range(repeat):
        ctx.convolution(tx, tw, tb, list(c["s"]), list(c["p"]), [1, 1], False, [0, 0], groups, ty)
    return ctx.last_kernel


# ---------------------------------------------------------------- HBM traffic
COPY_BYTES = 512 << 20
PROBE_REPS = 5


def traffic_probe(W, I, v):
    """Child run counted by rocprofv3: the headline's conv `v` (float32; "pair":
    2a and 2b recorded back to back, which the runtime runs as one paired
    launch) PROBE_REPS times, then a device copy of COPY_BYTES PROBE_REPS
    times (the calibration)."""
    ctx = W.Context(0)
    try:
        for name in (("2a", "2b") if v == "pair" else (v,)):
            build_conv(ctx, I, CONV2[name], "float32", 40 + 10 * (name == "2b"))
        ctx.set_graph_mode(False)
        for _ in range(PROBE_REPS):
            ctx.submit()
        ctx.sync()
        ctx.reset()
        src = ctx.tensor("float32", [COPY_BYTES // 4])
        dst = ctx.tensor("float32", [COPY_BYTES // 4])
        ctx.copy(src, dst)
        for _ in range(PROBE_REPS):
            ctx.submit()
        ctx.sync()
    finally:
        ctx.destroy()


# One configuration, recorded once and submitted PROBE_REPS times without a
# graph (one dispatch per launch): the child run that rocprofv3 --pmc counts.
KERNEL_PROBES = ("conv2a_f32", "conv2b_f32", "conv2ab_f32", "conv2a_f16", "conv2a_f16_b64", "conv2b_f16_b64", "addmm_nt",
                 "addmm_nn", "bmm", "dw3a", "dw3b", "dw3a_b256", "dw3b_b256")


def kernel_probe(W, I, name):
    ctx = W.Context(0)
    try:
        if name == "conv2ab_f32":  # 2a and 2b back to back: one paired launch
            build_conv(ctx, I, CONV2["2a"], "float32", 40)
            build_conv(ctx, I, CONV2["2b"], "float32", 50)
        elif name.startswith("conv"):
            build_conv(ctx, I, CONV2[name[4:6]], "float32" if name.endswith("f32") else "float16", 40,
                       batch=64 if name.endswith("_b64") else 1)
        elif name.startswith("addmm"):
            M, K, N = 4096, 768, 3072
            nt = name.endswith("nt")
            x = ctx.from_numpy(I.normal(1, (M, K)), "float16")
            w = ctx.from_numpy(I.normal(2, (N, K) if nt else (K, N), 0, 0.02), "float16")
            b = ctx.from_numpy(I.uniform(3, (N,), -0.1, 0.1), "float16")
            ctx.addmm(b, x, w, ctx.tensor("float16", [M, N]), trans_b=nt)
        elif name == "bmm":
            a = ctx.from_numpy(I.normal(1, (16, 1024, 64)), "float16")
            bb = ctx.from_numpy(I.normal(2, (16, 64, 1024)), "float16")
            ctx.bmm(a, bb, ctx.tensor("float16", [16, 1024, 1024]))
        else:
            batch = 256 if name.endswith("b256") else 1
            C, H, K, S = (256, 40, 3, 1) if name.startswith("dw3a") else (512, 20, 5, 2)
            OH = (H + 2 * (K // 2) - K) // S + 1
            x = ctx.from_numpy(I.normal(3, (batch, C, H, H)), "float16")
            w = ctx.from_numpy(I.uniform(4, (C, 1, K, K), -0.5, 0.5), "float16")
            ctx.convolution(x, w, None, [S, S], [K // 2, K // 2], [1, 1], False, [0, 0], C,
                            ctx.tensor("float16", [batch, C, OH, OH]))
        print(name, ctx.last_kernel, flush=True)
        ctx.set_graph_mode(False)
        for _ in range(PROBE_REPS):
            ctx.submit()
        ctx.sync()
    finally:
        ctx.destroy()


def measure_traffic(v):
    """HBM bytes per step of the headline conv `v` ("pair": the paired launch
    of 2a and 2b; else its convolution or GEMM dispatch, plus the split-K
    reduction when there is one) from two
    rocprofv3 --pmc runs
    (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each scaled by what the
    counter reads for a plain copy of COPY_BYTES (which moves exactly
    COPY_BYTES in each direction).  The copy's reading is the sum over the
    blit dispatches issued after the last conv dispatch (the data uploads
    before the conv are blits too), divided by PROBE_REPS."""
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if prof is None:
        return None
    res = {}
    env = dict(os.environ, TMPDIR="/tmp")
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="wgx_pmc_", dir="/tmp")
        try:
            cmd = ["timeout", "-s", "KILL", "90", prof, "--pmc", counter, "-d", d, "-o", "run",
                   "--output-format", "csv", "--", sys.executable, os.path.abspath(__file__),
                   "--traffic-probe", v]
            r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True, timeout=120)
            files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
            if r.returncode != 0 or not files:
                log(f"traffic: rocprofv3 {counter} failed (rc {r.returncode})")
                return None
            rows = []
            with open(files[0]) as f:
                for row in csv.DictReader(f):
                    if row["Counter_Name"] == counter:
                        rows.append((int(row["Dispatch_Id"]), row["Kernel_Name"],
                                     float(row["Counter_Value"])))
            rows.sort()
            conv = [(i, x) for i, n, x in rows
                    if any(k in n for k in ("k_gemm", "k_sgemm", "k_splitk", "k_conv_lds"))]
            last = max((i for i, _ in conv), default=None)
            copy = [x for i, n, x in rows if "copyBuffer" in n and last is not None and i > last]
            if not conv or not copy:
                log(f"traffic: no {counter} rows for the conv or the copy")
                return None
            res[counter] = (sum(x for _, x in conv) / PROBE_REPS, sum(copy) / PROBE_REPS)
        finally:
            shutil.rmtree(d, ignore_errors=True)
    f_k, f_c = res["FETCH_SIZE"]
    w_k, w_c = res["WRITE_SIZE"]
    fs, ws = COPY_BYTES / (f_c * 1024.0), COPY_BYTES / (w_c * 1024.0)
    return {"bytes": int(f_k * 1024 * fs + w_k * 1024 * ws),
            "fetch_kib": round(f_k, 1), "write_kib": round(w_k, 1),
            "copy_fetch_kib": round(f_c, 1), "copy_write_kib": round(w_c, 1),
            "fetch_scale": round(fs, 4), "write_scale": round(ws, 4)}


def time_ctx(ctx, reps, warm=3):
    for _ in range(warm):
        ctx.submit()
    ctx.sync()
    return ctx.time_submits(reps)


def measure(W, build, n_inst_amortised, reps_shape=50, reps_amort=5, graph=True):
    """At-shape: one instance, one launch per submit.  Amortised: a graph of
    n instances with distinct buffers, per-instance time (graph=False: the
    instances issued as direct launches, as a short command list runs)."""
    ctx = W.Context(0)
    try:
        ctx.set_graph_mode(graph)
        kernel = build(ctx, 0)
        shape_ms = time_ctx(ctx, reps_shape)
    finally:
        ctx.destroy()
    ctx = W.Context(0)
    try:
        ctx.set_graph_mode(graph)
        for i in range(n_inst_amortised):
            build(ctx, i)
        amort_ms = time_ctx(ctx, reps_amort, warm=1) / n_inst_amortised
    finally:
        ctx.destroy()
    return kernel, shape_ms, amort_ms


# ---------------------------------------------------------------- detail configs
def detail_configs(W, I, quick=False, yolo=True):
    out = {}
    scale = 0.25 if quick else 1.0

    def rec(name, kernel, shape_ms, amort_ms, flops, nbytes, bound, peak):
        d = {"kernel": kernel, "at_shape_ms": shape_ms, "amortised_ms": amort_ms,
             "GFLOPs_at_shape": flops / shape_ms / 1e6, "GFLOPs_amortised": flops / amort_ms / 1e6,
             "GBps_at_shape": nbytes / shape_ms / 1e6, "GBps_amortised": nbytes / amort_ms / 1e6,
             "bound": bound}
        if bound == "hbm":
            d["frac_of_peak_amortised"] = d["GBps_amortised"] / PEAK["hbm_GBps"]
        else:
            d["frac_of_peak_amortised"] = d["GFLOPs_amortised"] / 1e3 / peak
        out[name] = d
        log(f"{name:28s} {kernel:34s} shape {shape_ms*1e3:9.2f} us  amort {amort_ms*1e3:9.2f} us  "
            f"{d['GFLOPs_amortised']:10.1f} GFLOP/s {d['GBps_amortised']:9.1f} GB/s  "
            f"{100*d['frac_of_peak_amortised']:5.1f}% of {bound}")

    # config 1: mm fp32 512^3
    def b_mm(ctx, i):
        a = ctx.from_numpy(I.uniform(2 * i, (512, 512), -1, 1), "float32")
        b = ctx.from_numpy(I.uniform(2 * i + 1, (512, 512), -1, 1), "float32")
        o = ctx.tensor("float32", [512, 512])
        ctx.mm(a, b, o)
        return ctx.last_kernel
    k, s, a = measure(W, b_mm, max(8, int(100 * scale)))
    rec("1_mm_f32_512", k, s, a, 2 * 512 ** 3, 3 * 512 * 512 * 4, "mfma", PEAK["fp32_TFLOPs"])

    # config 2 in both dtypes
    for dt, es, peak in (("float32", 4, PEAK["fp32_TFLOPs"]), ("float16", 2, PEAK["fp16_TFLOPs"])):
        for v, c in CONV2.items():
            n = max(8, int(int(300e6 / conv_bytes(c, es)) * scale))
            k, s, a = measure(W, lambda ctx, i, c=c, dt=dt: build_conv(ctx, I, c, dt, 10 * i), n)
            rec(f"2{v[1]}_conv_{dt}", k, s, a, conv_flops(c), conv_bytes(c, es), "mfma", peak)
            # one launch carrying 64 batch-1 instances (batched-instance form)
            ctx = W.Context(0)
            try:
                kb = build_conv(ctx, I, c, dt, 7, batch=64)
                ms = time_ctx(ctx, 10)
            finally:
                ctx.destroy()
            out[f"2{v[1]}_conv_{dt}"]["batched64_ms_per_instance"] = ms / 64
            out[f"2{v[1]}_conv_{dt}"]["GFLOPs_batched64"] = conv_flops(c) * 64 / ms / 1e6
            out[f"2{v[1]}_conv_{dt}"]["frac_of_peak_batched64"] = conv_flops(c) * 64 / ms / 1e9 / peak
            log(f"{'':28s} batched x64: {ms/64*1e3:9.2f} us/instance  "
                f"{conv_flops(c)*64/ms/1e6:10.1f} GFLOP/s  {100*conv_flops(c)*64/ms/1e9/peak:5.1f}%")

    # config 3: depthwise fp16
    DW = {"3A": dict(x=(1, 256, 40, 40), w=(256, 1, 3, 3), s=(1, 1), p=(1, 1), y=(1, 256, 40, 40), groups=256),
          "3B": dict(x=(1, 512, 20, 20), w=(512, 1, 5, 5), s=(2, 2), p=(2, 2), y=(1, 512, 10, 10), groups=512)}
    for v, c in DW.items():
        nbytes = (int(np.prod(c["x"])) + int(np.prod(c["w"])) + int(np.prod(c["y"]))) * 2
        n = max(8, int(int(300e6 / nbytes) * scale))

        def b_dw(ctx, i, c=c):
            x = ctx.from_numpy(I.normal(10 * i, c["x"]), "float16")
            w = ctx.from_numpy(I.uniform(10 * i + 1, c["w"], -0.5, 0.5), "float16")
            b = ctx.from_numpy(np.zeros(c["w"][0], np.float32), "float16")
            y = ctx.tensor("float16", list(c["y"]))
            ctx.convolution(x, w, b, list(c["s"]), list(c["p"]), [1, 1], False, [0, 0], c["groups"], y)
            return ctx.last_kernel
        k, s, a = measure(W, b_dw, n)
        rec(f"{v}_depthwise_f16", k, s, a, conv_flops(c), nbytes, "hbm", None)
        # batched-instance form: one launch over 256 instances
        ctx = W.Context(0)
        try:
            cb = dict(c)
            xb = (256,) + tuple(c["x"][1:])
            x = ctx.from_numpy(I.normal(3, xb), "float16")
            w = ctx.from_numpy(I.uniform(4, c["w"], -0.5, 0.5), "float16")
            y = ctx.tensor("float16", [256] + list(c["y"][1:]))
            ctx.convolution(x, w, None, list(c["s"]), list(c["p"]), [1, 1], False, [0, 0], c["groups"], y)
            ms = time_ctx(ctx, 20)
        finally:
            ctx.destroy()
        bbytes = (int(np.prod(c["x"])) + int(np.prod(c["y"]))) * 2 * 256 + int(np.prod(c["w"])) * 2
        out[f"{v}_depthwise_f16"]["GBps_batched256"] = bbytes / ms / 1e6
        out[f"{v}_depthwise_f16"]["frac_of_peak_batched256"] = bbytes / ms / 1e6 / PEAK["hbm_GBps"]
        log(f"{'':28s} batched x256: {ms*1e3:9.2f} us  {bbytes/ms/1e6:9.1f} GB/s  "
            f"{100*bbytes/ms/1e6/PEAK['hbm_GBps']:5.1f}% of HBM")

    # config 4: addmm fp16, NN and NT
    M, K, N = 4096, 768, 3072
    for tb in (False, True):
        def b_addmm(ctx, i, tb=tb):
            x = ctx.from_numpy(I.normal(10 * i, (M, K)), "float16")
            wshape = (N, K) if tb else (K, N)
            w = ctx.from_numpy(I.normal(10 * i + 1, wshape, 0, 0.02), "float16")
            b = ctx.from_numpy(I.uniform(10 * i + 2, (N,), -0.1, 0.1), "float16")
            o = ctx.tensor("float16", [M, N])
            ctx.addmm(b, x, w, o, trans_b=tb)
            return ctx.last_kernel
        nb = (M * K + K * N + N + M * N) * 2
        k, s, a = measure(W, b_addmm, max(4, int(9 * scale)), reps_shape=20, reps_amort=3)
        rec(f"4_addmm_f16_{'NT' if tb else 'NN'}", k, s, a, 2.0 * M * N * K, nb, "mfma", PEAK["fp16_TFLOPs"])

    # config 4: bmm fp16
    def b_bmm(ctx, i):
        a = ctx.from_numpy(I.normal(10 * i, (16, 1024, 64)), "float16")
        b = ctx.from_numpy(I.normal(10 * i + 1, (16, 64, 1024)), "float16")
        o = ctx.tensor("float16", [16, 1024, 1024])
        ctx.bmm(a, b, o)
        return ctx.last_kernel
    nb = (2 * 16 * 1024 * 64 + 16 * 1024 * 1024) * 2
    k, s, a = measure(W, b_bmm, max(4, int(9 * scale)), reps_shape=20, reps_amort=3)
    rec("4_bmm_f16", k, s, a, 2.0 * 16 * 1024 * 1024 * 64, nb, "hbm", None)

    # config 5: the YOLO-N-style fp16 program through Node recordProgram
    y = yolo_frame(quick) if yolo else None
    if y is not None:
        out["5_yolo_n_f16"] = y
        log(f"{'5_yolo_n_f16':28s} {y['ops']} ops / {y['commands']} commands      "
            f"frame {y['frame_ms_wall']*1e3:9.1f} us wall (submit+sync), {y['frame_ms_device']*1e3:9.1f} us device  "
            f"{y['conv_GFLOPs_device']:8.1f} conv GFLOP/s")
    # and the reference's own converted yolo26n (fp16 program and weights)
    y = yolo26n_frame(quick) if yolo else None
    if y is not None:
        out["5_yolo26n_f16"] = y
        log(f"{'5_yolo26n_f16':28s} {y['ops']} ops / {y['commands']} commands      "
            f"frame {y['frame_ms_wall']*1e3:9.1f} us wall (submit+sync), {y['frame_ms_device']*1e3:9.1f} us device")
    return out


def yolo26n_frame(quick=False):
    """ms/frame of the reference's yolo26n float16 program (program-fp16.json
    and weights-fp16.bin as its converter wrote them, 397 operators, input
    [1,3,640,640]) through recordProgram in Node, measured like yolo_frame."""
    import shutil
    import subprocess
    import tempfile

    node = shutil.which("node")
    gold = os.path.join(ROOT, "tests", "golden", "yolo26n")
    if node is None or not os.path.isfile(os.path.join(gold, "program-fp16.json")):
        log("5_yolo26n_f16: node or the program files are missing, skipped")
        return None
    d = tempfile.mkdtemp(prefix="wgx_yolo26n_")
    try:
        shutil.copy(os.path.join(gold, "program-fp16.json"), os.path.join(d, "program.json"))
        os.symlink(os.path.join(gold, "weights-fp16.bin"), os.path.join(d, "weights.bin"))
        i = np.arange(3 * 640 * 640)
        ((i % 251) / 250 - 0.5).astype(np.float16).tofile(os.path.join(d, "input.bin"))
        runner = os.path.join(ROOT, "wgpu-executorch_amd", "js", "run_program.js")
        reps = 20 if quick else 100
        r = subprocess.run([node, runner, d, "--device", "0", "--warmup", "5", "--reps", str(reps)],
                           capture_output=True, text=True, timeout=300)
        if r.returncode != 0:
            raise RuntimeError("run_program.js failed: " + r.stderr[-2000:])
        res = json.loads(r.stdout.strip().splitlines()[-1])
    finally:
        shutil.rmtree(d, ignore_errors=True)
    res["unit"] = "ms/frame"
    return res


def yolo_frame(quick=False):
    """ms/frame of the synthetic YOLO-N-style fp16 program, input [1,3,640,640]:
    recorded once with WgpuExecutionContext.recordProgram in Node, one
    submit()+sync() per frame (median wall time) and device time per submit."""
    import importlib
    import shutil
    import subprocess
    import tempfile

    node = shutil.which("node")
    if node is None:
        log("5_yolo_n_f16: node is not installed, skipped")
        return None
    Y = importlib.import_module("wgpu_executorch_amd.yolo_program")
    d = tempfile.mkdtemp(prefix="wgx_yolo_")
    try:
        info = Y.write(d, img=640)
        runner = os.path.join(ROOT, "wgpu-executorch_amd", "js", "run_program.js")
        reps = 20 if quick else 100
        r = subprocess.run([node, runner, d, "--device", "0", "--warmup", "5", "--reps", str(reps)],
                           capture_output=True, text=True, timeout=300)
        if r.returncode != 0:
            raise RuntimeError("run_program.js failed: " + r.stderr[-2000:])
        res = json.loads(r.stdout.strip().splitlines()[-1])
    finally:
        shutil.rmtree(d, ignore_errors=True)
    res.update({"params": info["params"], "conv_gflop": info["conv_flops"] / 1e9,
                "conv_GFLOPs_device": info["conv_flops"] / res["frame_ms_device"] / 1e6,
                "unit": "ms/frame"})
    return res


def gemm_k_sweep(W, I):
    """Where the large-tile GEMM's time goes: the fp16 addmm NT form (X[4096,K]
    @ W^T, W^T stored [3072,K], + bias) for K from 64 to 3072, amortised (a
    graph of instances over >= 300 MB of buffers), one JSON line per K."""
    M, N = 4096, 3072
    for K in (64, 192, 384, 768, 1536, 3072):
        def b(ctx, i, K=K):
            x = ctx.from_numpy(I.normal(10 * i + 1, (M, K)), "float16")
            w = ctx.from_numpy(I.normal(10 * i + 2, (N, K), 0, 0.02), "float16")
            bias = ctx.from_numpy(I.uniform(10 * i + 3, (N,), -0.1, 0.1), "float16")
            ctx.addmm(bias, x, w, ctx.tensor("float16", [M, N]), trans_b=True)
            return ctx.last_kernel
        nbytes = (M * K + N * K + N + M * N) * 2
        k, s, a = measure(W, b, max(4, int(300e6 // nbytes) + 1), reps_shape=20, reps_amort=5)
        print(json.dumps({"K": K, "kernel": k, "at_shape_us": round(s * 1e3, 2), "amortised_us": round(a * 1e3, 2),
                          "TFLOPs_amortised": round(2.0 * M * N * K / (a * 1e-3) / 1e12, 1)}), flush=True)


# ---------------------------------------------------------------- vendor libraries
def vendor_configs():
    """The same shapes through PyTorch-ROCm's own kernels (hipBLASLt for the
    GEMMs, MIOpen for the convolutions), per launch, back-to-back launches
    timed with HIP events on torch's stream (warm caches, like the at-shape
    numbers above).  A point of comparison only: nothing of the product path
    runs through torch."""
    import torch
    import torch.nn.functional as F

    dev = "cuda"
    out = {}

    def t(fn, reps=100, warm=10):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps  # ms

    g = torch.Generator(device=dev).manual_seed(5)
    M, K, N = 4096, 768, 3072
    X = torch.randn(M, K, device=dev, dtype=torch.float16, generator=g)
    Wt = (torch.randn(N, K, device=dev, dtype=torch.float16, generator=g) * 0.02)
    Wkn = Wt.t().contiguous()
    b = torch.rand(N, device=dev, dtype=torch.float16, generator=g) * 0.2 - 0.1
    out["4_addmm_f16_NN"] = t(lambda: torch.addmm(b, X, Wkn))
    out["4_addmm_f16_NT"] = t(lambda: torch.addmm(b, X, Wt.t()))
    A = torch.randn(16, 1024, 64, device=dev, dtype=torch.float16, generator=g)
    B = torch.randn(16, 64, 1024, device=dev, dtype=torch.float16, generator=g)
    out["4_bmm_f16"] = t(lambda: torch.bmm(A, B))
    a = torch.rand(512, 512, device=dev, generator=g) * 2 - 1
    out["1_mm_f32_512"] = t(lambda: torch.mm(a, a))
    for dt, name in ((torch.float32, "float32"), (torch.float16, "float16")):
        for v, c in CONV2.items():
            x = torch.rand(c["x"], device=dev, dtype=dt, generator=g) * 2 - 1
            w = torch.rand(c["w"], device=dev, dtype=dt, generator=g) * 0.2 - 0.1
            bb = torch.rand(c["w"][0], device=dev, dtype=dt, generator=g) * 0.2 - 0.1
            out[f"2{v[1]}_conv_{name}"] = t(lambda: F.conv2d(x, w, bb, stride=c["s"], padding=c["p"]), reps=50)
    for nm, xs, ws, s_, p_ in (("3A_depthwise_f16", (1, 256, 40, 40), (256, 1, 3, 3), 1, 1),
                               ("3B_depthwise_f16", (1, 512, 20, 20), (512, 1, 5, 5), 2, 2)):
        x = torch.randn(xs, device=dev, dtype=torch.float16, generator=g)
        w = torch.rand(ws, device=dev, dtype=torch.float16, generator=g) - 0.5
        out[nm] = t(lambda: F.conv2d(x, w, None, stride=s_, padding=p_, groups=xs[1]), reps=50)
    torch.cuda.synchronize()
    return out


# ---------------------------------------------------------------- CPU baseline
def cpu_baseline(I, budget_s=20.0):
    """The oracle's WGSL restatement (f32, order-faithful) on this host's
    cores, over whole steps of the default workload until budget_s is used."""
    import oracle

    n_thr = oracle.num_threads()
    data = {}
    for v, c in CONV2.items():
        data[v] = (I.uniform(100, c["x"], -1, 1), I.kaiming_uniform(101, c["w"]),
                   I.uniform(102, (c["w"][0],), -0.1, 0.1))
    steps, t0 = 0, time.perf_counter()
    while True:
        for v, c in CONV2.items():
            x, w, b = data[v]
            oracle.emu_conv2d(0, x, w, b, c["s"], c["p"])
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 10000:
            break
    flops = sum(conv_flops(c) for c in CONV2.values()) * steps
    return {"value": flops / el / 1e9, "unit": "GFLOP/s", "cores": n_thr, "kind": "port",
            "sample": f"{steps} full steps (conv 2a + 2b, float32, batch 1) of the oracle's "
                      f"order-faithful C restatement of the reference WGSL kernels, "
                      f"{el:.1f} s on {n_thr} OpenMP threads; Dawn+SwiftShader is unavailable offline"}


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--detail", type=str, default=None, help="write per-config JSON here")
    ap.add_argument("--no-detail", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 FETCH/WRITE_SIZE runs")
    ap.add_argument("--vendor", action="store_true",
                    help="also time PyTorch-ROCm's hipBLASLt / MIOpen kernels on the same shapes (detail only)")
    ap.add_argument("--no-yolo", action="store_true", help="skip the YOLO-N program (config 5) in the detail")
    ap.add_argument("--kernel-probe", choices=KERNEL_PROBES, default=None,
                    help="record one configuration and submit it a few times (for rocprofv3 --pmc runs)")
    ap.add_argument("--gemm-k-sweep", action="store_true",
                    help="time the fp16 addmm NT form at M=4096, N=3072 for K = 64 ... 3072 (amortised) and exit")
    ap.add_argument("--yolo26n-only", action="store_true",
                    help="run only the reference's yolo26n float16 program (ms/frame) and exit")
    ap.add_argument("--vendor-probe", action="store_true",
                    help=argparse.SUPPRESS)  # the child run that times the vendor kernels
    ap.add_argument("--traffic-probe", choices=list(CONV2) + ["pair"], default=None,
                    help=argparse.SUPPRESS)  # the child run that rocprofv3 counts
    args = ap.parse_args()
    if args.vendor_probe:
        # torch ships its own HIP runtime: it runs in a process of its own,
        # one that never loads libwgx
        print(json.dumps(vendor_configs()), flush=True)
        return
    if args.yolo26n_only:
        # the frame runs in a Node child process; this one never touches the GPU
        print(json.dumps({"5_yolo26n_f16": yolo26n_frame(args.quick)}), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on exactly one GPU (the hot path is not sharded); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from __graft_entry__ import load_package

    pkg = load_package()
    W, I = pkg.wgx, pkg.inputs
    if args.traffic_probe:
        traffic_probe(W, I, args.traffic_probe)
        return
    if args.kernel_probe:
        kernel_probe(W, I, args.kernel_probe)
        return
    if args.gemm_k_sweep:
        gemm_k_sweep(W, I)
        return

    # ---- headline: config 2 (2a + 2b), float32, one submit per step
    ctx = W.Context(0)
    kernels = {}
    for v, c in CONV2.items():
        kernels[v] = build_conv(ctx, I, c, "float32", 40 + 10 * (v == "2b"))
    for _ in range(args.warmup):
        ctx.submit()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ctx.submit()
    ctx.sync()
    el = time.perf_counter() - t0
    # the same steps again between HIP events on the context's stream: the
    # per-launch time of the step as it runs back to back (operands warm)
    steps_ms = ctx.time_submits(args.steps)
    # 2a and 2b read and write disjoint buffers: the runtime may run them as
    # one paired launch (WGX_MERGE=0 keeps them apart)
    paired = ctx.paired_launches > 0
    ctx.destroy()
    ms_step = el * 1e3 / args.steps
    step_flops = sum(conv_flops(c) for c in CONV2.values())
    value = step_flops / (ms_step * 1e-3) / 1e9

    # ---- dominant kernel: average launch duration, HIP events recorded on the
    # context's own stream around one submit of a graph, two ways:
    #  amortised (quoted): AMORT instances over distinct buffers of >= 300 MB
    #    in all, so the 256 MB MALL cannot hold the working set and every
    #    launch reads its operands from HBM;
    #  warm: 20 launches of one instance (operands stay in L2 / MALL).
    # Both issue the instances as direct launches, the path a step's short
    # command list takes (a graph's kernel nodes run slower: the paired
    # launch 29.2 us in a graph, 26.8 us per step issued directly).
    per_kernel, warm = {}, {}
    reps_in_graph = 20
    if paired:
        # the step is one paired launch of 2a and 2b: that launch is the
        # dominant (only) kernel; warm: 20 pairs on one set of buffers,
        # amortised: a graph of (2a, 2b) instances over >= 300 MB
        kctx = W.Context(0)
        try:
            kctx.set_graph_mode(False)
            for _ in range(reps_in_graph):
                for v, c in CONV2.items():
                    build_conv(kctx, I, c, "float32", 40 + 10 * (v == "2b"))
            warm["pair"] = time_ctx(kctx, 20) / reps_in_graph
        finally:
            kctx.destroy()
        pair_bytes = sum(conv_bytes(c, 4) for c in CONV2.values())

        def build_pair(ctx, i):
            for v, c in CONV2.items():
                build_conv(ctx, I, c, "float32", 40 + 10 * i + 5 * (v == "2b"))
        _, _, per_kernel["pair"] = measure(W, build_pair, int(300e6 / pair_bytes) + 1, reps_shape=5, reps_amort=10,
                                           graph=False)
        dom, flops_dom, bytes_dom = "pair", step_flops, pair_bytes
        # the pair runs both parts in 4-wave blocks, the part with more input
        # channels (2b) on 32 x 32 tiles, the other on 32 x 64
        kname = "k_conv_lds_pair (conv 2a: 3x3s1 32x64 tiles + conv 2b: 3x3s2 32x32 tiles, 4-wave blocks)"
        covers, wl = "one dispatch: conv 2a and 2b paired", "conv 2a + conv 2b (one paired launch)"
    else:
        for v, c in CONV2.items():
            kctx = W.Context(0)
            try:
                kctx.set_graph_mode(False)
                build_conv(kctx, I, c, "float32", 40, repeat=reps_in_graph)
                warm[v] = time_ctx(kctx, 20) / reps_in_graph
            finally:
                kctx.destroy()
            n = int(300e6 / conv_bytes(c, 4)) + 1
            _, _, per_kernel[v] = measure(W, lambda ctx, i, c=c: build_conv(ctx, I, c, "float32", 40 + 10 * i), n,
                                          reps_shape=5, reps_amort=10, graph=False)
        dom = max(per_kernel, key=per_kernel.get)
        flops_dom, bytes_dom, kname = conv_flops(CONV2[dom]), conv_bytes(CONV2[dom], 4), kernels[dom]
        covers = ("GEMM dispatch + split-K reduction dispatch" if re.search(r"_k\d+$", kernels[dom])
                  else "one dispatch")
        wl = f"conv {dom}"
    dom_ms = per_kernel[dom]
    achieved = flops_dom / (dom_ms * 1e-3) / 1e12
    achieved_warm = flops_dom / (warm[dom] * 1e-3) / 1e12
    traffic = None if args.no_traffic else measure_traffic(dom)
    roofline = {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK["fp32_TFLOPs"],
                "unit": "TFLOP/s", "frac": round(achieved / PEAK["fp32_TFLOPs"], 4),
                "traffic": traffic["bytes"] if traffic else None,
                "kernel": kname, "workload": wl,
                "launch_us": round(dom_ms * 1e3, 2),
                "protocol": "amortised: direct launches of instances over >= 300 MB of distinct buffers",
                "frac_warm": round(achieved_warm / PEAK["fp32_TFLOPs"], 4),
                "launch_us_warm": round(warm[dom] * 1e3, 2),
                # the timed steps themselves (a step is the one paired launch
                # when paired; else both launches of the step)
                "launch_us_steps": round(steps_ms * 1e3, 2),
                "frac_steps": round(step_flops / (steps_ms * 1e-3) / 1e12 / PEAK["fp32_TFLOPs"], 4),
                "launch_covers": covers,
                "algorithmic_bytes": bytes_dom}
    if traffic:
        roofline["traffic_detail"] = traffic

    detail = {}
    if not args.no_detail:
        log("---- per-configuration detail (amortised = graph of instances over >= 300 MB)")
        detail = detail_configs(W, I, quick=args.quick, yolo=not args.no_yolo)
        if args.vendor:
            import subprocess
            r = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-probe"],
                               capture_output=True, text=True, timeout=600)
            if r.returncode != 0:
                raise RuntimeError("vendor probe failed: " + r.stderr[-2000:])
            vendor = json.loads(r.stdout.strip().splitlines()[-1])
            for k, ms in vendor.items():
                if k in detail:
                    detail[k]["vendor_ms"] = ms
                    detail[k]["vendor_over_ours_at_shape"] = ms / detail[k]["at_shape_ms"]
                    log(f"{k:28s} vendor library {ms*1e3:9.2f} us per launch   ours at shape "
                        f"{detail[k]['at_shape_ms']*1e3:9.2f} us, amortised {detail[k]['amortised_ms']*1e3:9.2f} us")
        if args.detail:
            with open(args.detail, "w") as f:
                json.dump(detail, f, indent=1)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(I, budget_s=15.0)

    line = {
        "metric": "mm/conv GFLOP/s & % roofline; depthwise HBM GB/s; YOLO-N-shaped fp16 ms/frame",
        "value": round(value, 2), "unit": "GFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "aten.convolution im2col-GEMM fp32 NCHW batch 1: "
                               "[1,64,80,80]*[128,64,3,3] s1p1 + [1,128,80,80]*[256,128,3,3] s2p1",
                   "kernels": kernels, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if detail:
        line["detail"] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                              for kk, vv in d.items()} for k, d in detail.items()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
