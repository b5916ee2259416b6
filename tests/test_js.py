"""Runs the Node boundary tests (tests/js/*.test.js) under pytest.

The CPU leg drives the N-API addon on a host-only device (argument and shape
validation, buffers, program parsing); the GPU leg runs every JS test,
including the known-answer kernels, on GPU 0.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "wgpu-executorch_amd", "js", "wgx_napi.node")
NODE = shutil.which("node")

needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


def _run(flag):
    if not os.path.exists(ADDON):
        pytest.fail("wgx_napi.node is not built (run __graft_entry__.build())")
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "js", "run.js"), flag],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert " 0 failed" in r.stdout


@needs_node
def test_js_boundary_host_device():
    _run("--cpu")


@needs_node
@pytest.mark.gpu
def test_js_boundary_gpu():
    _run("--gpu")
