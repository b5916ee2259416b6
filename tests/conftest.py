import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def kats():
    with open(os.path.join(ROOT, "tests", "golden", "reference_kats.json")) as f:
        return json.load(f)["cases"]


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


def load_pkg():
    from __graft_entry__ import load_package

    return load_package()


@pytest.fixture(scope="session")
def pkg():
    """The product package; its ops run only through libwgx.so."""
    return load_pkg()


@pytest.fixture(scope="session")
def gpu_ctx(pkg):
    ctx = pkg.wgx.Context(0)
    assert ctx.has_device and ctx.arch == "gfx950", ctx.arch
    yield ctx
    ctx.destroy()
