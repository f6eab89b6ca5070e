import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "quant-lib_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on cuda:0)")


@pytest.fixture(autouse=True)
def _announce_gpu_case(request):
    # Name the case before any GPU work so a run that dies mid-test still says which one.
    if request.node.get_closest_marker("gpu") is not None:
        sys.stderr.write(f"\n[gpu-case] {request.node.nodeid}\n")
        sys.stderr.flush()
    yield
