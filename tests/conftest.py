"""Shared pytest setup: markers and import paths.

``gpu``-marked tests need an MI355X and the built ``libmemopt_hip.so``; the
rest run on CPU. The package directory (holding the ``memopt_C`` shim) and
``oracle/`` are put on ``sys.path``.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "memopt-transformer-runtime_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(autouse=True)
def _fresh_pool(request):
    """Every GPU test starts without a pool. init_pool keeps a live pool of
    identical parameters (the reference's idempotence), so a test that expects
    untouched pages would otherwise see the pages of whichever test ran before
    it with the same parameters, and pass or fail with the order of the run."""
    if request.node.get_closest_marker("gpu") is not None:
        import memopt_C

        memopt_C.reset_pool()
    yield
