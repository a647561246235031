"""pytest configuration: import paths and the ``gpu`` marker.

GPU tests (``-m gpu``) run the HIP kernels through the C ABI on a ROCm device
and compare them with the CPU oracle; everything else runs on the CPU.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "sigma-0_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import pytest  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(params=["chunks", "walk", "segments"])
def bwd_route(request, monkeypatch):
    """Runs a backward test on every route of the library's backward: the
    chunk-parallel kernels, the reverse walk, and the walk split into sequence
    segments (forced here down to segments of two chunks, so that the short test
    sequences split too); the library reads M3_BWD_ROUTE at each call; unset, it
    picks by B * H and the length."""
    monkeypatch.setenv("M3_BWD_ROUTE", request.param)
    return request.param
