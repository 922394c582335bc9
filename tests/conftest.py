"""pytest configuration: the `gpu` marker, import paths, shared fixtures.

`-m "not gpu"` runs on any host (the oracle, host layouts, router, C-ABI exports).
`-m gpu` needs an MI355X; those tests call the library through its C ABI.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "mxfp6-gemm_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")
    config.addinivalue_line("markers", "slow: full-size benchmark shapes")


def pytest_collection_modifyitems(config, items):
    need_gpu = [it for it in items if "gpu" in it.keywords]
    if not need_gpu:
        return
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # torch missing: no GPU path at all
        has_gpu = False
    if not has_gpu:
        skip = pytest.mark.skip(reason="no GPU visible on this host")
        for it in need_gpu:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def mx():
    import mxfp6_amd
    mxfp6_amd.lib()
    return mxfp6_amd


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def ref_lib():
    import oracle
    r = oracle.ref()
    if r is None:
        pytest.skip("reference library oracle/_ref/libmxfp6ref.so not built")
    return r
