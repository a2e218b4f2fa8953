import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "qwen3.5-cpu-cpp_amd"), os.path.join(ROOT, "oracle"),
          os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    # A GPU test on a host without a device is skipped, never run on a fallback path.
    if not any("gpu" in item.keywords for item in items):
        return
    import helpers

    if helpers.gpu_count() > 0:
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def model_dirs(tmp_path_factory):
    """Synthetic checkpoints (seed 0, std 0.02) of the small named shapes, written once."""
    import pyq35

    base = tmp_path_factory.mktemp("models")
    out = {}
    for name in ("tiny", "tiny_gqa", "tiny_untied"):
        d = str(base / name)
        pyq35.synth_write_model(d, pyq35.dims_for(name), seed=0, std=0.02)
        out[name] = d
    return out
