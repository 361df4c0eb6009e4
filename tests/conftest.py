import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "mhc-mlx_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libmhc_hip.so")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible (torch.cuda.is_available() is False)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _hip_path_did_not_fall_back(request):
    """A GPU test must not pass on the module's reference fallback.

    MHCLayer / MHCRewire hand a call to the torch reference path (with one
    warning) when the HIP path raises or gets CPU tensors; the module flag
    records it.  Every test marked ``gpu`` starts with the flag clear and
    fails if it is set at the end, so parity evidence always comes from the
    library.  A test that exercises the fallback on purpose restores the
    flag with ``monkeypatch`` (undone before this check runs).
    """
    if "gpu" not in request.keywords:
        yield
        return
    from mhc_mlx_amd import layer as L

    L._METAL_FAILED = False
    yield
    assert not L._METAL_FAILED, "the HIP path fell back to the torch reference path during this GPU test"


@pytest.fixture
def knobs():
    """Set libmhc_hip launch-shape knobs for one test: ``knobs(name, value)``.

    Every knob of the library's table is restored when the test ends.
    """
    from mhc_mlx_amd import _lib

    saved = {name: _lib.get_knob(name) for name in _lib.knob_names()}
    yield _lib.set_knob
    for name, value in saved.items():
        _lib.set_knob(name, value)
