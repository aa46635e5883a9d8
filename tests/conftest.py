"""Shared test setup: the `gpu` marker and the repo root on sys.path.

GPU tests call libpanmuon through its C ABI on a real MI355X; run them with
`pytest -m gpu`. Without a HIP device they are skipped, never faked.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (HIP device) and the built libpanmuon.so")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no HIP device in this container")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


# torch's stock Muon functions, captured before any test installs the HIP path
# (patch_muon replaces these module globals for the rest of the process).
import torch.optim._muon as _torch_muon  # noqa: E402

TORCH_ZEROPOWER = _torch_muon._zeropower_via_newtonschulz
TORCH_SINGLE_TENSOR_MUON = _torch_muon._single_tensor_muon


@pytest.fixture
def torch_stock_muon():
    """Run a block with torch's stock Muon functions installed, restoring after."""
    import contextlib

    @contextlib.contextmanager
    def stock():
        saved = (_torch_muon._zeropower_via_newtonschulz, _torch_muon._single_tensor_muon)
        _torch_muon._zeropower_via_newtonschulz = TORCH_ZEROPOWER
        _torch_muon._single_tensor_muon = TORCH_SINGLE_TENSOR_MUON
        try:
            yield
        finally:
            _torch_muon._zeropower_via_newtonschulz, _torch_muon._single_tensor_muon = saved

    return stock

# torch's own fused Adam, captured before patch_adamw replaces the module global
import torch.optim.adam as _torch_adam  # noqa: E402

TORCH_FUSED_ADAM = _torch_adam._fused_adam


@pytest.fixture
def torch_fused_adam():
    """Run a block with torch's own fused Adam installed, restoring after."""
    import contextlib

    @contextlib.contextmanager
    def stock():
        saved = _torch_adam._fused_adam
        _torch_adam._fused_adam = TORCH_FUSED_ADAM
        try:
            yield
        finally:
            _torch_adam._fused_adam = saved

    return stock


@pytest.fixture(autouse=True)
def _restore_patch_muon_switches():
    """Restores the drop-in's module switches (NS_FORM, WORKSPACE_LIMIT) after
    every test, whatever the test set them to."""
    import pan2_amd.optim.patch_muon as pm

    saved = (pm.NS_FORM, pm.WORKSPACE_LIMIT)
    yield
    pm.NS_FORM, pm.WORKSPACE_LIMIT = saved
