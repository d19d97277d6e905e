"""pytest configuration: import paths and the `gpu` marker."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "vllm-ascend-hust-latchmoe_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible (gpu tests run on the MI355X box)")
    for it in gpu_items:
        it.add_marker(skip)


@pytest.fixture(autouse=True)
def _clear_device_flags(request):
    """GPU tests start with clear device status words: a test that drops
    pairs on purpose (masked combines, planted bad ids) must not make a
    later test's staging check fail."""
    if "gpu" in request.keywords:
        import torch

        if torch.cuda.is_available():
            from vllm_moe_offload_amd import native

            native.device_flags(clear=True)
    yield
