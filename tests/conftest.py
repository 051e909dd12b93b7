import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def ggml():
    from openasr_amd import ggml as g
    g.base()
    return g


@pytest.fixture(scope="session")
def gpu(ggml):
    """The MI355X plugin loaded through the verified loader. Fails (never
    skips) when the plugin or the device is missing: a GPU test must not
    pass on a fallback."""
    return ggml.plugin()


@pytest.fixture(scope="session")
def ref():
    from oracle import ref as r
    r.lib()
    return r
