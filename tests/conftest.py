import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP engine through the C ABI")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


@pytest.fixture()
def golden_package(tmp_path):
    """The reference's frozen two-layer JFM v2 package, decoded from its hex fixture."""
    src = os.path.join(GOLDEN, "jfm-v2-golden")
    for name in os.listdir(src):
        if name.endswith(".hex"):
            text = open(os.path.join(src, name)).read()
            data = bytes.fromhex("".join(text.split()))
            (tmp_path / name[:-4]).write_bytes(data)
    return str(tmp_path)
