import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "brisk-llm_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libbrisk_hip.so on cuda:0)")
    config.addinivalue_line("markers", "slow: full-size model (seconds to minutes)")


@pytest.fixture(scope="session")
def oracle_lib():
    import pyoracle
    return pyoracle.oracle_lib()
