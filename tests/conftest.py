import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


@pytest.fixture(autouse=True)
def _single_rank_env(monkeypatch):
    for key in ("RANK", "WORLD_SIZE", "LOCAL_RANK", "MINISPEED_DEVICE", "MINISPEED_BACKEND"):
        monkeypatch.delenv(key, raising=False)
