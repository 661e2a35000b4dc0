import os
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    # Tuning measures plans on the GPU and persists its decisions: keep the suite's plans the
    # planner's (deterministic), and any decision a test makes out of the user's cache.
    os.environ.setdefault("METILE_AMD_DISABLE_TUNING", "1")
    os.environ["METILE_AMD_CACHE_DIR"] = tempfile.mkdtemp(prefix="metile_amd_cache_")
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running case")
