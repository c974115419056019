import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def pytest_sessionfinish(session, exitstatus):
    """Writes the parity figures the tests recorded (model_parity.REPORT) as
    JSON lines to the file KDEC_PARITY_REPORT names, if any."""
    path = os.environ.get("KDEC_PARITY_REPORT")
    mp = sys.modules.get("model_parity")
    if not path or mp is None or not mp.REPORT:
        return
    import json
    with open(path, "a") as f:
        for row in mp.REPORT:
            f.write(json.dumps(row, default=float) + "\n")
