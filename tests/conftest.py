import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


def pytest_sessionfinish(session, exitstatus):
    path = os.environ.get("DCN2_PARITY_LOG")
    if not path:
        return
    import json

    from util import PARITY_LOG
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        json.dump(PARITY_LOG, f, indent=0)
