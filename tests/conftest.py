import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built HIP library")


def load_fixtures():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "cascade_fixtures.json")) as f:
        return json.load(f)
