import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
# every test call checks that its slot ids are unique (a host sync the product path skips)
os.environ.setdefault("NSSM_CHECK_SLOTS", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libnssm_hip.so)")
