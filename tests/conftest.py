import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    # Run the cheap GPU layout probes before the end-to-end parity tests so a
    # wrong MFMA layout is reported by name first.
    def key(item):
        return 0 if "probe" in item.nodeid else 1
    items.sort(key=key)
