import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")
    config.addinivalue_line("markers", "ref: needs the compiled reference under oracle/_ref")


def pytest_collection_modifyitems(config, items):
    import oracle
    if not oracle.ref_available():
        skip = pytest.mark.skip(reason="compiled reference oracle/_ref not built here")
        for it in items:
            if "ref" in it.keywords:
                it.add_marker(skip)
