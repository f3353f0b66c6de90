import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def tuning():
    """set(name, value) of a planner override (braidinfer_amd._lib.set_tuning)
    for one test; every override it touched is restored afterwards."""
    from braidinfer_amd import _lib
    saved = {}

    def set_(name, value):
        if name not in saved:
            saved[name] = _lib.get_tuning(name)
        _lib.set_tuning(name, value)

    yield set_
    for name, value in saved.items():
        _lib.set_tuning(name, value)


def pytest_terminal_summary(terminalreporter):
    """Lists how many elements each documented rounding allowance admitted
    (tests/helpers.py ALLOWANCE_LOG), per check, when any test used one."""
    from tests.helpers import ALLOWANCE_LOG
    if not ALLOWANCE_LOG:
        return
    used = [(w, u, n) for w, u, n in ALLOWANCE_LOG if u]
    terminalreporter.write_sep("-", f"rounding allowances: {len(ALLOWANCE_LOG)} checks offered one, "
                                    f"{len(used)} used it")
    for what, u, n in used:
        terminalreporter.write_line(f"  {what}: {u} of {n} elements beyond the strict bound")
