import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


def _print_case(item):
    # name the case before any GPU work, so a run that ends abruptly still says where it was
    print(f"\n[case] {item.nodeid}", flush=True)


def pytest_runtest_setup(item):
    if item.get_closest_marker("gpu") is not None:
        _print_case(item)


@pytest.fixture(scope="session")
def ctx():
    import rust_trainer_amd as rt

    c = rt.Context(0)
    yield c
    c.close()
