import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import moe_oracle

    return moe_oracle


@pytest.fixture(scope="session")
def moe():
    """The product package with its HIP library loaded (fails loudly if absent)."""
    import mixtureofexperts_amd as m

    m.lib()
    return m
