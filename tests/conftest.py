import faulthandler
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# A test that runs longer than this is taken to be hung: every thread's stack
# is printed (naming the test and where it sits) and the process exits, so a
# hang ends the run early instead of consuming the caller's whole time limit.
WATCHDOG_S = float(os.environ.get("POCR_TEST_WATCHDOG_S", "300"))

# Thread count of the oracle's worker pool in the test processes. Above one,
# every parallel oracle path (row-split matvecs, head-split attention) runs
# through the pool; results do not depend on the count.
ORACLE_THREADS = int(os.environ.get("POCR_ORACLE_THREADS", "4"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X")


@pytest.fixture(autouse=True)
def _hang_watchdog(request):
    if WATCHDOG_S > 0:
        faulthandler.dump_traceback_later(WATCHDOG_S, exit=True)
    yield
    if WATCHDOG_S > 0:
        faulthandler.cancel_dump_traceback_later()


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    oracle.set_threads(ORACLE_THREADS)
    return oracle


@pytest.fixture(scope="session")
def ctx():
    from rapidocrvl_amd import lib

    c = lib.Context(0)
    yield c
    c.close()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
