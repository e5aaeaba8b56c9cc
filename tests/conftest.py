import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as O
    O.lib()
    return O

REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libpicolm_ref.so")
needs_ref = pytest.mark.skipif(not os.path.exists(REF_LIB),
                               reason="reference harness not built (make -C oracle ref)")


@pytest.fixture(scope="session")
def gpu():
    """The product library on device 0 (tests marked gpu only)."""
    import picolm_amd as P
    if P.lib.plh_device_count() < 1:
        pytest.fail("no HIP device visible: gpu tests need an MI355X")
    P.init(0)
    return P
