import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libmi_sdvk.so")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device. On a GPU run a missing device or library is a failure,
    never a skip: the product path has no fallback."""
    from sdvk_amd import _lib, hip

    n = hip.device_count()
    assert n >= 1, "no HIP device visible"
    lib = _lib.load()
    name = hip.device_name(0)
    print(f"[gpu] device 0: {name}; libmi_sdvk version {lib.mi_version()}", flush=True)
    return lib


@pytest.fixture(scope="session")
def oracle():
    from oracle import binding

    binding.lib()
    return binding


def pytest_terminal_summary(terminalreporter):
    """Worst parity error per test function (max |err| over its checks,
    relative to RMS of the reference, and the share of its bar it used), so
    the margins show in a -q run's record."""
    from helpers import WORST

    if not WORST:
        return
    tr = terminalreporter
    tr.write_sep("-", "parity margins: worst max|err| / RMS per test function")
    for key, (e, tol, test) in sorted(WORST.items()):
        case = test.split("::")[-1]
        tr.write_line(f"{key:<64} {e:.3e}  bar {tol:.1e}  ({100 * e / tol:5.1f}% of the bar)  {case}")


@pytest.fixture
def tune(gpu):
    """tune(name, value): a plan override through mi_tuning_set for this test
    (value None clears it); every override is cleared when the test ends."""
    from sdvk_amd import ops

    ops.tuning_reset()
    yield ops.tuning_set
    ops.tuning_reset()
