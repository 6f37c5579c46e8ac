import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.build()
    oracle.set_threads(1)
    return oracle


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Totals of the gradient criterion over the session: entries compared,
    entries outside rtol 1e-4 / atol 1e-5 that their float32 error bound
    accepted, and the largest error/bound ratio among those."""
    pipeline = sys.modules.get("oracle_pipeline")
    checks = getattr(pipeline, "GRADIENT_CHECKS", None)
    if not checks:
        return
    entries = sum(c["n"] for c in checks)
    outside = sum(c["outside_tolerance"] for c in checks)
    failed = sum(c["outside_bound"] for c in checks)
    ratio = max(c["max_err_over_bound"] for c in checks)
    terminalreporter.write_line(
        f"gradient criterion: {len(checks)} checks, {entries} entries; {outside} outside rtol 1e-4/atol 1e-5, "
        f"all but {failed} of them within their float32 bound (max err/bound {ratio:.3f})")
