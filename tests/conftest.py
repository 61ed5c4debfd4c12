"""pytest configuration: markers, import paths, shared fixtures."""
import os
import sys

import pytest

TESTS = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(TESTS)
for p in (REPO, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    from oracle_bindings import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle_bindings import Ref
    if not Ref.available():
        pytest.skip("oracle/_ref not built (reference checkout not mounted)")
    return Ref()


@pytest.fixture(scope="session")
def tq4():
    import __graft_entry__
    return __graft_entry__.package()


def pytest_terminal_summary(terminalreporter):
    """Decode tolerance margins: achieved error as a fraction of its budget."""
    gh = sys.modules.get("gpu_helpers")
    rows = getattr(gh, "MARGINS", None) if gh else None
    if not rows:
        return
    tr = terminalreporter
    tr.section("decode tolerance margins (achieved / budget)")
    worst = sorted(rows, key=lambda r: -max(r[1] / r[3], r[2] / r[4]))
    fa = max(r[1] / r[3] for r in rows)
    fr = max(r[2] / r[4] for r in rows)
    tr.write_line(f"{len(rows)} comparisons; worst max-abs fraction {fa:.3f}, "
                  f"worst mean-rel fraction {fr:.3f}")
    for label, mx, mr, bx, br in worst[:25]:
        tr.write_line(f"  {label:<48s} max-abs {mx:.3e} ({mx / bx:6.3f})  "
                      f"mean-rel {mr:.3e} ({mr / br:6.3f})")
