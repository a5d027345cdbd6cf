import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running case")


def pytest_terminal_summary(terminalreporter):
    """Worst attention errors of each test that compared against the oracle:
    max-abs, the bar's floored max-rel, and the unfloored max-rel over
    |ref| >= 1e-2, next to the largest |ref| for scale."""
    lib = sys.modules.get("slm_testlib")
    worst = getattr(lib, "WORST", None)
    if not worst:
        return
    tr = terminalreporter
    tr.write_sep("-", "attention errors vs the oracle (worst per test)")
    tr.write_line(f"{'test':84s} {'n':>5s} {'max-abs':>9s} {'max-rel':>9s} "
                  f"{'unfloored':>9s} {'max|ref|':>9s}")
    for test, w in sorted(worst.items()):
        tr.write_line(f"{test[-84:]:84s} {w['n']:5d} {w['max_abs']:9.2e} {w['max_rel']:9.2e} "
                      f"{w['max_rel_unfloored']:9.2e} {w['max_ref']:9.2e}")
