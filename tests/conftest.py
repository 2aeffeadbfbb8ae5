import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "mac-ai-engineering_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device; run with -m gpu")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Every parity check's worst error as a fraction of its bar (tests/_parity.py), the closest to its bar last, and
    the run's worst overall: the margins reach the tail of the output that a driver keeps."""
    mod = sys.modules.get("_parity")
    recs = getattr(mod, "RECORDS", None)
    if not recs:
        return
    tr = terminalreporter
    tr.section(f"parity margins: worst error / bar of {len(recs)} checks (closest last)")
    for case, name, frac, err, bar in sorted(recs, key=lambda r: r[2]):
        tr.write_line(f"{frac:6.3f}  {name:>7} {err:.2e} / {bar:.2e}  {case}")
    case, name, frac, err, bar = max(recs, key=lambda r: r[2])
    tr.write_line(f"worst of the run: {name} at {frac:.3f} of its bar ({err:.2e} / {bar:.2e}) in {case}; "
                  f"log {mod.LOG}")
