"""Parity bookkeeping of the GPU tests: a case's per-tensor errors against its bars, checked, printed with the worst
margin, kept for the run's closing summary (tests/conftest.py prints every case's worst error / bar, the largest
last), and appended as one JSON line to the file that MACAI_PARITY_LOG names -- gpurun_out/parity.jsonl under the
repository root when it is unset (the reference's parity log, tests/test_chunking.py:15-16, 52-55) -- so a run records
how close to its bar every case came, not only pass or fail."""
import json
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LOG = os.environ.get("MACAI_PARITY_LOG") or os.path.join(ROOT, "gpurun_out", "parity.jsonl")
RECORDS = []     # (case, worst tensor, its error / bar, its error, its bar) of every check in this process


def _case():
    """The running test's id (pytest sets PYTEST_CURRENT_TEST to '<nodeid> (call)')."""
    return os.environ.get("PYTEST_CURRENT_TEST", "?").rsplit(" ", 1)[0]


def check(errs: dict, bars, case: str = None, **extra):
    """Assert every errs[name] <= its bar (bars: one number or {name: bar}); print each error and the worst
    error / bar ratio; keep the worst in RECORDS; append {"case", "errors", "bars", "worst", "worst_of_bar", **extra} to
    LOG."""
    case = case or _case()
    if not isinstance(bars, dict):
        bars = {n: bars for n in errs}
    frac = {n: (errs[n] / bars[n] if bars[n] > 0 else float("inf")) for n in errs}
    worst = max(frac, key=frac.get) if frac else None
    print(f"{case}: errors", {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    if worst is not None:
        print(f"{case}: worst margin {worst} at {frac[worst]:.3f} of its bar {bars[worst]:.2e}", flush=True)
        RECORDS.append((case, worst, frac[worst], errs[worst], bars[worst]))
    rec = {"case": case, "errors": errs, "bars": bars, "worst": worst,
           "worst_of_bar": None if worst is None else frac[worst], **extra}
    try:
        os.makedirs(os.path.dirname(LOG) or ".", exist_ok=True)
        with open(LOG, "a", encoding="utf-8") as fh:
            fh.write(json.dumps(rec) + "\n")
    except OSError as e:           # the log is a record, never a reason to fail a parity check
        print(f"parity log {LOG} not written: {e}", flush=True)
    bad = {n: (errs[n], bars[n]) for n in errs if not errs[n] <= bars[n]}
    assert not bad, f"{case}: (error, bar) over the bar: {bad}"
    return frac
