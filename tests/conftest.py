import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "stream-mm2026_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")
    config.addinivalue_line("markers", "slow: long CPU test")


def pytest_terminal_summary(terminalreporter):
    """The parameter error report of the GPU parity comparisons (tests/param_bar.py)."""
    mod = sys.modules.get("param_bar")
    if mod is None or not mod.RECORDS:
        return
    recs = mod.RECORDS
    n = sum(s["n"] for _, s in recs)
    ident = sum(s["identical"] * s["n"] for _, s in recs) / max(n, 1)
    over = sum(s["share_rel_over_1e6"] * s["n"] for _, s in recs)
    ratios = [s["min_update_ratio_over"] for _, s in recs if s["min_update_ratio_over"] is not None]
    tr = terminalreporter
    tr.section("parameter error vs the oracle (bar |dp| <= 2^-20 |update| + 2^-22 |p'|)")
    zero = sum(s.get("zero_target", 0) for _, s in recs)
    tr.write_line(f"{len(recs)} comparisons, {n:,} elements: {100 * ident:.3f} % bit-identical, "
                  f"max {max(s['max_ulps'] for _, s in recs)} ulp, max |dp|/|p'| (p' != 0) "
                  f"{max(s['rel_max'] for _, s in recs):.2e}, max bar use {max(s['bar_use'] for _, s in recs):.3f}")
    if zero:
        tr.write_line(f"p' = 0 in the oracle with dp != 0: {zero:,} elements, max |dp| "
                      f"{max(s.get('zero_target_max_abs', 0.0) for _, s in recs):.2e} (within the bar's update term)")
    tr.write_line(f"elements above 1e-6 relative: {int(round(over)):,} ({100 * over / max(n, 1):.4f} %), "
                  f"every one with |update| >= {min(ratios) if ratios else float('nan'):.2f} |p'| "
                  f"(a step through or next to zero)")
    worst = sorted(recs, key=lambda r: -r[1]["share_rel_over_1e6"])[:5]
    for label, s in worst:
        tr.write_line("  " + mod.format_stats(s, label))
