"""Measured forward errors, recorded by the GPU parity tests and printed at the
end of the pytest run (tests/conftest.py: pytest_terminal_summary), so that a
run's output shows the error envelope of every configuration it checked, not
only pass or fail (the reference prints O_diff and L_diff per config,
tests/test_fa3_db_full.py:47-49)."""

RECORDS = []


def record(tag, o_maxabs, l_maxrel=None, note=""):
    RECORDS.append((str(tag), float(o_maxabs), None if l_maxrel is None else float(l_maxrel), note))


def summary_lines():
    if not RECORDS:
        return []
    out = [f"forward error envelope ({len(RECORDS)} checks): O max-abs vs the oracle, "
           f"L max-rel = max |L - L_ref| / max(|L_ref|, 1)"]
    worst_o = max(r[1] for r in RECORDS)
    ls = [r[2] for r in RECORDS if r[2] is not None]
    for tag, o, l, note in RECORDS:
        ltxt = "" if l is None else f"  L max-rel {l:.2e}"
        out.append(f"  {tag}: O max-abs {o:.3e}{ltxt}{('  ' + note) if note else ''}")
    out.append(f"  worst: O max-abs {worst_o:.3e}, L max-rel {max(ls) if ls else float('nan'):.2e}")
    return out
