"""Worst parity error of every GPU test, collected while the tests run and printed at the end of
the session by tests/conftest.py (pytest_terminal_summary), so that the margins to each bound
appear in the run's output instead of only in captured test output. No torch import here: the
CPU suite's conftest loads it too."""
import os

# test id -> {"err", "bound", "dtype", "uniform", "checks", "what"}
RECORDS = {}


def current_test() -> str:
    """The running test's node id without pytest's " (call)" suffix."""
    return os.environ.get("PYTEST_CURRENT_TEST", "?").rsplit(" (", 1)[0]


def record(err: float, bound: float, dtype: str, uniform: float = None, what: str = "") -> None:
    """Keep the worst `err` (in units of the bound's metric) seen by the running test."""
    tid = current_test()
    r = RECORDS.get(tid)
    if r is None:
        RECORDS[tid] = r = {"err": err, "bound": bound, "dtype": dtype, "uniform": uniform, "checks": 0,
                            "what": what}
    elif not err <= r["err"]:          # NaN counts as worse than anything
        r.update(err=err, bound=bound, dtype=dtype, uniform=uniform, what=what or r["what"])
    r["checks"] += 1


def _fmt(x):
    return "n/a" if x is None else f"{x:.2e}"


def summary_lines():
    """Per test function (parametrizations folded), then one line per dtype, then the named
    full-size workloads last."""
    if not RECORDS:
        return []
    per_fn = {}
    for tid, r in RECORDS.items():
        fn = tid.split("[", 1)[0].replace("tests/", "")
        key = (fn, r["dtype"])
        w = per_fn.get(key)
        if w is None or not r["err"] <= w["err"]:
            per_fn[key] = dict(r, cases=(w["cases"] if w else 0) + 1, tid=tid)
        else:
            w["cases"] += 1
    lines = ["parity (worst over each test's checks; err = max |gpu-ref|/max(1,|ref|), for bf16 outputs net of "
             "half a bf16 ulp of ref; 'uniform' = the same without that term):"]
    for (fn, dt), w in sorted(per_fn.items()):
        lines.append(f"  {fn:<78s} {dt:<5s} err {_fmt(w['err'])} <= {w['bound']:.0e}  uniform {_fmt(w['uniform'])}"
                     f"  ({w['cases']} cases)")
    by_dtype = {}
    for tid, r in RECORDS.items():
        w = by_dtype.get(r["dtype"])
        if w is None or not r["err"] <= w["err"]:
            by_dtype[r["dtype"]] = dict(r, tid=tid)
    n = sum(r["checks"] for r in RECORDS.values())
    lines.append(f"parity summary: {n} checks in {len(RECORDS)} test cases")
    for dt, w in sorted(by_dtype.items()):
        lines.append(f"  worst {dt}: err {_fmt(w['err'])} (bound {w['bound']:.0e}, uniform {_fmt(w['uniform'])}) in "
                     f"{w['tid'].replace('tests/', '')}")
    for tid, r in sorted(RECORDS.items()):
        if r["what"]:
            lines.append(f"  {r['what']}: err {_fmt(r['err'])} <= {r['bound']:.0e} (uniform {_fmt(r['uniform'])})")
    return lines
