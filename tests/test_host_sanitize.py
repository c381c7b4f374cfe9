"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer
(no GPU): tests/sanitize/host_plan_fuzz.cpp drives the C ABI's planning entry
points (tile configuration, workspace size, ragged-round cut, block -> tile
map) and the launching entry points' argument checks over seeded random
shapes, strides and alignments, every forced tile included; a sanitizer
report or a result off the documented contract fails the run.  The driver is
built (about three minutes, once) by tests/sanitize/build_fuzz.py when
missing or older than its sources."""

import os
import subprocess
import sys


def test_host_planning_under_address_and_undefined_behaviour_sanitizers():
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize"))
    import build_fuzz

    fuzz = build_fuzz.build()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([fuzz, "4000"], capture_output=True, text=True, timeout=600, env=env)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "host_plan_fuzz: 4000 problems, 0 mismatches" in res.stdout, out[-4000:]
    # the draws reach every family, most tiles, split-K and header workspaces and both cuts
    import re

    picks = [int(x) for x in re.search(r"table picks by tile:((?: \d+)+)", res.stdout).group(1).split()]
    fams = [int(x) for x in re.search(r"families fast/generic/reg: (\d+) (\d+) (\d+)", res.stdout).groups()]
    ws = [int(x) for x in re.search(r"workspace none/header/split: (\d+) (\d+) (\d+)", res.stdout).groups()]
    cuts = [int(x) for x in re.search(r"cuts by columns/rows: (\d+) (\d+)", res.stdout).groups()]
    assert sum(p > 0 for p in picks) >= 6 and all(f > 0 for f in fams) and all(w > 0 for w in ws), res.stdout
    assert sum(cuts) > 0, res.stdout
