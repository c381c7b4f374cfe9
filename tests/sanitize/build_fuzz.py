"""Build tests/sanitize/host_plan_fuzz.cpp against the library source with
AddressSanitizer and UndefinedBehaviorSanitizer on the host code only (every
sanitizer flag goes through -Xarch_host; the GPU code is built as usual and
never launched), into tests/sanitize/_build/host_plan_fuzz.  Any sanitizer
report aborts the run (-fno-sanitize-recover).  CPU only."""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from f16acc_amd import build as libbuild  # noqa: E402

FUZZ_SRC = os.path.join(HERE, "host_plan_fuzz.cpp")
FUZZ = os.path.join(HERE, "_build", "host_plan_fuzz")
HOST_SANITIZE = []
for flag in ("-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"):
    HOST_SANITIZE += ["-Xarch_host", flag]


def stale():
    if not os.path.exists(FUZZ):
        return True
    built = os.path.getmtime(FUZZ)
    srcs = (libbuild.SRC, FUZZ_SRC, os.path.join(libbuild.INCLUDE, "f16acc.h"))
    return any(os.path.getmtime(s) > built for s in srcs)


def build(force=False):
    """Compile the fuzz driver when it is missing or older than its sources."""
    if not force and not stale():
        return FUZZ
    os.makedirs(os.path.dirname(FUZZ), exist_ok=True)
    cmd = [libbuild.hipcc(), *libbuild.COMMON_FLAGS, "-g", *HOST_SANITIZE, "-I", libbuild.INCLUDE, libbuild.SRC,
           FUZZ_SRC, "-o", FUZZ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("sanitizer build failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    return FUZZ


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
