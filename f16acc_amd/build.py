"""Build the HIP library libf16acc_amd.so for gfx950 with hipcc, in-tree.

    python f16acc_amd/build.py

The library is the whole native part of the package: kernels, per-shape tile
table and the C ABI declared in include/f16acc.h.
"""

import os
import shutil
import subprocess
import sys
import tempfile

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
SRC = os.path.join(PKG, "csrc", "f16acc_gemm.hip")
CHUNKRATE_SRC = os.path.join(PKG, "csrc", "chunkrate.hip")
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(PKG, "_build")
LIB = os.path.join(OUT_DIR, "libf16acc_amd.so")
CHUNKRATE = os.path.join(OUT_DIR, "chunkrate")  # MFMA / chunk-epilogue microbenchmark
ARCH = "gfx950"

# -packed-fp32-ops: hipcc may otherwise fuse FP32 pairs into v_pk_* ops
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wextra",
]
HIP_FLAGS = COMMON_FLAGS + ["-fPIC", "-shared"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise FileNotFoundError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def _compile(flags, src, out, verbose):
    """hipcc src -> out; the previous output is replaced atomically."""
    os.makedirs(OUT_DIR, exist_ok=True)
    fd, tmp = tempfile.mkstemp(suffix=".tmp", dir=OUT_DIR)
    os.close(fd)
    cmd = [hipcc(), *flags, "-I", INCLUDE, src, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        os.unlink(tmp)
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    if verbose:
        noise = ("packed-fp32-ops", "warning generated", "warnings generated")
        msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if not any(n in ln for n in noise)]
        if msgs:
            print("\n".join(msgs), file=sys.stderr)
    os.chmod(tmp, 0o755)
    os.replace(tmp, out)
    return out


def build(verbose=False):
    """Compile the library and the chunkrate microbenchmark."""
    _compile(COMMON_FLAGS, CHUNKRATE_SRC, CHUNKRATE, verbose)
    return _compile(HIP_FLAGS, SRC, LIB, verbose)


if __name__ == "__main__":
    print(build(verbose=True))
