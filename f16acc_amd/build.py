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
# The same source with the tile flag and FP32 redo compiled out
# (-DF16ACC_NO_REDO=1): only bench.py's redo-overhead A/B loads it.
LIB_NOREDO = os.path.join(OUT_DIR, "libf16acc_amd_noredo.so")
# ... and with the split redo in place of the in-kernel one for 256x256
# (-DF16ACC_SPLIT_REDO=1): only bench.py's overflow workload loads it.
LIB_SPLITREDO = os.path.join(OUT_DIR, "libf16acc_amd_splitredo.so")
# ... and with multi-round shapes on the one-tile-per-workgroup grid instead
# of the persistent kernel (-DF16ACC_NO_PERSISTENT=1): only bench.py's
# persistent A/B loads it.
LIB_NOPERSIST = os.path.join(OUT_DIR, "libf16acc_amd_nopersist.so")
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


def _start(flags, src, out):
    """Start hipcc src -> a temporary file next to out."""
    os.makedirs(OUT_DIR, exist_ok=True)
    fd, tmp = tempfile.mkstemp(suffix=".tmp", dir=OUT_DIR)
    os.close(fd)
    cmd = [hipcc(), *flags, "-I", INCLUDE, src, "-o", tmp]
    return cmd, tmp, out, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _finish(job, verbose):
    """Wait for a hipcc job; the previous output is replaced atomically."""
    cmd, tmp, out, proc = job
    text, _ = proc.communicate()
    if proc.returncode != 0:
        os.unlink(tmp)
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + text)
    if verbose:
        noise = ("packed-fp32-ops", "warning generated", "warnings generated")
        msgs = [ln for ln in text.splitlines() if not any(n in ln for n in noise)]
        if msgs:
            print("\n".join(msgs), file=sys.stderr)
    os.chmod(tmp, 0o755)
    os.replace(tmp, out)
    return out


def build(verbose=False):
    """Compile the library, its no-redo, split-redo and no-persistent twins
    and the chunkrate microbenchmark (five hipcc processes at once)."""
    jobs = [_start(HIP_FLAGS, SRC, LIB), _start(HIP_FLAGS + ["-DF16ACC_NO_REDO=1"], SRC, LIB_NOREDO),
            _start(HIP_FLAGS + ["-DF16ACC_SPLIT_REDO=1"], SRC, LIB_SPLITREDO),
            _start(HIP_FLAGS + ["-DF16ACC_NO_PERSISTENT=1"], SRC, LIB_NOPERSIST),
            _start(COMMON_FLAGS, CHUNKRATE_SRC, CHUNKRATE)]
    errors = []
    for job in jobs:
        try:
            _finish(job, verbose)
        except RuntimeError as e:
            errors.append(str(e))
    if errors:
        raise RuntimeError("\n".join(errors))
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
