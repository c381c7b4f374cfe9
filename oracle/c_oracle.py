"""Oracle (test infrastructure): ctypes binding of oracle/chunk32.c, the
scalar C restatement of the reference's chunk-32 GEMM (f16acc/kernel.py:37-105).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
"""

import ctypes
import os
import subprocess

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle_chunk32.so")
_lib = None


def build():
    """Compile the C restatement with gcc (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise FileNotFoundError(f"{LIB} is not built: run `make -C oracle`")
        lib = ctypes.CDLL(LIB)
        i64, vp = ctypes.c_int64, ctypes.c_void_p
        lib.oracle_mm.argtypes = [vp, vp, vp, vp] + [i64] * 9 + [ctypes.c_int, ctypes.c_int, i64, i64, i64, ctypes.c_int]
        lib.oracle_mm.restype = ctypes.c_int
        lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_f16.restype = ctypes.c_uint16
        lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.oracle_f16_to_f32.restype = ctypes.c_float
        _lib = lib
    return _lib


def mm(a16, b16, out_dtype=torch.float16, chunked=True, tile=(256, 256), mode="round_once",
       chunk=32, return_flags=False):
    """Same contract as oracle.chunk32.mm, evaluated by the scalar C code in a
    fixed sequential order.  Any strides of a16 / b16 are passed through."""
    lib = load()
    a16, b16 = a16.cpu(), b16.cpu()
    M, K = a16.shape
    N = b16.shape[1]
    bm, bn = tile
    c = torch.empty(M, N, dtype=out_dtype)
    flags = torch.zeros((M + bm - 1) // bm, (N + bn - 1) // bn, dtype=torch.uint8)
    rc = lib.oracle_mm(a16.data_ptr(), b16.data_ptr(), c.data_ptr(), flags.data_ptr(),
                       M, N, K, a16.stride(0), a16.stride(1), b16.stride(0), b16.stride(1),
                       c.stride(0), c.stride(1), int(out_dtype == torch.float32), int(chunked),
                       bm, bn, chunk, {"round_once": 0, "per_k16": 1}[mode])
    if rc != 0:
        raise ValueError("oracle_mm rejected its arguments")
    return (c, flags) if return_flags else c
