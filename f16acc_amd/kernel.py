"""The chunked FP16 GEMM op: `mm(a, b)` on HIP devices.

Host side of the reference's f16acc/kernel.py:84-105 (`mm`): the same
arguments, the same ValueError checks before any launch, a freshly allocated
contiguous output, and no synchronisation.  The Triton `_gemm` / `_redo`
launches are replaced by one call into libf16acc_amd.so (f16acc_gemm), which
runs the main pass and the FP32 redo of overflowing tiles in one kernel on
the current stream.
"""

import ctypes

import torch

from . import _lib

_OUT = {torch.float16: _lib.OUT_F16, torch.float32: _lib.OUT_F32}


def _validate(a, b, out_dtype):
    """Real checks, not asserts (python -O keeps them): a wrong shape or dtype
    would let the kernel read past the end of b (kernel.py:85-90)."""
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"mm needs (M, K) @ (K, N), got {tuple(a.shape)} @ {tuple(b.shape)}")
    if a.dtype != torch.float16 or b.dtype != torch.float16 or not (a.is_cuda and b.is_cuda) or a.device != b.device:
        raise ValueError("mm needs fp16 GPU tensors on the same device")
    if out_dtype not in _OUT:  # the reference does not check this; anything else would be misread
        raise ValueError(f"mm writes torch.float16 or torch.float32, not {out_dtype}")


def mm(a, b, out_dtype=torch.float16, chunked=True):
    """c = a @ b for fp16 a [M, K] and b [K, N] of any strides on one HIP device.

    out_dtype: torch.float16 (default) or torch.float32.
    chunked:   True  -> 32-long K chunks rounded to fp16 and added into an FP32
                        sum, tiles with an inf/NaN sum redone in FP32
               False -> plain FP32 accumulation
    Raises ValueError for bad shapes, dtypes or devices (kernel.py:87-90).
    """
    _validate(a, b, out_dtype)
    M, K = a.shape
    N = b.shape[1]
    c = torch.empty(M, N, device=a.device, dtype=out_dtype)
    if M == 0 or N == 0:
        return c
    _launch(a, b, c, None, M, N, K, chunked)
    return c


def mm_flags(a, b, out_dtype=torch.float16, chunked=True):
    """mm plus the per-tile redo flags (uint8 [tiles_m, tiles_n]): 1 where the
    tile's chunked FP32 sum held inf/NaN and was recomputed in FP32.  Same
    checks as mm; used by tests and benches to see which tiles were redone."""
    _validate(a, b, out_dtype)
    M, K = a.shape
    N = b.shape[1]
    cfg = tile_config(a, b)
    c = torch.empty(M, N, device=a.device, dtype=out_dtype)
    flags = torch.zeros(cfg["tiles_m"], cfg["tiles_n"], device=a.device, dtype=torch.uint8)
    if M and N:
        _launch(a, b, c, flags, M, N, K, chunked)
    return c, flags


def tile_config(a, b):
    """The per-shape tile choice the library makes for a @ b (replaces the
    reference's autotuned best_config, kernel.py:16-19, 101-102)."""
    M, K = a.shape
    N = b.shape[1]
    bm, bn, fam, thr = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    tm, tn = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(_lib.tile_config(M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
                                a.data_ptr(), b.data_ptr(), ctypes.byref(bm), ctypes.byref(bn),
                                ctypes.byref(tm), ctypes.byref(tn), ctypes.byref(fam), ctypes.byref(thr)))
    return {"bm": bm.value, "bn": bn.value, "tiles_m": tm.value, "tiles_n": tn.value,
            "family": ("fast", "generic")[fam.value], "threads": thr.value}


def _launch(a, b, c, flags, M, N, K, chunked):
    dev = a.device
    if torch.cuda.current_device() != dev.index:
        with torch.cuda.device(dev):
            return _launch(a, b, c, flags, M, N, K, chunked)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = _lib.gemm(a.data_ptr(), b.data_ptr(), c.data_ptr(), flags.data_ptr() if flags is not None else None,
                   M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1),
                   _OUT[c.dtype], int(bool(chunked)), stream)
    _lib.check(rc)
