"""ctypes binding of libf16acc_amd.so (the C ABI in include/f16acc.h).

There is no fallback: if the library is missing, importing this module
raises, and the package cannot be used.
"""

import ctypes
import os

from .build import LIB

if not os.path.exists(LIB):
    raise ImportError(f"{LIB} is not built; run `python f16acc_amd/build.py` (needs hipcc for gfx950)")

_dll = ctypes.CDLL(LIB)

_i64, _vp, _int = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
_P64 = ctypes.POINTER(ctypes.c_int64)
_PI = ctypes.POINTER(ctypes.c_int)

gemm = _dll.f16acc_gemm
gemm.argtypes = [_vp, _vp, _vp, _vp] + [_i64] * 9 + [_int, _int, _vp]
gemm.restype = _int

gemm_bias = _dll.f16acc_gemm_bias
gemm_bias.argtypes = [_vp, _vp, _vp, _vp, _vp] + [_i64] * 9 + [_int, _int, _vp]
gemm_bias.restype = _int

gemm_ws = _dll.f16acc_gemm_ws
gemm_ws.argtypes = [_vp, _vp, _vp, _vp, _vp] + [_i64] * 9 + [_int, _int, _vp, _vp, ctypes.c_size_t]
gemm_ws.restype = _int

gemm_noalloc = _dll.f16acc_gemm_noalloc
gemm_noalloc.argtypes = [_vp, _vp, _vp, _vp, _vp] + [_i64] * 9 + [_int, _int, _vp]
gemm_noalloc.restype = _int

workspace_size = _dll.f16acc_workspace_size
workspace_size.argtypes = [_i64] * 7 + [_vp, _vp, ctypes.POINTER(ctypes.c_size_t)]
workspace_size.restype = _int

gemm_tile = _dll.f16acc_gemm_tile
gemm_tile.argtypes = [_vp, _vp, _vp, _vp] + [_i64] * 9 + [_int, _int, _vp, _int]
gemm_tile.restype = _int

gemm_tile_ws = _dll.f16acc_gemm_tile_ws
gemm_tile_ws.argtypes = [_vp, _vp, _vp, _vp] + [_i64] * 9 + [_int, _int, _vp, _int, _vp, ctypes.c_size_t]
gemm_tile_ws.restype = _int

pack = _dll.f16acc_pack
pack.argtypes = [_vp, _vp] + [_i64] * 6 + [_vp]
pack.restype = _int

tile_config = _dll.f16acc_tile_config
tile_config.argtypes = [_i64] * 7 + [_vp, _vp, _int, _PI, _PI, _PI, _P64, _P64, _PI, _PI]
tile_config.restype = _int

block_tile = _dll.f16acc_block_tile
block_tile.argtypes = [_i64, _i64, _i64, _P64, _P64]
block_tile.restype = _int

tail_split = _dll.f16acc_tail_split
tail_split.argtypes = [_i64] * 7 + [_vp, _vp, _P64]
tail_split.restype = _int

strerror = _dll.f16acc_strerror
strerror.argtypes = [_int]
strerror.restype = ctypes.c_char_p

abi_version = _dll.f16acc_abi_version
abi_version.argtypes = []
abi_version.restype = _int

# Exported symbol names, as declared in include/f16acc.h.
EXPORTS = ("f16acc_gemm", "f16acc_gemm_bias", "f16acc_gemm_ws", "f16acc_gemm_noalloc", "f16acc_workspace_size", "f16acc_gemm_tile", "f16acc_gemm_tile_ws", "f16acc_pack", "f16acc_tile_config", "f16acc_block_tile", "f16acc_strerror",
           "f16acc_abi_version", "f16acc_tail_split")
ABI_VERSION = 7

OUT_F16, OUT_F32 = 0, 1
WS_HEADER = 4096  # F16ACC_WS_HEADER: the first bytes of a workspace, zero on first use
E_ARG, E_UNSUPPORTED, E_SCRATCH, E_DEVICE = -1, -2, -3, -4
TILES = ("256x256", "256x128", "128x256", "128x128", "generic", "64x64", "128x96k2", "64x32k4",
         "256x288")  # F16ACC_TILE_* ids
TILE_GENERIC = 4

if abi_version() != ABI_VERSION:
    raise ImportError(f"{LIB} has ABI version {abi_version()}, this package needs {ABI_VERSION}: rebuild it")


def check(rc):
    if rc != 0:
        raise RuntimeError(strerror(rc).decode())
