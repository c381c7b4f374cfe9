"""The chunked FP16 GEMM op: `mm(a, b)` on HIP devices.

Host side of the reference's f16acc/kernel.py:84-105 (`mm`): the same
arguments, the same ValueError checks before any launch, a freshly allocated
contiguous output, and no synchronisation.  The Triton `_gemm` / `_redo`
launches are replaced by one call into libf16acc_amd.so (f16acc_gemm), which
runs the main pass and the FP32 redo of overflowing tiles in one kernel on
the current stream.  Operands the fast kernels cannot read directly (rows not
16-byte aligned, e.g. K = 8961; odd strides) are first copied by the
library's pack kernel into zero-padded buffers that torch allocates.
"""

import ctypes

import torch

from . import _lib

_OUT = {torch.float16: _lib.OUT_F16, torch.float32: _lib.OUT_F32}

# Below this many multiply-adds the generic gather kernel beats a pack + fast
# kernel (the copy's launch and traffic are not repaid).
PACK_MIN_MACS = 1 << 24

# f16acc_tile_config's kernel families (F16ACC_FAMILY_* in include/f16acc.h)
_FAMILIES = ("fast", "generic", "reg")

# Workspace (f16acc_gemm_ws): the deferred redo list of flagged tiles, then
# the split-K FP32 partials; one per (device, stream): kernels
# on one stream run one after another, so consecutive calls on a stream can
# share it.  A workspace that a larger one replaces is kept, not freed: a HIP
# graph captured earlier holds its address and writes there on every replay,
# so its memory must never go to another tensor.  Sizes grow at least 2x, so
# few are kept.  A call under HIP graph capture gets the workspace of its
# capture (device, stream, capture id), used by no eager call and no other
# graph, so replays of different graphs, on any streams, and eager calls on
# the capture stream never share partials; it is kept for the life of the
# process, as the graph may be replayed at any time.
_workspaces = {}
_retired = []
_hip = None  # libamdhip64, for hipStreamGetCaptureInfo
_ws_sizes = {}  # problem key -> f16acc_workspace_size result
_WS_MEMO_MAX = 4096


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
    a, b, K = _operands(a, b, M, N, K)
    _launch(a, b, c, None, M, N, K, chunked, ws=_workspace(a, b, M, N, K))
    return c


def _workspace(a, b, M, N, K):
    """The split-K workspace for this problem on the current stream, or None
    when the library would not split it (its tiles already fill the GPU)."""
    key = (a.device.index, M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), a.data_ptr() % 16,
           b.data_ptr() % 16)
    nbytes = _ws_sizes.get(key)
    if nbytes is None:
        n = ctypes.c_size_t()
        _lib.check(_lib.workspace_size(M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), a.data_ptr(),
                                       b.data_ptr(), ctypes.byref(n)))
        if len(_ws_sizes) >= _WS_MEMO_MAX:
            _ws_sizes.clear()
        nbytes = _ws_sizes[key] = n.value
    if nbytes == 0:
        return None
    skey = (a.device.index, _stream(a.device))
    if torch.cuda.is_current_stream_capturing():
        skey += (_capture_id(skey[1]),)
    ws = _workspaces.get(skey)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _retired.append(ws)
        grown = 2 * ws.numel() if ws is not None else 0
        ws = torch.empty(max(nbytes, grown, 1 << 20), dtype=torch.uint8, device=a.device)
        ws[:_lib.WS_HEADER].zero_()  # the deferred redo list: empty (the library keeps it so)
        _workspaces[skey] = ws
    return ws


def _capture_id(stream):
    """Sequence id of the HIP graph capture running on `stream`
    (hipStreamGetCaptureInfo).  Called only while torch reports a capture on
    that stream; a runtime that then names no active capture is an error
    (a fresh key per call would leave one workspace per call behind)."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipStreamGetCaptureInfo.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int),
                                                 ctypes.POINTER(ctypes.c_ulonglong)]
        _hip.hipStreamGetCaptureInfo.restype = ctypes.c_int
    status, cid = ctypes.c_int(), ctypes.c_ulonglong()
    rc = _hip.hipStreamGetCaptureInfo(stream, ctypes.byref(status), ctypes.byref(cid))
    if rc != 0 or status.value != 1:  # hipStreamCaptureStatusActive is 1
        raise RuntimeError(f"f16acc: no HIP graph capture id for the capturing stream (hipError {rc}, "
                           f"status {status.value})")
    return cid.value


def mm_bias(a, b, bias, out_dtype=torch.float16, chunked=True):
    """mm(a, b) + bias with the add fused into the GEMM's store (f16acc_gemm_bias).

    bias: fp16 [N] on a's device.  For an fp16 output the result equals the
    reference's unfused `y = mm(a, b); y += bias` (f16acc/patch.py:28-30) bit
    for bit: the FP32 sum is rounded to fp16, the bias added in FP32 and the
    sum rounded again, as torch's fp16 add does."""
    _validate(a, b, out_dtype)
    N = b.shape[1]
    if (bias.dim() != 1 or bias.shape[0] != N or bias.dtype != torch.float16 or not bias.is_cuda
            or bias.device != a.device):
        raise ValueError(f"mm_bias needs an fp16 [{N}] bias on {a.device}, got {tuple(bias.shape)} {bias.dtype}")
    M, K = a.shape
    c = torch.empty(M, N, device=a.device, dtype=out_dtype)
    if M == 0 or N == 0:
        return c
    a, b, K = _operands(a, b, M, N, K)
    _launch(a, b, c, None, M, N, K, chunked, bias=bias.contiguous(), ws=_workspace(a, b, M, N, K))
    return c


def _canon(stride, extent, row):
    """The stride the library plans with: an extent-1 dimension's stride
    addresses nothing, so it counts as a plain row length `row`."""
    return stride if extent > 1 else row


def _fast_a(a, K):
    """a [M, K] as the fast kernels read it: K-contiguous 16-byte aligned rows
    that do not overlap (row stride >= K; a broadcast row, stride 0, or a
    sliding window does not qualify: the copies clip a tile by one record
    count, which needs disjoint rows)."""
    sam = _canon(a.stride(0), a.shape[0], -(-K // 8) * 8)
    return K % 8 == 0 and (a.stride(1) == 1 or K <= 1) and sam % 8 == 0 and sam >= K and a.data_ptr() % 16 == 0


def _fast_b(b, K, N):
    """b [K, N]: K-contiguous columns (w.t()) or N-contiguous rows, 16-byte
    aligned, with disjoint rows (sbn >= K, or sbk >= N for a row-major b)."""
    if b.data_ptr() % 16:
        return False
    sbk = _canon(b.stride(0), K, -(-N // 8) * 8)
    sbn = _canon(b.stride(1), N, -(-K // 8) * 8)
    kc = K % 8 == 0 and (sbk == 1 or K <= 1) and sbn % 8 == 0 and sbn >= K
    nc = N % 8 == 0 and (sbn == 1 or N <= 1) and sbk % 8 == 0 and sbk >= N
    return kc or nc


def _pack(src, rows, cols, s_r, s_c, ld):
    """Zero-padded contiguous [rows, ld] copy of a strided fp16 matrix (f16acc_pack)."""
    dst = torch.empty(rows, ld, device=src.device, dtype=torch.float16)
    stream = _stream(src.device)
    _lib.check(_lib.pack(src.data_ptr(), dst.data_ptr(), rows, cols, s_r, s_c, rows, ld, stream))
    return dst


def _pack_plan(a, b, M, N, K, tile=None):
    """(pack_a, pack_b, Kp, ld): which operands mm copies before the GEMM, the
    K it then runs with, and the row length of the copies.  Nothing is packed
    when the fast kernels can read a and b directly, when the library's
    register-staged loader reads them as they are (unit-stride rows at any
    even address, where the table picks 128x128 or 64x64) and that costs
    less than the copy (_reg_beats_pack; always for a forced tile), when the
    problem is too small to repay a copy, or when the generic tile is forced;
    otherwise K is padded to a multiple of 8 by zeros and every operand that
    is not fast (or all, when K changes) is packed.  The copies' rows are ld = K rounded up to
    64 elements long, so that every row starts on a 128-byte cache line (rows
    of 8968 halves straddle lines and doubled the GEMM's memory transactions
    on the 2049 x 1537 x 8961 config)."""
    if K == 0 or tile == "generic":
        return False, False, K, K
    ok_a, ok_b = _fast_a(a, K), _fast_b(b, K, N)
    if ok_a and ok_b:
        return False, False, K, K
    small = tile is None and M * N * K < PACK_MIN_MACS
    if (small or tile is not None or _reg_beats_pack(M, N, K)) and _raw_family(a, b, M, N, K, tile) == "reg":
        return False, False, K, K
    if small:
        return False, False, K, K
    Kp = -(-K // 8) * 8
    return Kp != K or not ok_a, Kp != K or not ok_b, Kp, -(-K // 64) * 64


def _reg_beats_pack(M, N, K):
    """Whether reading misaligned operands in place (register-staged loads:
    the GEMM runs ~1.4x longer than on packed copies) costs less than packing
    them (two copies of (M + N) x K halves read and written at ~6 TB/s, plus
    ~5 us of launches).  Measured on MI355X, w.t() operands with odd K: in
    place wins from 256^2 x 1001 (13.9 against 34.5 us per call) up to
    2048 x 1536 x 1537 (29.2 against 33.0 us); packing wins on
    2049 x 1537 x 8961 (115.5 against 126.4 us)."""
    return 0.4 * 2.0 * M * N * K / 500e12 < 4.0 * (M + N) * K / 6e12 + 5e-6


def _raw_family(a, b, M, N, K, tile):
    """Kernel family the library picks for a and b as they are (no packing):
    "reg" when its register-staged loader reads them directly (unit-stride
    rows at any even address, on the 128x128 and 64x64 tiles)."""
    fam = ctypes.c_int()
    _lib.check(_lib.tile_config(M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), a.data_ptr(),
                                b.data_ptr(), _tile_id(tile), None, None, None, None, None, ctypes.byref(fam), None))
    return _FAMILIES[fam.value]


def _operands(a, b, M, N, K, tile=None):
    """The operands the GEMM runs on (see _pack_plan): a as the [M, Kp] view
    of an [M, ld] buffer, b as the K-contiguous [Kp, N] view of an [N, ld]
    buffer when packed.  Returns (a, b, K) for the launch."""
    pack_a, pack_b, Kp, ld = _pack_plan(a, b, M, N, K, tile)
    if pack_a:
        with torch.cuda.device(a.device):
            a = _pack(a, M, K, a.stride(0), a.stride(1), ld)[:, :Kp]
    if pack_b:
        with torch.cuda.device(b.device):
            b = _pack(b, N, K, b.stride(1), b.stride(0), ld)[:, :Kp].t()  # element (n, k) = b[k][n]
    return a, b, Kp


def mm_flags(a, b, out_dtype=torch.float16, chunked=True, tile=None):
    """mm plus the per-tile redo flags (uint8 [tiles_m, tiles_n]): 1 where the
    tile's chunked FP32 sum held inf/NaN and was recomputed in FP32.  Same
    checks as mm; used by tests and benches to see which tiles were redone.
    tile: None for the per-shape table's choice, or a name of _lib.TILES to
    force that configuration (tuning, as the reference's autotuner does)."""
    _validate(a, b, out_dtype)
    M, K = a.shape
    N = b.shape[1]
    c = torch.empty(M, N, device=a.device, dtype=out_dtype)
    if M and N:
        a, b, K = _operands(a, b, M, N, K, tile)
    cfg = tile_config(a, b, tile)
    flags = torch.zeros(cfg["tiles_m"], cfg["tiles_n"], device=a.device, dtype=torch.uint8)
    if M and N:
        ws = _workspace(a, b, M, N, K) if tile is None else None
        _launch(a, b, c, flags, M, N, K, chunked, _tile_id(tile), ws=ws)
    return c, flags


def mm_tile(a, b, tile, out_dtype=torch.float16, chunked=True):
    """mm with the tile configuration forced to `tile` (a name of _lib.TILES)."""
    _validate(a, b, out_dtype)
    M, K = a.shape
    N = b.shape[1]
    c = torch.empty(M, N, device=a.device, dtype=out_dtype)
    if M and N:
        a, b, K = _operands(a, b, M, N, K, tile)
        _launch(a, b, c, None, M, N, K, chunked, _tile_id(tile))
    return c


def _tile_id(tile):
    if tile is None:
        return -1
    if tile not in _lib.TILES:
        raise ValueError(f"tile must be one of {_lib.TILES}, not {tile!r}")
    return _lib.TILES.index(tile)


def tile_config(a, b, tile=None):
    """The tile configuration mm uses for a @ b (replaces the reference's
    autotuned best_config, kernel.py:16-19, 101-102), or what a forced `tile`
    resolves to, for the operands the GEMM actually reads: when mm would pack
    a or b first, the packed copies' layout (contiguous, 16-byte aligned rows
    of Kp elements)."""
    M, K = a.shape
    N = b.shape[1]
    pack_a, pack_b, Kp, ld = _pack_plan(a, b, M, N, K, tile) if M and N else (False, False, K, K)
    sam, sak, pa = (ld, 1, 0) if pack_a else (a.stride(0), a.stride(1), a.data_ptr())
    sbk, sbn, pb = (1, ld, 0) if pack_b else (b.stride(0), b.stride(1), b.data_ptr())
    tid, bm, bn, fam, thr = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    tm, tn = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(_lib.tile_config(M, N, Kp, sam, sak, sbk, sbn, pa, pb, _tile_id(tile), ctypes.byref(tid),
                                ctypes.byref(bm), ctypes.byref(bn), ctypes.byref(tm), ctypes.byref(tn),
                                ctypes.byref(fam), ctypes.byref(thr)))
    return {"tile": _lib.TILES[tid.value], "bm": bm.value, "bn": bn.value, "tiles_m": tm.value,
            "tiles_n": tn.value, "family": _FAMILIES[fam.value], "threads": thr.value}


def _stream(dev):
    """hipStream_t of the current torch stream on dev, as an integer."""
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)  # ~0.2 us against ~2 us for the public path
    return raw(dev.index) if raw is not None else torch.cuda.current_stream(dev).cuda_stream


def _launch(a, b, c, flags, M, N, K, chunked, tile=-1, bias=None, ws=None):
    dev = a.device
    if torch.cuda.current_device() != dev.index:
        with torch.cuda.device(dev):
            return _launch(a, b, c, flags, M, N, K, chunked, tile, bias, ws)
    stream = _stream(dev)
    ptrs = (a.data_ptr(), b.data_ptr(), c.data_ptr(), flags.data_ptr() if flags is not None else None)
    args = (M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1),
            _OUT[c.dtype], int(bool(chunked)), stream)
    if ws is not None:
        rc = _lib.gemm_ws(ptrs[0], ptrs[1], bias.data_ptr() if bias is not None else None, ptrs[2], ptrs[3], *args,
                          ws.data_ptr(), ws.numel())
    elif bias is not None:
        rc = _lib.gemm_bias(ptrs[0], ptrs[1], bias.data_ptr(), ptrs[2], ptrs[3], *args)
    elif tile < 0:
        rc = _lib.gemm(*ptrs, *args)
    else:
        rc = _lib.gemm_tile(*ptrs, *args, tile)
    _lib.check(rc)
