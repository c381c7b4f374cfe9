"""f16acc_gemm_noalloc, the entry point that allocates nothing: the
workspace (deferred redo list, split-K partials) is the library's fixed
per-GPU scratch instead of a caller's.  Called through the C ABI, it returns
the same bits and tile flags as f16acc_gemm_ws with a caller workspace, on
two calls in a row (the second smaller), both split along K, and the GPU's
free memory does not change across a call; on a shape whose flagged tiles
are redone by the deferred list, it equals f16acc_gemm (redo in place) on
consecutive calls, so the scratch's list is left empty."""

import pytest
import torch

from f16acc_amd import _lib
from oracle import chunk32

pytestmark = pytest.mark.gpu


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).half()


def _call(entry, a, b, bias, c, flags, ws=None):
    M, K = a.shape
    N = b.shape[1]
    args = [a.data_ptr(), b.data_ptr(), bias.data_ptr() if bias is not None else None, c.data_ptr(),
            flags.data_ptr() if flags is not None else None, M, N, K, a.stride(0), a.stride(1), b.stride(0),
            b.stride(1), c.stride(0), c.stride(1), _lib.OUT_F32 if c.dtype == torch.float32 else _lib.OUT_F16, 1,
            torch.cuda.current_stream().cuda_stream]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    _lib.check(entry(*args))


def _split_bytes(a, b):
    import ctypes

    M, K = a.shape
    n = ctypes.c_size_t()
    _lib.check(_lib.workspace_size(M, b.shape[1], K, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
                                   a.data_ptr(), b.data_ptr(), ctypes.byref(n)))
    return max(n.value - _lib.WS_HEADER, 0)  # the split-K partials' bytes


def _overflow_case():
    """256 x 256 x 4096, b row-major, the reference's forced-overflow closed
    form (tests/test_f16acc.py:91-101) inside one K range: one tile flagged,
    its block exactly 100."""
    M, N, K = 256, 256, 4096
    a, b = rnd((M, K), 80, 0.1), rnd((K, N), 81, 0.1)
    a[100:110, :] = 100.0
    b[:, 150:160] = 0.0
    b[1024:1056, 150:160], b[1056:1088, 150:160] = 30.0, -30.0
    b[1087, 150:160] = -29.0
    return a, b


def test_noalloc_equals_workspace_entry_on_two_calls_in_a_row():
    from f16acc_amd.kernel import tile_config

    ws = torch.empty((32 << 20) + _lib.WS_HEADER, dtype=torch.uint8, device="cuda")
    ws[:_lib.WS_HEADER].zero_()
    # call 1: the Qwen2.5-1.5B down projection's shape (2048 x 1536 x 8960,
    # fused bias, fp16 out) with the weight row-major [K, N] (b = w.t() would
    # split K inside the workgroup instead), split in two on 128x128 tiles
    # (25.2 MB of partials)
    x, w, bias = rnd((2048, 8960), 82).cuda(), rnd((1536, 8960), 83, 0.02).cuda(), rnd((1536,), 84, 0.02).cuda()
    w_kn = w.t().contiguous()
    # call 2, smaller: 256 x 256 x 4096 (b row-major, fp32 out) with an
    # overflow in one split, split four ways
    oa, ob = _overflow_case()
    ga, gb = oa.cuda(), ob.cuda()
    cases = [(x, w_kn, bias, torch.float16), (ga, gb, None, torch.float32)]
    for i, (a, b, bi, dt) in enumerate(cases):
        assert _split_bytes(a, b) > 0, "expected a split-K plan"
        cfg = tile_config(a, b)
        M, N = a.shape[0], b.shape[1]
        c_ws = torch.full((M, N), float("nan"), device="cuda", dtype=dt)
        c_na = torch.full((M, N), float("nan"), device="cuda", dtype=dt)
        f_ws = torch.full((cfg["tiles_m"], cfg["tiles_n"]), 7, device="cuda", dtype=torch.uint8)
        f_na = torch.full_like(f_ws, 7)
        _call(_lib.gemm_ws, a, b, bi, c_ws, f_ws, ws)
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info()[0]
        _call(_lib.gemm_noalloc, a, b, bi, c_na, f_na)
        torch.cuda.synchronize()
        if i > 0:  # the first call on the device may load the library's code object
            assert torch.cuda.mem_get_info()[0] == free_before
        assert torch.equal(c_na, c_ws), i
        assert torch.equal(f_na, f_ws), i
    # the second call against the oracle, and its closed form exact
    ref, rflags = chunk32.mm(oa, ob, torch.float32, tile=(cfg["bm"], cfg["bn"]), return_flags=True)
    assert torch.equal(f_na.cpu(), rflags) and int(rflags.sum()) == 1
    assert torch.all(c_na[100:110, 150:160].cpu() == 100.0)
    assert chunk32.rel(c_na.cpu(), ref) < 1e-3
    # and the first call's result is still what mm returns
    from f16acc_amd.kernel import mm_bias

    again = torch.empty(2048, 1536, device="cuda", dtype=torch.float16)
    _call(_lib.gemm_noalloc, x, w_kn, bias, again, None)
    torch.cuda.synchronize()
    assert torch.equal(again, mm_bias(x, w_kn, bias))


def test_noalloc_unsplit_problem_equals_plain_entry():
    """A problem whose tiles fill the GPU takes no split (4096 x 4096 x 2560,
    one round of 256x256 tiles, fp16 out); its overflowing tiles are listed in
    the scratch's header and redone by a second launch.  Three calls in a row
    (overflow, clean, overflow) each equal f16acc_gemm, which redoes in place,
    bit for bit: the list is emptied after each call."""
    K = 2560
    a, b = rnd((4096, K), 85), rnd((K, 4096), 86)
    a[512:640] = 120.0  # 128 rows x 128 columns whose chunk sums pass 65504
    b[:, 1024:1152] = 120.0
    clean_a = rnd((4096, K), 87).cuda()
    a, b = a.cuda(), b.cuda()
    assert _split_bytes(a, b) == 0
    for x in (a, clean_a, a):
        c = torch.empty(4096, 4096, device="cuda", dtype=torch.float16)
        _call(_lib.gemm_noalloc, x, b, None, c, None)
        plain = torch.empty_like(c)
        _lib.check(_lib.gemm(x.data_ptr(), b.data_ptr(), plain.data_ptr(), None, 4096, 4096, K, K, 1, 4096, 1,
                             4096, 1, _lib.OUT_F16, 1, torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert torch.equal(c, plain)
