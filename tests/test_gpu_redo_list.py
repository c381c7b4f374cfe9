"""The deferred redo (a workspace's redo list): a chunked launch of at most
one round of 256x256 tiles lists its flagged tiles instead of redoing them in
place, and a second launch recomputes each in FP32 as four 128x128 quarters
(the reference's separate _redo launch, f16acc/kernel.py:75-81, 103-104).

Checked through the C ABI against f16acc_gemm (no workspace: redo in place),
bit for bit: many flagged tiles, ragged edges, both b layouts, fp16 / fp32
output, fused bias, every tile flagged, none flagged; the list left empty
after every call (consecutive calls on one workspace, and the header read
back); tile flags; and HIP graph replays of a listing call."""

import pytest
import torch

from f16acc_amd import _lib
from f16acc_amd.kernel import tile_config
from oracle import chunk32

pytestmark = pytest.mark.gpu


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).half()


def _ws():
    ws = torch.empty((1 << 20) + _lib.WS_HEADER, dtype=torch.uint8, device="cuda")
    ws[:_lib.WS_HEADER].zero_()
    return ws


def _counters_zero(ws):
    """The list's counters (the chunked launch's item counter and the 8 lines
    of length and readers: the first 8 bytes of each 128-byte line of the
    header's first 1152 bytes) are back to zero."""
    lines = ws[:1152].view(torch.int32).view(9, 32)[:, :2]
    return int(lines.abs().sum()) == 0


def _gemm(a, b, c, bias=None, flags=None, ws=None):
    M, K = a.shape
    N = b.shape[1]
    args = (M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1),
            _lib.OUT_F32 if c.dtype == torch.float32 else _lib.OUT_F16, 1, torch.cuda.current_stream().cuda_stream)
    fp = flags.data_ptr() if flags is not None else None
    bp = bias.data_ptr() if bias is not None else None
    if ws is None:
        rc = (_lib.gemm_bias(a.data_ptr(), b.data_ptr(), bp, c.data_ptr(), fp, *args) if bias is not None else
              _lib.gemm(a.data_ptr(), b.data_ptr(), c.data_ptr(), fp, *args))
    else:
        rc = _lib.gemm_ws(a.data_ptr(), b.data_ptr(), bp, c.data_ptr(), fp, *args, ws.data_ptr(), ws.numel())
    _lib.check(rc)


def _listed(M, N, K, a, b):
    import ctypes

    n = ctypes.c_size_t()
    _lib.check(_lib.workspace_size(M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), a.data_ptr(),
                                   b.data_ptr(), ctypes.byref(n)))
    return n.value == _lib.WS_HEADER


def _overflowing(M, N, K, rows, cols, seed):
    """a, b ~ N(0, 1) with 128-row blocks of a and 128-column blocks of b
    ~ U(200, 255): the 256x256 tiles holding an intersection overflow."""
    g = torch.Generator().manual_seed(seed)
    a, b = torch.randn(M, K, generator=g), torch.randn(K, N, generator=g)
    for r in rows:
        a[r * 128:(r + 1) * 128] = 200.0 + 55.0 * torch.rand(min(128, M - r * 128), K, generator=g)
    for q in cols:
        b[:, q * 128:(q + 1) * 128] = 200.0 + 55.0 * torch.rand(K, min(128, N - q * 128), generator=g)
    return a.half(), b.half()


CASES = [  # M, N, K, row blocks, column blocks, b = w.t(), out dtype, bias
    (4096, 4096, 2560, [3, 9, 17, 30], [0, 11, 22, 31], False, torch.float32, False),
    (4096, 4096, 2560, [3, 9, 17, 30], [0, 11, 22, 31], True, torch.float16, True),
    (3000, 3504, 2600, [0, 11, 23], [1, 13, 27], True, torch.float32, True),   # ragged edge tiles flagged, ragged K
    (3000, 3504, 2600, [0, 11, 23], [1, 13, 27], False, torch.float16, False),
]


def test_short_k_redoes_in_place_through_the_workspace_entry():
    """Below 40 stages of K (K = 2496) a one-round 256x256 problem does not
    list its flagged tiles: f16acc_gemm_ws redoes them in place, as
    f16acc_gemm does, and leaves the header's counters at zero; at K = 2560
    the same shape lists them.  Both equal f16acc_gemm bit for bit, with the
    same single flagged tile."""
    M = N = 4096
    for K, listed in ((2496, False), (2560, True)):
        a, b = _overflowing(M, N, K, [5], [7], 11)
        ga, gb = a.cuda(), b.cuda()
        assert _listed(M, N, K, ga, gb) == listed, K
        ws = _ws()
        c0 = torch.full((M, N), float("nan"), device="cuda", dtype=torch.float16)
        c1 = torch.full_like(c0, float("nan"))
        f0 = torch.zeros(16, 16, device="cuda", dtype=torch.uint8)
        f1 = torch.zeros_like(f0)
        _gemm(ga, gb, c0, None, f0)
        _gemm(ga, gb, c1, None, f1, ws)
        torch.cuda.synchronize()
        assert {tuple(t) for t in f0.nonzero().tolist()} == {(2, 3)}, K
        assert torch.equal(f1, f0) and torch.equal(c1, c0), K
        assert _counters_zero(ws), K


@pytest.mark.parametrize("M, N, K, rows, cols, b_t, out_dtype, biased", CASES)
def test_deferred_redo_equals_redo_in_place(M, N, K, rows, cols, b_t, out_dtype, biased):
    a, b = _overflowing(M, N, K, rows, cols, 5)
    ga, gb = a.cuda(), (b.t().contiguous().cuda().t() if b_t else b.cuda())
    cfg = tile_config(ga, gb)
    assert cfg["tile"] == "256x256" and cfg["tiles_m"] * cfg["tiles_n"] <= 256 and _listed(M, N, K, ga, gb)
    bias = rnd((N,), 6, 0.02).cuda() if biased else None
    ws = _ws()
    outs, fls = [], []
    for w in (None, ws, ws):  # in place, then twice through the list
        c = torch.full((M, N), float("nan"), device="cuda", dtype=out_dtype)
        fl = torch.zeros(cfg["tiles_m"], cfg["tiles_n"], device="cuda", dtype=torch.uint8)
        _gemm(ga, gb, c, bias, fl, w)
        outs.append(c)
        fls.append(fl)
    torch.cuda.synchronize()
    want = {(r // 2, q // 2) for r in rows for q in cols}
    assert {tuple(t) for t in fls[0].nonzero().tolist()} == want
    assert torch.equal(fls[1], fls[0]) and torch.equal(fls[2], fls[0])
    assert torch.equal(outs[1], outs[0]) and torch.equal(outs[2], outs[0])
    assert _counters_zero(ws)
    # the values themselves: redone tiles are the FP32 sums, the rest the oracle's
    ref, rflags = chunk32.mm(a, b, out_dtype, tile=(256, 256), return_flags=True)
    if biased:
        ref = (ref.float() + bias.cpu().float()).to(out_dtype)
    assert torch.equal(fls[0].cpu(), rflags)
    fin = torch.isfinite(ref)
    err = (outs[0].cpu()[fin].double() - ref[fin].double()).abs().max() / ref[fin].double().abs().max()
    assert float(err) < 1e-3


def test_one_tile_grid_between_full_grids_on_one_workspace():
    """256x256 forced (f16acc_gemm_tile_ws against f16acc_gemm_tile, which
    redoes in place): a 4096^3-row call, then a one-tile problem (a redo
    launch of 4 workgroups, fewer than the list's 8 lines: the lines no
    workgroup reads are cleared too), then the first call again; every call
    equals the in-place redo, so no line keeps a stale length."""
    ws = _ws()
    tile = _lib.TILES.index("256x256")
    big = _overflowing(4096, 4096, 2560, [3, 17], [6, 25], 9)
    small = _overflowing(256, 256, 2560, [0], [1], 10)
    for a, b in (big, small, big):
        ga, gb = a.cuda(), b.cuda()
        M, K = a.shape
        N = b.shape[1]
        c0 = torch.empty(M, N, device="cuda", dtype=torch.float32)
        c1 = torch.empty_like(c0)
        args = (M, N, K, K, 1, N, 1, N, 1, _lib.OUT_F32, 1, torch.cuda.current_stream().cuda_stream, tile)
        _lib.check(_lib.gemm_tile(ga.data_ptr(), gb.data_ptr(), c0.data_ptr(), None, *args))
        _lib.check(_lib.gemm_tile_ws(ga.data_ptr(), gb.data_ptr(), c1.data_ptr(), None, *args, ws.data_ptr(),
                                     ws.numel()))
        torch.cuda.synchronize()
        assert torch.equal(c0, c1), M
        assert _counters_zero(ws)


def test_every_tile_flagged_and_none_flagged():
    """All 256 tiles of 4096 x 4096 x 2560 listed (1024 quarters for the redo
    launch's 256 workgroups), then a clean call on the same workspace: each
    equals the in-place redo."""
    M = N = 4096
    K = 2560
    a = torch.full((M, K), 100.0, dtype=torch.float16)
    b = torch.full((K, N), 30.0, dtype=torch.float16)
    b.view(K // 32, 32, N)[1::2] = -30.0  # chunk sums of +-96000 (inf in fp16), exact total per pair
    clean = rnd((M, K), 7).cuda()
    ga, gb = a.cuda(), b.cuda()
    ws = _ws()
    for x in (ga, clean, ga):
        c0 = torch.empty(M, N, device="cuda", dtype=torch.float32)
        c1 = torch.empty_like(c0)
        fl0 = torch.zeros(16, 16, device="cuda", dtype=torch.uint8)
        fl1 = torch.zeros_like(fl0)
        _gemm(x, gb, c0, flags=fl0)
        _gemm(x, gb, c1, flags=fl1, ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(c0, c1) and torch.equal(fl0, fl1)
        assert int(fl0.sum()) == (256 if x is ga else 0)
        if x is ga:
            assert bool((c1 == 0.0).all())  # the chunk pairs cancel exactly in FP32
        assert _counters_zero(ws)


def test_graph_replays_of_a_listing_call_match_eager():
    """A listing call captured in a HIP graph and replayed several times, with
    eager calls on the same workspace in between: every replay equals eager
    (the redo launch empties the list on every replay)."""
    from f16acc_amd import kernel

    a, b = _overflowing(4096, 4096, 2560, [5, 20], [2, 29], 8)
    ga, gb = a.cuda(), b.cuda()
    want = kernel.mm(ga, gb, torch.float32)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kernel.mm(ga, gb, torch.float32)  # the capture stream's workspace exists before capture
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = kernel.mm(ga, gb, torch.float32)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        assert torch.equal(kernel.mm(ga, gb, torch.float32), want), i
