"""Operands whose rows overlap: broadcast views (row stride 0, x.expand(M, K))
and sliding windows (row stride smaller than a row).  The reference reaches
every element through its own pointer, a_ptr + rm * sam + rk * sak
(f16acc/kernel.py:41-47), so such views work there, and patch.linear relies
on "the kernel takes any strides" (f16acc/patch.py:28).

The library's direct-to-LDS copies clip a tile by one buffer record count,
which is exact only for disjoint rows, so these views go to the
register-staged loader, a packed copy or the gather kernel (the routing
itself is checked on the CPU in tests/test_boundary.py).  Each case runs
through the C ABI with the operands as given (the table's pick, and every
tile forced: the library's own routing) and through mm / mm_tile (which may
pack first), against the oracle, on every tile of the direct-to-LDS family."""

import pytest
import torch

import f16acc_amd as f16acc
from f16acc_amd import _lib
from f16acc_amd.kernel import mm_tile
from oracle import chunk32

pytestmark = pytest.mark.gpu
rel = chunk32.rel
TOL = 1e-3
FAST_TILES = ["256x256", "256x288", "128x96k2", "64x32k4", "128x128", "64x64", "256x128", "128x256"]
M, N, K = 512, 576, 320
CASES = ["a_broadcast", "a_window", "b_broadcast_rowmajor", "b_broadcast_wt", "b_window_wt", "b_window_rowmajor"]


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).half()


def overlap_case(name, m=M, n=N, k=K):
    """(a, b) CPU views of a case and a function returning their GPU twins
    (the same strides over a copy of the same storage)."""
    def window(rows, cols, seed):  # rows 8 elements apart over one flat buffer
        flat = rnd(((rows - 1) * 8 + cols,), seed)
        return flat, lambda t: t.as_strided((rows, cols), (8, 1))

    if name == "a_broadcast":  # x.expand(M, K): row stride 0
        v, b = rnd((k,), 1), rnd((k, n), 2)
        return v.expand(m, k), b, lambda: (v.cuda().expand(m, k), b.cuda())
    if name == "a_window":  # unfold-style rows: sam = 8 < K
        flat, view = window(m, k, 3)
        w = rnd((n, k), 4)
        return view(flat), w.t(), lambda: (view(flat.cuda()), w.cuda().t())
    if name == "b_broadcast_rowmajor":  # v.expand(K, N): sbk = 0
        a, v = rnd((m, k), 5), rnd((n,), 6)
        return a, v.expand(k, n), lambda: (a.cuda(), v.cuda().expand(k, n))
    if name == "b_broadcast_wt":  # v.expand(N, K).t(): one weight row for every column, sbn = 0
        a, v = rnd((m, k), 7), rnd((k,), 8)
        return a, v.expand(n, k).t(), lambda: (a.cuda(), v.cuda().expand(n, k).t())
    if name == "b_window_wt":  # weight rows 8 apart, passed as w.t(): sbn = 8 < K
        a = rnd((m, k), 9)
        flat, view = window(n, k, 10)
        return a, view(flat).t(), lambda: (a.cuda(), view(flat.cuda()).t())
    if name == "b_window_rowmajor":  # k-rows 8 apart: sbk = 8 < N
        a = rnd((m, k), 11)
        flat, view = window(k, n, 12)
        return a, view(flat), lambda: (a.cuda(), view(flat.cuda()))
    raise ValueError(name)


def _abi(ga, gb, tile):
    """The C ABI with the operands as given (f16acc_gemm, or f16acc_gemm_tile
    for a forced tile), FP32 output into a NaN-filled buffer."""
    c = torch.full((M, N), float("nan"), device="cuda", dtype=torch.float32)
    args = (ga.data_ptr(), gb.data_ptr(), c.data_ptr(), None, M, N, K, ga.stride(0), ga.stride(1), gb.stride(0),
            gb.stride(1), N, 1, _lib.OUT_F32, 1, torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.gemm(*args) if tile is None else _lib.gemm_tile(*args, _lib.TILES.index(tile)))
    return c


def bit_equal(x, y):
    return float((x.view(torch.int32) == y.view(torch.int32)).float().mean())


@pytest.mark.parametrize("tile", [None] + FAST_TILES)
@pytest.mark.parametrize("case", CASES)
def test_overlapping_rows_match_oracle(case, tile):
    """Values against the oracle (1e-3, and at least 99% of the FP32 outputs
    bit-equal: for these N(0, 1) inputs every FP32 sum of fp16-rounded chunk
    partials is exact, so the kernel can only differ where an MFMA partial and
    the host's land on two sides of an fp16 rounding boundary), and the
    structure a broadcast forces: every output row (a broadcast a) or column
    (a broadcast w.t()) equal to the first, bit for bit."""
    a, b, twin = overlap_case(case)
    ga, gb = twin()
    assert ga.stride() == a.stride() and gb.stride() == b.stride()
    assert torch.equal(ga.cpu(), a) and torch.equal(gb.cpu(), b)
    ref = chunk32.chunked_sum(a, b)
    assert bool(torch.isfinite(ref).all())
    c_abi = _abi(ga, gb, tile)
    c_mm = mm_tile(ga, gb, tile, torch.float32) if tile else f16acc.mm(ga, gb, torch.float32)
    c16 = mm_tile(ga, gb, tile) if tile else f16acc.mm(ga, gb)
    torch.cuda.synchronize()
    for name, c in (("abi", c_abi.cpu()), ("mm", c_mm.cpu())):
        assert rel(c, ref) < TOL, (case, tile, name)
        assert bit_equal(c, ref) > 0.99, (case, tile, name, bit_equal(c, ref))
    assert rel(c16.cpu(), ref.half()) < TOL, (case, tile)
    if case == "a_broadcast":
        assert bool((c_abi == c_abi[:1]).all()) and bool((c16 == c16[:1]).all()), (case, tile)
    if case == "b_broadcast_wt":
        assert bool((c_abi == c_abi[:, :1]).all()) and bool((c16 == c16[:, :1]).all()), (case, tile)


def test_patched_linear_on_an_expanded_activation():
    """nn.Linear(384, 640) on x[:1, :1].expand(2, 150, 384): the activation
    reaches mm as a (0, 1)-strided [300, 384] view.  Every output row is the
    single row's result, equal to the oracle plus the bias rounded as the
    reference's `y += b` (f16acc/patch.py:29-30), and to the same call on a
    contiguous copy of the activation."""
    x = rnd((1, 1, 384), 20)
    w, bias = rnd((640, 384), 21, 0.05), rnd((640,), 22, 0.02)
    lin = torch.nn.Linear(384, 640, device="cuda", dtype=torch.float16)
    with torch.no_grad():
        lin.weight.copy_(w.cuda())
        lin.bias.copy_(bias.cuda())
    gx = x.cuda().expand(2, 150, 384)
    assert gx.reshape(300, 384).stride() == (0, 1)
    f16acc.enable()
    try:
        before = f16acc.calls["chunked"]
        with torch.inference_mode():
            y = lin(gx)
            y2 = lin(gx.contiguous())
        assert f16acc.calls["chunked"] == before + 2
    finally:
        f16acc.disable()
    y, y2 = y.reshape(300, 640).cpu(), y2.reshape(300, 640).cpu()
    ref = (chunk32.mm(x.reshape(1, 384).expand(300, 384), w.t(), torch.float16).float() + bias.float()).half()
    assert bool((y == y[:1]).all()) and bool((y != 0).any())
    assert rel(y, ref) < TOL
    assert torch.equal(y, y2)
