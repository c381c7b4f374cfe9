"""The persistent kernel (gemm_persistent): chunked 256x256 on shapes of
more than one round of tiles, one workgroup per CU walking its
tiles and issuing each next tile's first copies ahead of the previous tile's
store.  Shapes just past one round (257..300 tiles) keep the oracle cheap;
the full-size 8192^3 and lm_head checks in test_gpu_parity.py run on it too.

Checked: values and flags against the oracle on ragged edges, both b
layouts, fp16 and fp32 output, fused bias; overflow redone exactly in tiles
of the later rounds, in every wave's sub-tile; and bit-equality with the
same source built to run every shape one tile per workgroup
(libf16acc_amd_nopersist.so, a build the benchmark's A/B uses), which
computes every tile with the same K loop, flag and redo."""

import ctypes

import pytest
import torch

import f16acc_amd as f16acc
from f16acc_amd import _lib, build
from f16acc_amd.kernel import mm_flags, mm_tile, tile_config
from oracle import chunk32

pytestmark = pytest.mark.gpu
rel = chunk32.rel
TOL = 1e-3
CUS = 256  # MI355X


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).half()


def _gpu_b(b, b_t):
    return b.t().contiguous().cuda().t() if b_t else b.cuda()


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def _round_two_tile(tiles_m, tiles_n):
    """A tile that the persistent grid (one workgroup per CU) runs in its
    second round: the tile of block CUS + 3."""
    tm, tn = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(_lib.block_tile(_cus() + 3, tiles_m, tiles_n, ctypes.byref(tm), ctypes.byref(tn)))
    return tm.value, tn.value


CASES = [  # (M, N, K, tile, b_t): more tiles than CUs
    (4352, 4096, 256, "256x256", False),  # 17 x 16 = 272 tiles, row-major b
    (4352, 4096, 256, "256x256", True),
    (4100, 4130, 200, "256x256", True),   # 17 x 17 tiles, ragged edges, a partial last stage
    (4100, 4130, 200, "256x256", False),
]


@pytest.mark.parametrize("M, N, K, tile, b_t", CASES)
def test_persistent_matches_oracle(M, N, K, tile, b_t):
    assert _cus() == CUS
    a, b = rnd((M, K), 1), rnd((K, N), 2)
    ga, gb = a.cuda(), _gpu_b(b, b_t)
    cfg = tile_config(ga, gb, tile)
    assert cfg["tile"] == tile and cfg["tiles_m"] * cfg["tiles_n"] > CUS
    ref = chunk32.chunked_sum(a, b)
    f32 = chunk32.fp32_sum(a, b)
    for out_dtype in (torch.float32, torch.float16):
        c, flags = mm_flags(ga, gb, out_dtype, tile=tile)
        assert int(flags.sum()) == 0
        assert rel(c.cpu(), ref.to(out_dtype)) < TOL, (M, N, K, tile, out_dtype)
        if out_dtype == torch.float32:
            same = float((c.cpu().view(torch.int32) == ref.view(torch.int32)).float().mean())
            assert same > 1 - 1e-3 * -(-K // 32), same
            assert float((c.cpu() - ref).norm()) < 0.2 * float((f32 - ref).norm())
        # the table's pick and the C ABI without tile flags take the same kernel
        c2 = mm_tile(ga, gb, tile, out_dtype)
        assert torch.equal(c2, c), (M, N, K, tile, out_dtype)


def test_persistent_fused_bias_equals_unfused_add():
    """The fused bias (the store rounds to fp16, adds the bias in FP32, rounds
    again) equals `y = mm(x, w.t()); y += b` (f16acc/patch.py:28-30) bit for
    bit on the persistent grid (8192 x 4096 x 128 with a row-major weight:
    512 tiles of 256x256, the table's pick)."""
    M, N, K = 8192, 4096, 128
    a, w, bias = rnd((M, K), 3), rnd((N, K), 4, 0.05), rnd((N,), 5, 0.02)
    ga, gbias = a.cuda(), bias.cuda()
    gb = w.t().contiguous().cuda()
    cfg = tile_config(ga, gb)
    assert cfg["tile"] == "256x256" and cfg["tiles_m"] * cfg["tiles_n"] > CUS
    y = f16acc.kernel.mm_bias(ga, gb, gbias)
    want = f16acc.mm(ga, gb)
    want += gbias
    assert torch.equal(y, want)


@pytest.mark.parametrize("tile, b_t", [("256x256", False), ("256x256", True)])
def test_persistent_overflow_in_later_rounds_is_redone_exactly(tile, b_t):
    """The overflow stress pattern on a grid of more than one round: 128-wide
    blocks of a's rows and b's columns ~ U(200, 255) (chunk sums past 65504):
    the flagged tiles are exactly those holding a block intersection, in
    every round, and equal the FP32-accumulate mode bit for bit (the redo runs
    all of K in one workgroup: same tile, same summation order)."""
    M, N, K = (4352, 4096, 256) if tile == "256x256" else (2304, 8640, 256)
    bn = 256 if tile == "256x256" else 288
    # 128-row / 128-column blocks, each column block inside one tile column;
    # plus one intersection in the tile the grid's block CUS + 3 runs
    rows, cols = ([1, 9, 16, 33], [0, 7, 21, 31]) if tile == "256x256" else ([1, 9, 16, 17], [0, 7, 21, 45])
    ti, tj = _round_two_tile(-(-M // 256), -(-N // bn))
    rows, cols = sorted(set(rows + [2 * ti])), sorted(set(cols + [-(-tj * bn // 128)]))
    assert all((128 * q) // bn == (128 * q + 127) // bn and 128 * q + 128 <= N for q in cols)
    g = torch.Generator().manual_seed(7)
    a, b = torch.randn(M, K, generator=g), torch.randn(K, N, generator=g)
    for r in rows:
        a[r * 128:(r + 1) * 128] = 200.0 + 55.0 * torch.rand(128, K, generator=g)
    for q in cols:
        b[:, q * 128:(q + 1) * 128] = 200.0 + 55.0 * torch.rand(K, 128, generator=g)
    a, b = a.half(), b.half()
    ga, gb = a.cuda(), _gpu_b(b, b_t)
    cfg = tile_config(ga, gb, tile)
    assert cfg["tile"] == tile and cfg["tiles_m"] * cfg["tiles_n"] > CUS
    bm, bn = cfg["bm"], cfg["bn"]
    c, flags = mm_flags(ga, gb, torch.float32, tile=tile)
    ref, rflags = chunk32.mm(a, b, torch.float32, tile=(bm, bn), return_flags=True)
    assert torch.equal(flags.cpu(), rflags)
    want = {(r * 128 // bm, q * 128 // bn) for r in rows for q in cols}
    assert {tuple(t) for t in flags.nonzero().tolist()} == want
    # some flagged tiles run in the second round of the persistent grid
    second = set()
    for blk in range(CUS, cfg["tiles_m"] * cfg["tiles_n"]):
        tm, tn = ctypes.c_int64(), ctypes.c_int64()
        _lib.check(_lib.block_tile(blk, cfg["tiles_m"], cfg["tiles_n"], ctypes.byref(tm), ctypes.byref(tn)))
        second.add((tm.value, tn.value))
    assert want & second
    c32 = mm_tile(ga, gb, tile, torch.float32, chunked=False)
    mask = flags.bool().repeat_interleave(bm, 0).repeat_interleave(bn, 1)[:M, :N]
    assert torch.equal(c[mask], c32[mask])
    assert rel(c.cpu()[~mask.cpu()], ref[~mask.cpu()]) < TOL
    # without tile flags (the C ABI's own path): the same bits
    assert torch.equal(mm_tile(ga, gb, tile, torch.float32), c)


WAVES = {"256x256": (4, 2)}


@pytest.mark.parametrize("tile, wm, wn", [(t, i, j) for t in WAVES for i in range(4) for j in range(2)])
def test_persistent_overflow_in_every_wave_of_a_second_round_tile(tile, wm, wn):
    """The reference's forced-overflow closed form (tests/test_f16acc.py:91-101)
    in one wave's sub-tile of a tile the persistent grid runs in its second
    round: that tile alone is flagged and its block comes out exactly 100."""
    bm, bn = (256, 256) if tile == "256x256" else (256, 288)
    M, N, K = (4352, 4096, 128) if tile == "256x256" else (2304, 8640, 128)
    tiles_m, tiles_n = -(-M // bm), -(-N // bn)
    ti, tj = _round_two_tile(tiles_m, tiles_n)
    r0, c0 = ti * bm + wm * (bm // 4) + 5, tj * bn + wn * (bn // 2) + 3
    a, b = rnd((M, K), 20, 0.5), rnd((K, N), 21, 0.5)
    a[r0:r0 + 10, :] = 100.0
    b[:, c0:c0 + 10] = 0.0
    b[:32, c0:c0 + 10], b[32:64, c0:c0 + 10], b[64:96, c0:c0 + 10], b[96:, c0:c0 + 10] = 30.0, -30.0, 30.0, -30.0
    b[127, c0:c0 + 10] = -29.0
    ga, gb = a.cuda(), _gpu_b(b, tile == "256x288")
    c, flags = mm_flags(ga, gb, torch.float32, tile=tile)
    assert flags.shape == (tiles_m, tiles_n)
    assert int(flags.sum()) == 1 and int(flags[ti, tj]) == 1, (tile, wm, wn)
    assert bool((c[r0:r0 + 10, c0:c0 + 10] == 100.0).all())
    ref = chunk32.mm(a, b, torch.float32, tile=(bm, bn))
    assert rel(c.cpu(), ref) < TOL


def _nopersist():
    lib = ctypes.CDLL(build.LIB_NOPERSIST)
    for name in ("f16acc_gemm", "f16acc_gemm_bias"):
        getattr(lib, name).argtypes = getattr(_lib, name[7:]).argtypes
        getattr(lib, name).restype = ctypes.c_int
    return lib


@pytest.mark.parametrize("M, N, K, b_t, out_dtype, biased", [
    (4352, 4096, 256, False, torch.float16, False),
    (4352, 4096, 256, True, torch.float32, False),
    (4100, 4130, 200, True, torch.float16, True),
    (4100, 4130, 200, False, torch.float32, True),
    (8192, 4096, 136, False, torch.float16, False),
])
def test_persistent_equals_one_tile_per_workgroup_bit_for_bit(M, N, K, b_t, out_dtype, biased):
    """The same call through the shipped library (persistent) and the build
    without the persistent kernel: identical bits, overflowing tiles included."""
    other = _nopersist()
    a, b = rnd((M, K), 30), rnd((K, N), 31)
    a[128:256] = 120.0  # one row block overflows with b's large columns
    b[:, 300:420] = 120.0
    ga, gb = a.cuda(), _gpu_b(b, b_t)
    bias = rnd((N,), 32, 0.02).cuda() if biased else None
    stream = torch.cuda.current_stream().cuda_stream
    code = _lib.OUT_F32 if out_dtype == torch.float32 else _lib.OUT_F16
    outs = []
    for gemm, gemm_bias in ((_lib.gemm, _lib.gemm_bias), (other.f16acc_gemm, other.f16acc_gemm_bias)):
        c = torch.empty(M, N, device="cuda", dtype=out_dtype)
        args = (M, N, K, ga.stride(0), ga.stride(1), gb.stride(0), gb.stride(1), N, 1, code, 1, stream)
        if biased:
            _lib.check(gemm_bias(ga.data_ptr(), gb.data_ptr(), bias.data_ptr(), c.data_ptr(), None, *args))
        else:
            _lib.check(gemm(ga.data_ptr(), gb.data_ptr(), c.data_ptr(), None, *args))
        outs.append(c)
    torch.cuda.synchronize()
    assert bool((~torch.isfinite(outs[0])).sum() == 0) or out_dtype == torch.float16
    assert torch.equal(outs[0], outs[1])
