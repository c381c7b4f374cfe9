"""Parity of the HIP kernels with the oracle (CPU restatement of the
reference's chunk-32 algorithm, f16acc/kernel.py:37-105 of the reference).

Inputs are generated on the CPU from a seed, cast to fp16 and copied to the
GPU, so the oracle and the kernel see identical bits.  Tolerances:
  * vs the oracle: max|x - ref| / max|ref| < 1e-3 (the reference's own
    metric, tests/test_f16acc.py:11-12); fp16 outputs may differ by one fp16
    ulp where the FP32 sums straddle a rounding boundary
  * vs FP64: the reference's bounds (2e-3 at odd sizes, tests/test_f16acc.py:21-24)
  * overflow closed forms: exact
"""

import ctypes

import pytest
import torch

import f16acc_amd as f16acc
from f16acc_amd import _lib
from f16acc_amd.kernel import mm_flags, tile_config
from oracle import chunk32

pytestmark = pytest.mark.gpu
rel = chunk32.rel
TOL = 1e-3


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).half()


def run(a_cpu, b_cpu, out_dtype=torch.float16, chunked=True, b_transposed=False):
    """Kernel result (CPU tensor), flags, and the tile shape it used.
    b_transposed: pass b as the w.t() view of a contiguous [N, K] tensor."""
    a = a_cpu.cuda()
    b = b_cpu.t().contiguous().cuda().t() if b_transposed else b_cpu.cuda()
    cfg = tile_config(a, b)
    c, flags = mm_flags(a, b, out_dtype, chunked)
    torch.cuda.synchronize()
    return c.cpu(), flags.cpu(), cfg


def oracle(a, b, out_dtype, cfg, chunked=True):
    return chunk32.mm(a, b, out_dtype, chunked=chunked, tile=(cfg["bm"], cfg["bn"]), return_flags=True)


def assert_carries_chunk_rounding(c, ref, f32, K, what):
    """An FP32 output c of the chunked kernel against the oracle's chunk sum
    ref and plain FP32 accumulation f32 (no tile flagged).  For N(0, 1)
    inputs every FP32 sum of fp16-rounded partials is exact, so c can only
    differ from ref where one of its chunks' FP32 partials rounds to the
    other fp16 neighbour in the MFMA than on the host (measured ~4e-4 of the
    elements per chunk on MI355X); FP32 accumulation keeps almost no bits.
    The max-norm error cannot tell the two apart (one such partial moves an
    element as much as the chunk rounding moves the worst one), the L2 norm
    and the bit count can."""
    c, ref, f32 = c.float().cpu(), ref.float().cpu(), f32.float().cpu()
    chunks = -(-K // 32)
    same = float((c.view(torch.int32) == ref.view(torch.int32)).float().mean())
    assert same > 1.0 - 1e-3 * chunks, (what, same)
    assert float((c - ref).norm()) < 0.2 * float((f32 - ref).norm()), what


ALL_TILES = ["256x256", "256x128", "128x256", "128x128", "generic", "64x64", "128x96k2", "64x32k4", "256x288"]


# Tiles that read a K-contiguous b only (the K-group tiles; 256x288, whose
# k-rows of 36 units do not fit the transpose-read swizzle), and the tile
# each runs as with a row-major b
KC_ONLY_FALLBACK = {"128x96k2": "128x128", "64x32k4": "64x64", "256x288": "256x256"}


def forced_tile_runs_as(tile, b_row_major):
    """The tile a forced tile runs as."""
    return KC_ONLY_FALLBACK.get(tile, tile) if b_row_major else tile


def tile_dims(tile):
    """(bm, bn) of a tile name."""
    if tile == "generic":
        return 128, 128
    bm, bn = tile.split("x")
    return int(bm), int(bn.split("k")[0])


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("b_transposed", [False, True])
def test_square_1024_matches_oracle_and_fp64(out_dtype, b_transposed):
    a, b = rnd((1024, 1024), 0), rnd((1024, 1024), 1)
    c, flags, cfg = run(a, b, out_dtype, b_transposed=b_transposed)
    ref, rflags = oracle(a, b, out_dtype, cfg)
    assert cfg["family"] == "fast"
    assert torch.equal(flags, rflags) and int(flags.sum()) == 0
    assert rel(c, ref) < TOL
    assert rel(c, a.double() @ b.double()) < 2e-3


@pytest.mark.parametrize("n", [4096, 8192])
def test_full_size_square_gemms_match_oracle_and_fp64(n):
    """The square workloads at their full sizes, n^3 with A, B ~ N(0, 1):
    fp16 and fp32 output, B row-major and as the w.t() view, each against the
    oracle's FP32 chunk sum (computed once: the layouts hold the same values)
    and against FP64 within the reference's published 5.1e-4 at 4096^3
    (README.md:29; 4.8e-4 measured in its tests/test_f16acc.py:39).  These
    seeds give at most 4.8e-4 against the oracle (one fp16 ulp at the top of
    the 8192^3 output, |c| up to 518) and 4.4e-4 against FP64; the oracle
    takes ~2 s at 4096^3 and ~11 s at 8192^3 on 16 host threads."""
    a, b = rnd((n, n), 50), rnd((n, n), 51)
    s = chunk32.chunked_sum(a, b)
    assert bool(torch.isfinite(s).all())
    # The reference's FP16 accumulator (tl.dot(..., out_dtype=fp16), kernel.py:49)
    # rounds inside a chunk too; the oracle's per-k16 model (two k16 steps per
    # chunk) reproduces its published 4.8e-4 at 4096^3.  The kernel rounds each
    # chunk once, and stays within the 1e-3 budget of that model as well.
    s16 = chunk32.chunked_sum(a, b, mode="per_k16") if n == 4096 else None
    f32 = chunk32.fp32_sum(a, b)
    ref64 = a.cuda().double() @ b.cuda().double()
    for b_t in (False, True):
        for out_dtype in (torch.float16, torch.float32):
            c, flags, cfg = run(a, b, out_dtype, b_transposed=b_t)
            assert cfg["tile"] == "256x256" and int(flags.sum()) == 0, (n, b_t, out_dtype, cfg)
            assert rel(c, s.to(out_dtype)) < TOL, (n, b_t, out_dtype)
            if out_dtype == torch.float32:
                assert_carries_chunk_rounding(c, s, f32, n, (n, b_t))
            if s16 is not None:
                assert rel(c, s16.to(out_dtype)) < TOL, (n, b_t, out_dtype, "per_k16")
            assert rel(c.cuda(), ref64) < 5.1e-4, (n, b_t, out_dtype)
            del c


@pytest.mark.parametrize("layer, n_out, n_in, biased", [("q/o", 1536, 1536, True), ("k/v", 256, 1536, True),
                                                        ("gate/up", 8960, 1536, False), ("down", 1536, 8960, False),
                                                        ("lm_head", 151936, 1536, False)])
def test_qwen_layer_shapes_match_oracle(layer, n_out, n_in, biased):
    """Qwen2.5-1.5B's linear layers at 2048 tokens: x ~ N(0, 1), weight
    N(0, 0.02) stored [out, in] and multiplied as w.t(), q/k/v with an
    N(0, 0.02) bias.  mm matches the oracle with no tile flagged, through
    whatever the shape plans (the K-group tiles for q/o, k/v and down,
    256x288 for gate/up, 256x256 for the lm_head); the fused bias equals the unfused
    `y = mm(x, w.t()); y += b` (f16acc/patch.py:28-30) bit for bit, and the
    patched nn.Linear returns those bits."""
    M = 2048
    x, w = rnd((M, n_in), 60), rnd((n_out, n_in), 61, 0.02)
    gx, gw = x.cuda(), w.cuda()
    c = f16acc.mm(gx, gw.t())
    s = chunk32.chunked_sum(x, w.t())
    assert bool(torch.isfinite(s).all())
    assert rel(c.cpu(), s.half()) < TOL, layer
    if layer != "lm_head":  # the FP16-accumulator model too (kernel.py:49); lm_head's is ~1 min on the host
        assert rel(c.cpu(), chunk32.chunked_sum(x, w.t(), mode="per_k16").half()) < TOL, layer
    if not biased:
        return
    bias = rnd((n_out,), 62, 0.02).cuda()
    fused = f16acc.kernel.mm_bias(gx, gw.t(), bias)
    unfused = c.clone()
    unfused += bias
    assert torch.equal(fused, unfused), layer
    lin = torch.nn.Linear(n_in, n_out, device="cuda", dtype=torch.float16)
    with torch.no_grad():
        lin.weight.copy_(gw)
        lin.bias.copy_(bias)
    f16acc.enable()
    try:
        before = f16acc.calls["chunked"]
        with torch.inference_mode():
            y = lin(gx)
        assert f16acc.calls["chunked"] == before + 1
    finally:
        f16acc.disable()
    assert torch.equal(y, fused), layer


@pytest.mark.parametrize("shape", [(1000, 777, 1234), (300, 256, 200), (129, 72, 136), (64, 40, 8),
                                   (257, 1536, 256), (33, 33, 33), (1, 64, 1)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_odd_and_edge_shapes(shape, out_dtype):
    M, K, N = shape
    a, b = rnd((M, K), 2), rnd((K, N), 3)
    for b_t in (False, True):
        c, flags, cfg = run(a, b, out_dtype, b_transposed=b_t)
        ref, rflags = oracle(a, b, out_dtype, cfg)
        assert torch.equal(flags, rflags)
        assert rel(c, ref) < TOL, (shape, b_t, cfg)
        assert rel(c, a.double() @ b.double()) < 2e-3


def test_fp32_accumulate_mode():
    a, b = rnd((512, 640), 4), rnd((640, 384), 5)
    c, _, _ = run(a, b, torch.float32, chunked=False)
    ref = a.float() @ b.float()
    assert rel(c, ref.double()) < 1e-5


def test_strided_operands_use_generic_path():
    # 300 x 233 x 200: below the size where mm packs strided operands
    a_big, b_big = rnd((300, 400), 6), rnd((200, 700), 7)
    a, b = a_big[:, ::2], b_big[:, 1::3]  # strides (400, 2) and (700, 3)
    ga, gb = a_big.cuda()[:, ::2], b_big.cuda()[:, 1::3]
    cfg = tile_config(ga, gb)
    assert cfg["family"] == "generic"
    c, flags = mm_flags(ga, gb, torch.float32)
    ref, rflags = oracle(a, b, torch.float32, cfg)
    assert torch.equal(flags.cpu(), rflags)
    assert rel(c.cpu(), ref) < TOL


def test_forced_overflow_closed_form_is_exact():
    # reference tests/test_f16acc.py:91-101: chunk sums are +96000 / -95900
    # (inf in fp16) but the exact result is 100
    w = torch.empty(128, 64, dtype=torch.float16)
    w[:, :32], w[:, 32:], w[:, 63] = 30.0, -30.0, -29.0
    x = torch.full((256, 64), 100.0, dtype=torch.float16)
    for out_dtype in (torch.float16, torch.float32):
        c, flags, cfg = run(x, w.t().contiguous(), out_dtype)
        assert torch.all(c == 100.0)
        assert flags.all()
        c, flags, cfg = run(x, w.t().contiguous(), out_dtype, b_transposed=True)
        assert torch.all(c == 100.0)


def test_chunk_whose_first_16_terms_overflow_is_not_flagged():
    """Where the chunk models part: a chunk whose first 16 terms sum past
    65504 but whose 32-term sum is 0.  An FP16 accumulator that rounds after
    16 terms (the oracle's per-k16 model of the reference's tl.dot with
    out_dtype=fp16, kernel.py:49) holds inf there, so the reference would
    flag the tile and redo it in FP32; the kernel rounds each chunk once
    (the oracle's round-once model), sees 0 and flags nothing.  Every output
    is exact either way (y == 100), so only the flags differ."""
    M, N, K = 256, 128, 64
    a = torch.full((M, K), 100.0, dtype=torch.float16)
    w = torch.zeros(N, K, dtype=torch.float16)
    w[:, :16], w[:, 16:32] = 50.0, -50.0  # 16 terms of 5000: 80000 > 65504, then back to 0
    w[:, 32] = 1.0
    ga, gw = a.cuda(), w.cuda()
    cfg = tile_config(ga, gw.t())
    c, flags = mm_flags(ga, gw.t(), torch.float32)
    once, fonce = chunk32.mm(a, w.t(), torch.float32, tile=(cfg["bm"], cfg["bn"]), return_flags=True)
    k16, fk16 = chunk32.mm(a, w.t(), torch.float32, tile=(cfg["bm"], cfg["bn"]), mode="per_k16",
                           return_flags=True)
    assert bool((fk16 == 1).all()) and int(fonce.sum()) == 0
    assert torch.equal(flags.cpu(), fonce)
    assert torch.all(c.cpu() == 100.0) and torch.equal(once, k16)


def test_nan_input_flags_its_tile():
    a, b = rnd((256, 128), 8), rnd((128, 256), 9)
    a[5, 7] = float("nan")
    c, flags, cfg = run(a, b, torch.float32)
    ref, rflags = oracle(a, b, torch.float32, cfg)
    assert torch.equal(flags, rflags) and flags.sum() >= 1
    assert torch.equal(torch.isnan(c), torch.isnan(ref))
    fin = ~torch.isnan(ref)
    assert rel(c[fin], ref[fin]) < TOL


def test_zero_sizes():
    a, b = torch.empty(256, 0, dtype=torch.float16), torch.empty(0, 16, dtype=torch.float16)
    c = f16acc.mm(a.cuda(), b.cuda())
    assert c.shape == (256, 16) and bool((c == 0).all())
    c = f16acc.mm(rnd((0, 64), 1).cuda(), rnd((64, 32), 2).cuda())
    assert c.shape == (0, 32)
    c = f16acc.mm(rnd((64, 64), 1).cuda(), rnd((64, 0), 2).cuda())
    assert c.shape == (64, 0)


@pytest.mark.parametrize("tile", ALL_TILES)
@pytest.mark.parametrize("K", [64, 128, 192, 200, 320, 1024])
def test_every_tile_matches_oracle(tile, K):
    """Each tile configuration, forced, on ragged M/N edges, for K of one to
    sixteen LDS stages (the three-stage rings of 256x128 / 128x256 see every
    fill and drain case), both B layouts, both output dtypes."""
    from f16acc_amd.kernel import mm_tile

    M, N = 300, 520
    a, b = rnd((M, K), 10 + K), rnd((K, N), 11 + K)
    ga = a.cuda()
    for b_t in (False, True):
        gb = b.t().contiguous().cuda().t() if b_t else b.cuda()
        cfg = tile_config(ga, gb, tile)
        assert cfg["tile"] == forced_tile_runs_as(tile, not b_t)
        for out_dtype in (torch.float32, torch.float16):
            c, flags = mm_flags(ga, gb, out_dtype, tile=tile)
            ref, rflags = oracle(a, b, out_dtype, cfg)
            assert torch.equal(flags.cpu(), rflags)
            assert rel(c.cpu(), ref) < TOL, (tile, K, b_t, out_dtype)
            if out_dtype == torch.float32:
                assert_carries_chunk_rounding(c, ref, a.float() @ b.float(), K, (tile, K, b_t))
        c32 = mm_tile(ga, gb, tile, torch.float32, chunked=False)
        assert rel(c32.cpu(), (a.float() @ b.float()).double()) < 1e-5


@pytest.mark.parametrize("tile", ["256x256", "256x288", "128x96k2", "64x32k4"])
def test_k_contiguous_slices_of_wider_buffers(tile):
    """a = x[:, :K] of a wider [M, K + 64] buffer and b = w[:, :K].t() of a
    wider [N, K + 40] weight: 16-byte aligned rows whose stride exceeds K,
    which the direct-to-LDS copies read in place (the copies clip at K by
    each stage's range and at M, N by the buffers' record counts).  Ragged
    M, N, a partial last stage (K = 200), both output dtypes, values and
    flags against the oracle."""
    M, N, K = 300, 333, 200
    xa, wb = rnd((M, K + 64), 130), rnd((N, K + 40), 131)
    gxa, gwb = xa.cuda(), wb.cuda()
    ga, gb = gxa[:, :K], gwb[:, :K].t()
    assert ga.stride() == (K + 64, 1) and gb.stride() == (1, K + 40)
    cfg = tile_config(ga, gb, tile)
    assert cfg["tile"] == tile and cfg["family"] == "fast"
    for out_dtype in (torch.float32, torch.float16):
        c, flags = mm_flags(ga, gb, out_dtype, tile=tile)
        ref, rflags = oracle(xa[:, :K], wb[:, :K].t(), out_dtype, cfg)
        assert torch.equal(flags.cpu(), rflags)
        assert rel(c.cpu(), ref) < TOL, (tile, out_dtype)


@pytest.mark.parametrize("tile", ALL_TILES)
def test_every_tile_stores_unaligned_rows_and_edges(tile):
    """fp16 rows of N = 517 halves start off 16-byte alignment, and M, N leave
    partial tiles: such tiles are staged through LDS and leave as 16-byte
    units at 2-byte aligned addresses, element by element at the edge.  The
    FP32 sums do not depend on the output dtype, so the fp16 output must be
    the fp32 output of the same tile rounded to fp16, bit for bit."""
    from f16acc_amd.kernel import mm_tile

    M, N, K = 300, 517, 200
    a, b = rnd((M, K), 30), rnd((K, N), 31)
    ga = a.cuda()
    for b_t in (False, True):
        gb = b.t().contiguous().cuda().t() if b_t else b.cuda()
        for chunked in (True, False):
            c16 = mm_tile(ga, gb, tile, torch.float16, chunked=chunked)
            c32 = mm_tile(ga, gb, tile, torch.float32, chunked=chunked)
            assert torch.equal(c16, c32.half()), (tile, b_t, chunked)
        ref, _ = oracle(a, b, torch.float16, tile_config(ga, gb, tile))
        assert rel(c16.cpu(), ref) < TOL


# Waves of each tile configuration (rows x columns of waves); wave (wm, wn)
# owns the (bm / rows) x (bn / columns) sub-tile at (wm, wn) of its tile.
WAVES = {"256x256": (4, 2), "256x128": (4, 2), "128x256": (2, 4), "128x128": (2, 2), "generic": (2, 2),
         "64x64": (2, 2), "128x96k2": (2, 2), "64x32k4": (2, 1), "256x288": (4, 2)}


def _wave_cases(tiles):
    out = []
    for tile in tiles:
        wmc, wnc = WAVES[tile]
        out += [(tile, wm, wn) for wm in range(wmc) for wn in range(wnc)]
    return out


def _overflow_block(tile, wm, wn, ti, tj):
    """First row and column of a 10 x 10 block inside wave (wm, wn)'s
    sub-tile of output tile (ti, tj)."""
    bm, bn = tile_dims(tile)
    wmc, wnc = WAVES[tile]
    return ti * bm + wm * (bm // wmc) + 5, tj * bn + wn * (bn // wnc) + 3


@pytest.mark.parametrize("tile, wm, wn", _wave_cases(ALL_TILES))
def test_every_tile_redoes_overflow_in_every_wave(tile, wm, wn):
    """Overflow closed form (reference tests/test_f16acc.py:91-101) placed in
    one wave's sub-tile of tile (1, 1) of a larger grid, for every wave of
    every tile: the flag one wave raises reaches the whole workgroup, so that
    tile is flagged and redone exactly, and no other tile is."""
    M, N, K = 512, 512, 128
    a = rnd((M, K), 20, 0.5)
    b = rnd((K, N), 21, 0.5)
    r0, c0 = _overflow_block(tile, wm, wn, 1, 1)
    a[r0:r0 + 10, :] = 100.0
    b[:, c0:c0 + 10] = 0.0
    b[:32, c0:c0 + 10], b[32:64, c0:c0 + 10], b[64:96, c0:c0 + 10], b[96:, c0:c0 + 10] = 30.0, -30.0, 30.0, -30.0
    b[127, c0:c0 + 10] = -29.0
    # b row-major, except for the tiles that read a K-contiguous b only
    ga, gb = a.cuda(), (b.t().contiguous().cuda().t() if tile in KC_ONLY_FALLBACK else b.cuda())
    cfg = tile_config(ga, gb, tile)
    assert cfg["tile"] == tile
    c, flags = mm_flags(ga, gb, torch.float32, tile=tile)
    ref, rflags = oracle(a, b, torch.float32, cfg)
    assert int(rflags.sum()) == 1 and rflags[1, 1] == 1
    assert torch.equal(flags.cpu(), rflags), (tile, wm, wn)
    assert torch.all(c[r0:r0 + 10, c0:c0 + 10].cpu() == 100.0)
    assert rel(c.cpu(), ref) < TOL


@pytest.mark.parametrize("tile, wm, wn", _wave_cases(["256x256", "256x288"]))
def test_overflow_in_the_last_column_of_the_last_stage(tile, wm, wn):
    """The chunked 256x256 and 256x288 loops multiply a stage's last column
    after the stage barrier, while they read the next stage's fragments (past
    the last stage: a slot of zeros).  The overflow closed form (reference
    tests/test_f16acc.py:91-101) lies in the last stage only (K = 320: chunks
    8 and 9, the earlier chunks of those rows are zeros), in the last row block
    and the last column of one wave's sub-tile of tile (1, 1): exactly that
    tile is flagged and its redone block is exact; both b layouts for 256x256."""
    bm, bn = tile_dims(tile)
    wmc, wnc = WAVES[tile]
    M, N, K = 2 * bm, 2 * bn, 320
    a = rnd((M, K), 44, 0.5)
    b = rnd((K, N), 45, 0.5)
    r0 = bm + wm * (bm // wmc) + bm // wmc - 14  # rows 50-59 of the wave's 64: its last row block
    c0 = bn + wn * (bn // wnc) + bn // wnc - 12  # columns in the wave's last 16-column block
    a[r0:r0 + 10, :] = 0.0
    a[r0:r0 + 10, 256:] = 100.0
    b[:, c0:c0 + 10] = 0.0
    b[256:288, c0:c0 + 10], b[288:320, c0:c0 + 10] = 30.0, -30.0
    b[319, c0:c0 + 10] = -29.0
    ga = a.cuda()
    for b_row_major in ((False, True) if tile == "256x256" else (False,)):
        gb = b.cuda() if b_row_major else b.t().contiguous().cuda().t()
        cfg = tile_config(ga, gb, tile)
        assert cfg["tile"] == tile
        c, flags = mm_flags(ga, gb, torch.float32, tile=tile)
        ref, rflags = oracle(a, b, torch.float32, cfg)
        assert int(rflags.sum()) == 1 and rflags[1, 1] == 1
        assert torch.equal(flags.cpu(), rflags), (tile, wm, wn, b_row_major)
        assert torch.all(c[r0:r0 + 10, c0:c0 + 10].cpu() == 100.0)
        assert rel(c.cpu(), ref) < TOL


K_GROUPS = {"128x96k2": 2, "64x32k4": 4}


@pytest.mark.parametrize("tile, wm, wn, group", [(t, wm, wn, g) for t, wm, wn in _wave_cases(list(K_GROUPS))
                                                 for g in range(K_GROUPS[t])])
def test_k_group_tiles_redo_overflow_in_every_group_and_wave(tile, wm, wn, group):
    """K-group tiles split K inside the workgroup: group g sums stages
    [2g, 2g + 2) of K = 128 * groups.  The overflow closed form (reference
    tests/test_f16acc.py:91-101) is placed in one group's K range only (the
    other groups' sums are exact zeros there), in one wave's sub-tile of
    tile (1, 1): the reduced sum is NaN, so exactly that tile is flagged,
    redone over all of K in FP32 and comes out exact; both b layouts (a
    row-major b runs 128x96k2 as 128x128)."""
    groups = K_GROUPS[tile]
    M, N, K = 512, 512, 128 * groups
    a = rnd((M, K), 40, 0.5)
    b = rnd((K, N), 41, 0.5)
    r0, c0 = _overflow_block(tile, wm, wn, 1, 1)
    k0 = 128 * group
    a[r0:r0 + 10, :] = 100.0
    b[:, c0:c0 + 10] = 0.0
    for q, v in enumerate((30.0, -30.0, 30.0, -30.0)):
        b[k0 + 32 * q:k0 + 32 * q + 32, c0:c0 + 10] = v
    b[k0 + 127, c0:c0 + 10] = -29.0
    ga = a.cuda()
    for b_row_major in (False, True):
        gb = b.cuda() if b_row_major else b.t().contiguous().cuda().t()
        cfg = tile_config(ga, gb, tile)
        assert cfg["tile"] == forced_tile_runs_as(tile, b_row_major)
        c, flags = mm_flags(ga, gb, torch.float32, tile=tile)
        ref, rflags = oracle(a, b, torch.float32, cfg)
        assert int(rflags.sum()) == 1 and rflags[r0 // cfg["bm"], c0 // cfg["bn"]] == 1
        assert torch.equal(flags.cpu(), rflags), (tile, wm, wn, group, b_row_major)
        assert torch.all(c[r0:r0 + 10, c0:c0 + 10].cpu() == 100.0)
        assert rel(c.cpu(), ref) < TOL


@pytest.mark.parametrize("tile", list(K_GROUPS))
@pytest.mark.parametrize("K", [0, 8, 64, 72, 136, 200, 448, 1536, 1560])
def test_k_group_tiles_with_uneven_and_empty_groups(tile, K):
    """K ranges that leave the last K groups with fewer stages or none
    (K = 64 on four groups: one stage; K = 0: none at all), a partial last
    stage, fp16 and fp32 out, chunked and FP32 modes, against the oracle."""
    from f16acc_amd.kernel import mm_tile

    M, N = 200, 136
    a, b = rnd((M, K), 50 + K), rnd((K, N), 51 + K)
    ga, gb = a.cuda(), b.t().contiguous().cuda().t()
    cfg = tile_config(ga, gb, tile)
    assert cfg["tile"] == tile or K == 0  # K = 0: no layout to read, any tile
    for out_dtype in (torch.float32, torch.float16):
        c, flags = mm_flags(ga, gb, out_dtype, tile=tile)
        ref, rflags = oracle(a, b, out_dtype, cfg)
        assert torch.equal(flags.cpu(), rflags)
        if K == 0:
            assert bool((c == 0).all())
        else:
            assert rel(c.cpu(), ref) < TOL, (tile, K, out_dtype)
    c32 = mm_tile(ga, gb, tile, torch.float32, chunked=False)
    if K:
        assert rel(c32.cpu(), (a.float() @ b.float()).double()) < 1e-5


def _packed_case(a, b):
    """The operands mm runs on after packing, and whether both are fast-path."""
    from f16acc_amd.kernel import _fast_a, _fast_b, _operands

    M, K = a.shape
    N = b.shape[1]
    a2, b2, K2 = _operands(a, b, M, N, K)
    return a2, b2, K2, _fast_a(a2, K2) and _fast_b(b2, K2, N)


@pytest.mark.parametrize("case", ["odd_k", "odd_k_wt", "row_major_odd_n", "offset_view", "strided"])
def test_misaligned_operands_match_oracle(case):
    """Operands the direct-to-LDS copies cannot read: unit-stride rows at any
    even address are read in place by the register-staged loader where the
    table picks 128x128 or 64x64; anything else (and every case on a forced
    256x256) is packed first (zero-padded K) and runs on a fast tile.  Both
    ways match the oracle."""
    from f16acc_amd.kernel import mm_tile

    M, K, N = 257, 1001, 193
    if case == "odd_k":  # a [M, K] with K % 8 != 0, b row-major
        a, b = rnd((M, K), 30), rnd((K, N), 31)
        ga, gb = a.cuda(), b.cuda()
    elif case == "odd_k_wt":  # b as the w.t() view of an [N, K] weight
        a, w = rnd((M, K), 32), rnd((N, K), 33)
        b = w.t()
        ga, gb = a.cuda(), w.cuda().t()
    elif case == "row_major_odd_n":  # row-major b with N % 8 != 0: transposing pack
        K = 1024
        a, b = rnd((M, K), 34), rnd((K, N), 35)
        ga, gb = a.cuda(), b.cuda()
    elif case == "offset_view":  # views starting one element in: misaligned pointers and strides
        K = 1024
        abig, bbig = rnd((M, K + 1), 36), rnd((K + 1, N + 7), 37)
        a, b = abig[:, 1:], bbig[1:, 3:3 + N]
        ga, gb = abig.cuda()[:, 1:], bbig.cuda()[1:, 3:3 + N]
    else:  # both operands strided in both dimensions
        abig, bbig = rnd((M, 2 * K), 38), rnd((K, 3 * N), 39)
        a, b = abig[:, ::2], bbig[:, 1::3]
        ga, gb = abig.cuda()[:, ::2], bbig.cuda()[:, 1::3]
    a2, b2, K2, fast = _packed_case(ga, gb)
    cfg = tile_config(ga, gb)
    if case == "strided":
        assert fast and K2 % 8 == 0 and K2 - a.shape[1] < 8 and cfg["family"] == "fast"
        # packed copies start every row on a 128-byte line
        assert a2.stride(0) % 64 == 0 and a2.data_ptr() % 128 == 0
        assert b2.stride(1) % 64 == 0 and b2.data_ptr() % 128 == 0
    else:
        assert cfg["family"] == "reg" and cfg["tile"] in ("128x128", "64x64"), cfg
        assert a2.data_ptr() == ga.data_ptr() and b2.data_ptr() == gb.data_ptr() and K2 == a.shape[1]
    for out_dtype in (torch.float32, torch.float16):
        c, flags = mm_flags(ga, gb, out_dtype)
        ref, rflags = oracle(a, b, out_dtype, cfg)
        assert torch.equal(flags.cpu(), rflags)
        assert rel(c.cpu(), ref) < TOL, (case, out_dtype)
        assert rel(c.cpu(), a.double() @ b.double()) < 2e-3
        # the same operands packed and run on 256x256
        c256 = mm_tile(ga, gb, "256x256", out_dtype)
        assert rel(c256.cpu(), oracle(a, b, out_dtype, tile_config(ga, gb, "256x256"))[0]) < TOL


# The 64x64 tile has a register loader for a K-contiguous b only (its 128
# registers per lane hold no more); forced with a row-major b it gathers.
_REG_CASES = [(tile, case) for tile in ("128x128", "64x64")
              for case in ("odd_k_wt", "odd_k_row_major", "offset_views", "odd_n_row_major")
              if not (tile == "64x64" and case in ("odd_k_row_major", "odd_n_row_major"))]


@pytest.mark.parametrize("tile, case", _REG_CASES)
def test_reg_loader_equals_packed_copies_bit_for_bit(tile, case):
    """The register-staged loader fills the LDS stages exactly as the
    direct-to-LDS copies fill them from packed, zero-padded operands, so the
    same tile gives the same bits either way: chunked and FP32 modes, ragged
    M, N and K (units cut at K and, for a row-major b, at N), overflow redo
    included (one row block of a is large enough to overflow its chunks)."""
    from f16acc_amd.kernel import _pack, mm_tile

    M, N, K = 200, 136, 777
    if case == "odd_n_row_major":
        N, K = 131, 320
    abig = rnd((M + 1, K + 3), 80)
    abig[64:80] *= 10000.0  # chunk sums past 65504 in one row block
    if case == "offset_views":
        ga = abig.cuda()[1:, 3:]
        bbig = rnd((N + 5, K + 1), 81)
        gb = bbig.cuda()[5:, 1:].t()
    else:
        ga = abig.cuda()[:M, :K]
        if case in ("odd_k_wt",):
            gb = rnd((N, K), 82).cuda().t()
        else:
            gb = rnd((K, N), 83).cuda()
    cfg = tile_config(ga, gb, tile)
    assert cfg["family"] == "reg", cfg
    ld = -(-K // 64) * 64
    pa = _pack(ga, M, K, ga.stride(0), ga.stride(1), ld)[:, :K + (-K % 8)]
    pb = _pack(gb, N, K, gb.stride(1), gb.stride(0), ld)[:, :K + (-K % 8)].t()
    assert tile_config(pa, pb, tile)["family"] == "fast"
    for chunked in (True, False):
        c_reg = mm_tile(ga, gb, tile, torch.float32, chunked=chunked)
        c_fast = mm_tile(pa, pb, tile, torch.float32, chunked=chunked)
        assert torch.equal(c_reg, c_fast), (tile, case, chunked)
    _, flags = mm_flags(ga, gb, torch.float32, tile=tile)
    ref, rflags = oracle(ga.cpu(), gb.cpu(), torch.float32, cfg)
    assert torch.equal(flags.cpu(), rflags) and int(flags.sum()) > 0
    assert rel(c_reg.cpu(), (ga.cpu().float() @ gb.cpu().float()).double()) < 1e-5


def test_odd_config_2049_1537_8961():
    """The odd Qwen-layer config (M=2049, N=1537, K=8961, weight stored
    [N, K]) against the oracle: K-padding by the pack must not change the
    last, one-element chunk."""
    a, w = rnd((2049, 8961), 40), rnd((1537, 8961), 41, 0.02)
    ga, gw = a.cuda(), w.cuda()
    from f16acc_amd.kernel import _pack, mm_tile

    c, flags = mm_flags(ga, gw.t(), torch.float32)
    cfg = tile_config(ga, gw.t())
    assert (cfg["family"], cfg["tile"]) == ("fast", "128x128")  # packed: cheaper than in place at this size
    ref, rflags = oracle(a, w.t(), torch.float32, cfg)
    assert int(flags.sum()) == 0 and int(rflags.sum()) == 0
    assert rel(c.cpu(), ref) < TOL
    # forced, the tile reads the rows in place: the same bits as the same
    # tile on packed copies, and the oracle's result
    assert tile_config(ga, gw.t(), "128x128")["family"] == "reg"
    c_reg = mm_tile(ga, gw.t(), "128x128", torch.float32)
    pa = _pack(ga, 2049, 8961, 8961, 1, 9024)[:, :8968]
    pw = _pack(gw, 1537, 8961, 8961, 1, 9024)[:, :8968]
    assert torch.equal(c_reg, mm_tile(pa, pw.t(), "128x128", torch.float32))
    assert rel(c_reg.cpu(), ref) < TOL


@pytest.mark.parametrize("n, blocks", [(1024, 2), (4096, 7)])
def test_overflow_stress_flags_exactly_the_block_intersections(n, blocks):
    """The overflow stress workload, n^3 with `blocks` of the n / 128
    row-blocks of a and column-blocks of b set to U(200, 255) (at 4096, 7 of
    32: 4.8 % of the 128 x 128 tiles): only the intersection tiles overflow;
    they are flagged like the oracle's, equal the unsplit FP32-accumulate
    mode bit for bit (the redo runs all of K in one workgroup: same tile,
    same summation order), and every other tile matches the oracle."""
    import bench
    from f16acc_amd.kernel import mm_tile

    a, b, rows, cols = bench.overflow_inputs(n=n, blocks=blocks)
    ga, gb = a.cuda(), b.cuda()
    cfg = tile_config(ga, gb)
    c, flags = mm_flags(ga, gb, torch.float32)
    c32 = mm_tile(ga, gb, cfg["tile"], torch.float32, chunked=False)
    ref, rflags = oracle(a, b, torch.float32, cfg)
    assert torch.equal(flags.cpu(), rflags)
    bm, bn = cfg["bm"], cfg["bn"]
    # each overflowing block is 128 x 128: it covers one tile of 128 or more,
    # or 128 / bm x 128 / bn smaller tiles
    sm, sn = max(1, 128 // bm), max(1, 128 // bn)
    want = {(r * 128 // bm + i, q * 128 // bn + j) for r in rows for q in cols for i in range(sm) for j in range(sn)}
    assert {tuple(t) for t in flags.nonzero().tolist()} == want
    mask = flags.bool().repeat_interleave(bm, 0).repeat_interleave(bn, 1)[:n, :n]
    assert torch.equal(c[mask], c32[mask])
    assert rel(c.cpu()[~mask.cpu()], ref[~mask.cpu()]) < TOL


@pytest.mark.parametrize("shape", [(256, 384, 640), (300, 1000, 77), (300, 200, 517), (1024, 1536, 256),
                                   (128, 0, 16)])
def test_fused_bias_equals_unfused_add_bit_for_bit(shape):
    """The patched nn.Linear adds its bias in the GEMM's store; the result must
    equal the reference's unfused y = mm(x2, w.t()); y += b exactly
    (f16acc/patch.py:28-30), including K = 0 (the zero-width layer)."""
    from f16acc_amd import patch

    M, K, N = shape
    x, w, bias = rnd((M, K), 50).cuda(), rnd((N, K), 51, 0.05).cuda(), rnd((N,), 52, 0.5).cuda()
    unfused = f16acc.mm(x, w.t())
    unfused += bias
    with torch.no_grad():
        fused = patch.linear(x, w, bias)
    assert torch.equal(fused, unfused)


@pytest.mark.parametrize("M, N, K, tile", [(2048, 8192, 1536, "256x256"), (2048, 8960, 1536, "256x288"),
                                           (2048, 1536, 1536, "128x96k2"), (2048, 256, 1536, "64x32k4"),
                                           (256, 4096, 5120, "128x128")])
def test_fused_bias_on_tiles_the_redo_recomputes(M, N, K, tile):
    """The fused bias where the overflow redo stores a tile a second time:
    the overflow closed form (reference tests/test_f16acc.py:91-101: chunk
    partials of +-96000, exact sum 100) in 8 x 8 blocks at the four corner
    tiles of each table pick (the last: 128x128 split along K).  The fused
    result equals the reference's unfused y = mm(x2, w.t()); y += b
    (f16acc/patch.py:28-30) bit for bit, in fp16 through the patched
    nn.Linear and in fp32 through mm_bias; the redone blocks hold exactly
    100 + b; exactly the four corner tiles are flagged."""
    from f16acc_amd import patch
    from f16acc_amd.kernel import mm_bias

    x, w, bias = rnd((M, K), 90), rnd((N, K), 91, 0.02), rnd((N,), 92, 0.5)
    pattern = torch.full((K,), 30.0)
    pattern.view(-1, 32)[1::2] = -30.0
    pattern[K - 1] = -29.0
    rows, cols = [(5, 13), (M - 13, M - 5)], [(7, 15), (N - 11, N - 3)]
    for r0, r1 in rows:
        x[r0:r1] = 100.0
    for c0, c1 in cols:
        w[c0:c1] = pattern.half()
    gx, gw, gbias = x.cuda(), w.cuda(), bias.cuda()
    cfg = tile_config(gx, gw.t())
    assert cfg["tile"] == tile
    _, flags = mm_flags(gx, gw.t())
    want = torch.zeros(cfg["tiles_m"], cfg["tiles_n"], dtype=torch.uint8)
    want[0, 0] = want[0, -1] = want[-1, 0] = want[-1, -1] = 1
    assert torch.equal(flags.cpu(), want)
    unfused = f16acc.mm(gx, gw.t())
    unfused += gbias
    with torch.no_grad():
        fused = patch.linear(gx, gw, gbias)
    assert torch.equal(fused, unfused)
    fused32 = mm_bias(gx, gw.t(), gbias, torch.float32)
    unfused32 = f16acc.mm(gx, gw.t(), torch.float32) + gbias.float()
    assert torch.equal(fused32, unfused32)
    for r0, r1 in rows:
        for c0, c1 in cols:
            exact = (torch.full((c1 - c0,), 100.0, dtype=torch.float16) + bias[c0:c1]).expand(r1 - r0, -1)
            assert torch.equal(fused[r0:r1, c0:c1].cpu(), exact)
            assert torch.equal(fused32[r0:r1, c0:c1].cpu(), (100.0 + bias[c0:c1].float()).expand(r1 - r0, -1))


def test_fused_bias_fp32_output_matches_oracle():
    from f16acc_amd.kernel import mm_bias

    a, w, bias = rnd((300, 520), 53), rnd((200, 520), 54), rnd((200,), 55)
    c = mm_bias(a.cuda(), w.cuda().t(), bias.cuda(), torch.float32)
    ref = chunk32.mm(a, w.t(), torch.float32, tile=(128, 128)) + bias.float()
    assert rel(c.cpu(), ref) < TOL
    with pytest.raises(ValueError):
        mm_bias(a.cuda(), w.cuda().t(), bias[:10].cuda())


def _split_plan(ga, gb):
    import ctypes

    from f16acc_amd import _lib

    M, K = ga.shape
    N = gb.shape[1]
    n = ctypes.c_size_t()
    _lib.check(_lib.workspace_size(M, N, K, ga.stride(0), ga.stride(1), gb.stride(0), gb.stride(1), ga.data_ptr(),
                                   gb.data_ptr(), ctypes.byref(n)))
    return max(n.value - _lib.WS_HEADER, 0)  # the split-K partials' bytes


@pytest.mark.parametrize("shape, b_layout", [((256, 256, 4096), "row-major"), ((1024, 256, 4096), "row-major"),
                                             ((300, 200, 4200), "row-major"), ((512, 384, 8960), "row-major"),
                                             ((256, 4096, 5120), "w.t()")])
def test_split_k_matches_oracle(shape, b_layout):
    """Shapes with few output tiles are split along K into chunk-aligned
    ranges; a second launch adds the FP32 partials per tile.  Results and
    flags match the oracle; repeated calls (sharing the stream's workspace)
    give identical bits.  (With b = w.t() most of these shapes take a K-group
    tile instead: b is row-major there, except for a shape whose two rounds
    of 64x32 tiles lose to a split in five.)"""
    M, N, K = shape
    a, w = rnd((M, K), 60 + K), rnd((N, K), 61 + K)
    ga, gb = a.cuda(), (w.cuda().t() if b_layout == "w.t()" else w.t().contiguous().cuda())
    a2, b2, K2, _ = _packed_case(ga, gb)
    assert _split_plan(a2, b2) > 0, "shape expected to be split"
    cfg = tile_config(a2, b2)
    for out_dtype in (torch.float32, torch.float16):
        c, flags = mm_flags(ga, gb, out_dtype)
        ref, rflags = oracle(a, w.t(), out_dtype, cfg)
        assert torch.equal(flags.cpu(), rflags)
        assert rel(c.cpu(), ref) < TOL, (shape, out_dtype)
        # the workspace is reused across calls: another split problem in between
        other_a, other_b = rnd((256, 4096), 1).cuda(), rnd((4096, 256), 2).cuda()
        assert _split_plan(other_a, other_b) > 0
        f16acc.mm(other_a, other_b)
        again = f16acc.mm(ga, gb, out_dtype)
        assert torch.equal(again, c)


def _gemm_tile_ws(ga, gb, c, flags, tile, ws):
    """f16acc_gemm_tile_ws through the C ABI: tile forced, split-K workspace."""
    from f16acc_amd import _lib

    M, K = ga.shape
    N = gb.shape[1]
    rc = _lib.gemm_tile_ws(ga.data_ptr(), gb.data_ptr(), c.data_ptr(), flags.data_ptr(), M, N, K, ga.stride(0),
                           ga.stride(1), gb.stride(0), gb.stride(1), c.stride(0), c.stride(1),
                           _lib.OUT_F32 if c.dtype == torch.float32 else _lib.OUT_F16, 1,
                           torch.cuda.current_stream().cuda_stream, _lib.TILES.index(tile), ws.data_ptr(), ws.numel())
    _lib.check(rc)


@pytest.mark.parametrize("tile, wm, wn", _wave_cases(["128x128", "256x128", "128x256"]))
def test_split_k_overflow_in_every_wave_of_a_split_tile(tile, wm, wn):
    """A chunk overflow inside one K range of a split tile, placed in each
    wave's sub-tile of the last tile in turn, on every tile that splits
    (128x128 is the table's pick here; 256x128 and 128x256 are forced): the
    summed tile is not finite, so the finishing launch flags it, whichever
    wave holds the overflow, and recomputes it over all of K in FP32, exactly
    (the reference's closed form, tests/test_f16acc.py:91-101, widened)."""
    M, N, K = 256, 256, 4096
    a = rnd((M, K), 70, 0.1)
    b = rnd((K, N), 71, 0.1)
    bm, bn = map(int, tile.split("x"))
    ti, tj = M // bm - 1, N // bn - 1
    r0, c0 = _overflow_block(tile, wm, wn, ti, tj)
    a[r0:r0 + 10, :] = 100.0
    b[:, c0:c0 + 10] = 0.0
    b[2048:2080, c0:c0 + 10], b[2080:2112, c0:c0 + 10] = 30.0, -30.0  # chunk sums of +-96000 in one split
    b[2111, c0:c0 + 10] = -29.0
    ga, gb = a.cuda(), b.cuda()
    cfg = tile_config(ga, gb, tile)
    if tile == "128x128":
        assert tile_config(ga, gb)["tile"] == tile and _split_plan(ga, gb) > 0
    ws = torch.full((32 << 20,), 0x7f, dtype=torch.uint8, device="cuda")
    ws[:_lib.WS_HEADER].zero_()  # an empty deferred redo list; garbage behind it
    c = torch.empty(M, N, device="cuda", dtype=torch.float32)
    flags = torch.zeros(cfg["tiles_m"], cfg["tiles_n"], device="cuda", dtype=torch.uint8)
    _gemm_tile_ws(ga, gb, c, flags, tile, ws)
    torch.cuda.synchronize()
    assert bool((ws != 0x7f).any()), "the split path did not run"
    ref, rflags = oracle(a, b, torch.float32, cfg)
    assert int(rflags.sum()) == 1 and rflags[ti, tj] == 1
    assert torch.equal(flags.cpu(), rflags), (tile, wm, wn)
    assert torch.all(c[r0:r0 + 10, c0:c0 + 10].cpu() == 100.0)
    assert rel(c.cpu(), ref) < TOL


def test_split_k_bias_and_ws_entry_without_workspace():
    """A biased projection with few output tiles and long K (256 x 4096 x
    5120) takes the split path through patch.linear and still equals the
    unfused y = mm(x2, w.t()); y += b bit for bit; f16acc_gemm_ws with no
    workspace is f16acc_gemm."""
    from f16acc_amd import _lib, patch

    x, w, bias = rnd((256, 5120), 72).cuda(), rnd((4096, 5120), 73, 0.02).cuda(), rnd((4096,), 74, 0.02).cuda()
    assert _split_plan(x, w.t()) > 0
    unfused = f16acc.mm(x, w.t())
    unfused += bias
    with torch.no_grad():
        assert torch.equal(patch.linear(x, w, bias), unfused)
    c = torch.empty(256, 4096, device="cuda", dtype=torch.float16)
    st = torch.cuda.current_stream().cuda_stream
    rc = _lib.gemm_ws(x.data_ptr(), w.data_ptr(), None, c.data_ptr(), None, 256, 4096, 5120, x.stride(0), 1,
                      1, 5120, 4096, 1, 0, 1, st, None, 0)
    assert rc == 0
    plain = torch.empty_like(c)
    assert _lib.gemm(x.data_ptr(), w.data_ptr(), plain.data_ptr(), None, 256, 4096, 5120, x.stride(0), 1, 1, 5120,
                     4096, 1, 0, 1, st) == 0
    assert torch.equal(c, plain)
    assert rel(c.cpu(), chunk32.mm(x.cpu(), w.cpu().t(), torch.float16, tile=(128, 128))) < TOL


def _tail_split(ga, gb):
    import ctypes

    from f16acc_amd import _lib

    n = ctypes.c_int64()
    M, K = ga.shape
    _lib.check(_lib.tail_split(M, gb.shape[1], K, ga.stride(0), ga.stride(1), gb.stride(0), gb.stride(1),
                               ga.data_ptr(), gb.data_ptr(), ctypes.byref(n)))
    return n.value


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("b_layout", ["w.t()", "row-major"])
def test_ragged_round_tail_split_equals_single_grid(out_dtype, b_layout):
    """Qwen2.5-1.5B gate/up (2048 x 8960 x 1536): 280 tiles of 256x256 for
    256 CUs.  With a row-major b, mm runs columns 0..8191 as one round of
    256x256 tiles and the last 768 as a second launch (B offset by 8192
    columns); with b = w.t() it runs one round of 256 tiles of 256x288 (the
    last column of tiles 32 wide) and no cut.  Every element is computed as
    in the single grid mm_flags launches (bit for bit) and matches the
    oracle."""
    x, w = rnd((2048, 1536), 80), rnd((8960, 1536), 81, 0.05)
    gx = x.cuda()
    gb = w.cuda().t() if b_layout == "w.t()" else w.t().contiguous().cuda()
    assert _tail_split(gx, gb) == (0 if b_layout == "w.t()" else 8192)
    assert tile_config(gx, gb)["tile"] == ("256x288" if b_layout == "w.t()" else "128x128")
    c = f16acc.mm(gx, gb, out_dtype)
    c1, flags = mm_flags(gx, gb, out_dtype)
    assert int(flags.sum()) == 0
    assert torch.equal(c, c1)
    assert rel(c.cpu(), chunk32.mm(x, w.t(), out_dtype, tile=(128, 128))) < TOL


def test_ragged_round_tail_split_redoes_overflow_in_both_launches():
    """The reference's forced-overflow closed form (tests/test_f16acc.py:91-101:
    chunk sums of +-96000, exact result 100) in output columns 500..509 (the
    256x256 launch) and 8500..8509 (the tail launch): both come out exact."""
    x, w = rnd((2048, 1536), 82, 0.5), rnd((8960, 1536), 83, 0.5)
    x[100:110, :] = 100.0
    for c0 in (500, 8500):
        cols = slice(c0, c0 + 10)
        w[cols, :] = 0.0
        w[cols, 0:32], w[cols, 32:64], w[cols, 64:96], w[cols, 96:128] = 30.0, -30.0, 30.0, -30.0
        w[cols, 127] = -29.0
    gx, gb = x.cuda(), w.t().contiguous().cuda()  # row-major b: the cut
    assert _tail_split(gx, gb) == 8192
    c = f16acc.mm(gx, gb, torch.float32)
    assert torch.all(c[100:110, 500:510] == 100.0) and torch.all(c[100:110, 8500:8510] == 100.0)
    assert rel(c.cpu(), chunk32.mm(x, w.t(), torch.float32, tile=(128, 128))) < TOL


def test_ragged_round_tail_split_fused_bias():
    """The tail launch gets the bias from its first column on: the fused
    result still equals the unfused y = mm(x2, b); y += bias bit for bit.
    patch.linear's own layout (b = w.t()) runs the same projection as one
    256x288 round, whose last column of tiles is 32 wide: the fused bias is
    bit-equal there too."""
    from f16acc_amd import _lib, patch

    x, w, bias = rnd((2048, 1536), 84).cuda(), rnd((8960, 1536), 85, 0.02).cuda(), rnd((8960,), 86, 0.5).cuda()
    b_rm = w.t().contiguous()
    assert _tail_split(x, b_rm) == 8192
    unfused = f16acc.mm(x, b_rm)
    unfused += bias
    fused = torch.empty_like(unfused)
    st = torch.cuda.current_stream().cuda_stream
    assert _lib.gemm_bias(x.data_ptr(), b_rm.data_ptr(), bias.data_ptr(), fused.data_ptr(), None, 2048, 8960,
                          1536, x.stride(0), 1, 8960, 1, 8960, 1, 0, 1, st) == 0
    assert torch.equal(fused, unfused)
    assert _tail_split(x, w.t()) == 0 and tile_config(x, w.t())["tile"] == "256x288"
    unfused = f16acc.mm(x, w.t())
    unfused += bias
    with torch.no_grad():
        assert torch.equal(patch.linear(x, w, bias), unfused)



@pytest.mark.parametrize("shape", [(300, 200, 517), (512, 384, 256), (1024, 1024, 1024)])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_c_abi_writes_any_output_strides(shape, out_dtype):
    """f16acc_gemm writes c at any element strides (scm, scn): column-major,
    rows padded to a pitch that breaks 16-byte alignment, every other
    column.  The tile and its arithmetic depend on a and b only, so each
    result equals the same call's contiguous output bit for bit, and every
    element of the surrounding buffer that is not part of c keeps its
    sentinel."""
    from f16acc_amd import _lib

    M, N, K = shape
    a, w = rnd((M, K), 70).cuda(), rnd((N, K), 71).cuda()
    b = w.t()
    out = _lib.OUT_F32 if out_dtype == torch.float32 else _lib.OUT_F16
    stream = torch.cuda.current_stream().cuda_stream
    want = torch.empty(M, N, device="cuda", dtype=out_dtype)
    _lib.check(_lib.gemm(a.data_ptr(), b.data_ptr(), want.data_ptr(), None, M, N, K, a.stride(0), a.stride(1),
                         b.stride(0), b.stride(1), N, 1, out, 1, stream))
    sentinel = -7.0
    layouts = {"column-major": (N * M, 1, M, lambda buf: buf.view(N, M).t()),
               "pitch N+3": (M * (N + 3), N + 3, 1, lambda buf: buf.view(M, N + 3)[:, :N]),
               "every other column": (M * 2 * N, 2 * N, 2, lambda buf: buf.view(M, 2 * N)[:, ::2])}
    for name, (numel, scm, scn, view) in layouts.items():
        buf = torch.full((numel + 64,), sentinel, device="cuda", dtype=out_dtype)
        body = buf[32:32 + numel]
        _lib.check(_lib.gemm(a.data_ptr(), b.data_ptr(), body.data_ptr(), None, M, N, K, a.stride(0), a.stride(1),
                             b.stride(0), b.stride(1), scm, scn, out, 1, stream))
        torch.cuda.synchronize()
        c = view(body)
        assert torch.equal(c, want), (name, shape, out_dtype)
        written = torch.zeros(numel, dtype=torch.bool, device="cuda")
        view(written.view(-1)).fill_(True)
        untouched = torch.cat([buf[:32], body[~written], buf[32 + numel:]])
        assert bool((untouched == sentinel).all()), (name, shape, out_dtype)


def test_launch_stream_is_the_current_torch_stream():
    """The launch goes on torch's current stream of the operands' device (the
    raw query the Python layer uses agrees with the public one), also inside
    a stream context."""
    from f16acc_amd.kernel import _stream

    dev = torch.device("cuda", 0)
    assert _stream(dev) == torch.cuda.current_stream(dev).cuda_stream
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert _stream(dev) == s.cuda_stream == torch.cuda.current_stream(dev).cuda_stream
        a, b = rnd((300, 520), 97).cuda(), rnd((520, 200), 98).cuda()
        c = f16acc.mm(a, b)
    s.synchronize()
    assert rel(c.cpu(), chunk32.mm(a.cpu(), b.cpu(), torch.float16, tile=(128, 128))) < TOL


def test_concurrent_calls_on_two_streams_from_two_threads():
    """mm keeps no shared state (the reference hands best_config to its redo
    launch through a global, README.md:48): two host threads calling it on
    their own streams, split-K and two-launch shapes included, get the same
    bits as one thread alone."""
    import threading

    shapes = [(2048, 256, 4096), (2048, 8960, 1536), (300, 520, 640)]
    inputs = [(rnd((M, K), 90 + i).cuda(), rnd((N, K), 95 + i, 0.05).cuda().t()) for i, (M, N, K) in enumerate(shapes)]
    want = [f16acc.mm(a, b) for a, b in inputs]
    torch.cuda.synchronize()
    got = [[None] * len(inputs) for _ in range(2)]
    errors = []

    def worker(k):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for rep in range(3):
                    for i, (a, b) in enumerate(inputs):
                        got[k][i] = f16acc.mm(a, b)
            s.synchronize()
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for k in range(2):
        for i in range(len(inputs)):
            assert torch.equal(got[k][i], want[i]), (k, shapes[i])


def test_hip_graph_capture_replays_match_eager():
    """mm captured in a HIP graph (one split-K shape, one two-launch shape,
    one plain and one bias-fused call) and replayed three times, with eager
    work on the same inputs between replays: every replay equals the eager
    result bit for bit.  The library records no memset nodes; its workspace
    and outputs come from the graph's pool."""
    from f16acc_amd import patch

    x1, w1 = rnd((2048, 4096), 100).cuda(), rnd((256, 4096), 101, 0.02).cuda()
    x2, w2 = rnd((2048, 1536), 102).cuda(), rnd((8960, 1536), 103, 0.02).cuda()
    x3, w3, b3 = rnd((512, 640), 104).cuda(), rnd((384, 640), 105, 0.05).cuda(), rnd((384,), 106, 0.5).cuda()

    def run():
        with torch.no_grad():
            return f16acc.mm(x1, w1.t()), f16acc.mm(x2, w2.t()), patch.linear(x3, w3, b3), f16acc.mm(x3, w3.t())

    eager = run()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()  # warm-up on the capture stream: its workspace exists before capture
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = run()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)
        again = run()  # eager work between replays
        torch.cuda.synchronize()
        for o, e in zip(again, eager):
            assert torch.equal(o, e)


def test_graph_keeps_its_split_k_workspace_when_a_larger_one_replaces_it():
    """A graph captured with a split-K mm writes its FP32 partials to the
    stream's workspace on every replay.  A later eager call on that stream
    that needs a larger workspace must not free the captured one: a tensor
    allocated afterwards, of the old workspace's size, keeps its contents
    across replays, and every replay still equals the eager result."""
    from f16acc_amd import kernel

    # weights row-major [K, N] (b = w.t() would split K inside the workgroup
    # on these shapes, with no workspace)
    x1, w1 = rnd((2048, 4096), 110).cuda(), rnd((4096, 256), 111, 0.02).cuda()  # 8 MiB of partials
    x2, w2 = rnd((1024, 16384), 112).cuda(), rnd((16384, 512), 113, 0.02).cuda()  # 32 MiB
    eager1 = f16acc.mm(x1, w1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    key = (x1.device.index, side.cuda_stream)
    with torch.cuda.stream(side):
        f16acc.mm(x1, w1)  # the workspace exists before capture
        captured = kernel._workspaces[key]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            out = f16acc.mm(x1, w1)
        eager2 = f16acc.mm(x2, w2)
        assert kernel._workspaces[key] is not captured and kernel._workspaces[key].numel() > captured.numel()
        victim = torch.full((captured.numel(),), 0x5A, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager1)
        assert bool((victim == 0x5A).all())
    assert torch.equal(f16acc.mm(x2, w2), eager2)


def test_graphs_captured_on_one_stream_get_their_own_split_k_workspaces():
    """torch.cuda.graph captures on one shared side stream by default.  Two
    graphs with a split-K mm each get a workspace of their own, distinct from
    the eager one, so replaying both at once on two streams while an eager
    split-K call runs cannot mix their FP32 partials: every replay equals the
    eager result, bit for bit."""
    from f16acc_amd import kernel

    # weights row-major [K, N]: 2048 x 256 x 4096 splits K (8 MiB of partials)
    x1, w1 = rnd((2048, 4096), 120).cuda(), rnd((4096, 256), 121, 0.02).cuda()
    x2, w2 = rnd((2048, 4096), 122).cuda(), rnd((4096, 256), 123, 0.02).cuda()
    e1, e2 = f16acc.mm(x1, w1), f16acc.mm(x2, w2)
    before = {id(t) for t in kernel._workspaces.values()}
    g1, g2 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        o1 = f16acc.mm(x1, w1)
    with torch.cuda.graph(g2):
        o2 = f16acc.mm(x2, w2)
    new = [t for t in kernel._workspaces.values() if id(t) not in before]
    assert len(new) == 2 and new[0].data_ptr() != new[1].data_ptr()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        s1.wait_stream(torch.cuda.current_stream())
        s2.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s1):
            g1.replay()
        with torch.cuda.stream(s2):
            g2.replay()
        e3 = f16acc.mm(x1, w1)  # eager, at the same time, on the current stream
        torch.cuda.synchronize()
        assert torch.equal(o1, e1) and torch.equal(o2, e2) and torch.equal(e3, e1)


def _random_operand(g, rows, cols, kind, seed):
    """A [rows, cols] fp16 CPU tensor laid out as `kind` (its GPU twin has the
    same strides): contiguous, transposed view, strided view, offset view,
    broadcast view (one row or one column expanded: a stride of 0) or
    sliding window (rows 8 elements apart, overlapping when cols > 8)."""
    if kind == "broadcast":
        if seed % 2:
            return rnd((cols,), seed).expand(rows, cols)
        return rnd((rows, 1), seed).expand(rows, cols)
    if kind == "window":
        return rnd((8 * max(rows - 1, 0) + cols,), seed).as_strided((rows, cols), (8, 1))
    n = 3 * max(rows, cols) + 5
    base = rnd((n, n), seed)
    if kind == "contiguous":
        return base[:rows, :cols].contiguous()
    if kind == "transposed":
        return base[:cols, :rows].contiguous().t()
    if kind == "strided":
        return base[: 2 * rows : 2, : 3 * cols : 3]
    return base[1 : rows + 1, 3 : cols + 3]  # offset view: misaligned rows


@pytest.mark.parametrize("case", range(40))
def test_randomized_shapes_layouts_and_tiles_match_oracle(case):
    """Seeded random problems: M, N in 1..300, K in 0..700 (ragged chunks and
    stages), each operand contiguous / transposed / strided / offset /
    broadcast / sliding window, fp16 or
    fp32 output, chunked or not, the table's tile or a forced one; values and
    tile flags against the oracle, some tiles overflowing on purpose."""
    import random

    from f16acc_amd import _lib

    r = random.Random(1000 + case)
    M, N, K = r.randint(1, 300), r.randint(1, 300), r.choice([0, 1, 7, 32, 33, 64, 96, 200, r.randint(1, 700)])
    kinds = ["contiguous", "transposed", "strided", "offset", "broadcast", "window"]
    ka, kb = r.choice(kinds), r.choice(kinds)
    a = _random_operand(None, M, K, ka, 2000 + case)
    b = _random_operand(None, K, N, kb, 3000 + case)
    assert a.shape == (M, K) and b.shape == (K, N)
    # one overflowing block of rows x cols (chunk sums past 65504), written
    # only into operands whose elements each have their own memory
    disjoint = ka not in ("broadcast", "window") and kb not in ("broadcast", "window")
    if K >= 64 and r.random() < 0.3 and disjoint:
        i0, j0 = r.randrange(M), r.randrange(N)
        a[i0 : i0 + 4, :] = 60.0
        b[:, j0 : j0 + 4] = 60.0
    out_dtype = r.choice([torch.float16, torch.float32])
    chunked = r.random() < 0.8
    tile = r.choice([None, None] + list(_lib.TILES))

    def twin(t):
        # same strides and offset on the GPU: copy the whole base storage
        base = t.as_strided((t.untyped_storage().nbytes() // 2,), (1,), 0)
        g = base.cuda()
        return g.as_strided(t.shape, t.stride(), t.storage_offset())

    ga, gb = twin(a), twin(b)
    assert torch.equal(ga.cpu(), a) and torch.equal(gb.cpu(), b)
    cfg = tile_config(ga, gb, tile)
    c, flags = mm_flags(ga, gb, out_dtype, chunked, tile=tile)
    ref, rflags = oracle(a, b, out_dtype, cfg, chunked=chunked)
    assert c.shape == (M, N) and c.dtype == out_dtype
    assert torch.equal(flags.cpu(), rflags), (case, M, N, K, tile)
    finite = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(c.cpu()), finite), (case, M, N, K, tile)
    if bool(finite.any()) and float(ref[finite].abs().max()) > 0:
        err = (c.cpu()[finite].double() - ref[finite].double()).abs().max() / ref[finite].double().abs().max()
        assert err < TOL, (case, M, N, K, tile, out_dtype, chunked, float(err))
    else:
        assert torch.equal(c.cpu()[finite], ref[finite])


def _twin(t):
    """The GPU copy of a CPU view: the whole base storage copied, the same
    strides and offset."""
    base = t.as_strided((t.untyped_storage().nbytes() // 2,), (1,), 0)
    return base.cuda().as_strided(t.shape, t.stride(), t.storage_offset())


def _check_against_oracle(c, ref, what):
    finite = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(c.cpu()), finite), what
    if bool(finite.any()) and float(ref[finite].abs().max()) > 0:
        err = (c.cpu()[finite].double() - ref[finite].double()).abs().max() / ref[finite].double().abs().max()
        assert err < TOL, (what, float(err))
    else:
        assert torch.equal(c.cpu()[finite], ref[finite]), what


@pytest.mark.parametrize("case", range(40))
def test_randomized_long_k_on_few_tiles_through_mm_and_bias(case):
    """Seeded random problems with few tiles and a long K (M, N in 1..520,
    K in 1024..6000: split-K plans and the K-group tiles), any operand layout
    (b mostly K-contiguous, as the K-group tiles need), fp16 or fp32 output,
    chunked or not, some tiles overflowing: the single grid with tile flags
    (forced tile or the table's) against the oracle; mm itself (its
    workspace: split-K partials, the deferred redo list) against the oracle
    too; and for fp16 output the fused bias equal to mm + bias bit for bit."""
    import random

    r = random.Random(4000 + case)
    M, N, K = r.randint(1, 520), r.randint(1, 520), r.randint(1024, 6000)
    kinds = ["contiguous", "transposed", "strided", "offset", "broadcast", "window"]
    ka = r.choice(kinds)
    kb = "transposed" if r.random() < 0.7 else r.choice(kinds)
    a = _random_operand(None, M, K, ka, 8000 + case)
    b = _random_operand(None, K, N, kb, 9000 + case)
    if r.random() < 0.3 and ka not in ("broadcast", "window") and kb not in ("broadcast", "window"):
        i0, j0 = r.randrange(M), r.randrange(N)
        a[i0 : i0 + 4, :] = 60.0
        b[:, j0 : j0 + 4] = 60.0
    out_dtype = r.choice([torch.float16, torch.float32])
    chunked = r.random() < 0.85
    tile = r.choice([None, None, None] + list(_lib.TILES))
    what = (case, M, N, K, ka, kb, out_dtype, chunked, tile)
    ga, gb = _twin(a), _twin(b)
    cfg = tile_config(ga, gb, tile)
    c, flags = mm_flags(ga, gb, out_dtype, chunked, tile=tile)
    ref, rflags = oracle(a, b, out_dtype, cfg, chunked=chunked)
    assert torch.equal(flags.cpu(), rflags), what
    _check_against_oracle(c, ref, what)
    _check_against_oracle(f16acc.mm(ga, gb, out_dtype, chunked=chunked), ref, what)
    if out_dtype == torch.float16 and chunked:
        bias = rnd((N,), 10000 + case, 0.1).cuda()
        want = f16acc.mm(ga, gb)
        want += bias
        assert torch.equal(f16acc.kernel.mm_bias(ga, gb, bias), want), what


@pytest.mark.parametrize("b_layout", ["w.t()", "row-major"])
def test_ragged_round_row_cut_equals_single_grid(b_layout):
    """A tall problem (8960 x 2048 x 1536: 35 x 8 tiles of 256x256 for 256
    CUs) is cut along M: rows 0..8191 as one round of 256x256 tiles, the last
    768 as a second launch (a offset by 8192 rows, c by 8192 rows).  Every
    element is computed as in the single grid, bit for bit; the fused bias
    is per column, so it applies unchanged to both launches."""
    from f16acc_amd import patch

    x, w, bias = rnd((8960, 1536), 110), rnd((2048, 1536), 111, 0.05), rnd((2048,), 112, 0.5)
    gx = x.cuda()
    gb = w.cuda().t() if b_layout == "w.t()" else w.t().contiguous().cuda()
    assert _tail_split(gx, gb) == -8192
    c = f16acc.mm(gx, gb)
    c1, flags = mm_flags(gx, gb)
    assert int(flags.sum()) == 0
    assert torch.equal(c, c1)
    assert rel(c.cpu(), chunk32.mm(x, w.t(), torch.float16, tile=(128, 128))) < TOL
    if b_layout == "w.t()":
        unfused = c.clone()
        unfused += bias.cuda()
        with torch.no_grad():
            assert torch.equal(patch.linear(gx, w.cuda(), bias.cuda()), unfused)
    # the forced-overflow closed form in the first and in the second launch
    xo, wo = x.clone(), w.clone()
    for r0 in (300, 8500):
        xo[r0 : r0 + 10, :] = 100.0
    wo[40:50, :] = 0.0
    wo[40:50, 0:32], wo[40:50, 32:64], wo[40:50, 64:96], wo[40:50, 96:128] = 30.0, -30.0, 30.0, -30.0
    wo[40:50, 127] = -29.0
    co = f16acc.mm(xo.cuda(), wo.cuda().t(), torch.float32)
    assert torch.all(co[300:310, 40:50] == 100.0) and torch.all(co[8500:8510, 40:50] == 100.0)


@pytest.mark.parametrize("M, N, K, b_layout, tile, split", [
    (256, 1024, 2048, "row", "64x64", False),     # a partial 64x64 round over a 128x128 K split
    (3072, 1024, 4096, "t", "64x64", False),      # three 64x64 per CU over one 128x128 per CU
    (4096, 3072, 1024, "t", "256x256", False),    # a lone last 128x128 round: 256x256, redo in place (short K)
    (4096, 3072, 2560, "row", "256x256", False),  # ... from K 2560 the deferred redo list
    (256, 11008, 8192, "row", "128x128", True),   # long K keeps the 128x128 K split
])
def test_partial_round_picks_match_oracle(M, N, K, b_layout, tile, split):
    """mm on shapes the table prices by partial rounds (fp16 out): the pick,
    its whole output against the same tile forced (bit for bit where mm does
    not split K, within the tolerance where it does: the split reassociates
    the FP32 chunk sums), and corner and middle blocks of the output against
    the oracle on the same rows and columns (chunk sums are per element)."""
    a = rnd((M, K), 7100 + K)
    b = rnd((K, N), 7200 + N, 0.02)
    ga = a.cuda()
    gb = b.cuda() if b_layout == "row" else b.t().contiguous().cuda().t()
    assert tile_config(ga, gb)["tile"] == tile
    n = ctypes.c_size_t()
    _lib.check(_lib.workspace_size(M, N, K, ga.stride(0), ga.stride(1), gb.stride(0), gb.stride(1), ga.data_ptr(),
                                   gb.data_ptr(), ctypes.byref(n)))
    assert (n.value > _lib.WS_HEADER) == split, n.value
    c = f16acc.mm(ga, gb)
    forced = f16acc.kernel.mm_tile(ga, gb, tile)
    torch.cuda.synchronize()
    if split:
        _check_against_oracle(c, forced.cpu().float(), (M, N, K, "split vs forced"))
    else:
        assert torch.equal(c, forced), (M, N, K)
    for r0, c0 in ((0, 0), (M - 128, N - 128), (M // 2 // 64 * 64, N // 2 // 64 * 64)):
        ref = chunk32.mm(a[r0:r0 + 128], b[:, c0:c0 + 128], torch.float16, tile=(128, 128))
        _check_against_oracle(c[r0:r0 + 128, c0:c0 + 128], ref, (M, N, K, r0, c0))


@pytest.mark.parametrize("case", range(30))
def test_randomized_large_grids_through_the_table(case):
    """Seeded random shapes of one round or more (M, N in 256..6144, K in
    512..4096, a multiple of 8), b row-major or w.t(), fp16 out: mm as
    planned (any tile, a ragged-round cut, a deferred redo launch, a K split)
    against the pick forced alone -- bit for bit when the plan is one
    unsplit launch of that tile -- and, on corner and middle blocks, against
    the oracle on the same rows and columns.  Where mm packs an operand
    first (a row-major b with N not a multiple of 8), the forced run may read
    it in place on another tile, and the two are compared to the tolerance."""
    import random

    r = random.Random(9100 + case)
    M, N, K = r.randint(256, 6144), r.randint(256, 6144), 8 * r.randint(64, 512)
    b_layout = r.choice(["row", "t"])
    what = (case, M, N, K, b_layout)
    a = rnd((M, K), 9200 + case)
    b = rnd((K, N), 9300 + case, 0.05)
    ga = a.cuda()
    gb = b.cuda() if b_layout == "row" else b.t().contiguous().cuda().t()
    pick = tile_config(ga, gb)["tile"]
    one_launch = False
    if b_layout == "t" or N % 8 == 0:  # read as given: the plan below is the one mm runs
        n, cut = ctypes.c_size_t(), ctypes.c_int64()
        _lib.check(_lib.workspace_size(M, N, K, ga.stride(0), ga.stride(1), gb.stride(0), gb.stride(1),
                                       ga.data_ptr(), gb.data_ptr(), ctypes.byref(n)))
        _lib.check(_lib.tail_split(M, N, K, ga.stride(0), ga.stride(1), gb.stride(0), gb.stride(1), ga.data_ptr(),
                                   gb.data_ptr(), ctypes.byref(cut)))
        one_launch = n.value <= _lib.WS_HEADER and cut.value == 0
    c = f16acc.mm(ga, gb)
    forced = f16acc.kernel.mm_tile(ga, gb, pick)
    torch.cuda.synchronize()
    if one_launch:
        assert torch.equal(c, forced), (what, pick)
    else:
        _check_against_oracle(c, forced.cpu().float(), (what, pick))
    for r0, c0 in ((0, 0), (M - 96, N - 96), (M // 2, N // 2)):
        ref = chunk32.mm(a[r0:r0 + 96], b[:, c0:c0 + 96], torch.float16, tile=(96, 96))
        _check_against_oracle(c[r0:r0 + 96, c0:c0 + 96], ref, (what, pick, r0, c0))
