"""The chunk rounding itself, pinned on the GPU.

A 1e-3 tolerance against the oracle cannot tell the reference's chunk-32
rounding (f16acc/kernel.py:49: each 32-term chunk rounded to fp16, then added
in FP32) from plain FP32 accumulation: on N(0, 1) inputs the two differ by
2-8e-4.  These tests can:

* closed forms, compared exactly: the oracle's pinned cases
  (tests/test_oracle.py) in every element of a tile grid, each column one
  form, each row scaled by its own power of two (scaling commutes with fp16
  rounding away from the subnormal range), repeated over three 64-long
  stages, on every tile and both b layouts:
    A  chunks 2049 (tie -> 2048) and 2047      chunk-32 4095, FP32 4096
    B  2049 (-> 2048), then 1 at k = 32        chunk-32 2049, FP32 2050, boundary one late 2050
    C  one chunk of 2051 (tie -> 2052)         chunk-32 2052, FP32 2051, rounded per 16 terms 2050
* the K = 33 chunk boundary on operands the copies cannot read (packed,
  register-staged or gathered);
* random inputs, FP32 output: the kernel's bits against the oracle's.  With
  fp16-rounded partials every FP32 sum is exact for these inputs, so the
  kernel and the oracle can differ only where a chunk's FP32 partial lands on
  the other side of an fp16 rounding boundary in the MFMA than on the host
  (whose partials come from an FP32 matmul in another order).  At K = 1024
  (32 chunks an element) at least 98 % of the elements must be bit-equal to
  the oracle, and 99 % to the same sums with every partial rounded once from
  its exact value (oracle paired_sum, exact_partials; measured on MI355X:
  98.6 % and 99.4 %), against 0.02 % for FP32 accumulation.  The max-norm
  error cannot make this distinction: one partial on the other side of a
  rounding boundary moves an element by as much as the chunk rounding moves
  the worst element; the L2 norm can (kernel within a fifth of FP32
  accumulation's distance from the oracle);
* subnormal chunk partials (inputs ~ N(0, 1) * 2^-9: partials ~ 2^-15.5,
  below binary16's 2^-14), where rounding to the subnormal grid dominates
  the error: the same bounds.
"""

import pytest
import torch

import f16acc_amd as f16acc
from f16acc_amd.kernel import mm_flags, mm_tile, tile_config
from oracle import chunk32

rel = chunk32.rel
ALL_TILES = ["256x256", "256x128", "128x256", "128x128", "generic", "64x64", "128x96k2", "64x32k4", "256x288"]
FORMS = [  # one 64-long stage of a b column: (values, chunk-32 sum, FP32 sum)
    ([1.0] * 31 + [2018.0] + [1.0] * 31 + [2016.0], 4095.0, 4096.0),
    ([1.0] * 31 + [2018.0] + [1.0] + [0.0] * 31, 2049.0, 2050.0),
    ([1.0] * 15 + [2034.0] + [2.0] + [0.0] * 47, 2052.0, 2051.0),
]
SCALES = [1.0, 2.0, -4.0, 0.5]
K_GROUPS = {"128x96k2": 2, "64x32k4": 4}  # tiles that sum K ranges in groups


def closed_form_operands(M, N, stages):
    """a [M, 64 * stages] with row m = SCALES[m % 4]; b [K, N] with column n =
    FORMS[n % 3] repeated per stage; and the exact chunk-32 and FP32 results."""
    K = 64 * stages
    s = torch.tensor([SCALES[m % 4] for m in range(M)])
    a = s.view(M, 1).expand(M, K).contiguous().half()
    col = torch.tensor([FORMS[n % 3][0] for n in range(N)]).t()  # [64, N]
    b = col.repeat(stages, 1).half().contiguous()
    chunked = s.view(M, 1) * stages * torch.tensor([FORMS[n % 3][1] for n in range(N)]).view(1, N)
    fp32 = s.view(M, 1) * stages * torch.tensor([FORMS[n % 3][2] for n in range(N)]).view(1, N)
    return a, b, chunked.float(), fp32.float()


def test_closed_forms_hold_in_the_oracle():
    a, b, chunked, fp32 = closed_form_operands(12, 9, 3)
    assert torch.equal(chunk32.chunked_sum(a, b), chunked)
    assert torch.equal(chunk32.fp32_sum(a, b), fp32)
    per16 = chunk32.chunked_sum(a, b, mode="per_k16")
    assert not torch.equal(per16, chunked)  # form C: 2050 per 16 terms


@pytest.mark.gpu
@pytest.mark.parametrize("tile", [None] + ALL_TILES)
def test_chunk_rounding_closed_forms_on_every_tile(tile):
    M, N = 300, 520
    a, b, chunked, fp32 = closed_form_operands(M, N, 3)
    ga = a.cuda()
    for b_t in (False, True):
        gb = b.t().contiguous().cuda().t() if b_t else b.cuda()
        c, flags = mm_flags(ga, gb, torch.float32, tile=tile)
        assert int(flags.sum()) == 0, (tile, b_t)
        assert torch.equal(c.cpu(), chunked), (tile, b_t, tile_config(ga, gb, tile))
        c32 = mm_tile(ga, gb, tile, torch.float32, chunked=False) if tile else f16acc.mm(ga, gb, torch.float32,
                                                                                         chunked=False)
        assert torch.equal(c32.cpu(), fp32), (tile, b_t)


@pytest.mark.gpu
@pytest.mark.parametrize("tile", [None, "128x128", "64x64", "generic", "256x256"])
def test_chunk_boundary_at_k33_on_operands_the_copies_cannot_read(tile):
    """K = 33: one whole chunk of 2049 (-> 2048) and a one-term chunk of 1.
    K is not a multiple of 8, so the operands are packed, read in place or
    gathered; a boundary one term late would give 2050."""
    M, N, K = 200, 136, 33
    a = torch.ones(M, K, dtype=torch.float16)
    b = torch.ones(K, N, dtype=torch.float16)
    b[31, :] = 2018.0
    ga, gb = a.cuda(), b.cuda()
    for gbv in (gb, b.t().contiguous().cuda().t()):
        c = mm_tile(ga, gbv, tile, torch.float32) if tile else f16acc.mm(ga, gbv, torch.float32)
        assert bool((c == 2049.0).all()), tile
        c32 = mm_tile(ga, gbv, tile, torch.float32, chunked=False) if tile else f16acc.mm(ga, gbv, torch.float32,
                                                                                          chunked=False)
        assert bool((c32 == 2050.0).all()), tile


def _bits(x, y):
    return float((x.view(torch.int32) == y.view(torch.int32)).float().mean())


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).half()


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [1.0, 2.0 ** -9], ids=["normal", "subnormal_partials"])
@pytest.mark.parametrize("tile", ALL_TILES)
def test_random_inputs_carry_the_chunk_rounding_bit_for_bit(tile, scale):
    M, N, K = 300, 520, 1024
    a, b = rnd((M, K), 40, scale), rnd((K, N), 41, scale)
    ref = chunk32.chunked_sum(a, b)
    f32 = chunk32.fp32_sum(a, b)
    if scale != 1.0:  # most chunk partials are binary16 subnormals
        p0 = (a[:, :32].float() @ b[:32].float()).abs()
        assert float((p0 < 2.0 ** -14).float().mean()) > 0.5
    assert _bits(f32, ref) < 0.01  # FP32 accumulation keeps few elements' bits
    ga = a.cuda()
    exact = {}
    for b_t in (False, True):
        gb = b.t().contiguous().cuda().t() if b_t else b.cuda()
        kg = K_GROUPS.get(tile_config(ga, gb, tile)["tile"], 1)
        if kg not in exact:
            exact[kg] = chunk32.paired_sum(a, b, kgroups=kg, exact_partials=True)
        c, flags = mm_flags(ga, gb, torch.float32, tile=tile)
        c = c.cpu()
        assert int(flags.sum()) == 0
        frac, frac_exact = _bits(c, ref), _bits(c, exact[kg])
        assert frac > 0.98 and frac_exact > 0.99, (tile, b_t, scale, frac, frac_exact)
        # the elements that differ are off by one partial's fp16 rounding,
        # far less in total than the chunk rounding FP32 accumulation skips
        assert float((c - ref).norm()) < 0.2 * float((f32 - ref).norm()), (tile, b_t, scale)
