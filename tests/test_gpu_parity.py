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

import pytest
import torch

import f16acc_amd as f16acc
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
    a_big, b_big = rnd((300, 512), 6), rnd((256, 700), 7)
    a, b = a_big[:, ::2], b_big[:, 1::3]  # strides (512, 2) and (700, 3)
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
