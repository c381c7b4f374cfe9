"""Golden fixtures (tests/golden/cases.npz, written by make_golden.py from the
scalar C oracle): the oracles must reproduce them, and the HIP kernels must
match them within the parity tolerance."""

import pytest
import torch

from oracle import c_oracle, chunk32
from tests.golden.make_golden import TILE, load

CASES = load()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_oracles_reproduce_golden(case):
    name, a, b, od, c, flags = case
    got, gflags = c_oracle.mm(a, b, od, tile=TILE, return_flags=True)
    assert torch.equal(got.view(torch.int16) if od == torch.float16 else got.view(torch.int32),
                       c.view(torch.int16) if od == torch.float16 else c.view(torch.int32))
    assert torch.equal(gflags, flags)
    got_t, tflags = chunk32.mm(a, b, od, tile=TILE, return_flags=True)
    assert chunk32.rel_finite(got_t, c) < 1e-6 and torch.equal(tflags, flags)


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_kernel_matches_golden(case):
    from f16acc_amd.kernel import mm_flags, tile_config

    name, a, b, od, c, flags = case
    ga = a.cuda()
    gb = b.t().contiguous().cuda().t() if b.stride(0) == 1 and b.shape[0] > 1 else b.contiguous().cuda()
    # the fixtures' flags are per 128x128 tile: force that tile
    cfg = tile_config(ga, gb, "128x128")
    assert (cfg["bm"], cfg["bn"]) == tuple(TILE)
    got, gflags = mm_flags(ga, gb, od, tile="128x128")
    assert torch.equal(gflags.cpu(), flags)
    assert chunk32.rel_finite(got.cpu(), c) < 1e-3
    # the table's own choice (64x64 on these small grids): a tile's flag is
    # "some chunk sum in it is non-finite", so its flags OR-pooled onto the
    # 128x128 grid are the fixture's
    cfg = tile_config(ga, gb)
    got, gflags = mm_flags(ga, gb, od)
    assert chunk32.rel_finite(got.cpu(), c) < 1e-3
    fm, fn = TILE[0] // cfg["bm"], TILE[1] // cfg["bn"]
    g = gflags.cpu()
    g = torch.nn.functional.pad(g, (0, -g.shape[1] % fn, 0, -g.shape[0] % fm))
    pooled = g.view(g.shape[0] // fm, fm, g.shape[1] // fn, fn).amax(dim=(1, 3))
    assert torch.equal(pooled, flags)
