"""Pins of the oracle (CPU restatements of the reference's chunk-32 GEMM,
f16acc/kernel.py:37-105 of the reference) against things fixed outside it:

* binary16 conversions against numpy's IEEE implementation (exhaustive /
  dense random), the library routine the C code restates;
* closed forms whose value changes under each plausible mistake: chunk
  length 16 or 64 instead of 32, a chunk boundary off by one, rounding per
  16 terms instead of per 32, redo of single elements instead of whole tiles,
  flagging fp16 output overflow, forgetting the zero-fill past K;
* the reference's own closed form (tests/test_f16acc.py:91-101) and error
  levels (tests/test_f16acc.py:26-40, README.md:29);
* brute force on tiny inputs with numpy scalars, in a different formulation
  (explicit sequential float32 / float16 scalar arithmetic).
"""

import numpy as np
import pytest
import torch

from oracle import c_oracle, chunk32

rel = chunk32.rel
ORACLES = [pytest.param(chunk32.mm, id="torch"), pytest.param(c_oracle.mm, id="c")]


@pytest.fixture(scope="module", autouse=True)
def _built():
    c_oracle.build()


def test_f16_to_f32_exhaustive():
    lib = c_oracle.load()
    allh = np.arange(65536, dtype=np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    got = np.array([lib.oracle_f16_to_f32(int(h)) for h in allh], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne():
    lib = c_oracle.load()
    rng = np.random.default_rng(0)
    exps = rng.integers(-30, 18, 40000)
    x = (rng.random(40000) * 2 - 1) * np.exp2(exps)
    x = x.astype(np.float32)
    # ties and boundaries: halfway points between neighbouring binary16 values
    h = np.arange(0, 0x7c00, 97, dtype=np.uint16).view(np.float16).astype(np.float32)
    hn = np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float32)
    mids = ((h.astype(np.float64) + hn.astype(np.float64)) / 2).astype(np.float32)
    edge = np.array([65504, 65519.996, 65520, 65536, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26, 1 + 2.0 ** -11,
                     1 + 3 * 2.0 ** -11, -0.0, np.inf, -np.inf], np.float32)
    allx = np.concatenate([x, -x, mids, -mids, edge])
    with np.errstate(over="ignore"):
        want = allx.astype(np.float16).view(np.uint16)
    got = np.array([lib.oracle_f32_to_f16(float(v)) for v in allx], np.uint16)
    assert np.array_equal(got, want)


def _ones_col(vals):
    """a = ones [1, K], b = vals as a [K, 1] column: c = sum over k of vals."""
    v = torch.tensor(vals, dtype=torch.float32).half()
    return torch.ones(1, len(vals), dtype=torch.float16), v.view(-1, 1)


@pytest.mark.parametrize("mm", ORACLES)
def test_chunk_rounding_closed_forms(mm):
    # chunk 1 = 31 ones + 2018 = 2049 -> fp16 tie -> 2048;  chunk 2 = 32 terms = 2047 (exact)
    # chunk-32: 2048 + 2047 = 4095;  one 64-chunk: 4096;  FP32 accumulation: 4096
    a, b = _ones_col([1.0] * 31 + [2018.0] + [1.0] * 31 + [2016.0])
    assert mm(a, b, torch.float32).item() == 4095.0
    assert mm(a, b, torch.float32, chunked=False).item() == 4096.0
    # chunk boundary: K = 33, first 32 terms sum to 2049 (-> 2048), term 33 = 1
    # correct: 2049;  boundary one later (33 terms in chunk 1): 2050
    a, b = _ones_col([1.0] * 31 + [2018.0] + [1.0])
    assert mm(a, b, torch.float32).item() == 2049.0
    # round-once vs per-16: first 16 terms = 15 ones + 2034 = 2049, last 16 sum to 2
    # round-once: 2051 -> tie -> 2052;  per-16: 2048 + 2 = 2050
    a, b = _ones_col([1.0] * 15 + [2034.0] + [2.0] + [0.0] * 15)
    assert mm(a, b, torch.float32).item() == 2052.0
    assert mm(a, b, torch.float32, mode="per_k16").item() == 2050.0


@pytest.mark.parametrize("mm", ORACLES)
def test_zero_fill_past_k_and_empty_k(mm):
    # K = 5: one short chunk; anything but a zero-filled tail changes the sum
    a, b = _ones_col([1.0, 2.0, 3.0, 4.0, 2038.0])  # 2048 exact
    assert mm(a, b, torch.float32).item() == 2048.0
    c = mm(torch.empty(3, 0, dtype=torch.float16), torch.empty(0, 4, dtype=torch.float16), torch.float32)
    assert c.shape == (3, 4) and bool((c == 0).all())


@pytest.mark.parametrize("mm", ORACLES)
def test_reference_forced_overflow_closed_form(mm):
    # reference tests/test_f16acc.py:91-101: chunk sums +96000 / -95900 are inf in
    # fp16, the exact result is 100; the tile must be redone whole in FP32
    w = torch.empty(128, 64, dtype=torch.float16)
    w[:, :32], w[:, 32:], w[:, 63] = 30.0, -30.0, -29.0
    x = torch.full((256, 64), 100.0, dtype=torch.float16)
    c, flags = mm(x, w.t(), tile=(128, 128), return_flags=True)
    assert bool((c == 100.0).all()) and bool(flags.all())
    assert not torch.isfinite(chunk32.chunked_sum(x, w.t())).any()  # without the redo


@pytest.mark.parametrize("mm", ORACLES)
def test_redo_covers_the_whole_tile_only(mm):
    # 8 x 8 output, tiles 4 x 4.  Column 0 of b overflows a chunk (2 x 32 x 1024 =
    # 65536 -> inf in fp16 but finite in FP32) for row 0 only; every other
    # element is the 2049 closed form (chunk-32: 2048, FP32: 2049).
    K = 32
    a = torch.ones(8, K, dtype=torch.float16)
    b = torch.ones(K, 8, dtype=torch.float16)
    b[K - 1, :] = 2018.0  # 31 + 2018 = 2049 in every column
    a[0, :] = 2.0
    b[:, 0] = 1024.0  # row 0 x col 0: 32 * 2 * 1024 = 65536 -> inf in fp16
    c, flags = mm(a, b, torch.float32, tile=(4, 4), return_flags=True)
    assert flags.tolist() == [[1, 0], [0, 0]]
    assert c[0, 0].item() == 65536.0  # redone in FP32
    assert c[1, 1].item() == 2049.0  # same tile: redone in FP32, not 2048
    assert c[1, 5].item() == 2048.0  # tile (0, 1): chunked
    assert c[5, 1].item() == 2048.0  # tile (1, 0): chunked
    assert c[0, 5].item() == 2.0 * 31 + 2.0 * 2018 - 2.0  # 4096 + ... see below
    # row 0, col 5: 2 * (31 * 1 + 2018) = 4098 -> fp16 tie between 4096 and 4100 -> 4096


def test_row0_col5_closed_form_value():
    # the value asserted above, derived: chunk partial 4098 -> binary16 spacing 4 at
    # 4096, tie -> even significand -> 4096 = 2*31 + 2*2018 - 2
    assert float(np.float16(4098.0)) == 4096.0


@pytest.mark.parametrize("mm", ORACLES)
def test_fp16_output_overflow_is_not_flagged(mm):
    # three chunks of 30000 (exact in fp16): FP32 sum 90000 is finite -> no flag,
    # but the fp16 output is inf (kernel.py:70-72: the flag looks at the FP32 sum)
    a, b = _ones_col(([1.0] * 31 + [29969.0]) * 3)
    c, flags = mm(a, b, torch.float16, tile=(1, 1), return_flags=True)
    assert torch.isinf(c).all() and flags.sum() == 0
    assert mm(a, b, torch.float32).item() == 90000.0


@pytest.mark.parametrize("mm", ORACLES)
def test_nan_input_flags_every_tile_it_reaches(mm):
    g = torch.Generator().manual_seed(3)
    a = torch.randn(8, 64, generator=g).half()
    b = torch.randn(64, 12, generator=g).half()
    a[5, 10] = float("nan")  # reaches row 5: tiles (1, 0), (1, 1), (1, 2) of 4 x 4
    c, flags = mm(a, b, torch.float32, tile=(4, 4), return_flags=True)
    assert flags.tolist() == [[0, 0, 0], [1, 1, 1]]
    assert torch.isnan(c[5]).all() and not torch.isnan(c[torch.arange(8) != 5]).any()


def _brute(a, b, out_dtype, chunk=32, tile=(2, 2), mode="round_once"):
    """Scalar restatement with numpy float32/float16 scalars."""
    a = a.numpy().astype(np.float32)
    b = b.numpy().astype(np.float32)
    M, K = a.shape
    N = b.shape[1]
    s = np.zeros((M, N), np.float32)
    for i in range(M):
        for j in range(N):
            tot = np.float32(0)
            for k0 in range(0, K, chunk):
                p = np.float32(0)
                for k in range(k0, min(K, k0 + chunk)):
                    p = np.float32(p + np.float32(a[i, k] * b[k, j]))
                    if mode == "per_k16" and (k - k0) % 16 == 15 and k + 1 < min(K, k0 + chunk):
                        p = np.float32(np.float16(p))
                with np.errstate(over="ignore"):
                    tot = np.float32(tot + np.float32(np.float16(p)))
            s[i, j] = tot
    for ti in range(0, M, tile[0]):
        for tj in range(0, N, tile[1]):
            blk = s[ti:ti + tile[0], tj:tj + tile[1]]
            if not np.isfinite(blk).all():
                for i in range(ti, min(M, ti + tile[0])):
                    for j in range(tj, min(N, tj + tile[1])):
                        t = np.float32(0)
                        for k in range(K):
                            t = np.float32(t + np.float32(a[i, k] * b[k, j]))
                        s[i, j] = t
    with np.errstate(over="ignore"):
        return torch.from_numpy(s.astype(np.float16 if out_dtype == torch.float16 else np.float32))


@pytest.mark.parametrize("shape", [(3, 5, 2), (4, 33, 3), (5, 70, 4), (2, 64, 5)])
@pytest.mark.parametrize("mode", ["round_once", "per_k16"])
def test_brute_force_tiny(shape, mode):
    M, K, N = shape
    g = torch.Generator().manual_seed(M * 100 + K)
    a = (torch.randn(M, K, generator=g) * 8).half()
    b = (torch.randn(K, N, generator=g) * 8).half()
    if K >= 33:
        a[0, :] = 200.0  # row 0 chunks overflow for large b entries
        b[:, 0] = 250.0
    for od in (torch.float32, torch.float16):
        want = _brute(a, b, od, mode=mode)
        got_c = c_oracle.mm(a, b, od, tile=(2, 2), mode=mode)
        assert torch.equal(got_c.view(torch.int16 if od == torch.float16 else torch.int32),
                           want.view(torch.int16 if od == torch.float16 else torch.int32))
        got_t = chunk32.mm(a, b, od, tile=(2, 2), mode=mode)
        assert chunk32.rel_finite(got_t, want) < 1e-6


@pytest.mark.parametrize("mode", ["round_once", "per_k16"])
def test_torch_and_c_oracles_agree_on_strided_inputs(mode):
    g = torch.Generator().manual_seed(11)
    a = torch.randn(70, 200, generator=g).half()[:, ::2]  # strides (200, 2)
    w = torch.randn(45, 100, generator=g).half()
    # round-once: identical; per-16: the two FP32 orders of a 16-term partial
    # can round an intermediate fp16 differently (one fp16 ulp of a partial)
    tol = 1e-6 if mode == "round_once" else 1e-3
    for od in (torch.float16, torch.float32):
        ct = chunk32.mm(a, w.t(), od, mode=mode, tile=(32, 16))
        cc = c_oracle.mm(a, w.t(), od, mode=mode, tile=(32, 16))
        assert rel(ct, cc.double()) < tol


def test_error_levels_at_1024_match_fp64_bounds():
    g = torch.Generator().manual_seed(0)
    a = torch.randn(1024, 1024, generator=g).half()
    b = torch.randn(1024, 1024, generator=g).half()
    ref = a.double() @ b.double()
    ours = rel(chunk32.mm(a, b, torch.float32), ref)
    fp32 = rel(chunk32.mm(a, b, torch.float32, chunked=False), ref)
    # plain fp16 accumulation over the whole K, in K order (what chunking avoids)
    acc = torch.zeros(1024, 1024, dtype=torch.float16)
    for k in range(1024):
        acc = (acc.float() + a[:, k:k + 1].float() * b[k:k + 1, :].float()).half()
    plain = rel(acc, ref)
    assert ours < 2e-3  # tests/test_f16acc.py:21-24 bound
    assert fp32 < ours < 3 * max(fp32, 1e-4)
    assert ours * 5 < plain  # tests/test_f16acc.py:38 relation


@pytest.mark.slow
def test_reference_accuracy_figures_at_4096():
    """The reference measured 4.8e-4 (tests/test_f16acc.py:39) and 5.1e-4
    (README.md:29) for fp16 output at 4096^3 against FP64; the per-k16 model
    of its FP16 accumulator lands on that figure, round-once a little lower."""
    torch.set_num_threads(8)
    g = torch.Generator().manual_seed(0)
    a = torch.randn(4096, 4096, generator=g).half()
    b = torch.randn(4096, 4096, generator=g).half()
    ref = a.double() @ b.double()
    per16 = rel(chunk32.mm(a, b, mode="per_k16"), ref)
    once = rel(chunk32.mm(a, b), ref)
    assert 4.4e-4 < per16 < 5.2e-4
    assert 3.5e-4 < once <= per16


@pytest.mark.parametrize("kgroups", [1, 2, 3, 4])
def test_paired_sum_is_the_chunk_sum_reassociated(kgroups):
    """paired_sum adds the same fp16-rounded chunk partials in another FP32
    order (pairs of chunks, K ranges summed apart): equal to chunked_sum
    wherever every sum is exact (small integers), and a dropped or doubled
    chunk, a misplaced range or pairs across stage boundaries would break
    that equality on these ragged K."""
    g = torch.Generator().manual_seed(kgroups)
    for K in (1, 31, 64, 65, 200, 333):
        a = torch.randint(-3, 4, (9, K), generator=g).half()
        b = torch.randint(-3, 4, (K, 7), generator=g).half()
        want = chunk32.chunked_sum(a, b)
        assert torch.equal(chunk32.paired_sum(a, b, kgroups), want), K
        assert torch.equal(chunk32.paired_sum(a, b, kgroups, exact_partials=True), want), K
    # a chunk that overflows fp16 in one range: inf, as in the chunk sum
    a = torch.ones(2, 256, dtype=torch.float16)
    b = torch.ones(256, 2, dtype=torch.float16)
    b[200:232, 0] = 3000.0
    assert torch.isinf(chunk32.paired_sum(a, b, kgroups)[:, 0]).all()
    assert torch.equal(chunk32.paired_sum(a, b, kgroups)[:, 1], chunk32.chunked_sum(a, b)[:, 1])
