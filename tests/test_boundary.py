"""The drop-in boundary without a GPU: the C ABI library loads and exports
every symbol include/f16acc.h declares, rejects bad arguments before any
launch, maps blocks to tiles bijectively, and the Python surface raises the
reference's errors and routes calls the reference's way
(f16acc/kernel.py:84-90, f16acc/patch.py:17-40 of the reference).
"""

import ctypes
import os
import re

import pytest
import torch

import f16acc_amd as f16acc
from f16acc_amd import _lib, patch
from f16acc_amd.kernel import tile_config

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "f16acc.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(f16acc_\w+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    names = header_functions()
    assert names, "no declarations parsed"
    dll = ctypes.CDLL(_lib.LIB)
    for name in names:
        assert hasattr(dll, name), name
    assert sorted(_lib.EXPORTS) == names
    assert _lib.abi_version() == _lib.ABI_VERSION == 7


def test_gemm_rejects_bad_arguments_before_launching():
    args = dict(M=16, N=16, K=16, sam=16, sak=1, sbk=16, sbn=1, scm=16, scn=1)

    def call(ptrs=(8, 8, 8), out=0, chunked=1, **kw):
        a = {**args, **kw}
        return _lib.gemm(ptrs[0], ptrs[1], ptrs[2], None, a["M"], a["N"], a["K"], a["sam"], a["sak"], a["sbk"],
                         a["sbn"], a["scm"], a["scn"], out, chunked, None)

    assert call(M=-1) == _lib.E_ARG
    assert call(K=-5) == _lib.E_ARG
    assert call(out=2) == _lib.E_ARG
    assert call(chunked=7) == _lib.E_ARG
    assert call(ptrs=(0, 8, 8)) == _lib.E_ARG  # null a with K > 0
    assert call(ptrs=(8, 8, 0)) == _lib.E_ARG  # null c
    assert call(M=0) == 0 and call(N=0) == 0  # empty output: nothing launched
    assert _lib.strerror(_lib.E_ARG).decode().startswith("f16acc")
    a = args
    assert _lib.gemm_bias(8, 8, None, 8, None, a["M"], a["N"], a["K"], a["sam"], a["sak"], a["sbk"], a["sbn"],
                          a["scm"], a["scn"], 0, 1, None) == _lib.E_ARG  # bias entry without a bias
    for bad_tile in (-1, len(_lib.TILES), 99):  # forced tile out of range
        assert _lib.gemm_tile(8, 8, 8, None, a["M"], a["N"], a["K"], a["sam"], a["sak"], a["sbk"], a["sbn"],
                              a["scm"], a["scn"], 0, 1, None, bad_tile) == _lib.E_ARG
        assert _lib.gemm_tile_ws(8, 8, 8, None, a["M"], a["N"], a["K"], a["sam"], a["sak"], a["sbk"], a["sbn"],
                                 a["scm"], a["scn"], 0, 1, None, bad_tile, None, 0) == _lib.E_ARG
    # the allocation-free entry: bad sizes rejected, an empty output is a no-op
    assert _lib.gemm_noalloc(8, 8, None, 8, None, -1, a["N"], a["K"], a["sam"], a["sak"], a["sbk"], a["sbn"],
                             a["scm"], a["scn"], 0, 1, None) == _lib.E_ARG
    assert _lib.gemm_noalloc(8, 8, None, 8, None, 0, a["N"], a["K"], a["sam"], a["sak"], a["sbk"], a["sbn"],
                             a["scm"], a["scn"], 0, 1, None) == 0
    for code in (_lib.E_SCRATCH, _lib.E_DEVICE):
        assert _lib.strerror(code).decode().startswith("f16acc: ")
    # a workspace that is not 256-byte aligned
    assert _lib.gemm_tile_ws(8, 8, 8, None, a["M"], a["N"], a["K"], a["sam"], a["sak"], a["sbk"], a["sbn"],
                             a["scm"], a["scn"], 0, 1, None, 3, 8, 1 << 20) == _lib.E_ARG


def test_block_to_tile_map_is_a_bijection():
    """Brute force over grids, including ones not divisible by the 8 XCDs or
    the group width (the reference's _tile, kernel.py:22-34, covers every tile
    once; so must the XCD-aware map)."""
    tm, tn = ctypes.c_int64(), ctypes.c_int64()
    for gm in list(range(1, 18)) + [32, 33, 63]:
        for gn in list(range(1, 18)) + [35, 70]:
            seen = set()
            for b in range(gm * gn):
                assert _lib.block_tile(b, gm, gn, ctypes.byref(tm), ctypes.byref(tn)) == 0
                assert 0 <= tm.value < gm and 0 <= tn.value < gn
                seen.add((tm.value, tn.value))
            assert len(seen) == gm * gn
    assert _lib.block_tile(6, 2, 3, ctypes.byref(tm), ctypes.byref(tn)) == _lib.E_ARG


def test_block_map_keeps_each_xcd_on_a_compact_patch():
    """4096^2 with 256 x 256 tiles: 16 x 16 tiles, 32 per XCD; each XCD's
    tiles should touch few A row-blocks and B column-blocks."""
    tm, tn = ctypes.c_int64(), ctypes.c_int64()
    for xcd in range(8):
        rows, cols = set(), set()
        for b in range(xcd, 256, 8):
            _lib.block_tile(b, 16, 16, ctypes.byref(tm), ctypes.byref(tn))
            rows.add(tm.value)
            cols.add(tn.value)
        assert len(rows) * len(cols) == 32


class _Fake:
    """Stands in for a tensor in tile_config (shape, strides, data_ptr)."""

    def __init__(self, shape, strides, ptr=4096):
        self.shape, self._strides, self._ptr = shape, strides, ptr

    def stride(self, i):
        return self._strides[i]

    def data_ptr(self):
        return self._ptr


@pytest.mark.parametrize("M,N,K,sa,sb,fam,tile", [
    (4096, 4096, 4096, (4096, 1), (4096, 1), "fast", "256x256"),   # row-major b (NC loader)
    (4096, 4096, 4096, (4096, 1), (1, 4096), "fast", "256x256"),   # w.t() (KC loader)
    (8192, 8192, 8192, (8192, 1), (8192, 1), "fast", "256x256"),
    (2048, 151936, 1536, (1536, 1), (1, 1536), "fast", "256x256"),  # lm_head
    (2048, 8960, 1536, (1536, 1), (1, 1536), "fast", "256x288"),   # Qwen gate/up: 256 tiles, one round (280 of 256x256)
    (2048, 8960, 1536, (1536, 1), (8960, 1), "fast", "128x128"),   # row-major b: no 256x288; ragged 2nd round
    (1024, 11008, 4096, (4096, 1), (1, 4096), "fast", "256x256"),  # 172 256-tiles: one partial round beats 688 128-tiles
    (2048, 2048, 1536, (1536, 1), (1, 1536), "fast", "128x128"),   # 256 128-tiles: one per CU, no 64x64 (22.8 vs 24.1 us)
    (1024, 4096, 4096, (4096, 1), (1, 4096), "fast", "128x128"),   # one per CU: no K split either (51.4 vs 54.1 us)
    (2048, 1536, 1536, (1536, 1), (1, 1536), "fast", "128x96k2"),  # Qwen q/o: 256 128x96 tiles, two K groups
    (2048, 1536, 1536, (1536, 1), (1536, 1), "fast", "64x64"),     # row-major b: no K groups; 192 128-tiles
    (2048, 256, 1536, (1536, 1), (1, 1536), "fast", "64x32k4"),    # Qwen k/v: 256 64x32 tiles, four K groups
    (2048, 256, 1536, (1536, 1), (256, 1), "fast", "64x64"),       # row-major b: no K groups
    (256, 1024, 4096, (4096, 1), (1, 4096), "fast", "64x32k4"),    # llama-3-8B k/v, 256 tokens: 128 tiles
    (256, 512, 3584, (3584, 1), (1, 3584), "fast", "64x32k4"),     # Qwen2.5-7B k/v, 256 tokens: 64 tiles
    (256, 4096, 4096, (4096, 1), (1, 4096), "fast", "64x32k4"),    # 512 64x32 tiles: two rounds tie a split in four
    (1024, 1024, 4096, (4096, 1), (1, 4096), "fast", "64x32k4"),   # llama-3-8B k/v, 1024 tokens: two rounds
    (256, 3584, 3584, (3584, 1), (1, 3584), "fast", "64x32k4"),    # Qwen2.5-7B q/o, 256 tokens: beats a split in three
    (256, 4096, 5120, (5120, 1), (1, 5120), "fast", "128x128"),    # two rounds of 64x32 lose to a split in five
    (256, 4096, 11008, (11008, 1), (1, 11008), "fast", "128x128"), # llama-2-7B down, 256 tokens: split in eight
    (256, 11008, 4096, (4096, 1), (1, 4096), "fast", "128x96k2"),  # llama-2-7B gate/up, 256 tokens: 230 tiles
    (2048, 1536, 8960, (8960, 1), (1, 8960), "fast", "128x96k2"),  # Qwen down: K groups, no second launch
    (4096, 512, 3584, (3584, 1), (1, 3584), "fast", "64x64"),      # Qwen2.5-7B k/v, 4096 tokens: 192 128x96 tiles lose
    (1536, 1024, 1024, (1024, 1), (1, 1024), "fast", "64x64"),     # to 512 (384) of 64x64, 2 per CU: 30.3 / 10.3 us
    (1536, 1536, 4096, (4096, 1), (1, 4096), "fast", "128x96k2"),  # 576 64x64 tiles (3 on some CUs): 128x96 keeps it
    (512, 5120, 1024, (1024, 1), (1, 1024), "fast", "128x96k2"),   # ... also at K 1024 (64x64 won on two boxes, lost on one)
    (1024, 1024, 1536, (1536, 1), (1, 1536), "fast", "64x64"),     # two rounds of 64x32 at K 1536: 64x64 (11.2 vs 12.7)
    (1024, 1024, 2048, (2048, 1), (1, 2048), "fast", "64x32k4"),   # ... from K 2048 64x32 stays
    (2048, 1536, 8960, (8960, 1), (1536, 1), "fast", "128x128"),   # row-major b: 128x128 split in two
    (4096, 3072, 4096, (4096, 1), (1, 4096), "fast", "256x256"),   # 768 128-tiles leave a lone last round: 192 of
    (8192, 1536, 1536, (1536, 1), (1536, 1), "fast", "256x256"),   # 256x256 win (124.6 vs 132.8 us; 52.1 vs 56.7)
    (3072, 1024, 4096, (4096, 1), (1024, 1), "fast", "64x64"),     # 768 64x64 tiles, 3 per CU: 46.4 vs 48.2 us
    (256, 1024, 2048, (2048, 1), (1024, 1), "fast", "64x64"),      # 64x64 1 per CU over a split in two: 13.0 vs 19.0
    (256, 11008, 8192, (8192, 1), (11008, 1), "fast", "128x128"),  # long K: a split in two beats 3 64x64 per CU
    (128, 1536, 1536, (1536, 1), (1536, 1), "fast", "64x64"),      # 128 rows, row-major b
    (2049, 1537, 8961, (8961, 1), (1, 8961), "fast", "128x128"),   # rows not 16-byte aligned: packed first
    (300, 1537, 8961, (8961, 1), (1, 8961), "reg", "128x128"),     # read in place (cheaper than a copy)
    (2048, 256, 1537, (1537, 1), (1, 1537), "reg", "64x64"),       # k/v shape, odd K, w.t()
    (2048, 256, 1537, (1537, 1), (256, 1), "reg", "128x128"),      # row-major b: 64x64 has no room
    (64, 40, 24, (24, 1), (40, 1), "fast", "64x64"),               # too small to repay a copy: as given
    (300, 200, 256, (512, 2), (700, 3), "generic", "generic"),      # strided operands
])
def test_tile_table(M, N, K, sa, sb, fam, tile):
    cfg = tile_config(_Fake((M, K), sa), _Fake((K, N), sb))
    assert cfg["family"] == fam and cfg["tile"] == tile
    assert cfg["tiles_m"] == -(-M // cfg["bm"]) and cfg["tiles_n"] == -(-N // cfg["bn"])


@pytest.mark.parametrize("tile", ["256x256", "256x128", "128x256", "128x128", "generic", "64x64", "128x96k2",
                                  "64x32k4", "256x288"])
def test_forced_tile_resolves(tile):
    bm, bn = (128, 128) if tile == "generic" else (int(tile.split("x")[0]), int(tile.split("x")[1].split("k")[0]))
    # w.t() (K-contiguous b): every tile as forced
    cfg = tile_config(_Fake((4096, 1024), (1024, 1)), _Fake((1024, 2048), (1, 1024)), tile)
    assert cfg["tile"] == tile and (cfg["bm"], cfg["bn"]) == (bm, bn)
    assert cfg["family"] == ("generic" if tile == "generic" else "fast")
    # a row-major b: the K-group tiles run as 128x128 and 64x64 (their K
    # groups read a K-contiguous b only), 256x288 as 256x256
    cfg = tile_config(_Fake((4096, 1024), (1024, 1)), _Fake((1024, 2048), (2048, 1)), tile)
    assert cfg["tile"] == {"128x96k2": "128x128", "64x32k4": "64x64", "256x288": "256x256"}.get(tile, tile)
    # strided operands: mm packs them for a forced fast tile, so the tile holds
    cfg = tile_config(_Fake((300, 256), (512, 2)), _Fake((256, 200), (700, 3)), tile)
    assert cfg["tile"] == tile
    # the library itself, handed operands it cannot copy 16 bytes at a time,
    # falls back to the generic kernel
    tid = ctypes.c_int()
    _lib.check(_lib.tile_config(300, 200, 256, 512, 2, 700, 3, 0, 0, _lib.TILES.index(tile), ctypes.byref(tid),
                                None, None, None, None, None, None))
    assert _lib.TILES[tid.value] == "generic"
    with pytest.raises(ValueError):
        tile_config(_Fake((4096, 1024), (1024, 1)), _Fake((1024, 2048), (2048, 1)), "32x32")


def test_misaligned_pointer_is_packed_read_in_place_or_gathered():
    # mm copies a misaligned operand into an aligned buffer when the table
    # picks a tile without the register-staged loader (256x256 here) and the
    # GEMM is big enough to repay the copy; the library, handed the pointer
    # itself, gathers there
    cfg = tile_config(_Fake((4096, 4096), (4096, 1), ptr=4098), _Fake((4096, 4096), (4096, 1)))
    assert cfg["family"] == "fast"
    fam = ctypes.c_int()
    _lib.check(_lib.tile_config(4096, 4096, 4096, 4096, 1, 4096, 1, 4098, 0, -1, None, None, None, None, None,
                                ctypes.byref(fam), None))
    assert fam.value == 1  # F16ACC_FAMILY_GENERIC
    # where the table picks 128x128 or 64x64, unit-stride rows are read in
    # place at any even address (a row-major b moves 64x64 to 128x128)
    cfg = tile_config(_Fake((64, 64), (64, 1), ptr=4098), _Fake((64, 64), (64, 1)))
    assert (cfg["family"], cfg["tile"]) == ("reg", "128x128")
    cfg = tile_config(_Fake((64, 64), (64, 1), ptr=4098), _Fake((64, 64), (1, 64)))
    assert (cfg["family"], cfg["tile"]) == ("reg", "64x64")
    # forced tiles, operands as given: 64x64 with a row-major b and 256x256
    # gather (mm packs first for a forced tile)
    for b_strides, tile in (((64, 1), "64x64"), ((1, 64), "256x256")):
        _lib.check(_lib.tile_config(64, 64, 64, 64, 1, *b_strides, 4098, 4096, _lib.TILES.index(tile), None, None,
                                    None, None, None, ctypes.byref(fam), None))
        assert fam.value == 1, tile
        assert tile_config(_Fake((64, 64), (64, 1), ptr=4098), _Fake((64, 64), b_strides), tile)["family"] == "fast"


_OVERLAP = {  # (a strides, b strides) of [512, 320] @ [320, 576] views whose rows overlap
    "a_broadcast": ((0, 1), (576, 1)),          # x.expand(M, K)
    "a_window": ((8, 1), (1, 320)),             # rows 8 apart (unfold)
    "b_broadcast_rowmajor": ((320, 1), (0, 1)),  # v.expand(K, N)
    "b_broadcast_wt": ((320, 1), (1, 0)),        # v.expand(N, K).t()
    "b_window_wt": ((320, 1), (1, 8)),           # weight rows 8 apart, as w.t()
    "b_window_rowmajor": ((320, 1), (8, 1)),     # k-rows 8 apart
}


@pytest.mark.parametrize("case", list(_OVERLAP))
def test_overlapping_rows_never_take_the_direct_copies(case):
    """The copies clip a tile by one record count, exact only for disjoint
    rows: with a row stride of 0 or under a row the library routes every
    table pick and every forced tile elsewhere (register-staged, gather), and
    mm's own test of the layouts agrees (it packs such operands or leaves
    them to the library)."""
    from f16acc_amd.kernel import _fast_a, _fast_b

    sa, sb = _OVERLAP[case]
    M, N, K = 512, 576, 320
    fam = ctypes.c_int()
    for tile in [-1] + [i for i, t in enumerate(_lib.TILES) if t != "generic"]:
        _lib.check(_lib.tile_config(M, N, K, *sa, *sb, 4096, 8192, tile, None, None, None, None, None,
                                    ctypes.byref(fam), None))
        assert fam.value != 0, (case, tile)  # not F16ACC_FAMILY_FAST
    assert not (_fast_a(_Fake((M, K), sa), K) and _fast_b(_Fake((K, N), sb), K, N))


@pytest.mark.parametrize("M, N, K, sa, sb", [
    (1, 1536, 1536, (0, 1), (1, 1536)),    # one row broadcast from a vector: stride 0 addresses nothing
    (1, 1536, 1536, (4096, 1), (1, 1536)),  # x[:1] of a wider buffer
    (512, 1, 1536, (1536, 1), (1, 1)),      # b a contiguous [K, 1] column
    (512, 1, 1536, (1536, 1), (1, 0)),      # b = v.expand(1, K).t()
])
def test_single_rows_and_columns_take_the_direct_copies(M, N, K, sa, sb):
    """The stride of an extent-1 dimension is replaced by a row length before
    planning, so a single row or column keeps the fast path whatever stride
    torch reports for it (and its record count covers the row)."""
    from f16acc_amd.kernel import _fast_a, _fast_b

    fam = ctypes.c_int()
    _lib.check(_lib.tile_config(M, N, K, *sa, *sb, 4096, 8192, -1, None, None, None, None, None,
                                ctypes.byref(fam), None))
    assert fam.value == 0
    assert _fast_a(_Fake((M, K), sa), K) and _fast_b(_Fake((K, N), sb), K, N)


def test_bad_inputs_raise_value_error():
    # reference tests/test_f16acc.py:42-47 (runs here on CPU tensors: the device
    # check fires first for CPU operands, the shape check for mismatched K)
    a = torch.randn(256, 64).half()
    for bad in (torch.randn(32, 64).half(), torch.randn(64, 64), torch.randn(64, 64).half()):
        with pytest.raises(ValueError):
            f16acc.mm(a, bad)
    with pytest.raises(ValueError):
        f16acc.mm(a, torch.randn(64, 8).half(), out_dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        f16acc.mm(torch.randn(4, 4, 4).half(), torch.randn(4, 4).half())


def test_patch_enable_disable_and_cpu_fallback():
    for k in patch.calls:
        patch.calls[k] = 0
    lin = torch.nn.Linear(64, 32).half()
    f16acc.enable()
    try:
        assert torch.nn.functional.linear is patch.linear
        with torch.no_grad():
            y = lin(torch.randn(256, 64).half())  # CPU input: stays on the original
        assert y.shape == (256, 32)
        assert patch.calls == {"chunked": 0, "original": 1}
    finally:
        f16acc.disable()
    assert torch.nn.functional.linear is patch._orig
    assert patch.MIN_ROWS == 128
    assert f16acc.calls is patch.calls
    assert set(f16acc.__all__) == {"mm", "enable", "disable", "calls"}


@pytest.mark.parametrize("M,N,K,want,want_kc", [
    (2048, 8960, 1536, 8192, 0),       # Qwen2.5-1.5B gate/up: 280 tiles of 256x256 on 256 CUs (256 of 256x288)
    (8192, 8960, 1536, 8192, 0),       # 1120 tiles: four rounds plus 96 (four rounds of 256x288)
    (2048, 8960, 8960, 8192, 0),       # long K: the tail may split along K instead
    (4096, 4096, 4096, 0, 0),          # whole rounds
    (2048, 151936, 1536, 0, 0),        # lm_head: the ragged round is half full, a tail gains < 3 %
    (2048, 1536, 1536, 0, 0),          # under one round
    (8960, 2048, 1536, -8192, -8192),  # tall: the row cut fills the first round, the column cut would not
    (8960, 4096, 1536, -8192, -8192),  # only the row cut gains
    (4096, 8960, 1536, 8192, 0),       # only the column cut gains (two rounds of 256x288)
    (4096, 11008, 4096, 0, 0),         # a 69%-full last round costs less than the cut (404.8 against 419.5 us)
    (4096, 18944, 3584, 0, 0),
])
def test_ragged_round_tail_plan(M, N, K, want, want_kc):
    """Where f16acc_gemm cuts a ragged last 256x256 round into a second launch
    (no GPU here: the planner assumes 256 CUs): with a row-major b, and with
    b = w.t(), where 256x288 tiles fill the rounds instead on some shapes."""
    n = ctypes.c_int64(-1)
    _lib.check(_lib.tail_split(M, N, K, K, 1, N, 1, 0, 0, ctypes.byref(n)))
    assert n.value == want
    _lib.check(_lib.tail_split(M, N, K, K, 1, 1, K, 0, 0, ctypes.byref(n)))
    assert n.value == want_kc
    assert _lib.tail_split(-1, N, K, K, 1, 1, K, 0, 0, ctypes.byref(n)) == -1  # F16ACC_E_ARG



@pytest.mark.parametrize("M,N,K,in_place", [
    (256, 256, 1001, True),      # a copy costs more than the GEMM
    (2048, 1536, 1537, True),    # Qwen q/o with odd K: close, in place wins
    (1024, 4096, 1001, True),
    (2049, 1537, 8961, False),   # the odd config: the copy is cheaper than ~1.4x GEMM time
    (2048, 1536, 8959, False),
    (8192, 8192, 8191, False),
])
def test_in_place_reads_only_where_they_beat_a_copy(M, N, K, in_place):
    """mm reads unit-stride misaligned rows in place (register-staged loads)
    when that is cheaper than packing them: decided per shape from the
    measured costs, then only where the library reports the 'reg' family."""
    from f16acc_amd.kernel import _pack_plan, _reg_beats_pack

    assert _reg_beats_pack(M, N, K) == in_place
    a = _Fake((M, K), (K, 1))         # rows K halves long: misaligned for odd K
    b = _Fake((K, N), (1, K))         # w.t() of an [N, K] weight
    pack_a, pack_b, Kp, ld = _pack_plan(a, b, M, N, K)
    fam = tile_config(a, b)["family"]
    if in_place and fam == "reg":
        assert (pack_a, pack_b, Kp) == (False, False, K)
    else:
        assert pack_a and pack_b and Kp % 8 == 0 and ld % 64 == 0 and fam == "fast"


def test_k_split_only_where_cus_would_idle():
    """The split-K workspace is asked for only when the pick's tiles leave some
    CUs without a workgroup (Qwen2.5 down with a row-major weight: 192 tiles
    of 128x128 for 256 CUs), not when every CU already has one (1024 x 4096 x
    4096: 256 tiles), nor where a K-group tile splits K inside the workgroup
    (down, 2048 x 256 x 4096, 1024 x 256 x 4096 and 256 x 4096 x 4096 with
    b = w.t(), the last on two rounds of 64x32 tiles); 256 x 4096 x 5120 would
    need two rounds of 64x32 tiles that lose to a split in five, so it
    splits."""
    n = ctypes.c_size_t()
    for (M, N, K), b_kc, split in (((2048, 1536, 8960), False, True), ((2048, 1536, 8960), True, False),
                                   ((1024, 4096, 4096), True, False), ((2048, 256, 4096), True, False),
                                   ((1024, 256, 4096), True, False), ((2048, 256, 4096), False, True),
                                   ((256, 4096, 4096), True, False), ((256, 4096, 5120), True, True)):
        sbk, sbn = (1, K) if b_kc else (N, 1)
        _lib.check(_lib.workspace_size(M, N, K, K, 1, sbk, sbn, 0, 0, ctypes.byref(n)))
        assert (n.value > 0) == split, (M, N, K, b_kc)


def _pick_and_splits(M, N, K):
    """(tile, splits) the library plans for x [M, K] @ w.t(), w [N, K]."""
    tid, bm, bn, fam, thr = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    tm, tn = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(_lib.tile_config(M, N, K, K, 1, 1, K, 0, 0, -1, ctypes.byref(tid), ctypes.byref(bm), ctypes.byref(bn),
                                ctypes.byref(tm), ctypes.byref(tn), ctypes.byref(fam), ctypes.byref(thr)))
    n = ctypes.c_size_t()
    _lib.check(_lib.workspace_size(M, N, K, K, 1, 1, K, 0, 0, ctypes.byref(n)))
    part = max(n.value - _lib.WS_HEADER, 0)
    return _lib.TILES[tid.value], part // (tm.value * tn.value * bm.value * bn.value * 4) if part else 1


@pytest.mark.parametrize("M, N, K, tile, splits", [
    (1024, 3584, 3584, "128x128", 1),    # Qwen2.5-7B q/o, 1024 tokens: 224 tiles, short K: 42.8 us whole, 46.6 split
    (256, 14336, 4096, "128x128", 1),    # llama-3-8B gate/up, 256 tokens: 224 tiles: 48.7 us whole, 50.2 split
    (1024, 3584, 18944, "128x128", 2),   # Qwen2.5-7B down, 1024 tokens: 224 tiles, long K: 185.0 us split, 205.2 whole
    (256, 4096, 11008, "128x128", 8),    # llama-2-7B down, 256 tokens: 64 tiles: 45.5 us split, 114.1 whole
    (2049, 1537, 8968, "128x128", 2),    # the packed odd config: 221 tiles, long K
    (1536, 11008, 1536, "256x288", 1),   # 234 tiles of 256x288, one round: 64.8 us, 88.7 on 64x64
    (1536, 11008, 4096, "256x288", 1),   # 153.4 us, 221.8 on 64x64
])
def test_k_split_only_where_it_pays(M, N, K, tile, splits):
    """A grid with fewer tiles than CUs is split along K only when the time
    it saves exceeds the split's fixed cost (the FP32 partials' traffic and
    the finishing launch): not at 224 of 256 CUs with a short K, yes with a
    long K or a grid of a quarter of the CUs.  A 256x288 grid of one partial
    round is weighed against 64x64 at 256x256's rate (the table read past its
    four-entry rate array there, a fault the host sanitizer build found, and
    sent these shapes to 64x64)."""
    assert _pick_and_splits(M, N, K) == (tile, splits)


def test_workspace_holds_the_redo_list_where_it_is_deferred():
    """f16acc_workspace_size: one round of 256x256 tiles (4096^3) needs the
    header alone (its flagged tiles are listed and redone by a second launch),
    from 40 stages of K (K > 2496: 2560 lists, 2496 does not) up; shorter K
    redoes in place (the second launch's fixed cost would pass 3 % of the
    call); more rounds (8192^3: the persistent kernel redoes in place) and
    shapes whose tiles fill the CUs on other tiles need nothing; a split-K
    plan needs the header plus its partials."""
    n = ctypes.c_size_t()
    for (M, N, K, sbk, sbn), want in (((4096, 4096, 4096, 4096, 1), "header"), ((4096, 4096, 4096, 1, 4096), "header"),
                                      ((4096, 4096, 2560, 4096, 1), "header"), ((4096, 4096, 2496, 4096, 1), "none"),
                                      ((4096, 4096, 1024, 4096, 1), "none"),
                                      ((8192, 8192, 8192, 8192, 1), "none"), ((2048, 2048, 1536, 1, 1536), "none"),
                                      ((2048, 1536, 8960, 1536, 1), "split")):
        _lib.check(_lib.workspace_size(M, N, K, K, 1, sbk, sbn, 0, 0, ctypes.byref(n)))
        got = "none" if n.value == 0 else "header" if n.value == _lib.WS_HEADER else "split"
        assert got == want, (M, N, K, n.value)
