"""The chunk-epilogue microbenchmark (f16acc_amd/csrc/chunkrate.hip; the
MI355X analogue of the reference's bench/rate.py and bench/chunkrate.py:39-43)
runs on the GPU: its numerics self-check passes (the pair selector MFMA and
the sparse quad selector leave exactly the FP32 sum of the FP16-rounded chunk
partials in every register, bit for bit on integer inputs, within 2 ulp on
N(0, 1) inputs), and so do the lane-local identity sums of its part 3
(16x16x16 and 4x4x4 MFMAs adding one chunk each: exactly the two FP32
additions in chunk order); plain FP32-accumulating MFMAs issue at >= 0.9 of
the 16-cycle MFMA rate, so the epilogue figures it prints are measured
against a saturated matrix pipe."""

import os
import re
import subprocess

import pytest

from f16acc_amd.build import CHUNKRATE

pytestmark = pytest.mark.gpu


def test_chunkrate_self_check_and_mfma_issue_rate():
    assert os.path.exists(CHUNKRATE), f"{CHUNKRATE} is not built"
    res = subprocess.run([CHUNKRATE], capture_output=True, text=True, timeout=100)
    out = res.stdout
    print(out)
    assert res.returncode == 0, out + res.stderr
    assert "self-check ok" in out
    checks = re.findall(r"self-check \((\S+) inputs\): (\d+) of 512 sums off, (\d+) of 1024 partials rounded", out)
    assert [c[0] for c in checks] == ["integer", "N(0,1)"]
    assert all(int(c[1]) == 0 for c in checks) and all(int(c[2]) > 0 for c in checks)
    ident = re.findall(r"identity-sum check \((\S+) inputs\): (\d+) of 512 sums off", out)
    assert [c[0] for c in ident] == ["integer", "N(0,1)"] and all(int(c[1]) == 0 for c in ident), ident
    for name in ("v_mfma_f32_16x16x16_f16", "v_mfma_f32_4x4x4_16b_f16", "2 x 16x16x16 identity", "2 x 4x4x4 identity"):
        assert len(re.findall(re.escape(name) + r"\s+[0-9.]+", out)) == 2, name  # one and two waves per SIMD
    rates = [float(x) for x in re.findall(r"FP32-accumulating MFMAs\s+[0-9.]+\s+([0-9.]+)", out)]
    assert len(rates) == 2, out  # one and two waves per SIMD
    assert min(rates) >= 0.9, rates
    shipped = [float(x) for x in re.findall(r"cvt_pk x4 \+ selector MFMA\s+[0-9.]+\s+([0-9.]+)", out)]
    assert len(shipped) == 2 and all(0.5 < r <= 2 / 3 + 0.01 for r in shipped), shipped
