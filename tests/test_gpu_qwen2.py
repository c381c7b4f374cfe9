"""Patched vs unpatched prefill of a random-init Qwen2.5-1.5B-architecture
model: the full model (28 decoder layers, 2048 tokens) and a 2-layer,
256-token cut.  Every nn.Linear goes through f16acc_amd.mm; logits must agree
with the unpatched FP16 model and with FP32 as closely as the unpatched model
does (the reference's bench/llm.py:33-64 measures the same on a real
checkpoint, README.md:35: 99.9 % top-1 agreement)."""

import pytest
import torch

pytestmark = pytest.mark.gpu

# Random-init logits have small margins, so FP16 noise alone moves some
# top-1 picks: the unpatched FP16 model agrees with FP32 on ~92 % of the
# 2048 positions.  The patched model must stay within this much of the
# unpatched one's agreement with FP32, and its mean cross-entropy within
# this much of the unpatched one's distance to FP32.
TOP1_MARGIN = 0.02
CE_MARGIN = 2e-3


def check(r, calls):
    assert r["calls_in_one_forward"] == {"chunked": calls, "original": 0}
    assert r["top1_patched_vs_unpatched"] >= 0.98
    assert r["top1_patched_vs_fp32"] >= r["top1_unpatched_vs_fp32"] - TOP1_MARGIN
    gap_unpatched = abs(r["mean_ce_unpatched"] - r["mean_ce_fp32"])
    assert abs(r["mean_ce_patched"] - r["mean_ce_fp32"]) <= gap_unpatched + CE_MARGIN
    assert r["max_abs_logit_diff_patched_vs_fp32"] <= 1.5 * r["max_abs_logit_diff_unpatched_vs_fp32"] + 0.05


def test_qwen2_two_layer_prefill_ab():
    pytest.importorskip("transformers")
    import bench

    r = bench.qwen2_prefill_ab(layers=2, tokens=256, reps=1)
    check(r, 2 * 7 + 1)  # 2 layers x 7 projections + lm_head, all with 256 >= MIN_ROWS rows


def test_qwen2_full_prefill_ab():
    """The configured model at its real size: 28 layers, 2048 seeded tokens,
    batch 1, 197 routed nn.Linear calls per forward (28 x 7 + lm_head)."""
    pytest.importorskip("transformers")
    import bench

    r = bench.qwen2_prefill_ab(layers=28, tokens=2048, reps=1)
    print({k: v for k, v in r.items() if k != "calls_in_one_forward"})
    check(r, 28 * 7 + 1)
    torch.cuda.empty_cache()
