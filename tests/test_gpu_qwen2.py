"""Patched vs unpatched prefill of a random-init Qwen2.5-1.5B-architecture
model, cut to two decoder layers and 256 tokens (the full 28-layer, 2048-token
A/B is bench.py --workload qwen2_prefill).  Every nn.Linear goes through
f16acc_amd.mm; logits must agree with the unpatched FP16 model and with FP32
as closely as the unpatched model does (the reference's bench/llm.py:33-64
measures the same on a real checkpoint)."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_qwen2_two_layer_prefill_ab():
    pytest.importorskip("transformers")
    import bench

    r = bench.qwen2_prefill_ab(layers=2, tokens=256, reps=1)
    # 2 layers x 7 projections + lm_head, all with 256 >= MIN_ROWS rows
    assert r["calls_in_one_forward"] == {"chunked": 15, "original": 0}
    assert r["top1_patched_vs_unpatched"] >= 0.98
    assert r["top1_patched_vs_fp32"] >= r["top1_unpatched_vs_fp32"] - 0.02
    assert abs(r["mean_ce_patched"] - r["mean_ce_fp32"]) < 1e-2
