"""Route FP16 nn.Linear through the chunked GEMM.

    import f16acc_amd as f16acc; f16acc.enable()

Same behaviour as the reference's f16acc/patch.py:17-40: only
torch.nn.functional.linear is replaced (nn.Linear.forward calls it through
the module attribute).  Calls whose input is not fp16 on a GPU, whose weight
is not fp16, that run with gradients enabled, or that have fewer than
MIN_ROWS rows (decode steps: memory-bound) go to the original F.linear and
are counted under calls["original"]; the rest go through mm and are counted
under calls["chunked"].  An fp16 bias is added in the GEMM's store with the
rounding of the reference's separate `y += b` (patch.py:29-30), so results are
the same bit for bit.  Overflow is repaired inside the kernel, so there is no
host sync per call.
"""

import torch
import torch.nn.functional as F

from .kernel import mm, mm_bias

MIN_ROWS = 128
_orig = F.linear
calls = {"chunked": 0, "original": 0}


def linear(x, w, b=None):
    """F.linear(x, w, b) = x @ w.T + b, on the chunked kernel when eligible."""
    rows = x.shape[:-1].numel()
    eligible = (x.is_cuda and x.dtype == torch.float16 and w.dtype == torch.float16 and rows >= MIN_ROWS
                and not torch.is_grad_enabled())
    if not eligible:
        calls["original"] += 1
        return _orig(x, w, b)
    x2 = x.reshape(rows, x.shape[-1])
    if (b is not None and b.dtype == torch.float16 and b.dim() == 1 and b.shape[0] == w.shape[0] and b.is_cuda
            and b.device == x.device):
        # bias fused into the GEMM's store, rounded as the unfused y += b would be
        y = mm_bias(x2, w.t(), b)
    else:
        y = mm(x2, w.t())  # w.t() is a (1, K)-strided view; mm takes any strides
        if b is not None:
            y += b
    calls["chunked"] += 1
    return y.view(*x.shape[:-1], w.shape[0])


def enable():
    F.linear = linear


def disable():
    F.linear = _orig
