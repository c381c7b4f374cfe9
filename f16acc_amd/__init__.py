"""f16acc for MI355X: the chunked FP16 GEMM of the reference f16acc package,
on hand-written gfx950 HIP kernels.

Same surface as the reference's f16acc/__init__.py:8-11:
    mm(a, b, out_dtype=torch.float16, chunked=True)
    enable(), disable(), calls
Each 32-long K chunk of a dot product is rounded to FP16 and the chunks are
added in FP32; a tile whose FP32 sum overflows is redone with FP32
accumulation inside the same launch.
"""

from . import patch
from .kernel import mm
from .patch import calls, disable, enable

__all__ = ["mm", "enable", "disable", "calls"]
