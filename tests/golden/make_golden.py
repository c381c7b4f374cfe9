"""Writes tests/golden/cases.npz: small seeded chunk-32 GEMM cases with the
expected outputs and tile flags of the scalar C oracle (oracle/chunk32.c, the
restatement of the reference's f16acc/kernel.py:37-105).

    python tests/golden/make_golden.py

Each case stores a and b as raw binary16 bits (b in the layout the kernel
will see: "row" = b is [K, N] row-major, "t" = b is w.t() of a row-major
[N, K] w), the output dtype, the flag tile shape, and the expected c / flags.
The flag tile shape is the one the HIP library picks for the case (128 x 128
for every case here), so flags compare one to one.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import c_oracle  # noqa: E402

TILE = (128, 128)


def cases():
    g = torch.Generator().manual_seed(2024)

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g) * scale).half()

    out = []
    out.append(("square_f32", rn(96, 64), rn(64, 80), "row", torch.float32))
    out.append(("weight_view_f16", rn(130, 96), rn(136, 96, scale=0.05), "t", torch.float16))
    out.append(("ragged_k_f32", rn(70, 40), rn(40, 72), "row", torch.float32))
    out.append(("edge_tiles_f16", rn(129, 64), rn(64, 136), "row", torch.float16))
    # overflow: rows 0..7 x cols 0..7 of a 136 x 136 output blow every chunk up
    a, b = rn(136, 48), rn(48, 136)
    a[:8, :] = 120.0
    b[:, :8] = 110.0  # 32 * 120 * 110 = 422400 > 65504 -> tile (0, 0) redone in FP32
    out.append(("overflow_tile_f32", a, b, "row", torch.float32))
    w = torch.empty(128, 64, dtype=torch.float16)
    w[:, :32], w[:, 32:], w[:, 63] = 30.0, -30.0, -29.0
    out.append(("reference_closed_form_f16", torch.full((256, 64), 100.0, dtype=torch.float16), w, "t",
                torch.float16))
    return out


def main():
    c_oracle.build()
    arrays = {}
    names = []
    for name, a, bm, layout, od in cases():
        b = bm.t() if layout == "t" else bm
        c, flags = c_oracle.mm(a, b, od, tile=TILE, return_flags=True)
        names.append(name)
        arrays[f"{name}.a"] = a.view(torch.int16).numpy()
        arrays[f"{name}.b"] = bm.contiguous().view(torch.int16).numpy()
        arrays[f"{name}.layout"] = np.array(layout)
        arrays[f"{name}.out"] = np.array("f32" if od == torch.float32 else "f16")
        arrays[f"{name}.c"] = (c.view(torch.int32) if od == torch.float32 else c.view(torch.int16)).numpy()
        arrays[f"{name}.flags"] = flags.numpy()
    arrays["names"] = np.array(names)
    arrays["tile"] = np.array(TILE)
    np.savez_compressed(os.path.join(HERE, "cases.npz"), **arrays)
    print("wrote", len(names), "cases")


def load():
    """The cases as CPU tensors: list of (name, a, b, out_dtype, c, flags)."""
    z = np.load(os.path.join(HERE, "cases.npz"))
    res = []
    for name in z["names"]:
        name = str(name)
        a = torch.from_numpy(z[f"{name}.a"]).view(torch.float16)
        bm = torch.from_numpy(z[f"{name}.b"]).view(torch.float16)
        b = bm.t() if str(z[f"{name}.layout"]) == "t" else bm
        f32 = str(z[f"{name}.out"]) == "f32"
        c = torch.from_numpy(z[f"{name}.c"]).view(torch.float32 if f32 else torch.float16)
        res.append((name, a, b, torch.float32 if f32 else torch.float16, c, torch.from_numpy(z[f"{name}.flags"])))
    return res


if __name__ == "__main__":
    main()
