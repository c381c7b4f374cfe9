"""Oracle (test infrastructure): a PyTorch-CPU restatement of the reference's
chunk-32 GEMM.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it; it is the checker and never the product path.

Follows the reference f16acc/kernel.py:
  _loop   kernel.py:37-54   K walked in chunks of 32 (BLOCK_K, kernel.py:17);
                            loads past K read 0 (kernel.py:45-47), so a ragged
                            last chunk simply has fewer terms; each chunk's
                            FP16-accumulated partial is promoted to FP32 and
                            added to the FP32 sum in K order (kernel.py:49)
  _gemm   kernel.py:63-72   tile flag = any element of the FP32 tile sum not
                            finite (abs(x) < inf is false for NaN, kernel.py:70)
  _redo   kernel.py:75-81   flagged tiles recomputed whole with FP32 accumulate
  _store  kernel.py:57-60   cast of the FP32 tile to the output dtype (RNE)
  mm      kernel.py:84-105  chunked=False is plain FP32 accumulation, no flag

Chunk partial models (an FP16 accumulator's rounding is not observable off the
reference's GPU, so both bounds are offered):
  "round_once": FP32 partial over the chunk, rounded once to FP16 (RNE)
  "per_k16":    rounded to FP16 after each 16 terms (two m16n8k16 steps)
"""

import torch

CHUNK = 32
MODES = ("round_once", "per_k16")


def _f16(x):
    """Round an FP32 tensor to FP16 (RNE, overflow to inf) and back to FP32."""
    return x.half().float()


def fp32_sum(a16, b16):
    """Plain FP32 accumulation of fp16 operands: kernel.py:50-51 (chunked=False)
    and the redo pass kernel.py:80."""
    return a16.float() @ b16.float()


def chunked_sum(a16, b16, chunk=CHUNK, mode="round_once", group=8):
    """FP32 sum over K of FP16-rounded chunk partials (kernel.py:44-53).

    `group` chunks are evaluated per batched product to bound memory; the
    chunks are still added into the running sum one by one in K order.
    """
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}")
    if mode == "per_k16" and chunk % 16:
        raise ValueError("per_k16 needs a chunk that is a multiple of 16")
    M, K = a16.shape
    N = b16.shape[1]
    s = torch.zeros(M, N, dtype=torch.float32)
    nchunks = (K + chunk - 1) // chunk
    for g0 in range(0, nchunks, group):
        g1 = min(nchunks, g0 + group)
        for c in range(g0, g1):
            k0, k1 = c * chunk, min(K, (c + 1) * chunk)
            if mode == "round_once":
                p = _f16(a16[:, k0:k1].float() @ b16[k0:k1, :].float())
            else:
                p = torch.zeros(M, N, dtype=torch.float32)
                for h0 in range(k0, k1, 16):
                    h1 = min(k1, h0 + 16)
                    p = _f16(p + a16[:, h0:h1].float() @ b16[h0:h1, :].float())
            s += p
    return s


def paired_sum(a16, b16, kgroups=1, exact_partials=False):
    """The same FP16-rounded chunk partials as chunked_sum (round_once), summed
    in the order of a kernel that adds chunk pairs: for each 64-long K stage,
    s = fp32(s + H_2p + H_2p+1) with one rounding, stages in K order.  With
    kgroups > 1 the stages are dealt to kgroups consecutive ranges of
    ceil(stages / kgroups) each, every range summed this way from zero, and
    the range sums added in range order in FP32.  exact_partials: each chunk's
    FP32 partial is the exactly summed dot product rounded once to FP32
    (instead of torch's FP32 matmul).

    This is not the reference's order (that is chunked_sum: one chunk at a
    time, kernel.py:49); it differs from it by FP32 reassociation only, and is
    equal to it wherever every sum is exact.  Tests use it to compare the
    kernel's bits, where the reference's order only bounds them."""
    M, K = a16.shape
    N = b16.shape[1]
    nst = (K + 2 * CHUNK - 1) // (2 * CHUNK)
    per = -(-nst // kgroups) if nst else 0
    total = torch.zeros(M, N, dtype=torch.float32)
    for g in range(kgroups):
        s = torch.zeros(M, N, dtype=torch.float64)  # FP32 values, added exactly in FP64
        for st in range(g * per, min(nst, (g + 1) * per)):
            acc = s.clone()
            for k0 in (2 * st * CHUNK, (2 * st + 1) * CHUNK):
                if k0 >= K:
                    continue
                k1 = min(K, k0 + CHUNK)
                if exact_partials:
                    p = (a16[:, k0:k1].double() @ b16[k0:k1, :].double()).float()
                else:
                    p = a16[:, k0:k1].float() @ b16[k0:k1, :].float()
                acc += _f16(p).double()
            s = acc.float().double()  # one rounding per stage
        total = total + s.float() if g else s.float()
    return total


def tile_flags(s, bm, bn):
    """One flag per (bm x bn) tile, row-major tile order: any element not
    finite (kernel.py:70-71)."""
    M, N = s.shape
    tm, tn = (M + bm - 1) // bm, (N + bn - 1) // bn
    bad = ~torch.isfinite(s)
    flags = torch.zeros(tm, tn, dtype=torch.uint8)
    if M and N:
        pad = torch.zeros(tm * bm, tn * bn, dtype=torch.bool)
        pad[:M, :N] = bad
        flags = pad.view(tm, bm, tn, bn).any(dim=3).any(dim=1).to(torch.uint8)
    return flags


def mm(a16, b16, out_dtype=torch.float16, chunked=True, tile=(256, 256), mode="round_once",
       return_flags=False):
    """c = a16 @ b16 with the reference's semantics (kernel.py:84-105).

    a16 [M, K] and b16 [K, N] are fp16 CPU tensors of any strides.  `tile` is
    the flag/redo granularity (the reference's autotuned BM x BN).
    """
    if a16.dim() != 2 or b16.dim() != 2 or a16.shape[1] != b16.shape[0]:
        raise ValueError(f"oracle mm needs (M, K) @ (K, N), got {tuple(a16.shape)} @ {tuple(b16.shape)}")
    if a16.dtype != torch.float16 or b16.dtype != torch.float16:
        raise ValueError("oracle mm needs fp16 operands")
    a16, b16 = a16.cpu(), b16.cpu()
    bm, bn = tile
    if not chunked:
        s = fp32_sum(a16, b16)
        flags = torch.zeros((a16.shape[0] + bm - 1) // bm, (b16.shape[1] + bn - 1) // bn, dtype=torch.uint8)
    else:
        s = chunked_sum(a16, b16, mode=mode)
        flags = tile_flags(s, bm, bn)
        for ti, tj in flags.nonzero().tolist():  # _redo: whole tile, FP32 accumulate
            r0, c0 = ti * bm, tj * bn
            s[r0:r0 + bm, c0:c0 + bn] = fp32_sum(a16[r0:r0 + bm], b16[:, c0:c0 + bn])
    c = s.to(out_dtype)
    return (c, flags) if return_flags else c


def rel(x, ref):
    """The reference's error metric, tests/test_f16acc.py:11-12:
    max|x - ref| / max|ref| in float64."""
    x, ref = x.double(), ref.double()
    den = ref.abs().max()
    return ((x - ref).abs().max() / den).item() if den > 0 else (x - ref).abs().max().item()


def rel_finite(x, ref):
    """rel over the elements finite in ref, after checking that the others
    match exactly (inf with the same sign, NaN where ref is NaN); returns inf
    when they do not."""
    x, ref = x.double().cpu(), ref.double().cpu()
    fin = torch.isfinite(ref)
    same_nonfinite = torch.equal(torch.isnan(x), torch.isnan(ref)) and torch.equal(
        x[torch.isinf(ref)], ref[torch.isinf(ref)])
    if not same_nonfinite or not torch.isfinite(x[fin]).all():
        return float("inf")
    return rel(x[fin], ref[fin]) if fin.any() else 0.0
