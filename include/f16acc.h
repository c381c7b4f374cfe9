/*
 * f16acc for MI355X (gfx950): C ABI of the chunked FP16 GEMM.
 *
 * Plain C types only (pointers, 64-bit sizes and strides in elements), so any
 * host language can bind it; the Python package binds it through ctypes.
 * Every entry point is reentrant: the library keeps no per-call state.
 *
 * Return codes: 0 on success, a positive hipError_t value when the HIP
 * runtime failed, or one of the negative F16ACC_E_* codes below for
 * arguments the library rejects before launching anything.
 */
#ifndef F16ACC_H
#define F16ACC_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define F16ACC_OUT_F16 0
#define F16ACC_OUT_F32 1

#define F16ACC_E_ARG (-1)        /* negative size, null pointer with work to do, bad enum */
#define F16ACC_E_UNSUPPORTED (-2) /* a layout / extent this build cannot address */
#define F16ACC_E_SCRATCH (-3)     /* f16acc_gemm_noalloc: split plan larger than its fixed scratch */
#define F16ACC_E_DEVICE (-4)      /* f16acc_gemm_noalloc: stream on another device than the current one */

/* Tile configurations of the per-shape table (f16acc_tile_config reports
 * which one a problem uses; f16acc_gemm_tile forces one). */
#define F16ACC_TILE_256x256 0
#define F16ACC_TILE_256x128 1
#define F16ACC_TILE_128x256 2
#define F16ACC_TILE_128x128 3
#define F16ACC_TILE_GENERIC 4 /* 128x128, any strides, element gather */
#define F16ACC_TILE_64x64 5   /* small grids: 4 waves of 32x32, 4 workgroups per CU */
#define F16ACC_TILE_128x96_K2 6 /* two K groups of 4 waves of 64x48 splitting K inside the
                                   workgroup; K-contiguous b (else runs as 128x128) */
#define F16ACC_TILE_64x32_K4 7  /* four K groups of 2 waves of 32x32 splitting K inside the
                                   workgroup; K-contiguous b (else runs as 64x64) */
#define F16ACC_TILE_256x288 8    /* 8 waves of 64x144; K-contiguous b (else runs as 256x256) */
#define F16ACC_NUM_TILES 9

/* The first F16ACC_WS_HEADER bytes of a workspace (f16acc_gemm_ws,
 * f16acc_gemm_tile_ws) hold the list of tiles whose FP32 redo is deferred to
 * a second launch; they must be zero when the workspace is first used, and
 * every call leaves them zero.  Split-K partials follow them. */
#define F16ACC_WS_HEADER 4096

#define F16ACC_FAMILY_FAST 0    /* direct global -> LDS copies of 16-byte units */
#define F16ACC_FAMILY_GENERIC 1 /* strided element gather through registers */
#define F16ACC_FAMILY_REG 2     /* unit-stride rows at any even address: 16-byte loads
                                   through registers (128x128 and 64x64 tiles) */

/*
 * c[M,N] = a[M,K] @ b[K,N]; a and b binary16, c binary16 or binary32.
 *
 * Replaces the reference's host op and its two Triton launches,
 * f16acc/kernel.py:84-105 (mm -> _gemm[grid] at :99 and _redo[grid] at
 * :103-104).  Shape / dtype / device validation stays in the Python layer
 * (kernel.py:87-90 raise ValueError there); this function re-checks only what
 * it needs to stay in bounds.
 *
 *   a, b, c           device pointers (HIP), element strides may be anything,
 *                     including the stride-(1, K) view w.t() of an nn.Linear
 *                     weight (kernel.py:84, patch.py:28)
 *   tile_flags        optional (may be NULL): receives one byte per output
 *                     tile, row-major over the tile grid of f16acc_tile_config,
 *                     1 where the tile's chunked FP32 sum held inf or NaN and
 *                     was recomputed with FP32 accumulation (kernel.py:70-71,
 *                     75-81); sized f16acc_tile_config's tiles_m * tiles_n
 *   M, N, K           sizes; M == 0 or N == 0 launches nothing, K == 0 writes 0
 *   sam, sak          a strides (elements): a[i][k] = a[i*sam + k*sak]
 *   sbk, sbn          b strides: b[k][j] = b[k*sbk + j*sbn]
 *   scm, scn          c strides
 *   out_dtype         F16ACC_OUT_F16 or F16ACC_OUT_F32 (kernel.py:93 c dtype)
 *   chunked           1: 32-long K chunks rounded to binary16 and added into
 *                     an FP32 sum, non-finite tiles redone in FP32 on the same
 *                     stream without a host sync (kernel.py:49, 70-81);
 *                     0: plain FP32 accumulation (kernel.py:50-51)
 *   stream            hipStream_t to launch on (NULL = the null stream)
 *
 * All offsets are 64-bit, so outputs past 2^31 elements are addressed
 * correctly (kernel.py:97-98 switches Triton to int64 for that).
 */
int f16acc_gemm(const void* a, const void* b, void* c, uint8_t* tile_flags,
                int64_t M, int64_t N, int64_t K,
                int64_t sam, int64_t sak, int64_t sbk, int64_t sbn,
                int64_t scm, int64_t scn,
                int out_dtype, int chunked, void* stream);

/*
 * f16acc_gemm plus a bias: c[i][j] = a[i] . b[:, j] + bias[j], bias a
 * contiguous binary16 [N] vector (non-NULL).  Replaces the reference's
 * nn.Linear routing, f16acc/patch.py:28-30 (y = mm(x2, w.t()); y += b), with
 * the add fused into the GEMM's store and the same rounding: for a binary16
 * output the FP32 sum is rounded to binary16, the bias added in FP32 and the
 * result rounded again (torch's fp16 y += b), so results equal the unfused
 * sequence bit for bit.  A binary32 output adds the bias to the FP32 sum.
 */
int f16acc_gemm_bias(const void* a, const void* b, const void* bias, void* c, uint8_t* tile_flags,
                     int64_t M, int64_t N, int64_t K,
                     int64_t sam, int64_t sak, int64_t sbk, int64_t sbn,
                     int64_t scm, int64_t scn,
                     int out_dtype, int chunked, void* stream);

/*
 * Workspace that f16acc_gemm_ws uses for this problem: F16ACC_WS_HEADER
 * bytes plus the split-K partials, or 0 when it needs none.  Shapes with
 * few output tiles (k/v projections, 2048 x 256) leave most CUs idle;
 * splitting K into chunk-aligned ranges fills them.  Shapes of at most one
 * round of 256x256 tiles and K > 2496 (4096^3) use the header alone: their
 * tiles that overflow are listed there and redone by a second launch (see
 * f16acc_gemm_ws); at shorter K that launch would cost more than the
 * in-place redo it replaces.
 */
int f16acc_workspace_size(int64_t M, int64_t N, int64_t K,
                          int64_t sam, int64_t sak, int64_t sbk, int64_t sbn,
                          const void* a, const void* b, size_t* bytes);

/*
 * f16acc_gemm (bias NULL) or f16acc_gemm_bias (bias non-NULL), with a
 * workspace (256-byte aligned, ws_bytes >= f16acc_workspace_size, its first
 * F16ACC_WS_HEADER bytes zero on first use); with a NULL or smaller
 * workspace it does exactly what they do.
 *   - A split problem runs two launches on `stream`: workgroups sum K ranges
 *     of whole chunk pairs (so the chunks are the reference's,
 *     f16acc/kernel.py:44-49) into FP32 partials in the workspace; then one
 *     workgroup per tile adds them in split order, flags the tile when the
 *     total is not finite and recomputes it over all of K with FP32
 *     accumulation (kernel.py:70-81), and stores it.
 *   - A problem of at most one round of 256x256 tiles and K > 2496 runs as
 *     f16acc_gemm, except that a flagged tile is appended to the header's
 *     list instead of being redone by its own workgroup, and a second launch
 *     always follows:
 *     each flagged tile is recomputed in FP32 as four 128x128 quarters by
 *     four workgroups, and the launch's workgroups leave at once when the list
 *     is empty (the reference's separate _redo launch, kernel.py:75-81,
 *     103-104).  The last of them empties the list again.
 * Calls that overlap in time need separate workspaces.
 */
int f16acc_gemm_ws(const void* a, const void* b, const void* bias, void* c, uint8_t* tile_flags,
                   int64_t M, int64_t N, int64_t K,
                   int64_t sam, int64_t sak, int64_t sbk, int64_t sbn,
                   int64_t scm, int64_t scn,
                   int out_dtype, int chunked, void* stream, void* workspace, size_t ws_bytes);

/*
 * f16acc_gemm_ws without a caller workspace and without any allocation: the
 * workspace is a fixed scratch array of 32 MiB plus F16ACC_WS_HEADER bytes
 * that the library's code object holds in device memory on every GPU where
 * it is loaded, in every process, until the process ends.  No counterpart in the reference; it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results as
 * f16acc_gemm_ws (bias may be NULL).
 *
 *   - The first call on a device looks up that device's scratch address
 *     (hipGetSymbolAddress); the current device must be the stream's
 *     (F16ACC_E_DEVICE otherwise).
 *   - A split plan larger than the scratch returns F16ACC_E_SCRATCH before
 *     any launch (on a 256-CU MI355X every plan fits: at most 32 MiB).
 *   - Calls that overlap in time on one GPU share its scratch and race:
 *     serialise them (one stream, or events).  The scratch keeps the last
 *     call's partials and needs no clearing.
 */
int f16acc_gemm_noalloc(const void* a, const void* b, const void* bias, void* c, uint8_t* tile_flags,
                        int64_t M, int64_t N, int64_t K,
                        int64_t sam, int64_t sak, int64_t sbk, int64_t sbn,
                        int64_t scm, int64_t scn,
                        int out_dtype, int chunked, void* stream);

/*
 * The tile configuration f16acc_gemm picks for a problem: replaces the
 * reference's autotuned CONFIGS table and best_config handoff
 * (f16acc/kernel.py:16-19, 63, 101-102) with a fixed per-shape table.
 * forced_tile = -1 asks for the table's choice; an F16ACC_TILE_* value asks
 * what f16acc_gemm_tile would run with that tile (a fast tile the operands'
 * strides or alignment do not allow falls back to F16ACC_TILE_GENERIC).
 * Writes the tile id, the workgroup tile (bm x bn), the tile grid, the
 * kernel family (F16ACC_FAMILY_*) and the threads per workgroup.  Any output
 * pointer may be NULL.
 */
int f16acc_tile_config(int64_t M, int64_t N, int64_t K,
                       int64_t sam, int64_t sak, int64_t sbk, int64_t sbn,
                       const void* a, const void* b, int forced_tile,
                       int* tile, int* bm, int* bn, int64_t* tiles_m, int64_t* tiles_n,
                       int* family, int* threads);

/*
 * f16acc_gemm with the tile configuration forced to `tile` (F16ACC_TILE_*)
 * instead of the per-shape table's choice; same results up to the redo
 * granularity (tile_flags follows the forced tile grid).  For tuning and
 * benchmarking the table, as the reference's autotuner times every entry of
 * CONFIGS on first use (f16acc/kernel.py:16-19, 63).
 */
int f16acc_gemm_tile(const void* a, const void* b, void* c, uint8_t* tile_flags,
                     int64_t M, int64_t N, int64_t K,
                     int64_t sam, int64_t sak, int64_t sbk, int64_t sbn,
                     int64_t scm, int64_t scn,
                     int out_dtype, int chunked, void* stream, int tile);

/*
 * f16acc_gemm_tile with a split-K workspace, as f16acc_gemm_ws: a forced
 * 256x128, 128x256 or 128x128 tile whose tiles leave CUs idle splits K the
 * way the table's own 128x128 pick does (the 256x256 and 64x64 tiles never
 * split).  A workspace of 32 MiB + F16ACC_WS_HEADER covers every split on a
 * 256-CU GPU; a smaller one runs the problem unsplit.  For tuning, and for testing the
 * split path on every tile that has one.
 */
int f16acc_gemm_tile_ws(const void* a, const void* b, void* c, uint8_t* tile_flags,
                        int64_t M, int64_t N, int64_t K,
                        int64_t sam, int64_t sak, int64_t sbk, int64_t sbn,
                        int64_t scm, int64_t scn,
                        int out_dtype, int chunked, void* stream, int tile,
                        void* workspace, size_t ws_bytes);

/*
 * Operand packing for the fast kernels: dst[r][c] = src[r*s_r + c*s_c] for
 * r < rows, c < cols, zero elsewhere in the rows_pad x ld destination
 * (contiguous, row stride ld; ld a multiple of 8, dst 16-byte aligned).
 * The fast kernels need 16-byte aligned rows and K a multiple of 8; an
 * operand that misses this (odd K, odd strides, offset views) is packed once
 * with K padded by zeros (exact: zeros add nothing to a chunk's sum) and the
 * GEMM runs on the copy.  The reference needs no counterpart: Triton's
 * masked loads (f16acc/kernel.py:45-47) read any layout directly, at the
 * cost this copy avoids.  The caller owns dst (the Python layer allocates it
 * with torch).  Launches on `stream`; no synchronisation.
 */
int f16acc_pack(const void* src, void* dst, int64_t rows, int64_t cols,
                int64_t s_r, int64_t s_c, int64_t rows_pad, int64_t ld, void* stream);

/*
 * Output tile processed by workgroup `block` of a launch over a
 * tiles_m x tiles_n grid (the XCD-aware, group-M swizzled order the kernels
 * use).  Exposed so the mapping can be checked on the host; the reference's
 * counterpart is _tile, f16acc/kernel.py:22-34.  Returns F16ACC_E_ARG when
 * block is outside [0, tiles_m * tiles_n).
 */
int f16acc_block_tile(int64_t block, int64_t tiles_m, int64_t tiles_n,
                      int64_t* tile_m, int64_t* tile_n);

/*
 * Launch plan check: where f16acc_gemm (without tile flags) cuts a problem
 * whose 256x256 tiles fill whole rounds of the CUs plus a small ragged
 * round.  *nsplit > 0: output columns [0, nsplit) run as 256x256 tiles and
 * [nsplit, N) as a second launch with the table's choice for that shape;
 * *nsplit < 0: the same with rows [0, -nsplit) and [-nsplit, M); 0: one
 * grid.  No counterpart in the reference (one Triton grid per call);
 * exposed for host-side checks.
 */
int f16acc_tail_split(int64_t M, int64_t N, int64_t K, int64_t sam, int64_t sak, int64_t sbk, int64_t sbn,
                      const void* a, const void* b, int64_t* nsplit);

/* Short text for a return code of this library (never NULL). */
const char* f16acc_strerror(int code);

/* ABI version: bumped whenever a signature or the tile ids above change. */
int f16acc_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* F16ACC_H */
