/*
 * Oracle (test infrastructure, never the product path): a scalar C
 * restatement of the reference's chunk-32 GEMM.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * It follows f16acc/kernel.py of the reference:
 *   _loop  kernel.py:37-54  K is walked in chunks of CHUNK (BLOCK_K = 32,
 *                           kernel.py:17); loads past K read 0 (kernel.py:45-47);
 *                           each chunk is an FP16-accumulated partial that is
 *                           promoted to FP32 and added to an FP32 sum
 *                           (kernel.py:49).  Here the partial is summed in FP32
 *                           in k order and rounded once to FP16 (round-to-
 *                           nearest-even), the "round-once" model of an FP16
 *                           accumulator; mode 1 rounds after every 16 terms
 *                           (two m16n8k16 steps per chunk, the per-k16 model).
 *   _gemm  kernel.py:63-72  a tile is flagged when any element of its FP32
 *                           sum is not finite (|x| < inf is false; NaN too).
 *   _redo  kernel.py:75-81  a flagged tile is recomputed whole with plain FP32
 *                           accumulation, every element of it.
 *   _store kernel.py:57-60  the FP32 tile is cast to the output dtype (RNE).
 * Compiled with -ffp-contract=off so every product and sum is a separate
 * IEEE FP32 operation in a fixed order.
 */
#include <stdint.h>
#include <string.h>

/* IEEE binary16 <-> binary32, written from the format definition. */
float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0x1fu) {
    bits = sign | 0x7f800000u | (man << 13); /* inf / NaN (payload kept) */
  } else if (exp != 0) {
    bits = sign | ((exp + 112u) << 23) | (man << 13); /* normal: rebias 15 -> 127 */
  } else if (man == 0) {
    bits = sign; /* signed zero */
  } else {
    /* subnormal: value = man * 2^-24; normalise into an FP32 normal */
    int e = -1;
    do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
    man &= 0x3ffu;
    bits = sign | ((uint32_t)(112 - e) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) /* inf stays inf; NaN stays a quiet NaN */
    return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  int e = (int)exp - 127; /* unbiased exponent */
  if (e >= 16) return (uint16_t)(sign | 0x7c00u); /* >= 65536: overflow */
  if (e >= -14) {
    /* normal range of binary16: keep 10 mantissa bits, round the 13 dropped */
    uint32_t m = man >> 13, rest = man & 0x1fffu;
    uint32_t h = ((uint32_t)(e + 15) << 10) | m;
    if (rest > 0x1000u || (rest == 0x1000u && (m & 1u))) h += 1u; /* may carry into exp / inf */
    return (uint16_t)(sign | h);
  }
  if (e < -25) return sign; /* below half the smallest subnormal: rounds to zero */
  /* subnormal result: value = sig * 2^(e-23) with sig the 24-bit significand;
     the binary16 subnormal unit is 2^-24, so keep sig >> (-e - 1) ... rounded */
  uint32_t sig = man | 0x800000u;
  int shift = -e - 1; /* 14..24 */
  uint32_t q = sig >> shift, rem = sig & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1u;
  return (uint16_t)(sign | q);
}

static float round_f16(float x) { return oracle_f16_to_f32(oracle_f32_to_f16(x)); }

static int finite32(float x) { return x - x == 0.0f; } /* false for inf and NaN */

/*
 * c[M,N] = a[M,K] @ b[K,N] with the strides given in elements.
 * out_fp32: 0 -> c is binary16, 1 -> c is binary32.
 * chunked:  1 -> chunk semantics + tile flag + FP32 redo, 0 -> plain FP32.
 * bm, bn:   flag/redo tile shape; flags (may be NULL) receives one byte per
 *           tile in row-major tile order.
 * mode:     0 -> round-once chunks, 1 -> per-16 rounding inside a chunk.
 * Returns 0, or -1 on bad arguments.
 */
int oracle_mm(const uint16_t* a, const uint16_t* b, void* c, uint8_t* flags,
              int64_t M, int64_t N, int64_t K, int64_t sam, int64_t sak,
              int64_t sbk, int64_t sbn, int64_t scm, int64_t scn,
              int out_fp32, int chunked, int64_t bm, int64_t bn, int64_t chunk, int mode) {
  if (M < 0 || N < 0 || K < 0 || bm <= 0 || bn <= 0 || chunk <= 0) return -1;
  if (mode == 1 && chunk % 16 != 0) return -1;
  int64_t tm = (M + bm - 1) / bm, tn = (N + bn - 1) / bn;
  for (int64_t ti = 0; ti < tm; ++ti) {
    for (int64_t tj = 0; tj < tn; ++tj) {
      int64_t i0 = ti * bm, j0 = tj * bn;
      int64_t i1 = i0 + bm < M ? i0 + bm : M, j1 = j0 + bn < N ? j0 + bn : N;
      int flag = 0;
      for (int pass = 0; pass < 2; ++pass) {
        int fp32 = !chunked || pass == 1;
        for (int64_t i = i0; i < i1; ++i) {
          for (int64_t j = j0; j < j1; ++j) {
            float s = 0.0f;
            if (fp32) {
              for (int64_t k = 0; k < K; ++k)
                s += oracle_f16_to_f32(a[i * sam + k * sak]) * oracle_f16_to_f32(b[k * sbk + j * sbn]);
            } else {
              for (int64_t k0 = 0; k0 < K; k0 += chunk) {
                int64_t k1 = k0 + chunk < K ? k0 + chunk : K; /* the zero-filled tail adds nothing */
                float p = 0.0f;
                for (int64_t k = k0; k < k1; ++k) {
                  p += oracle_f16_to_f32(a[i * sam + k * sak]) * oracle_f16_to_f32(b[k * sbk + j * sbn]);
                  if (mode == 1 && ((k - k0) % 16) == 15 && k + 1 < k1) p = round_f16(p);
                }
                s += round_f16(p);
              }
              if (!finite32(s)) flag = 1;
            }
            int64_t off = i * scm + j * scn;
            if (out_fp32) ((float*)c)[off] = s;
            else ((uint16_t*)c)[off] = oracle_f32_to_f16(s);
          }
        }
        if (!chunked || !flag) break; /* pass 1 is the FP32 redo of a flagged tile */
      }
      if (flags) flags[ti * tn + tj] = (uint8_t)flag;
    }
  }
  return 0;
}
