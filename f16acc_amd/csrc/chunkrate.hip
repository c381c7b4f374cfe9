// chunkrate: what the chunk-32 emulation costs on the MFMA pipe of gfx950.
//
// The MI355X counterpart of the reference's bench/rate.py (MMA rate with
// FP32 vs FP16 accumulation) and bench/chunkrate.py (cost of promoting FP16
// accumulators to FP32 every few K steps).  gfx950 has no FP16-accumulating
// MFMA, so the question becomes: how fast can a 16x16x32 chunk MFMA with a
// zero accumulator be followed by the FP16 rounding of its result and the
// FP32 sum, compared with plain FP32-accumulating MFMAs?
//
// Register-only loops (no memory traffic), every instruction in inline asm so
// the issue order is exactly the program order.  Each measurement reports
// shader-clock cycles (s_memtime) per "block step" per SIMD: two chunk MFMAs
// of one 16x16 output block (ideal 32 cycles) plus whatever the variant adds.
//
//   part 0  numerics self-check of the two summation forms (pair selector
//           MFMA, sparse quad selector v_smfmac) against a scalar host sum
//           of the same FP16-rounded chunk partials; exits 1 on a mismatch
//   part 1  which VALU instruction classes overlap an MFMA: per step one MFMA
//           then four VALU ops of one class (16 cycles if fully hidden)
//   part 2  complete chunk epilogues, software pipelined (the epilogue of
//           block j-2 runs next to the MFMAs of block j)
//   part 3  the smaller f16 MFMAs (16x16x16, 4x4x4 in 16 blocks): cycles per
//           instruction, and epilogues that add a chunk pair with two of
//           them as lane-local identity sums instead of one 16x16x32
//           selector (the self-check covers those sums too)
//
//   usage: chunkrate            (needs one gfx950 GPU; prints a table)

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

#define CHECK(x)                                                                   \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                                \
    }                                                                              \
  } while (0)

constexpr int kIters = 20000;
constexpr int kThreads = 256;

// ---- part 1: MFMA + four VALU ops of one class -----------------------------
#define MFMA_ACC(acc, a, b) asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b))

template <int T>
__device__ __forceinline__ void valu4(float& x0, float& x1, float& x2, float& x3, unsigned& h0, unsigned& h1) {
#define V4(s) asm volatile(s : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(h0), "+v"(h1))
  if (T == 0) V4("v_add_f32 %0, %0, %1\n v_add_f32 %1, %1, %2\n v_add_f32 %2, %2, %3\n v_add_f32 %3, %3, %0");
  if (T == 1) V4("v_cvt_pk_f16_f32 %4, %0, %1\n v_cvt_pk_f16_f32 %5, %2, %3\n v_cvt_pk_f16_f32 %4, %1, %2\n v_cvt_pk_f16_f32 %5, %3, %0");
  if (T == 2) V4("v_dot2c_f32_f16 %0, %4, %5\n v_dot2c_f32_f16 %1, %5, %4\n v_dot2c_f32_f16 %2, %4, %5\n v_dot2c_f32_f16 %3, %5, %4");
  if (T == 3) V4("v_fma_mix_f32 %0, %4, %5, %0 op_sel_hi:[1,1,0]\n v_fma_mix_f32 %1, %4, %5, %1 op_sel_hi:[1,1,0]\n v_fma_mix_f32 %2, %4, %5, %2 op_sel_hi:[1,1,0]\n v_fma_mix_f32 %3, %4, %5, %3 op_sel_hi:[1,1,0]");
  if (T == 4) V4("v_add_u32 %4, %4, %5\n v_add_u32 %5, %5, %4\n v_xor_b32 %4, %4, %5\n v_add_u32 %5, %5, %4");
  if (T == 5) V4("v_pk_add_f16 %4, %4, %5\n v_pk_add_f16 %5, %5, %4\n v_pk_add_f16 %4, %4, %5\n v_pk_add_f16 %5, %5, %4");
  if (T == 6) V4("v_cvt_f32_f16 %0, %4\n v_cvt_f32_f16 %1, %5\n v_cvt_f32_f16 %2, %4\n v_cvt_f32_f16 %3, %5");
  if (T == 7) V4("v_fma_f32 %0, %0, %1, %2\n v_fma_f32 %1, %1, %2, %3\n v_fma_f32 %2, %2, %3, %0\n v_fma_f32 %3, %3, %0, %1");
#undef V4
}
constexpr const char* kValuNames[] = {"v_add_f32", "v_cvt_pk_f16_f32", "v_dot2c_f32_f16", "v_fma_mix_f32",
                                      "v_add_u32 / v_xor_b32", "v_pk_add_f16", "v_cvt_f32_f16", "v_fma_f32"};

// MODE 0: MFMA + VALU interleaved, 1: MFMA only, 2: VALU only
template <int T, int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void overlap_kernel(
    float* out, int iters, unsigned long long* cyc) {
  const int lane = threadIdx.x & 63;
  f16x8 a0, a1;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a0[e] = (f16)(0.01f * (lane + e));
    a1[e] = (f16)(0.02f * (lane - e));
  }
  f32x4 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, (float)j};
  float x0 = lane, x1 = 1.f, x2 = 2.f, x3 = 3.f;
  unsigned h0 = 0x3c003c00u + lane, h1 = 0x3c003c00u;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (MODE != 2) MFMA_ACC(acc[j], a0, a1);
      if (MODE != 1) valu4<T>(x0, x1, x2, x3, h0, h1);
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = x0 + x1 + x2 + x3 + (float)(h0 ^ h1);
#pragma unroll
  for (int j = 0; j < 16; ++j) s += acc[j][0] + acc[j][3];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}

// ---- part 2: complete chunk epilogues ----------------------------------------
#define MFMA_ZERO(d, a, b) asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b))
#define CVT_PK(h, x, y) asm volatile("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(h) : "v"(x), "v"(y))
#define MIX_LO(s, h) asm volatile("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]" : "+v"(s) : "v"(h))
#define MIX_HI(s, h) asm volatile("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(s) : "v"(h))
#define DOT2(s, h) asm volatile("v_dot2c_f32_f16 %0, %1, %2" : "+v"(s) : "v"(h), "v"(ones))
#define SMFMAC(acc, a, b, idx) \
  asm volatile("v_smfmac_f32_16x16x64_f16 %0, %1, %2, %3" : "+v"(acc) : "v"(a), "v"(b), "v"(idx))
#define M16X16X16(acc, a, b) asm volatile("v_mfma_f32_16x16x16_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b))
#define M4X4X4(acc, a, b) asm volatile("v_mfma_f32_4x4x4_16b_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b))

// Identity A operands of the lane-local sums (part 3).  v_mfma_f32_16x16x16_f16:
// lane 16q+n holds A[n][4q+e], B[4q+e][n] and D[4q+r][n]; with A[i][k] = (i == k)
// each lane adds its own four B halves to its own four D registers.
// v_mfma_f32_4x4x4_16b_f16 (block l/4): lane l holds A[l%4][e], B[e][l%4] and
// D[r][l%4]; A[i][k] = (i == k) does the same.
__device__ __forceinline__ f16x4 identity_16x16x16(int lane) {
  f16x4 a;
#pragma unroll
  for (int e = 0; e < 4; ++e) a[e] = ((lane & 15) == 4 * (lane >> 4) + e) ? (f16)1.0f : (f16)0.0f;
  return a;
}
__device__ __forceinline__ f16x4 identity_4x4x4(int lane) {
  f16x4 a;
#pragma unroll
  for (int e = 0; e < 4; ++e) a[e] = ((lane & 3) == e) ? (f16)1.0f : (f16)0.0f;
  return a;
}

// Sparse selector of a chunk quad: with B = {X_odd, X_even} (the rounded
// pairs of one 16x16 block from two consecutive stages, dense 16x16x32 B
// layout each: elements 0-7 are K 0-31, elements 8-15 are K 32-63), A row i
// is 1 at K = 2i, 2i+1, 32+2i, 33+2i: lane 16q+i holds K 16q..16q+15 as four
// groups of 4 with two stored values each; rows i with q == i/8 or
// q == 2 + i/8 store (1, 1) at positions 2(i%2), 2(i%2)+1 of group (i%8)/2.
__device__ __forceinline__ void quad_selector(int lane, f16x8& a, int& idx) {
  const int q = lane >> 4, i = lane & 15, g = (i & 7) >> 1, p = 2 * (i & 1);
  const bool on = q == (i >> 3) || q == 2 + (i >> 3);
  idx = 0;
#pragma unroll
  for (int c = 0; c < 8; ++c) a[c] = (on && c / 2 == g) ? (f16)1.0f : (f16)0.0f;
#pragma unroll
  for (int gg = 0; gg < 4; ++gg) idx |= (gg == g ? (p | ((p + 1) << 2)) : (0 | (1 << 2))) << (4 * gg);
}

// E: 0 FP32-accumulating MFMAs (the reference's chunked=False), 1 cvt_pk + dot2,
//    2 cvt_pk + fma_mix, 3 cvt_pk + selector MFMA (the shipped epilogue),
//    4 cvt_pk alone (no sum: a lower bound),
//    5 cvt_pk + sparse selector (one v_smfmac_f32_16x16x64_f16 per block per
//      two stages; the two stages' rounded pairs joined into one 8-register
//      operand), 6 as 5 with the rounding written straight into that operand
//    (5 and 6 run an even and an odd stage per iteration: 2 NB steps),
//    7 cvt_pk x4 (each chunk's four values into two dwords) + two
//      v_mfma_f32_16x16x16_f16 identity sums, 8 the same with two
//      v_mfma_f32_4x4x4_16b_f16
template <int E>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void epilogue_kernel(
    float* out, int iters, unsigned long long* cyc) {
  constexpr int NB = 8;
  const int lane = threadIdx.x & 63;
  f16x8 a0, a1, b[NB], sel;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a0[e] = (f16)(0.01f * (lane + e));
    a1[e] = (f16)(0.02f * (lane - e));
    sel[e] = (4 * (lane >> 4) + (e >> 1) == (lane & 15)) ? (f16)1.0f : (f16)0.0f;
  }
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) b[j][e] = (f16)(0.001f * (lane * (j + 1) + e));
  const unsigned ones = 0x3c003c00u;
  f32x4 p0[NB], p1[NB], S[NB];
  u32x4 h[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    p0[j] = p1[j] = S[j] = f32x4{0.f, 0.f, 0.f, (float)j};
    h[j] = u32x4{0u, 0u, 0u, 0u};
  }
  f16x8 sel4;
  int idx;
  quad_selector(lane, sel4, idx);
  const f16x4 id = E == 7 ? identity_16x16x16(lane) : identity_4x4x4(lane);
  u32x4 hs[NB];
  u32x8 X[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    hs[j] = u32x4{0u, 0u, 0u, 0u};
    X[j] = u32x8{0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  }
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
    if (E == 5 || E == 6) {
#pragma unroll
      for (int pass = 0; pass < 2; ++pass)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int q = (j + NB - 2) % NB;
          MFMA_ZERO(p0[j], b[j], a0);
          if (E == 5) {
            u32x4& d = pass ? h[q] : hs[q];
            CVT_PK(d[0], p0[q][0], p1[q][0]);
            CVT_PK(d[1], p0[q][1], p1[q][1]);
          } else {
            CVT_PK(X[q][4 * pass + 0], p0[q][0], p1[q][0]);
            CVT_PK(X[q][4 * pass + 1], p0[q][1], p1[q][1]);
          }
          MFMA_ZERO(p1[j], b[j], a1);
          if (E == 5) {
            u32x4& d = pass ? h[q] : hs[q];
            CVT_PK(d[2], p0[q][2], p1[q][2]);
            CVT_PK(d[3], p0[q][3], p1[q][3]);
          } else {
            CVT_PK(X[q][4 * pass + 2], p0[q][2], p1[q][2]);
            CVT_PK(X[q][4 * pass + 3], p0[q][3], p1[q][3]);
          }
          if (pass == 1) {
            const int r = (j + NB - 3) % NB;
            if (E == 5) {
              const u32x8 bb = __builtin_shufflevector(h[r], hs[r], 0, 1, 2, 3, 4, 5, 6, 7);
              SMFMAC(S[r], sel4, bb, idx);
            } else {
              SMFMAC(S[r], sel4, X[r], idx);
            }
          }
        }
      continue;
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int q = (j + NB - 2) % NB;  // block whose epilogue runs now: its MFMAs are 4 MFMAs old
      if (E == 0) {
        MFMA_ACC(S[j], b[j], a0);
        MFMA_ACC(S[j], b[j], a1);
        continue;
      }
      MFMA_ZERO(p0[j], b[j], a0);
      if (E == 3) {
        CVT_PK(h[q][0], p0[q][0], p1[q][0]);
        CVT_PK(h[q][1], p0[q][1], p1[q][1]);
      } else if (E == 7 || E == 8) {
        CVT_PK(h[q][0], p0[q][0], p0[q][1]);
        CVT_PK(h[q][1], p0[q][2], p0[q][3]);
      } else {
        CVT_PK(h[q][0], p0[q][0], p1[q][0]);
        CVT_PK(h[q][1], p0[q][1], p1[q][1]);
        CVT_PK(h[q][2], p0[q][2], p1[q][2]);
        CVT_PK(h[q][3], p0[q][3], p1[q][3]);
      }
      MFMA_ZERO(p1[j], b[j], a1);
      if (E == 1) {
        DOT2(S[q][0], h[q][0]); DOT2(S[q][1], h[q][1]); DOT2(S[q][2], h[q][2]); DOT2(S[q][3], h[q][3]);
      } else if (E == 2) {
        MIX_LO(S[q][0], h[q][0]); MIX_HI(S[q][0], h[q][0]); MIX_LO(S[q][1], h[q][1]); MIX_HI(S[q][1], h[q][1]);
        MIX_LO(S[q][2], h[q][2]); MIX_HI(S[q][2], h[q][2]); MIX_LO(S[q][3], h[q][3]); MIX_HI(S[q][3], h[q][3]);
      } else if (E == 3) {
        CVT_PK(h[q][2], p0[q][2], p1[q][2]);
        CVT_PK(h[q][3], p0[q][3], p1[q][3]);
        const int r = (j + NB - 3) % NB;  // rounded during the previous step
        MFMA_ACC(S[r], sel, h[r]);
      } else if (E == 7 || E == 8) {
        CVT_PK(h[q][2], p1[q][0], p1[q][1]);
        CVT_PK(h[q][3], p1[q][2], p1[q][3]);
        const int r = (j + NB - 3) % NB;
        const u32x2 x0 = {h[r][0], h[r][1]}, x1 = {h[r][2], h[r][3]};
        if (E == 7) {
          M16X16X16(S[r], id, x0);
          M16X16X16(S[r], id, x1);
        } else {
          M4X4X4(S[r], id, x0);
          M4X4X4(S[r], id, x1);
        }
      }
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NB; ++j) s += S[j][0] + S[j][3] + p0[j][1] + p1[j][2] + (float)h[j][1] + (float)hs[j][2] + (float)X[j][5];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}

// ---- part 3: cycles per MFMA of each f16 shape ------------------------------
// OP 0: v_mfma_f32_16x16x32_f16, 1: v_mfma_f32_16x16x16_f16,
// 2: v_mfma_f32_4x4x4_16b_f16; 16 independent accumulators back to back.
template <int OP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void mfma_rate_kernel(
    float* out, int iters, unsigned long long* cyc) {
  const int lane = threadIdx.x & 63;
  f16x8 a8, b8;
  f16x4 a4, b4;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a8[e] = (f16)(0.01f * (lane + e));
    b8[e] = (f16)(0.02f * (lane - e));
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a4[e] = a8[e];
    b4[e] = b8[e];
  }
  f32x4 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, (float)j};
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (OP == 0) MFMA_ACC(acc[j], a8, b8);
      if (OP == 1) M16X16X16(acc[j], a4, b4);
      if (OP == 2) M4X4X4(acc[j], a4, b4);
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += acc[j][0] + acc[j][3];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}

// ---- part 0: numerics self-check ----------------------------------------------
// One wave: four chunk MFMAs (zero accumulator) of per-lane fragments a[c],
// b[c]; the pair selector adds the FP16-rounded partials of chunks 0 and 1
// to s_in, the sparse quad selector those of all four chunks: the same
// instructions, operands and selector matrices as the timed loops above
// (written with builtins here, so the compiler places the wait states
// between an MFMA and the instructions reading its result).  Written out:
// the FP32 partials and both sums, so the host can check them register by
// register: whatever element a lane's register r holds, the selector must
// leave
//   s_in[r] + f16(P0[r]) + f16(P1[r])      (pair)
//   s_in[r] + f16(P0[r]) + ... + f16(P3[r]) (quad)
// in that same register; and the lane-local identity sums of part 3, one
// MFMA per chunk (16x16x16 and 4x4x4 forms), must leave
//   (s_in[r] + f16(P0[r])) + f16(P1[r])     (two FP32 additions in order)
__global__ __launch_bounds__(64) void selfcheck_kernel(const f16x8* in_a, const f16x8* in_b, const f32x4* s_in,
                                                       f32x4* p_out, f32x4* s_pair, f32x4* s_quad, f32x4* s_id) {
  typedef f16 f16x16 __attribute__((ext_vector_type(16)));
  typedef f16 f16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const int lane = threadIdx.x;
  f16x8 sel;
#pragma unroll
  for (int e = 0; e < 8; ++e) sel[e] = (4 * (lane >> 4) + (e >> 1) == (lane & 15)) ? (f16)1.0f : (f16)0.0f;
  f16x8 sel4;
  int idx;
  quad_selector(lane, sel4, idx);
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 p[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    p[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(in_b[c * 64 + lane], in_a[c * 64 + lane], zero, 0, 0, 0);
    p_out[c * 64 + lane] = p[c];
  }
  f16x8 even, odd;  // v_cvt_pk_f16_f32 of (P0, P1) and (P2, P3), register r -> elements 2r, 2r+1
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const f16x2 e = __builtin_convertvector((f32x2){p[0][r], p[1][r]}, f16x2);
    const f16x2 o = __builtin_convertvector((f32x2){p[2][r], p[3][r]}, f16x2);
    even[2 * r] = e[0];
    even[2 * r + 1] = e[1];
    odd[2 * r] = o[0];
    odd[2 * r + 1] = o[1];
  }
  s_pair[lane] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, even, s_in[lane], 0, 0, 0);
  const f16x16 bb = __builtin_shufflevector(odd, even, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
  s_quad[lane] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(sel4, bb, s_in[lane], idx, 0, 0);
  const f16x4 id16 = identity_16x16x16(lane), id4 = identity_4x4x4(lane);
  f32x4 t16 = s_in[lane], t4 = s_in[lane];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    f16x4 x;
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = (f16)p[c][r];
    t16 = __builtin_amdgcn_mfma_f32_16x16x16f16(id16, x, t16, 0, 0, 0);
    t4 = __builtin_amdgcn_mfma_f32_4x4x4f16(id4, x, t4, 0, 0, 0);
  }
  s_id[lane] = t16;
  s_id[64 + lane] = t4;
}

// Host side of part 0.  Integer-valued inputs keep every partial and sum
// exact in FP32 while the partials pass 2048, where binary16 rounds to even
// integers: the sums must then match bit for bit.  Random N(0, 1) inputs
// check the same within 2 ulp of the FP32 sum (the MFMA may round a
// three- or five-term sum once where the host rounds it once too, in a
// different association).  Returns the number of mismatches.
int selfcheck(bool integers, unsigned seed, double* worst_ulp) {
  std::vector<f16x8> ha(4 * 64), hb(4 * 64);
  std::vector<f32x4> hs(64), hp(4 * 64), hpair(64), hquad(64), hid(128);
  unsigned st = seed;
  auto rnd = [&]() {  // xorshift32
    st ^= st << 13;
    st ^= st >> 17;
    st ^= st << 5;
    return st;
  };
  auto gauss = [&]() {  // sum of 12 uniforms, minus 6: approximately N(0, 1)
    double x = 0;
    for (int i = 0; i < 12; ++i) x += (rnd() & 0xffffff) / 16777216.0;
    return x - 6.0;
  };
  for (int i = 0; i < 4 * 64; ++i)
    for (int e = 0; e < 8; ++e) {
      // integer partials up to 32 * 15 * 31 = 14880, mostly past 2048
      ha[i][e] = integers ? (f16)(float)(rnd() % 16) : (f16)(float)gauss();
      hb[i][e] = integers ? (f16)(float)(rnd() % 32) : (f16)(float)gauss();
    }
  for (int i = 0; i < 64; ++i)
    for (int r = 0; r < 4; ++r) hs[i][r] = integers ? (float)((int)(rnd() % 2001) - 1000) : (float)(100.0 * gauss());
  f16x8 *da, *db;
  f32x4 *ds, *dp, *dpair, *dquad, *did;
  CHECK(hipMalloc(&da, ha.size() * sizeof(f16x8)));
  CHECK(hipMalloc(&db, hb.size() * sizeof(f16x8)));
  CHECK(hipMalloc(&ds, hs.size() * sizeof(f32x4)));
  CHECK(hipMalloc(&dp, hp.size() * sizeof(f32x4)));
  CHECK(hipMalloc(&dpair, 64 * sizeof(f32x4)));
  CHECK(hipMalloc(&dquad, 64 * sizeof(f32x4)));
  CHECK(hipMalloc(&did, 128 * sizeof(f32x4)));
  CHECK(hipMemcpy(da, ha.data(), ha.size() * sizeof(f16x8), hipMemcpyHostToDevice));
  CHECK(hipMemcpy(db, hb.data(), hb.size() * sizeof(f16x8), hipMemcpyHostToDevice));
  CHECK(hipMemcpy(ds, hs.data(), hs.size() * sizeof(f32x4), hipMemcpyHostToDevice));
  hipLaunchKernelGGL(selfcheck_kernel, dim3(1), dim3(64), 0, 0, da, db, ds, dp, dpair, dquad, did);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  CHECK(hipMemcpy(hp.data(), dp, hp.size() * sizeof(f32x4), hipMemcpyDeviceToHost));
  CHECK(hipMemcpy(hpair.data(), dpair, 64 * sizeof(f32x4), hipMemcpyDeviceToHost));
  CHECK(hipMemcpy(hquad.data(), dquad, 64 * sizeof(f32x4), hipMemcpyDeviceToHost));
  CHECK(hipMemcpy(hid.data(), did, 128 * sizeof(f32x4), hipMemcpyDeviceToHost));
  for (void* q : {(void*)da, (void*)db, (void*)ds, (void*)dp, (void*)dpair, (void*)dquad, (void*)did}) CHECK(hipFree(q));
  int bad = 0, rounded = 0, bad_id = 0;
  *worst_ulp = 0;
  for (int l = 0; l < 64; ++l)
    for (int r = 0; r < 4; ++r) {
      double h[4];
      for (int c = 0; c < 4; ++c) {
        h[c] = (double)(float)(f16)hp[c * 64 + l][r];  // RNE to binary16, as v_cvt_pk_f16_f32
        rounded += h[c] != (double)hp[c * 64 + l][r];
      }
      // the identity sums: two FP32 additions in chunk order, bit for bit
      const float seq = (hs[l][r] + (float)h[0]) + (float)h[1];
      bad_id += (hid[l][r] != seq) + (hid[64 + l][r] != seq);
      const double pair = (double)hs[l][r] + h[0] + h[1];
      const double quad = pair + h[2] + h[3];
      for (int which = 0; which < 2; ++which) {
        const double want = which ? quad : pair;
        const float got = which ? hquad[l][r] : hpair[l][r];
        const double ulp = std::fmax(std::fabs(std::nextafter((float)want, INFINITY) - (float)want), 1e-30);
        const double err = std::fabs((double)got - want) / ulp;
        *worst_ulp = err > *worst_ulp ? err : *worst_ulp;
        if (integers ? (double)got != want : err > 2.0) ++bad;
      }
    }
  if (integers && rounded == 0) {
    std::printf("self-check: no partial was rounded, the inputs do not exercise the rounding\n");
    ++bad;
  }
  std::printf("self-check (%s inputs): %d of 512 sums off, %d of 1024 partials rounded to binary16, "
              "worst %.2f ulp\n", integers ? "integer" : "N(0,1)", bad, rounded, *worst_ulp);
  std::printf("identity-sum check (%s inputs): %d of 512 sums off (16x16x16 and 4x4x4 forms, exact)\n",
              integers ? "integer" : "N(0,1)", bad_id);
  return bad + bad_id;
}

struct Bufs {
  float* out = nullptr;
  unsigned long long* cyc = nullptr;
  int blocks = 0;
};

// Cycles per inner step per SIMD: the slowest workgroup's s_memtime span over
// its iterations, divided by the steps its SIMD ran (waves_per_simd waves).
template <class K>
double measure(K kernel, const Bufs& b, int steps_per_iter, int waves_per_simd) {
  hipLaunchKernelGGL(kernel, dim3(b.blocks), dim3(kThreads), 0, 0, b.out, 10, b.cyc);  // warm-up
  CHECK(hipDeviceSynchronize());
  hipLaunchKernelGGL(kernel, dim3(b.blocks), dim3(kThreads), 0, 0, b.out, kIters, b.cyc);
  CHECK(hipDeviceSynchronize());
  std::vector<unsigned long long> c(b.blocks);
  CHECK(hipMemcpy(c.data(), b.cyc, c.size() * sizeof(c[0]), hipMemcpyDeviceToHost));
  unsigned long long mx = 0;
  for (auto x : c) mx = x > mx ? x : mx;
  return (double)mx / ((double)kIters * steps_per_iter * waves_per_simd);
}

template <int T>
void part1_row(const Bufs& b, int w) {
  const double both = measure(overlap_kernel<T, 0>, b, 16, w);
  const double valu = measure(overlap_kernel<T, 2>, b, 16, w);
  std::printf("  %-22s %8.2f %12.2f\n", kValuNames[T], both, valu);
}

}  // namespace

int main() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, 0));
  std::printf("chunkrate on %s (%s), %d CUs; cycles are shader clocks (s_memtime) per SIMD\n", prop.name,
              prop.gcnArchName, cus);
  std::printf("part 0: pair selector MFMA and sparse quad selector vs a host sum of the rounded partials\n");
  double ulp_int = 0, ulp_rand = 0;
  const int bad = selfcheck(true, 12345u, &ulp_int) + selfcheck(false, 777u, &ulp_rand);
  if (bad) {
    std::printf("self-check FAILED\n");
    return 1;
  }
  std::printf("self-check ok\n");
  for (int w = 1; w <= 2; ++w) {
    Bufs b;
    b.blocks = cus * w;  // 4 waves per workgroup: w waves per SIMD
    CHECK(hipMalloc(&b.out, (size_t)b.blocks * kThreads * sizeof(float)));
    CHECK(hipMalloc(&b.cyc, (size_t)b.blocks * sizeof(unsigned long long)));
    std::printf("\n== %d wave(s) per SIMD\n", w);
    std::printf("part 1: one MFMA 16x16x32 (16 cycles) + four VALU ops; cycles per step\n");
    std::printf("  %-22s %8s %12s\n", "VALU op", "MFMA+4op", "4 ops alone");
    std::printf("  %-22s %8.2f\n", "(MFMA alone)", measure(overlap_kernel<0, 1>, b, 16, w));
    part1_row<0>(b, w);
    part1_row<1>(b, w);
    part1_row<2>(b, w);
    part1_row<3>(b, w);
    part1_row<4>(b, w);
    part1_row<5>(b, w);
    part1_row<6>(b, w);
    part1_row<7>(b, w);
    std::printf("part 2: chunk-pair epilogues; cycles per block step (2 chunk MFMAs = 32 ideal), fraction of peak\n");
    const char* names[] = {"FP32-accumulating MFMAs", "cvt_pk x4 + dot2 x4", "cvt_pk x4 + fma_mix x8",
                           "cvt_pk x4 + selector MFMA", "cvt_pk x4 alone (bound)",
                           "cvt_pk x4 + 1/2 smfmac (copy)", "cvt_pk x4 + 1/2 smfmac (in place)"};
    double c[7];
    c[0] = measure(epilogue_kernel<0>, b, 8, w);
    c[1] = measure(epilogue_kernel<1>, b, 8, w);
    c[2] = measure(epilogue_kernel<2>, b, 8, w);
    c[3] = measure(epilogue_kernel<3>, b, 8, w);
    c[4] = measure(epilogue_kernel<4>, b, 8, w);
    c[5] = measure(epilogue_kernel<5>, b, 16, w);
    c[6] = measure(epilogue_kernel<6>, b, 16, w);
    for (int i = 0; i < 7; ++i) std::printf("  %-33s %8.2f  %.3f\n", names[i], c[i], 32.0 / c[i]);
    std::printf("part 3: cycles per MFMA (16 independent accumulators)\n");
    std::printf("  %-33s %8.2f\n", "v_mfma_f32_16x16x32_f16", measure(mfma_rate_kernel<0>, b, 16, w));
    std::printf("  %-33s %8.2f\n", "v_mfma_f32_16x16x16_f16", measure(mfma_rate_kernel<1>, b, 16, w));
    std::printf("  %-33s %8.2f\n", "v_mfma_f32_4x4x4_16b_f16", measure(mfma_rate_kernel<2>, b, 16, w));
    std::printf("  chunk-pair epilogues with lane-local identity sums; cycles per block step, fraction of peak\n");
    const double e7 = measure(epilogue_kernel<7>, b, 8, w), e8 = measure(epilogue_kernel<8>, b, 8, w);
    std::printf("  %-33s %8.2f  %.3f\n", "cvt_pk x4 + 2 x 16x16x16 identity", e7, 32.0 / e7);
    std::printf("  %-33s %8.2f  %.3f\n", "cvt_pk x4 + 2 x 4x4x4 identity", e8, 32.0 / e8);
    CHECK(hipFree(b.out));
    CHECK(hipFree(b.cyc));
  }
  return 0;
}
