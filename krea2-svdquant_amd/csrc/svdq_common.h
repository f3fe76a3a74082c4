// Shared device helpers for the gfx950 SVDQuant kernels.
//
// Storage conventions (the reference checkpoint layout, runtime/load.py:90-126):
//   activations / smooth / l1 / l2 / bias : bf16, carried as uint16_t bits
//   weight scales                         : fp16 bits
//   packed INT4                           : uint8, byte j = (q[2j]+8) | (q[2j+1]+8) << 4
//
// MFMA register layouts used throughout (CDNA 32x32 family, wave64):
//   A operand of a 32x32xK MFMA: lane l supplies row (l % 32); lanes 0-31 and
//   32-63 supply two disjoint halves of the K slice.  B likewise with columns.
//   The kernels only rely on A and B using the SAME (lane-half, element) -> k
//   assignment, which makes the product independent of the hardware's
//   internal k order.
//   D (32x32 accumulator, 16 regs/lane): reg r of lane l holds
//   row = 8*(r/4) + 4*(l/32) + (r%4), col = l % 32.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svdq {

typedef int      i32x4  __attribute__((ext_vector_type(4)));
typedef int      i32x16 __attribute__((ext_vector_type(16)));
typedef float    f32x2  __attribute__((ext_vector_type(2)));
typedef float    f32x4  __attribute__((ext_vector_type(4)));
typedef float    f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16   bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16   bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2  __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4  __attribute__((ext_vector_type(4)));
typedef uint32_t u32x6  __attribute__((ext_vector_type(6)));
typedef uint32_t u32x8  __attribute__((ext_vector_type(8)));

// ---- bf16 / fp16 bit helpers ------------------------------------------------
__device__ __forceinline__ float bf16lo(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float bf16hi(uint32_t d) { return __uint_as_float(d & 0xFFFF0000u); }
__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// Two floats -> two bf16 (round to nearest even: v_cvt_pk_bf16_f32), low half = lo.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  bf16x2 b = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, b);
}
// Round one float to the nearest bf16 value, returned as float.
__device__ __forceinline__ float round_bf16(float f) {
  return bf16lo(pack_bf16x2(f, 0.0f));
}
__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// ---- division ---------------------------------------------------------------
// Correctly rounded float32 quotient x / s given rs = RN(1/s) (one multiply and two
// FMAs): Markstein's correction step (P. Markstein, "Computation of elementary functions on
// the IBM RISC System/6000 processor", IBM J. Res. Dev. 34(1), 1990) -- the residual
// r = x - q0 s is exact in an FMA and q0 + r rs rounds to the correctly rounded quotient.  Exhaustively verified for every pair of bf16-representable operands whose
// quotient is a normal float32 (tests/test_division_exact.py); callers guarantee that
// range and use the IEEE division otherwise.
__device__ __forceinline__ float div_rcp(float x, float s, float rs) {
  float q0 = x * rs;
  float r = __builtin_fmaf(-q0, s, x);
  return __builtin_fmaf(r, rs, q0);
}

// ---- MFMA wrappers ----------------------------------------------------------
__device__ __forceinline__ i32x16 mfma_i8_32x32x32(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_bf16_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// K = 8 form of the bf16 MFMA (same 8 passes as K = 16 on gfx950, half the operand registers):
// lane l holds row / column l % 32, k = 4 (l / 32) .. + 3, as two bf16 pairs.
__device__ __forceinline__ f32x16 mfma_bf16_32x32x8(u32x2 a, u32x2 b, f32x16 c) {
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c, 0,
                                                  0, 0);
}

__device__ __forceinline__ f32x16 mfma_fp8_32x32x64(const u32x4 (&a)[2], const u32x4 (&b)[2], f32x16 c) {
  typedef int i32x8 __attribute__((ext_vector_type(8)));
  const i32x8 av = {(int)a[0][0], (int)a[0][1], (int)a[0][2], (int)a[0][3],
                    (int)a[1][0], (int)a[1][1], (int)a[1][2], (int)a[1][3]};
  const i32x8 bv = {(int)b[0][0], (int)b[0][1], (int)b[0][2], (int)b[0][3],
                    (int)b[1][0], (int)b[1][1], (int)b[1][2], (int)b[1][3]};
  // format 0/0 = e4m3 x e4m3; E8M0 scale 127 = 2^0 on both sides
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 0, 0, 0, 127, 0, 127);
}

// e3m2 x e3m2 (FP6, format 3 on both sides): a lane's 32 codes are 6 dwords, given as the
// 16-byte and 8-byte parts the GEMM reads from its two LDS planes; the instruction reads 6
// registers, the two upper lanes of the 8-lane operand are left undefined.
__device__ __forceinline__ f32x16 mfma_fp6_32x32x64(u32x4 aq, u32x2 ar, u32x4 bq, u32x2 br, f32x16 c) {
  typedef int i32x8 __attribute__((ext_vector_type(8)));
  const u32x4 ar4 = __builtin_shufflevector(ar, ar, 0, 1, -1, -1);
  const u32x4 br4 = __builtin_shufflevector(br, br, 0, 1, -1, -1);
  const i32x8 av = __builtin_bit_cast(i32x8, __builtin_shufflevector(aq, ar4, 0, 1, 2, 3, 4, 5, -1, -1));
  const i32x8 bv = __builtin_bit_cast(i32x8, __builtin_shufflevector(bq, br4, 0, 1, 2, 3, 4, 5, -1, -1));
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 3, 3, 0, 127, 0, 127);
}

// e3m2 operand of 32 codes given as floats (k = 2i in x[i], k = 2i + 1 in y[i]):
// v_cvt_scalef32_2xpk16_bf6 writes field 2i from x[i] and field 2i + 1 from y[i] (contiguous
// 6-bit fields over 6 dwords), so field f holds k = f, the operand layout of the FP6 MFMA.
// Exact: every INT4 code is an e3m2 value (8 = 1.0 x 2^3, 7 = 1.11b x 2^2, ...).
__device__ __forceinline__ u32x6 codes_to_e3m2(f32x16 x, f32x16 y) {
  return __builtin_bit_cast(u32x6, __builtin_amdgcn_cvt_scalef32_2xpk16_bf6_f32(x, y, 1.0f));
}

// ---- INT4 code conversion (8-bit MFMA operands) ---------------------------------
// Both operands of the W4A4 GEMM are 8-bit per element in LDS.  A packed dword holds 8
// offset-binary nibbles u = q + 8 for k0..k7 (k0 in the low nibble); it becomes two
// dwords [k0,k2,k4,k6] and [k1,k3,k5,k7].  The activation pass writes its operand bytes in
// the same order, so the k permutation cancels in the dot product.
//
// e4m3 (OCP, bias 7) holds every q in [-8, 7] exactly.  v_perm_b32 is a byte table
// lookup over 8 bytes; two tables (u < 8: q = u - 8 < 0, u >= 8: q = u - 8 >= 0) and a
// per-byte select on bit 3 of u cover all 16 codes.
__device__ __forceinline__ uint32_t nib4_to_e4m3(uint32_t u) {
  const uint32_t j = u & 0x07070707u;
  const uint32_t pos = __builtin_amdgcn_perm(0x4e4c4a48u, 0x44403800u, j);  // q = 0..7
  const uint32_t neg = __builtin_amdgcn_perm(0xb8c0c4c8u, 0xcaccced0u, j);  // q = -8..-1
  const uint32_t mask = __builtin_amdgcn_perm(0u, 0u, ((u >> 3) & 0x01010101u) | 0x0c0c0c0cu);
  return (pos & mask) | (neg & ~mask);
}
__device__ __forceinline__ void nib8_to_e4m3(uint32_t x, uint32_t& lo, uint32_t& hi) {
  lo = nib4_to_e4m3(x);
  hi = nib4_to_e4m3(x >> 4);
}
// Same bytes as int8 16*q (two's complement nibble moved to the high half of the byte).
__device__ __forceinline__ void nib8_to_i8x16(uint32_t x, uint32_t& lo, uint32_t& hi) {
  const uint32_t t = x ^ 0x88888888u;
  lo = (t << 4) & 0xF0F0F0F0u;
  hi = t & 0xF0F0F0F0u;
}

// gfx950 v_permlane32_swap: exchange lanes 32..63 of `a` with lanes 0..31 of `b`.
__device__ __forceinline__ void permlane32_swap(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}

// Split 8 floats into bf16 hi + bf16 lo parts (x ~= hi + lo to ~2^-17 relative).
__device__ __forceinline__ void split_hi_lo(const float* v, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t h = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    hi[i] = h;
    lo[i] = pack_bf16x2(v[2 * i] - bf16lo(h), v[2 * i + 1] - bf16hi(h));
  }
}

// VGPR banks of the rescale FMA acc += P * S.  The FMA reads three VGPRs; the register file
// has four banks (register index mod 4) and three operands in one bank issue at about half
// rate (measured: 1.85x the time of three distinct banks).  The allocator starts the MFMA result
// tuples P and S and the accumulator tuple in the same bank, so register r of each lands in
// one bank.  Two rotations put the operands of every FMA in three consecutive banks:
//  * S one register ahead: the scale MFMA's A operand (rows of sx) is read with the rows
//    permuted so that S register r + 1 holds the row of P register r (D layout: register r of
//    lane half h holds row 8 (r / 4) + 4 h + r % 4);
//  * the accumulator two registers ahead: logical register r lives in acc[(r + 2) % 16], undone
//    once before the epilogue.
__device__ __forceinline__ int scale_row_perm(int row) {   // row in 0..31
  const int reg = 4 * (row >> 3) + (row & 3);              // D register of this row
  const int prev = (reg + 15) & 15;                        // one register earlier
  return 8 * (prev >> 2) + (row & 4) + (prev & 3);
}
__device__ __forceinline__ void rescale_acc(f32x16& acc, const f32x16& P, const f32x16& S) {
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[(r + 2) & 15] = __builtin_fmaf(P[r], S[(r + 1) & 15], acc[(r + 2) & 15]);
}
__device__ __forceinline__ void unrotate_acc(f32x16 (&acc)[2][2]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x16 t;
#pragma unroll
      for (int r = 0; r < 16; ++r) t[r] = acc[i][j][(r + 2) & 15];
      acc[i][j] = t;
    }
}

// XCD-aware block order: hardware hands consecutive workgroup ids to the 8 XCDs round-robin;
// remap so that each XCD receives a contiguous range of output tiles (shared A rows / B columns
// stay within one L2), then walk tiles in column-major groups of `group_m` block-rows.
__device__ __forceinline__ void tile_of_linear(int lin, int nbm, int nbn, int group_m, int& bm, int& bn) {
  const int per_group = group_m * nbn;
  const int gid = lin / per_group;
  const int first_m = gid * group_m;
  const int gm = min(nbm - first_m, group_m);
  const int in = lin % per_group;
  bm = first_m + in % gm;
  bn = in / gm;
}
__device__ __forceinline__ void tile_coords(int bid, int nbm, int nbn, int group_m, int& bm, int& bn) {
  const int nblk = nbm * nbn;
  int lin = bid;
  if (nblk % 8 == 0) lin = (bid % 8) * (nblk / 8) + bid / 8;
  tile_of_linear(lin, nbm, nbn, group_m, bm, bn);
}

}  // namespace svdq
