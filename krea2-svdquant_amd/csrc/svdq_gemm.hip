// W4A4 and W4A16 SVDQuant GEMMs for gfx950 with the low-rank / LoRA / bias epilogue.
//
// W4A4 (replaces the residual GEMM of quant/svd.py:158 with activation codes, and the
// low-rank add of kernels/triton/generic_int4.py:84-133):
//   y[m,n] = sum_g sx[m,g] sw[n,g] sum_{k in g} qx[m,k] qw[n,k]      (exact integer group sums
//            on the FP8 (e4m3) or INT8 MFMA, rescaled into an fp32 accumulator)
//          + mid[m,:] . l1cat[n,:]  + bias[n]                       (bf16 MFMA, mid split
//                                                                    into bf16 hi + lo)
// W4A16 (the pytorch_sim math, quant/svd.py:119-163):
//   y = x_hat @ W^T with W = bf16(q * bf16(sw)) dequantized in registers while staging the
//   tile into LDS (pack.py:26-44 with dtype=bf16), same epilogue.
//
// Both kernels permute k inside each chunk of 8 columns (even k first) when they unpack
// INT4 nibbles; the activation operand is written in the same order, so the permutation
// cancels in every dot product.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "svdq_common.h"
#include "svdq_kernels.h"

namespace svdq {
namespace {


__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
// byte E of v as a float (one v_cvt_f32_ubyteE)
template <int E>
__device__ __forceinline__ float ubyte_f32(uint32_t v) { return (float)((v >> (8 * E)) & 0xFFu); }



// a / d for d >= 1 where it rounds to the same bf16 as the IEEE float quotient RN(a / d); *exact
// is cleared where that is not shown and the caller must divide.  The product f = a * v_rcp_f32(d)
// lies within 2 ulps of a / d (1 ulp for the reciprocal, 1/2 for the product) and so within 3 of
// RN(a / d); bf16 rounding is monotone and changes only where the low 16 bits cross 0x8000, so
// when f's low 16 bits are more than 8 away from 0x8000 both round to the same bf16.  Not shown:
// d >= 2^100, |a| >= 2^100, inf / NaN, and results below 2^-100 (the reciprocal may leave the
// normal range).
__device__ __forceinline__ float div_bf16_fast(float a, float d, bool& exact) {
  const float f = a * __builtin_amdgcn_rcpf(d);
  const uint32_t lo = __float_as_uint(f) & 0xFFFFu;
  // bitwise & / |: the conditions evaluate branch-free
  exact = (int)(d < 0x1p100f) & (int)(fabsf(a) < 0x1p100f) & ((int)(fabsf(f) >= 0x1p-100f) | (int)(a == 0.0f)) &
          (int)(lo - 0x7FF8u > 16u);
  return f;
}

// GemmParams::epi on one element: y = the bf16-rounded layer output, a = the aux element, g = the
// column's evec element.  Each op rounds its result to bf16 as the unfused torch ops on bf16
// tensors do (float math inside one op, bf16 out): sigmoid and silu as 1 / (1 + exp(-v)) and
// v / (1 + exp(-v)) in float, the gated residual in one step as torch.addcmul.  The caller rounds
// the returned value.
// epi 1 and 2 are evaluated for a chunk of 8 elements at a time by epi_apply_op.
__device__ __forceinline__ float epi_op(int epi, float y, float a, float g) {
  if (epi == 1) return a * round_bf16(1.0f / (1.0f + expf(-y)));   // a * sigmoid(y)
  if (epi == 2) return round_bf16(a / (1.0f + expf(-a))) * y;      // silu(a) * y
  return __builtin_fmaf(g, y, a);                                   // addcmul(a, g, y)
}

// epi on a chunk of 8 bf16 outputs v with their aux elements a and evec elements g.  The op is
// chosen once per chunk, so each op's code appears once per call site.
// For the sigmoid and silu quotients the 8 reciprocal products come first, branch-free; only
// when one of the lane's 8 is not shown exact does the lane divide (all 8, keeping the
// reciprocal products that were exact).
template <int E>
__device__ __forceinline__ u32x4 epi_apply_op(u32x4 v, u32x4 a, u32x4 g) {
  float y[8], x[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    y[2 * d] = bf16lo(v[d]);
    y[2 * d + 1] = bf16hi(v[d]);
    x[2 * d] = bf16lo(a[d]);
    x[2 * d + 1] = bf16hi(a[d]);
  }
  float o[8];
  if constexpr (E == 3) {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = epi_op(3, y[e], x[e], e % 2 ? bf16hi(g[e / 2]) : bf16lo(g[e / 2]));
  } else {
    // sigmoid(y) = 1 / (1 + exp(-y)); silu(x) = x / (1 + exp(-x))
    float num[8], den[8], q[8];
    bool all = true;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      num[e] = E == 1 ? 1.0f : x[e];
      den[e] = 1.0f + expf(-(E == 1 ? y[e] : x[e]));
      bool ok;
      q[e] = div_bf16_fast(num[e], den[e], ok);
      all = all & ok;
    }
    if (!all) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        bool ok;
        div_bf16_fast(num[e], den[e], ok);
        if (!ok) q[e] = num[e] / den[e];
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = E == 1 ? x[e] * round_bf16(q[e]) : round_bf16(q[e]) * y[e];
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) v[d] = pack_bf16x2(o[2 * d], o[2 * d + 1]);
  return v;
}
__device__ __forceinline__ u32x4 epi_apply(const GemmParams& p, u32x4 v, u32x4 a, u32x4 g) {
  if (p.epi == 1) return epi_apply_op<1>(v, a, g);
  if (p.epi == 2) return epi_apply_op<2>(v, a, g);
  return epi_apply_op<3>(v, a, g);
}

// Whether the chunk of 8 outputs at columns n..n+7 takes its aux / evec by 16-byte loads.
__device__ __forceinline__ bool epi_vec(const GemmParams& p, int n) { return p.aux_vec && n + 8 <= p.N; }

// aux and evec elements of the chunk at (m, n..n+7) loaded element by element (the chunks
// epi_vec rejects; columns >= N read as 0 and are not stored).
__device__ __forceinline__ void epi_load_elems(const GemmParams& p, int m, int n, u32x4& a, u32x4& g) {
  const uint16_t* ar = p.aux + (long)m * p.ldaux + n;
  a = u32x4{};
  g = u32x4{};
  for (int e = 0; e < min(8, p.N - n); ++e) {
    a[e / 2] |= (uint32_t)ar[e] << (16 * (e % 2));
    if (p.epi == 3) g[e / 2] |= (uint32_t)p.evec[n + e] << (16 * (e % 2));
  }
}

// acc (2x2 sub-tiles of the wave) += mid @ l1cat^T, + bias, then store through the wave's 4 KB
// LDS region `stage` (coalesced 16-byte row chunks).  mid is the activation
// pass's finalized operand, bf16 hi and lo planes per row ([M, 2, RTp]); both planes go through
// the bf16 MFMA, so the low-rank term carries the f32 mid to 2^-18.  Two 16-column steps per
// iteration, their twelve loads issued together (one memory latency per 32 columns of RTp).
template <bool OUT_F32, bool EPI = false>
__device__ __forceinline__ void epilogue(const GemmParams& p, f32x16 (&acc)[2][2], int m0, int n0,
                                         int lr, int h, uint8_t* stage, const uint8_t* lmid = nullptr,
                                         const uint8_t* ll1 = nullptr, int wr = 0, int wc = 0,
                                         int mlim = 0x7FFFFFFF) {
  const int RTp = p.RTp;
  const int mend = min(p.M, mlim);   // rows m >= mend are not stored (past M, or another wave's)
  // Staged bf16 stores with an elementwise op: the aux chunks of the lane's 8 output chunks (and
  // its evec chunk) are loaded here, ahead of the low-rank MFMAs, so that one memory latency
  // covers them all.  Left to the store loop, each load would wait behind the previous chunk's
  // store (the compiler must assume aux and y may overlap) and the tile would pay 8 latencies.
  // Lane (h, lr) stores chunk c = lr % 8 of rows 8 it + 4 h + lr / 8 in each 32-row pass.
  constexpr bool PRE = EPI && !OUT_F32;
  u32x4 apre[PRE ? 8 : 1], gpre = u32x4{};
  if constexpr (PRE) {
    const int n = n0 + 8 * (lr & 7);
    if (epi_vec(p, n)) {
      if (p.epi == 3) gpre = ld16(p.evec + n);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int m = m0 + 32 * (u >> 2) + 8 * (u & 3) + 4 * h + (lr >> 3);
        apre[u] = m < mend ? ld16(p.aux + (long)m * p.ldaux + n) : u32x4{};
      }
    }
  }
  if (lmid != nullptr) {
    // RTp == 32, operands prefetched into LDS by the GEMM's last stage: the tile's mid rows
    // (128 bytes: hi plane, lo plane; 16-byte chunk c of row r at c ^ ((r >> 1) & 7)) and l1cat
    // rows (64 bytes; chunk c of row r at c ^ ((r >> 2) & 3)); wr / wc = the wave's first
    // row / column in the tile.  Conflict-free: 16 consecutive rows hit 16 distinct bank groups.
    u32x4 ahi[2][2], alo[2][2], b[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wr + 32 * i + lr, sw = (r >> 1) & 7;
        ahi[u][i] = ld16(lmid + r * 128 + 16 * ((2 * u + h) ^ sw));
        alo[u][i] = ld16(lmid + r * 128 + 16 * ((4 + 2 * u + h) ^ sw));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = wc + 32 * j + lr;
        b[u][j] = ld16(ll1 + c * 64 + 16 * ((2 * u + h) ^ ((c >> 2) & 3)));
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = mfma_bf16_32x32x16(ahi[u][i], b[u][j], acc[i][j]);
          acc[i][j] = mfma_bf16_32x32x16(alo[u][i], b[u][j], acc[i][j]);
        }
  }
  const uint16_t* arow[2];
  const uint16_t* brow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) arow[i] = p.midp + (long)min(m0 + 32 * i + lr, p.M - 1) * (2 * RTp) + 8 * h;
#pragma unroll
  for (int j = 0; j < 2; ++j) brow[j] = p.l1cat + (long)min(n0 + 32 * j + lr, p.N - 1) * RTp + 8 * h;
  for (int s = 0; s < (lmid != nullptr ? 0 : RTp / 16); s += 2) {
    u32x4 ahi[2][2], alo[2][2], b[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ahi[u][i] = ld16(arow[i] + 16 * (s + u));
        alo[u][i] = ld16(arow[i] + RTp + 16 * (s + u));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) b[u][j] = ld16(brow[j] + 16 * (s + u));
    }
    // all twelve loads in flight before the first MFMA waits on one of them
    asm volatile("" : "+v"(ahi[0][0]), "+v"(ahi[0][1]), "+v"(ahi[1][0]), "+v"(ahi[1][1]), "+v"(alo[0][0]),
                 "+v"(alo[0][1]), "+v"(alo[1][0]), "+v"(alo[1][1]), "+v"(b[0][0]), "+v"(b[0][1]), "+v"(b[1][0]),
                 "+v"(b[1][1]));
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = mfma_bf16_32x32x16(ahi[u][i], b[u][j], acc[i][j]);
          acc[i][j] = mfma_bf16_32x32x16(alo[u][i], b[u][j], acc[i][j]);
        }
  }
  float bv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + 32 * j + lr;
    bv[j] = p.bias && n < p.N ? bf16f(p.bias[n]) : 0.0f;
  }
  // Staged: in passes of 4 KB (32 rows of bf16, 16 rows of f32 out of the wave's 64), the values
  // go to the wave's LDS region (rows of 64 values; 16-byte chunk c of row r at c ^ (CPR / 2) when
  // (r >> 2) is odd, so the two half-waves, 4 rows apart, write disjoint banks) and come back as
  // 16-byte row chunks for coalesced stores.
  constexpr int ES = OUT_F32 ? 4 : 2;         // bytes per value
  constexpr int CPR = 64 * ES / 16;           // 16-byte chunks per row
  constexpr int VPC = 16 / ES;                // values per chunk
  constexpr int RP = 4096 / (64 * ES);        // rows per pass: 32 or 16
  constexpr int RPB = 16 * RP / 32;           // accumulator registers per 32-row sub-tile and pass
  const bool vec = (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 && p.ldy % VPC == 0;
#pragma unroll
  for (int q = 0; q < 64 / RP; ++q) {
    const int i = q * RP / 32, rq = (q * RP) % 32;   // sub-tile, first row of the pass in it
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = RPB * (rq / RP); r < RPB * (rq / RP + 1); ++r) {
        const int row = 8 * (r >> 2) + 4 * h + (r & 3) - rq, col = 32 * j + lr;
        const int pos = (col / VPC) ^ ((row >> 2) & 1 ? CPR / 2 : 0);
        uint8_t* dst = stage + row * (64 * ES) + pos * 16 + (col % VPC) * ES;
        const float v = acc[i][j][r] + bv[j];
        if (OUT_F32) *reinterpret_cast<float*>(dst) = v;
        else *reinterpret_cast<uint16_t*>(dst) = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu);
      }
    auto put = [&](u32x4 v, int m, int n) {
      uint8_t* out = reinterpret_cast<uint8_t*>(p.y) + ((long)m * p.ldy + n) * ES;
      if (vec && n + VPC <= p.N) {
        st16(out, v);
      } else {
#pragma unroll
        for (int e = 0; e < VPC; ++e) {
          if (n + e >= p.N) break;
          if (OUT_F32) reinterpret_cast<uint32_t*>(out)[e] = v[e];
          else reinterpret_cast<uint16_t*>(out)[e] = (uint16_t)(v[e / 2] >> (16 * (e % 2)));
        }
      }
    };
    if constexpr (PRE) {
      // A loop kept rolled over the pass's 4 chunks, so that the op's code appears once per pass
      // (unrolled, the epilogue's code outgrew the instruction cache); the prefetched aux
      // chunks move down one register per chunk.
      static_assert(CPR == 8 && VPC == 8 && RP == 32, "bf16 passes");
      u32x4 a0 = apre[4 * q], a1 = apre[4 * q + 1], a2 = apre[4 * q + 2], a3 = apre[4 * q + 3];
#pragma unroll 1
      for (int it = 0; it < 4; ++it) {
        const int row = 8 * it + 4 * h + (lr >> 3), c = lr & 7;
        const int pos = c ^ ((row >> 2) & 1 ? CPR / 2 : 0);
        const u32x4 v = *reinterpret_cast<const u32x4*>(stage + row * (64 * ES) + pos * 16);
        const int m = m0 + 32 * i + rq + row, n = n0 + c * VPC;
        if (m < mend) {
          u32x4 a = a0, g = gpre;
          if (!epi_vec(p, n)) epi_load_elems(p, m, n, a, g);
          put(epi_apply(p, v, a, g), m, n);
        }
        a0 = a1;
        a1 = a2;
        a2 = a3;
      }
    } else {
#pragma unroll
      for (int it = 0; it < RP * CPR / 64; ++it) {
        const int idx = 64 * it + (h << 5 | lr), row = idx / CPR, c = idx % CPR;
        const int pos = c ^ ((row >> 2) & 1 ? CPR / 2 : 0);
        const u32x4 v = *reinterpret_cast<const u32x4*>(stage + row * (64 * ES) + pos * 16);
        const int m = m0 + 32 * i + rq + row, n = n0 + c * VPC;
        if (m < mend) put(v, m, n);
      }
    }
  }
}

// --------------------------------------------------------------------------- W4A4
// Global -> LDS DMA (global_load_lds_dword / _dwordx4): lane L of the wave writes its 4 (16)
// bytes from base + off at LDS address lds + 4 L (16 L); `lds` (wave-uniform) goes in M0, as
// an operand, so the compiler owns that register.  Issued as inline asm so that the compiler
// neither orders later LDS reads after it (it cannot tell the pipeline stages apart) nor
// counts it in its own waits: the kernel waits explicitly.
// Two hazards the compiler cannot see, because it does not look inside inline asm:
//  * gfx9 requires 1 wait state between an SALU instruction that writes M0 and an LDS DMA that
//    reads it.  The compiler writes M0 (`s_mov_b32 m0, sN`) right before the asm block, so every
//    DMA starts with `s_nop 0`.
//  * gfx9 requires 5 wait states between a VALU instruction that writes an SGPR and a VMEM
//    instruction that reads it.  Under SGPR pressure the compiler restores a spilled base pointer
//    with v_readlane right before a DMA, which then reads a stale address (builds where that
//    happened faulted the GPU).  NOP = true starts the DMA with `s_nop 4` instead (5 wait states,
//    about 2% of the e3m2 GEMM's time); the kernels whose build restores SGPRs before a DMA (the
//    fused-epilogue variants) set it.
// tests/test_dma_hazards.py walks every DMA of the built library back over all its predecessor
// paths and fails if one can read a VALU-written SGPR within 5 wait states or an SALU-written M0
// within 1.
template <bool NOP = false>
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  if (NOP) asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
  else asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
template <bool NOP = false>
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  if (NOP) asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
  else asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}

// W4A4 GEMM (exact INT4-code products on the FP8 or INT8 MFMA).
//
// Block tile 256 x 128, 8 waves in a 4 x 2 grid, wave tile 64 x 64 = 2 x 2 sub-tiles of
// 32 x 32.  K advances 128 columns per pipeline stage (two groups of 64 or one of 128).  A
// stage is moved global -> LDS entirely by DMA (activation codes, expanded weight codes, both
// scale operands) into a ring of three LDS buffers; the DMA of stage s + 2 is issued during
// stage s, in four parts spread over its four half-group steps (issuing a stage's 64 DMA
// instructions per CU in one burst stalls the address unit and every wave behind it).  Each
// wave issues the same number of DMA instructions per stage, so `s_waitcnt vmcnt` with the
// count of the stage still in flight retires the one needed next.  Global bases are scalars
// advanced per stage; per-lane offsets are constants.
//
// LDS operand tiles: rows of 128 bytes = 8 chunks of 16; chunk c of row r sits at chunk
// position c ^ ((r >> 1) & 7).  The 16 lanes of a ds_read_b128 phase read one logical chunk
// of 16 consecutive rows and hit 16 distinct 4-bank groups.
//
// Per group and sub-tile: P = codes_x . codes_w (exact integer sums) on the FP8 MFMA (or the
// INT8 MFMA, int32 converted to fp32), S = sx (x) sw on a bf16 MFMA with K = 2: A = (sx, sx)
// then zeros, B = (hi(sw), lo(sw)) then zeros (zero for lanes 32-63), so S = sx hi + sx lo
// exactly; acc += P * S (one VALU FMA per output and group).
//   MODE 0: operands e4m3, v_mfma_f32_32x32x64_f8f6f4 (P already float32);
//   MODE 1: operands int8 16*q, 2x v_mfma_i32_32x32x32_i8 (P int32, converted; 1/256 in S).
//
// Schedule: every wave runs the same free sequence of half-group steps (one row sub-tile i
// against both column sub-tiles): products and scales on the MFMA, then the rescale FMAs.  The
// two waves of a SIMD drift apart and one's FMAs run under the other's MFMAs; a workgroup
// barrier once per stage (re-aligning all waves costs a few percent, measured) is the only
// synchronisation.  With G == 64 the next half-group's fragments are read from LDS at the top
// of each step into the second register set, a full step ahead of their use; the barrier sits
// before the last step of a stage, after which the first fragments of the next stage are read.
// With G == 128 (twice the fragment registers, one set) the next fragments are read after the
// step's MFMAs, and the barrier follows the last step's MFMAs.
template <int G, int MODE, bool OUT_F32, bool EPI = false>
__global__ void __launch_bounds__(512, 1) w4a4_kernel(GemmParams p) {
  constexpr int TBM = 256, TBN = 128, NT = 512, NBUF = 3;
  constexpr int KB = 128;                     // K columns per pipeline stage
  constexpr int GPS = KB / G;                 // groups per stage
  constexpr int HPS = 2 * GPS;                // half-group steps per stage
  constexpr int KS = G / 64;                  // 64-column MFMA steps per group
  constexpr int ADMA = TBM * KB / (16 * NT);  // A: 16-byte DMA chunks per thread per stage (4)
  constexpr int BDMA = TBN * KB / (16 * NT);  // B: 16-byte DMA chunks per thread per stage (2)
  constexpr int DMA = ADMA + BDMA + 2;        // DMA instructions per thread per stage
  static_assert(ADMA == 4 && BDMA == 2, "the DMA parts below assume 4 A and 2 B chunks per thread");
  constexpr int XS = TBM + 4, WS = TBN + 4;   // scale words per group; the last 4 are zero
  constexpr int ABUF = TBM * KB, BBUF = TBN * KB;
  __shared__ __attribute__((aligned(1024))) uint8_t sA[NBUF * ABUF];
  __shared__ __attribute__((aligned(1024))) uint8_t sB[NBUF * BBUF];
  __shared__ __attribute__((aligned(16))) uint32_t sX[NBUF][GPS][XS];   // (sx, sx) bf16 pairs
  __shared__ __attribute__((aligned(16))) uint32_t sW[NBUF][GPS][WS];   // (hi, lo) of sw

  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int nbm = (p.M + TBM - 1) / TBM, nbn = (p.N + TBN - 1) / TBN;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 4, bm, bn);
  const int m0 = bm * TBM, n0 = bn * TBN;
  const int K = p.K, ngroups = K / G, nstages = (K + KB - 1) / KB, H = 2 * ngroups;

  // Operand DMA: wave w, chunk i -> 8 rows of a stage tile (lane / 8 = row, lane % 8 = chunk).
  uint32_t arow_o[ADMA], brow_o[BDMA];
  int ac16[ADMA], bc16[BDMA];
#pragma unroll
  for (int i = 0; i < ADMA; ++i) {
    const int row = 8 * (ADMA * wave + i) + lane / 8;
    ac16[i] = 16 * ((lane % 8) ^ ((row >> 1) & 7));
    arow_o[i] = (uint32_t)min(m0 + row, p.M - 1) * (uint32_t)K;
  }
#pragma unroll
  for (int i = 0; i < BDMA; ++i) {
    const int row = 8 * (BDMA * wave + i) + lane / 8;
    bc16[i] = 16 * ((lane % 8) ^ ((row >> 1) & 7));
    brow_o[i] = (uint32_t)min(n0 + row, p.N - 1) * (uint32_t)K;
  }
  // Scale DMA: one dword per lane; wave w covers words 64 w .. 64 w + 63 of the stage's
  // GPS x TBM (GPS x TBN) scale tile, wrapping (the duplicate words hold the same values).
  const int xs = (64 * wave + lane) % (GPS * TBM), ws = (64 * wave + lane) % (GPS * TBN);
  const int xj = xs / TBM, wj = ws / TBN;
  const uint32_t xrowc = (uint32_t)min(m0 + xs % TBM, p.M - 1), wrowc = (uint32_t)min(n0 + ws % TBN, p.N - 1);
  const int xjs = ((64 * wave) % (GPS * TBM)) / TBM, wjs = ((64 * wave) % (GPS * TBN)) / TBN;
  const int xbase = (64 * wave) % (GPS * TBM) % TBM, wbase = (64 * wave) % (GPS * TBN) % TBN;
  if (tid < NBUF * GPS * 4) {
    sX[tid / (4 * GPS)][(tid / 4) % GPS][TBM + tid % 4] = 0u;
    sW[tid / (4 * GPS)][(tid / 4) % GPS][TBN + tid % 4] = 0u;
  }
  const uint32_t ldsA = lds_offset(sA), ldsB = lds_offset(sB), ldsX = lds_offset(&sX[0][0][0]),
                 ldsW = lds_offset(&sW[0][0][0]);

  // Part q of stage s's DMA into ring buffer `buf`: q0 = both scale tiles + A chunk 0 (3
  // instructions), q1 = A chunks 1-2, q2 = A chunk 3 + B chunk 0, q3 = B chunk 1.  Columns past
  // K (a last stage of one group of 64) re-read the stage's last 16 bytes; never consumed.
  auto gload_part = [&](int s, int buf, int q) {
    const int col0 = s * KB;
    const int lim = col0 + KB > K ? K - col0 - 16 : KB;
    const uint8_t* qa_s = p.qa + col0;
    const uint8_t* qw_s = p.qwe + col0;
    if (q == 0) {
      const int g0 = s * GPS;
      const int jmax = ngroups - 1 - g0;
      const uint32_t* sx_s = p.sxp + (long)g0 * p.M;
      const uint32_t* sw_s = p.swp + (long)g0 * p.N;
      dma4<EPI>(sx_s, 4 * ((uint32_t)min(xj, jmax) * (uint32_t)p.M + xrowc), ldsX + 4 * ((buf * GPS + xjs) * XS + xbase));
      dma4<EPI>(sw_s, 4 * ((uint32_t)min(wj, jmax) * (uint32_t)p.N + wrowc), ldsW + 4 * ((buf * GPS + wjs) * WS + wbase));
    }
#pragma unroll
    for (int i = 0; i < ADMA; ++i)
      if ((i + 1) / 2 == q) dma16<EPI>(qa_s, arow_o[i] + min(ac16[i], lim), ldsA + buf * ABUF + (ADMA * wave + i) * 1024);
#pragma unroll
    for (int i = 0; i < BDMA; ++i)
      if (q == 2 + i) dma16<EPI>(qw_s, brow_o[i] + min(bc16[i], lim), ldsB + buf * BBUF + (BDMA * wave + i) * 1024);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int sw_ = (lr >> 1) & 7;
  int fa[4], fb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int u = 4 * (q >> 1) + (q & 1);
    fa[q] = (64 * wm + lr) * 128 + 16 * ((u + 2 * h) ^ sw_);
    fb[q] = (64 * wn + lr) * 128 + 16 * ((u + 2 * h) ^ sw_);
  }
  // Scale-MFMA operands: persistent tuples, word 0 reloaded from LDS, words 1-3 stay zero.
  // A = (sx, sx) of the lane's row; B = (hi, lo) of the lane's column for lanes 0-31 and zero
  // for lanes 32-63 (they read the zero word).
  const int xo0 = 4 * (64 * wm + scale_row_perm(lr)), xo1 = xo0 + 128;   // rows permuted: see rescale_acc
  const int wo0 = 4 * (h ? TBN : 64 * wn + lr), wo1 = 4 * (h ? TBN : 64 * wn + 32 + lr);
  u32x4 xop[2] = {u32x4{}, u32x4{}};

  // Fragments.  G == 64 (RM): the next half-group's fragments are read a step ahead into the
  // other set: A by half-group parity, B and the weight scales by group parity.  G == 128: one
  // set (the registers do not fit twice).
  constexpr bool RM = G == 64;
  constexpr int NS = RM ? 2 : 1;
  u32x4 fa_[NS][KS][2], fb_[NS][2][KS][2], wop_[NS][2];
#pragma unroll
  for (int q = 0; q < NS; ++q) wop_[q][0] = wop_[q][1] = u32x4{};
  // half-group (s, gi, i) -> fragment sets: A set ai, B / weight-scale set bi
  auto read_half = [&](int s, int gi, int i, int ai, int bi) {
    const int buf = s % NBUF;
    const uint8_t* a0 = sA + buf * ABUF;
    const uint8_t* b0 = sB + buf * BBUF;
    const uint8_t* x0 = reinterpret_cast<const uint8_t*>(&sX[buf][gi][0]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int q = 2 * (G / 64 * gi + ks) + t;
        fa_[ai][ks][t] = ld16(a0 + fa[q] + 4096 * i);
        if (i == 0) {
#pragma unroll
          for (int j = 0; j < 2; ++j) fb_[bi][j][ks][t] = ld16(b0 + fb[q] + 4096 * j);
        }
      }
    xop[i][0] = *reinterpret_cast<const uint32_t*>(x0 + (i ? xo1 : xo0));
    if (i == 0) {
      const uint8_t* w0 = reinterpret_cast<const uint8_t*>(&sW[buf][gi][0]);
      wop_[bi][0][0] = *reinterpret_cast<const uint32_t*>(w0 + wo0);
      wop_[bi][1][0] = *reinterpret_cast<const uint32_t*>(w0 + wo1);
    }
  };
  // Product of sub-tile (i, j): FP8 -> fp32 sums directly; INT8 -> int32 sums (converted later).
  auto mfma_p8 = [&](int ai, int bi, int j) {
    f32x16 pf = mfma_fp8_32x32x64(fa_[ai][0], fb_[bi][j][0], f32x16{});
#pragma unroll
    for (int ks = 1; ks < KS; ++ks) pf = mfma_fp8_32x32x64(fa_[ai][ks], fb_[bi][j][ks], pf);
    return pf;
  };
  auto mfma_pi = [&](int ai, int bi, int j) {
    i32x16 pi = i32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        pi = mfma_i8_32x32x32(__builtin_bit_cast(i32x4, fa_[ai][ks][t]), __builtin_bit_cast(i32x4, fb_[bi][j][ks][t]), pi);
    return pi;
  };
  // Fence on every fragment register (both sets): reads issued before it have landed at it.
#define SVDQ_FRAGS_1 "+v"(fa_[0][0][0]), "+v"(fa_[0][0][1]), "+v"(fb_[0][0][0][0]), "+v"(fb_[0][0][0][1]), \
    "+v"(fb_[0][1][0][0]), "+v"(fb_[0][1][0][1]), "+v"(xop[0]), "+v"(xop[1]), "+v"(wop_[0][0]), "+v"(wop_[0][1])
#define SVDQ_FRAGS_2 "+v"(fa_[NS - 1][0][0]), "+v"(fa_[NS - 1][0][1]), "+v"(fb_[NS - 1][0][0][0]), \
    "+v"(fb_[NS - 1][0][0][1]), "+v"(fb_[NS - 1][1][0][0]), "+v"(fb_[NS - 1][1][0][1]), "+v"(wop_[NS - 1][0]), \
    "+v"(wop_[NS - 1][1])
  auto frag_fence = [&]() {
    if (RM) asm volatile("" : SVDQ_FRAGS_1, SVDQ_FRAGS_2::"memory");
    else asm volatile("" : SVDQ_FRAGS_1::"memory");
  };
#undef SVDQ_FRAGS_1
#undef SVDQ_FRAGS_2

  // Stages 0 and 1 in flight, stage 0 landed everywhere; stage 2 goes out during stage 0.
#pragma unroll
  for (int q = 0; q < 4; ++q) gload_part(0, 0, q);
  if (nstages > 1) {
#pragma unroll
    for (int q = 0; q < 4; ++q) gload_part(1, 1, q);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA) : "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __syncthreads();
  read_half(0, 0, 0, 0, 0);
  for (int s = 0; s < nstages; ++s) {
    const bool more = s + 1 < nstages;
    const bool ahead = s + 2 < nstages;       // stage s + 2 exists: its DMA goes out in this stage
#pragma unroll
    for (int hh = 0; hh < HPS; ++hh) {
      const int hg = s * HPS + hh;            // half-group index
      if (hh > 0 && hg >= H) break;           // K has an odd number of groups of 64
      const int i = hh & 1, gi = hh >> 1;
      const int ai = RM ? i : 0, bi = RM ? gi : 0;
      const bool last = hh == HPS - 1;
      // This step's fragments in place and the previous step's rescale issued before the next
      // reads go out (keeps one register set live per step).
      asm volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]), "+v"(fa_[ai][0][0]),
                   "+v"(fa_[ai][KS - 1][1]), "+v"(fb_[bi][0][0][0]), "+v"(fb_[bi][0][KS - 1][1]), "+v"(fb_[bi][1][0][0]),
                   "+v"(fb_[bi][1][KS - 1][1]), "+v"(xop[i]), "+v"(wop_[bi][0]), "+v"(wop_[bi][1])::"memory");
      if (RM) {
        if (last) {
          if (more) {
            // Stage s + 1 landed here (parts 0-2 of stage s + 2 may be in flight; part 3 goes
            // out below) and every wave's reads of stage s are complete before the barrier;
            // then stage s + 1's first fragments.
            if (ahead) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA - 1) : "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            frag_fence();
            asm volatile("s_barrier" ::: "memory");
            read_half(s + 1, 0, 0, 0, 0);
          }
        } else if (hg + 1 < H) {
          read_half(s, (hh + 1) >> 1, (hh + 1) & 1, (hh + 1) & 1, (hh + 1) >> 1);
        }
      }
      f32x16 P[2], S[2];
      i32x16 PI[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (MODE == 0) P[j] = mfma_p8(ai, bi, j);
        else PI[j] = mfma_pi(ai, bi, j);
        S[j] = mfma_bf16_32x32x16(xop[i], wop_[bi][j], f32x16{});
      }
      // Stage s + 2 -> buffer (s + 2) % 3, last read in stage s - 1 (before this stage's
      // opening barrier).
      if (RM) {
        if (ahead) gload_part(s + 2, (s + 2) % NBUF, hh);
      } else {
        if (ahead) {
          gload_part(s + 2, (s + 2) % NBUF, 2 * hh);
          gload_part(s + 2, (s + 2) % NBUF, 2 * hh + 1);
        }
        if (!last) {
          read_half(s, 0, 1, 0, 0);
        } else if (more) {
          // the step's MFMAs issued (their operands are overwritten next), stage s + 1 landed
          if (MODE == 0) asm volatile("" : "+v"(P[0]), "+v"(P[1]), "+v"(S[0]), "+v"(S[1])::"memory");
          else asm volatile("" : "+v"(PI[0]), "+v"(PI[1]), "+v"(S[0]), "+v"(S[1])::"memory");
          if (ahead) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(DMA) : "memory");
          else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
          read_half(s + 1, 0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x16 pf = MODE == 0 ? P[j] : __builtin_convertvector(PI[j], f32x16);
        rescale_acc(acc[i][j], pf, S[j]);
      }
    }
  }
  // No DMA is in flight (none goes out in the last stage); once every wave is past its last
  // reads, the operand buffers hold the output staging regions.
  __syncthreads();
  unrotate_acc(acc);
  epilogue<OUT_F32, EPI>(p, acc, m0 + 64 * wm, n0 + 64 * wn, lr, h, sA + wave * 4096);
}

// The low-rank term mid @ l1cat^T of one 64 x 64 output block with its operands in LDS, 32 ranks:
// the tile's mid rows (128 bytes: hi plane, lo plane; 16-byte chunk c of row r at
// c ^ ((r >> 1) & 7)) and l1cat rows (64 bytes; chunk c of row r at c ^ ((r >> 2) & 3)); wr / wc =
// the block's first row / column in the tile.  Each accumulator takes hi_k then lo_k for the two
// 16-rank steps, as in epilogue().
__device__ __forceinline__ void lowrank_lds(f32x16 (&acc)[2][2], int lr, int h, const uint8_t* lmid,
                                            const uint8_t* ll1, int wr, int wc) {
  u32x4 ahi[2][2], alo[2][2], b[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = wr + 32 * i + lr, sw = (r >> 1) & 7;
      ahi[u][i] = ld16(lmid + r * 128 + 16 * ((2 * u + h) ^ sw));
      alo[u][i] = ld16(lmid + r * 128 + 16 * ((4 + 2 * u + h) ^ sw));
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = wc + 32 * j + lr;
      b[u][j] = ld16(ll1 + c * 64 + 16 * ((2 * u + h) ^ ((c >> 2) & 3)));
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc[i][j] = mfma_bf16_32x32x16(ahi[u][i], b[u][j], acc[i][j]);
        acc[i][j] = mfma_bf16_32x32x16(alo[u][i], b[u][j], acc[i][j]);
      }
}


// W4A4 GEMM on the FP6 MFMA (e3m2 operands, v_mfma_scale_f32_32x32x64_f8f6f4 with format 3 on
// both sides): the INT4 codes are exact e3m2 values and the FP6 MFMA runs at twice the FP8 rate.
// The arithmetic (exact group sums P, scale products S on the bf16 MFMA, acc += P * S), the wave
// grid, the free-running schedule and the epilogue are those of w4a4_kernel; the operands come in
// the planar e3m2 layout of the activation pass, so the stage tiles are rows-contiguous planes:
//   A: for each of the stage's 4 k-steps t and halves h, a plane of 256 rows x 16 bytes (Q) and
//      one of 256 rows x 8 bytes (P) -- a lane's 6-register operand is its row's Q and P parts;
//   B: the same with 128 rows.
// A ds_read_b128 phase (16 lanes, 16 consecutive rows) and a ds_read_b64 phase (32 lanes, 32
// rows) read contiguous bytes: no bank conflicts and no swizzle.  A stage is 256 columns of K
// in a ring of two LDS buffers (80000 bytes each); stage s + 1 is moved in by DMA in parts
// during the first half-group steps of stage s (wave w streams plane w of every operand and a
// share of the scale tiles: 12 DMA instructions per wave per stage for G = 64) and waited for
// before the barrier that ends stage s.  Rows of the planes are padded to an even count so that a
// 16-byte DMA lane carries two 8-byte P rows.
//
// FULL (K a multiple of 2 KB): every stage holds KB columns and the stages pair up, so the main
// loop runs two stages per iteration with the buffer of each a compile-time constant (LDS
// offsets fold into the read and DMA instructions), no step carries a bound check, the last
// stage is peeled (no DMA, the epilogue's prefetch), and the DMA sources are wave-uniform
// pointers advanced one stage at a time.  Other K take the general loop.
// CH: RTp of 64 .. 256 (a multiple of 32, no store ops), the low-rank term streamed through the
// two LDS buffers in chunks of 32 ranks after the main loop (chunk 0 prefetched by the last stage
// as for RTp = 32); a separate build, so that the other kernels keep their code.
template <int G, bool OUT_F32, bool FULL, bool EPI = false, bool CH = false>
__device__ __forceinline__ void w4a4_e3m2_tile(const GemmParams& p, int bm, int bn) {
  constexpr int TBM = 256, TBN = 128, NBUF = 2;
  constexpr int KB = 256;                     // K columns per pipeline stage
  constexpr int KT = KB / 64;                 // k-steps per stage
  constexpr int GPS = KB / G;                 // groups per stage
  constexpr int HPS = 2 * GPS;                // half-group steps per stage
  constexpr int KS = G / 64;                  // k-steps per group
  constexpr int AQ = KT * 2 * TBM * 16, AP = KT * 2 * TBM * 8, BQ = KT * 2 * TBN * 16, BP = KT * 2 * TBN * 8;
  constexpr int XS = TBM + 4, WS = TBN + 4;   // scale words per group; the last 4 are zero
  constexpr int SXD = (GPS * TBM + 511) / 512, SWD = (GPS * TBN + 511) / 512;   // scale DMAs per wave
  constexpr int NDMA = 4 + 2 + 2 + 1 + SXD + SWD;                               // DMAs per wave per stage
  constexpr int NPART = HPS > 2 ? HPS - 2 : 1;                                  // steps that issue DMA
  constexpr int PER = (NDMA + NPART - 1) / NPART;
  static_assert(KT * 2 == 8, "one plane per wave");
  __shared__ __attribute__((aligned(1024))) uint8_t sAQ[NBUF][AQ];
  __shared__ __attribute__((aligned(1024))) uint8_t sAP[NBUF][AP];
  __shared__ __attribute__((aligned(1024))) uint8_t sBQ[NBUF][BQ];
  __shared__ __attribute__((aligned(1024))) uint8_t sBP[NBUF][BP];
  __shared__ __attribute__((aligned(16))) uint32_t sX[NBUF][GPS][XS];   // (sx, sx) bf16 pairs
  __shared__ __attribute__((aligned(16))) uint32_t sW[NBUF][GPS][WS];   // (hi, lo) of sw

  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = bm * TBM, n0 = bn * TBN;
  const int K = p.K, ngroups = K / G, nkt = K / 64, nstages = (K + KB - 1) / KB, H = 2 * ngroups;
  const int Mp = (p.M + 1) & ~1, Np = (p.N + 1) & ~1;

  // Operand DMA, wave w <-> plane w = (k-step w / 2, half w % 2) of each operand.  Per-lane byte
  // offsets within a plane (rows clamped into the operand; clamped rows are never stored).
  uint32_t aq_o[4], ap_o[2], bq_o[2];
#pragma unroll
  for (int c = 0; c < 4; ++c) aq_o[c] = (uint32_t)min(m0 + 64 * c + lane, p.M - 1) * 16u;
#pragma unroll
  for (int c = 0; c < 2; ++c) ap_o[c] = (uint32_t)min(m0 + 128 * c + 2 * lane, Mp - 2) * 8u;
#pragma unroll
  for (int c = 0; c < 2; ++c) bq_o[c] = (uint32_t)min(n0 + 64 * c + lane, p.N - 1) * 16u;
  const uint32_t bp_o = (uint32_t)min(n0 + 2 * lane, Np - 2) * 8u;
  const long aP0 = (long)nkt * 2 * Mp * 16, bP0 = (long)nkt * 2 * Np * 16;   // P region offsets
  const bool epi_lds = CH || p.RTp == 32;   // the epilogue's mid / l1cat rows fit the free buffer
  const int nch = p.RTp / 32;                // CH: chunks of 32 ranks
  if (tid < NBUF * GPS * 4) {
    sX[tid / (4 * GPS)][(tid / 4) % GPS][TBM + tid % 4] = 0u;
    sW[tid / (4 * GPS)][(tid / 4) % GPS][TBN + tid % 4] = 0u;
  }
  const uint32_t ldsAQ = lds_offset(sAQ), ldsAP = lds_offset(sAP), ldsBQ = lds_offset(sBQ),
                 ldsBP = lds_offset(sBP), ldsX = lds_offset(&sX[0][0][0]), ldsW = lds_offset(&sW[0][0][0]);

  // DMA d (0 .. NDMA-1) of stage s into buffer buf: 0-3 A Q rows 64 d.., 4-5 A P rows 128 (d-4)..,
  // 6-7 B Q rows 64 (d-6).., 8 B P, then the scale words (64 per instruction, wrapping).
  auto dma = [&](int s, int buf, int d) {
    const int kt = min(s * KT + (wave >> 1), nkt - 1);    // a k-step past K re-reads the last one
    const long pl = (long)(kt * 2 + (wave & 1));
    if (d < 4) {
      dma16<EPI>(p.qa + pl * Mp * 16, aq_o[d], ldsAQ + buf * AQ + (wave * TBM + 64 * d) * 16);
    } else if (d < 6) {
      dma16<EPI>(p.qa + aP0 + pl * Mp * 8, ap_o[d - 4], ldsAP + buf * AP + (wave * TBM + 128 * (d - 4)) * 8);
    } else if (d < 8) {
      dma16<EPI>(p.qwe + pl * Np * 16, bq_o[d - 6], ldsBQ + buf * BQ + (wave * TBN + 64 * (d - 6)) * 16);
    } else if (d == 8) {
      dma16<EPI>(p.qwe + bP0 + pl * Np * 8, bp_o, ldsBP + buf * BP + wave * TBN * 8);
    } else {
      const int g0 = s * GPS, jmax = ngroups - 1 - g0;
      if (d < 9 + SXD) {
        const int w0 = (512 * (d - 9) + 64 * wave) % (GPS * TBM), j = w0 / TBM, r0 = w0 % TBM;
        const uint32_t off = 4u * ((uint32_t)min(j, jmax) * (uint32_t)p.M + (uint32_t)min(m0 + r0 + lane, p.M - 1));
        dma4<EPI>(p.sxp + (long)g0 * p.M, off, ldsX + 4 * ((buf * GPS + j) * XS + r0));
      } else {
        const int w0 = (512 * (d - 9 - SXD) + 64 * wave) % (GPS * TBN), j = w0 / TBN, r0 = w0 % TBN;
        const uint32_t off = 4u * ((uint32_t)min(j, jmax) * (uint32_t)p.N + (uint32_t)min(n0 + r0 + lane, p.N - 1));
        dma4<EPI>(p.swp + (long)g0 * p.N, off, ldsW + 4 * ((buf * GPS + j) * WS + r0));
      }
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int xo0 = 4 * (64 * wm + scale_row_perm(lr)), xo1 = xo0 + 128;   // rows permuted: see rescale_acc
  const int wo0 = 4 * (h ? TBN : 64 * wn + lr), wo1 = 4 * (h ? TBN : 64 * wn + 32 + lr);
  u32x4 xop[2] = {u32x4{}, u32x4{}};

  // Fragments: Q (16 bytes) and P (8 bytes) parts per k-step.  G == 64 (RM): the next
  // half-group's fragments are read a step ahead into the other set (A by half-group parity, B
  // and the weight scales by group parity); G == 128: one set.
  constexpr bool RM = G == 64;
  constexpr int NS = RM ? 2 : 1;
  u32x4 faq[NS][KS], fbq[NS][2][KS], wop_[NS][2];
  u32x2 fap[NS][KS], fbp[NS][2][KS];
#pragma unroll
  for (int q = 0; q < NS; ++q) wop_[q][0] = wop_[q][1] = u32x4{};
  auto read_half = [&](int buf, int gi, int i, int ai, int bi) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int pl = (gi * KS + ks) * 2 + h;
      const int ra = pl * TBM + 64 * wm + 32 * i + lr;
      faq[ai][ks] = *reinterpret_cast<const u32x4*>(&sAQ[buf][ra * 16]);
      fap[ai][ks] = *reinterpret_cast<const u32x2*>(&sAP[buf][ra * 8]);
      if (i == 0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int rb = pl * TBN + 64 * wn + 32 * j + lr;
          fbq[bi][j][ks] = *reinterpret_cast<const u32x4*>(&sBQ[buf][rb * 16]);
          fbp[bi][j][ks] = *reinterpret_cast<const u32x2*>(&sBP[buf][rb * 8]);
        }
      }
    }
    const uint8_t* x0 = reinterpret_cast<const uint8_t*>(&sX[buf][gi][0]);
    xop[i][0] = *reinterpret_cast<const uint32_t*>(x0 + (i ? xo1 : xo0));
    if (i == 0) {
      const uint8_t* w0 = reinterpret_cast<const uint8_t*>(&sW[buf][gi][0]);
      wop_[bi][0][0] = *reinterpret_cast<const uint32_t*>(w0 + wo0);
      wop_[bi][1][0] = *reinterpret_cast<const uint32_t*>(w0 + wo1);
    }
  };
  auto mfma_p6 = [&](int ai, int bi, int j) {
    f32x16 pf = mfma_fp6_32x32x64(faq[ai][0], fap[ai][0], fbq[bi][j][0], fbp[bi][j][0], f32x16{});
#pragma unroll
    for (int ks = 1; ks < KS; ++ks) pf = mfma_fp6_32x32x64(faq[ai][ks], fap[ai][ks], fbq[bi][j][ks], fbp[bi][j][ks], pf);
    return pf;
  };
  // Fence on every fragment register (both sets): reads issued before it have landed at it.
#define SVDQ_FRAGS6_1 "+v"(faq[0][0]), "+v"(fap[0][0]), "+v"(fbq[0][0][0]), "+v"(fbp[0][0][0]), "+v"(fbq[0][1][0]), \
    "+v"(fbp[0][1][0]), "+v"(xop[0]), "+v"(xop[1]), "+v"(wop_[0][0]), "+v"(wop_[0][1])
#define SVDQ_FRAGS6_2 "+v"(faq[NS - 1][0]), "+v"(fap[NS - 1][0]), "+v"(fbq[NS - 1][0][0]), "+v"(fbp[NS - 1][0][0]), \
    "+v"(fbq[NS - 1][1][0]), "+v"(fbp[NS - 1][1][0]), "+v"(wop_[NS - 1][0]), "+v"(wop_[NS - 1][1])
  auto frag_fence = [&]() {
    if (RM) asm volatile("" : SVDQ_FRAGS6_1, SVDQ_FRAGS6_2::"memory");
    else asm volatile("" : SVDQ_FRAGS6_1::"memory");
  };
#undef SVDQ_FRAGS6_1
#undef SVDQ_FRAGS6_2

  // last stage, RTp == 32: the epilogue's low-rank operands -> the free buffer (its A Q area:
  // 256 mid rows of 128 bytes; its B Q area: 128 l1cat rows of 64 bytes), swizzled for the
  // epilogue's reads
  // (CH: chunk cc = ranks 32 cc .. 32 cc + 31 of mid rows of 4 RTp bytes and l1cat rows of 2 RTp
  // bytes, in the same LDS layout)
  auto epi_prefetch = [&](int fbuf, int cc) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = (4 * wave + c) * 64 + lane, r = idx >> 3, ch = (idx & 7) ^ ((r >> 1) & 7);
      if constexpr (CH) {
        const uint32_t src = (uint32_t)min(m0 + r, p.M - 1) * (uint32_t)(4 * p.RTp) +
                             (uint32_t)((ch & 4) ? 2 * p.RTp : 0) + 64u * cc + 16u * (ch & 3);
        dma16<EPI>(p.midp, src, ldsAQ + fbuf * AQ + (4 * wave + c) * 1024);
      } else {
        dma16<EPI>(p.midp, (uint32_t)min(m0 + r, p.M - 1) * 128u + 16u * ch, ldsAQ + fbuf * AQ + (4 * wave + c) * 1024);
      }
    }
    const int idx = wave * 64 + lane, r = idx >> 2, ch = (idx & 3) ^ ((r >> 2) & 3);
    if constexpr (CH)
      dma16<EPI>(p.l1cat, (uint32_t)min(n0 + r, p.N - 1) * (uint32_t)(2 * p.RTp) + 64u * cc + 16u * ch,
                 ldsBQ + fbuf * BQ + wave * 1024);
    else
      dma16<EPI>(p.l1cat, (uint32_t)min(n0 + r, p.N - 1) * 64u + 16u * ch, ldsBQ + fbuf * BQ + wave * 1024);
  };
  // This step's fragments in place and the previous step's rescale issued before the next reads
  // go out (keeps one register set live per step).
  auto step_fence = [&](int i, int ai, int bi) {
    asm volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]), "+v"(faq[ai][0]),
                 "+v"(fap[ai][KS - 1]), "+v"(fbq[bi][0][0]), "+v"(fbp[bi][0][KS - 1]), "+v"(fbq[bi][1][0]),
                 "+v"(fbp[bi][1][KS - 1]), "+v"(xop[i]), "+v"(wop_[bi][0]), "+v"(wop_[bi][1])::"memory");
  };

  // Stage 0 landed everywhere; stage s + 1 goes out during stage s.
#pragma unroll
  for (int d = 0; d < NDMA; ++d) dma(0, 0, d);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  read_half(0, 0, 0, 0, 0);

  if constexpr (FULL) {
    // DMA sources of stage 1 (advanced per stage) and wave-uniform LDS bases.
    const uint8_t* gAQ = p.qa + (long)(8 + wave) * Mp * 16;
    const uint8_t* gAP = p.qa + aP0 + (long)(8 + wave) * Mp * 8;
    const uint8_t* gBQ = p.qwe + (long)(8 + wave) * Np * 16;
    const uint8_t* gBP = p.qwe + bP0 + (long)(8 + wave) * Np * 8;
    const uint32_t* gX = p.sxp + (long)GPS * p.M;
    const uint32_t* gW = p.swp + (long)GPS * p.N;
    const uint32_t lAQ = ldsAQ + wave * TBM * 16, lAP = ldsAP + wave * TBM * 8, lBQ = ldsBQ + wave * TBN * 16,
                   lBP = ldsBP + wave * TBN * 8;
    uint32_t sx_o[SXD], lX[SXD], sw_o[SWD], lW[SWD];
#pragma unroll
    for (int d = 0; d < SXD; ++d) {
      const int w0 = (512 * d + 64 * wave) % (GPS * TBM), j = w0 / TBM, r0 = w0 % TBM;
      sx_o[d] = 4u * ((uint32_t)j * (uint32_t)p.M + (uint32_t)min(m0 + r0 + lane, p.M - 1));
      lX[d] = ldsX + 4 * (j * XS + r0);
    }
#pragma unroll
    for (int d = 0; d < SWD; ++d) {
      const int w0 = (512 * d + 64 * wave) % (GPS * TBN), j = w0 / TBN, r0 = w0 % TBN;
      sw_o[d] = 4u * ((uint32_t)j * (uint32_t)p.N + (uint32_t)min(n0 + r0 + lane, p.N - 1));
      lW[d] = ldsW + 4 * (j * WS + r0);
    }
    const long stA = 8L * Mp, stB = 8L * Np;   // bytes per stage / 16 (Q) and / 8 (P)
    // Per-lane LDS bases of the fragment reads; every read is base + a compile-time offset
    // (buffer, plane, sub-tile).  The bases are re-declared opaque at each stage so that the
    // compiler folds the offsets into the instructions instead of keeping one address register
    // per offset across the loop.
    typedef const __attribute__((address_space(3))) uint8_t* lds_u8;
    typedef const __attribute__((address_space(3))) u32x4* lds_u32x4;
    typedef const __attribute__((address_space(3))) u32x2* lds_u32x2;
    typedef const __attribute__((address_space(3))) uint32_t* lds_u32;
    lds_u8 rAQ = (lds_u8)&sAQ[0][(h * TBM + 64 * wm + lr) * 16];
    lds_u8 rAP = (lds_u8)&sAP[0][(h * TBM + 64 * wm + lr) * 8];
    lds_u8 rBQ = (lds_u8)&sBQ[0][(h * TBN + 64 * wn + lr) * 16];
    // (the two column sub-tiles' 8-byte parts get separate bases: merged into one ds_read2_b64,
    // they would have to be copied next to their 16-byte parts)
    lds_u8 rBP = (lds_u8)&sBP[0][(h * TBN + 64 * wn + lr) * 8], rBP1 = rBP + 32 * 8;
    lds_u8 rX = (lds_u8)&sX[0][0][0] + xo0;
    lds_u8 rW0 = (lds_u8)&sW[0][0][0] + wo0, rW1 = (lds_u8)&sW[0][0][0] + wo1;
    auto read_half_full = [&](int buf, int gi, int i, int ai, int bi) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int pl2 = (gi * KS + ks) * 2;   // plane pair of this k-step; the lane's half picks one
        faq[ai][ks] = *(lds_u32x4)(rAQ + buf * AQ + (pl2 * TBM + 32 * i) * 16);
        fap[ai][ks] = *(lds_u32x2)(rAP + buf * AP + (pl2 * TBM + 32 * i) * 8);
        if (i == 0) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            fbq[bi][j][ks] = *(lds_u32x4)(rBQ + buf * BQ + (pl2 * TBN + 32 * j) * 16);
            fbp[bi][j][ks] = *(lds_u32x2)((j ? rBP1 : rBP) + buf * BP + pl2 * TBN * 8);
          }
        }
      }
      xop[i][0] = *(lds_u32)(rX + 4 * ((buf * GPS + gi) * XS) + (i ? xo1 - xo0 : 0));
      if (i == 0) {
        wop_[bi][0][0] = *(lds_u32)(rW0 + 4 * ((buf * GPS + gi) * WS));
        wop_[bi][1][0] = *(lds_u32)(rW1 + 4 * ((buf * GPS + gi) * WS));
      }
    };
    auto dma_next = [&](int nb, int d) {
      if (d < 4) dma16<EPI>(gAQ, aq_o[d], lAQ + nb * AQ + 64 * d * 16);
      else if (d < 6) dma16<EPI>(gAP, ap_o[d - 4], lAP + nb * AP + 128 * (d - 4) * 8);
      else if (d < 8) dma16<EPI>(gBQ, bq_o[d - 6], lBQ + nb * BQ + 64 * (d - 6) * 16);
      else if (d == 8) dma16<EPI>(gBP, bp_o, lBP + nb * BP);
      else if (d < 9 + SXD) dma4<EPI>(gX, sx_o[d - 9], lX[d - 9] + 4 * nb * GPS * XS);
      else dma4<EPI>(gW, sw_o[d - 9 - SXD], lW[d - 9 - SXD] + 4 * nb * GPS * WS);
    };
    auto stage = [&](auto buf_c, auto last_c) {
      constexpr int buf = decltype(buf_c)::value, nbuf = buf ^ 1;
      constexpr bool LASTST = decltype(last_c)::value;
      asm volatile("" : "+v"(rAQ), "+v"(rAP), "+v"(rBQ), "+v"(rBP), "+v"(rBP1), "+v"(rX), "+v"(rW0), "+v"(rW1));
#pragma unroll
      for (int hh = 0; hh < HPS; ++hh) {
        const int i = hh & 1, gi = hh >> 1;
        const int ai = RM ? i : 0, bi = RM ? (gi & 1) : 0;
        const bool last = hh == HPS - 1;
        step_fence(i, ai, bi);
        if (RM) {
          if (last) {
            if (!LASTST) {
              asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
              frag_fence();
              asm volatile("s_barrier" ::: "memory");
              read_half_full(nbuf, 0, 0, 0, 0);
            }
          } else {
            read_half_full(buf, (hh + 1) >> 1, (hh + 1) & 1, (hh + 1) & 1, ((hh + 1) >> 1) & 1);
          }
        }
        f32x16 P[2], S[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          P[j] = mfma_p6(ai, bi, j);
          S[j] = mfma_bf16_32x32x16(xop[i], wop_[bi][j], f32x16{});
        }
        if (!LASTST && hh < NPART) {
#pragma unroll
          for (int d = hh * PER; d < (hh + 1) * PER; ++d)
            if (d < NDMA) dma_next(nbuf, d);
        }
        if (LASTST && hh == 0 && epi_lds) epi_prefetch(nbuf, 0);
        if (!RM) {
          if (!last) {
            read_half_full(buf, (hh + 1) >> 1, (hh + 1) & 1, 0, 0);
          } else if (!LASTST) {
            asm volatile("" : "+v"(P[0]), "+v"(P[1]), "+v"(S[0]), "+v"(S[1])::"memory");
            asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
            read_half_full(nbuf, 0, 0, 0, 0);
          }
        }
        // the rescale FMAs at raised priority: they issue ahead of the other wave's fragment reads
        // and DMA while its MFMAs run (2-3% on ff.up)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          rescale_acc(acc[i][j], P[j], S[j]);
        __builtin_amdgcn_s_setprio(0);
      }
      if (!LASTST) {
        gAQ += stA * 16;
        gAP += stA * 8;
        gBQ += stB * 16;
        gBP += stB * 8;
        gX += (long)GPS * p.M;
        gW += (long)GPS * p.N;
      }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using NO = std::integral_constant<bool, false>;
    using YES = std::integral_constant<bool, true>;
    for (int s = 0; s + 2 < nstages; s += 2) {
      stage(B0{}, NO{});
      stage(B1{}, NO{});
    }
    stage(B0{}, NO{});
    stage(B1{}, YES{});
  } else {
  for (int s = 0; s < nstages; ++s) {
    const bool more = s + 1 < nstages;
    const int buf = s & 1, nbuf = buf ^ 1;
#pragma unroll
    for (int hh = 0; hh < HPS; ++hh) {
      const int hg = s * HPS + hh;            // half-group index
      if (hh > 0 && hg >= H) break;           // the last stage holds fewer groups
      const int i = hh & 1, gi = hh >> 1;
      const int ai = RM ? i : 0, bi = RM ? (gi & 1) : 0;
      const bool last = hh == HPS - 1;
      step_fence(i, ai, bi);
      if (RM) {
        if (last) {
          if (more) {
            // stage s + 1 landed everywhere and every wave's reads of stage s are complete
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            frag_fence();
            asm volatile("s_barrier" ::: "memory");
            read_half(nbuf, 0, 0, 0, 0);
          }
        } else if (hg + 1 < H) {
          read_half(buf, (hh + 1) >> 1, (hh + 1) & 1, (hh + 1) & 1, ((hh + 1) >> 1) & 1);
        }
      }
      f32x16 P[2], S[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        P[j] = mfma_p6(ai, bi, j);
        S[j] = mfma_bf16_32x32x16(xop[i], wop_[bi][j], f32x16{});
      }
      // stage s + 1 -> buffer nbuf, last read in stage s - 1 (before the barrier that ended it)
      if (more && hh < NPART) {
#pragma unroll
        for (int d = hh * PER; d < (hh + 1) * PER; ++d)
          if (d < NDMA) dma(s + 1, nbuf, d);
      }
      if (!more && epi_lds && hh == 0) epi_prefetch(nbuf, 0);
      if (!RM) {
        if (!last) {
          if (hg + 1 < H) read_half(buf, (hh + 1) >> 1, (hh + 1) & 1, 0, 0);
        } else if (more) {
          // the step's MFMAs issued (their operands are overwritten next), stage s + 1 landed
          asm volatile("" : "+v"(P[0]), "+v"(P[1]), "+v"(S[0]), "+v"(S[1])::"memory");
          asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
          read_half(nbuf, 0, 0, 0, 0);
        }
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        rescale_acc(acc[i][j], P[j], S[j]);
      __builtin_amdgcn_s_setprio(0);
    }
  }
  }
  // Only the epilogue operands' DMA can be in flight; once every wave is past its last reads,
  // the last stage's A planes hold the output staging regions.
  const int lbuf = (nstages - 1) & 1;
  if (epi_lds) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  unrotate_acc(acc);
  if constexpr (CH) {
    // the low-rank term in chunks of 32 ranks: chunk cc in buffer lbuf ^ 1 ^ (cc & 1), chunk cc + 1's
    // DMA into the other while chunk cc's MFMAs run (the last stage's buffer is free past the
    // barrier above); each accumulator takes hi_k then lo_k for k = 0, 16, .. as in epilogue();
    // then bias, staging (the last stage's A planes) and stores
    for (int cc = 0; cc < nch; ++cc) {
      const int cb = lbuf ^ 1 ^ (cc & 1);
      if (cc + 1 < nch) epi_prefetch(cb ^ 1, cc + 1);
      lowrank_lds(acc, lr, h, &sAQ[cb][0], &sBQ[cb][0], 64 * wm, 64 * wn);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // chunk cc + 1 landed
      __syncthreads();                                     // and every wave is done with chunk cc
    }
    GemmParams pe = p;
    pe.RTp = 0;
    epilogue<OUT_F32, EPI>(pe, acc, m0 + 64 * wm, n0 + 64 * wn, lr, h, &sAQ[lbuf][0] + wave * 4096);
  } else {
    epilogue<OUT_F32, EPI>(p, acc, m0 + 64 * wm, n0 + 64 * wn, lr, h, &sAQ[lbuf][0] + wave * 4096,
                           epi_lds ? &sAQ[lbuf ^ 1][0] : nullptr, epi_lds ? &sBQ[lbuf ^ 1][0] : nullptr, 64 * wm,
                           64 * wn);
  }
}

template <int G, bool OUT_F32, bool FULL, bool EPI = false, bool CH = false>
__global__ void __launch_bounds__(512, 1) w4a4_e3m2_kernel(GemmParams p) {
  const int nbm = (p.M + 255) / 256, nbn = (p.N + 127) / 128;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 4, bm, bn);
  w4a4_e3m2_tile<G, OUT_F32, FULL, EPI, CH>(p, bm, bn);
}

// Sibling layers (same rows M, same K and group) in one launch: the layers' 256 x 128 tiles are
// numbered back to back (layer i from tile0[i]), that order is spread over the XCDs as in
// tile_coords, and each workgroup runs one tile of one layer with that layer's parameters.  The
// tiles are the single-layer kernel's, so every output is bit-identical to a launch per layer;
// what changes is that the layers' tiles share the rounds of workgroups over the CUs.  CH: the
// low-rank term in LDS chunks (every layer's RTp a multiple of 32 up to 256).
template <int G, bool OUT_F32, bool CH = false>
__global__ void __launch_bounds__(512, 1) w4a4_e3m2_siblings_kernel(GemmSiblings gs) {
  const int total = gs.tile0[gs.count];
  int lin = blockIdx.x;
  if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
  int i = 0;
#pragma unroll
  for (int c = 1; c < MAX_SIBLINGS; ++c) i += (c < gs.count && lin >= gs.tile0[c]) ? 1 : 0;
  i = __builtin_amdgcn_readfirstlane(i);
  const GemmParams& p = gs.layer[i];
  const int nbm = (p.M + 255) / 256, nbn = (p.N + 127) / 128;
  int bm, bn;
  tile_of_linear(lin - gs.tile0[i], nbm, nbn, 4, bm, bn);
  w4a4_e3m2_tile<G, OUT_F32, true, false, CH>(p, bm, bn);
}

// W4A4 GEMM, wide tiles (group 64, K a multiple of 256): block tile 256 x 256, 8 waves in a
// 2 x 4 grid, wave tile 128 x 64 = 4 x 2 sub-tiles of 32 x 32.  Same arithmetic as
// w4a4_e3m2_tile (FP6 product MFMA, bf16 scale MFMA, acc += P * S per group), same planar
// operands and epilogue; what changes is the reuse per byte staged: each A fragment read from
// LDS feeds 2 MFMAs and each B fragment 4 (2 and 2 in the 256 x 128 tile), and each byte the DMA
// brings in feeds 256 output columns instead of 128.  Per 32 x 32 x 64 block that is a third fewer
// DMA and a quarter fewer LDS read instructions, and the tile's fixed cost (first stage,
// epilogue) is spread over twice the work.
//
// Stage = 128 columns of K (2 groups), two LDS buffers of 53312 bytes:
//   A Q planes [k-step][half][256 rows][16 B], A P planes [k-step][half][256 rows][8 B], then B
//   the same with 256 columns, then the scale words: (sx, sx) pairs [group][256 + 4] and
//   (hi, lo) weight-scale pairs [group][256 + 4] (the last 4 words of each zero).
// Wave w moves, per stage: rows 128 (w & 1) .. + 127 of plane w >> 1 of each operand (2 + 1 DMA
// each for A and B) and 64 words of the scale tiles (group w >> 2, words 64 (w & 3) ..): 8 DMA
// instructions, issued 2 per step over the stage's first 4 steps and waited for before the
// barrier that ends the stage.
// Steps: (group gi, row sub-tile i), 8 per stage; a step issues the row sub-tile's two product
// and two scale MFMAs against both column sub-tiles, then its 32 rescale FMAs.  A fragments and
// the sx operand of the next step are read at the top of the step into the other register set;
// the B fragments and weight-scale operands of the next group are read in the group's last step,
// after its MFMAs have taken the current ones (one set).
// CH: RTp of 64 .. 256 (a multiple of 32), the low-rank term streamed through the two LDS buffers
// in chunks of 32 ranks after the main loop (chunk 0 prefetched by the last stage as for RTp = 32,
// chunk c + 1's DMA under chunk c's MFMAs); without it those ranks read their operands from global
// memory in the epilogue.  A separate build, so that the RTp = 32 kernel keeps its code.
template <bool OUT_F32, bool CH = false>
__device__ __forceinline__ void w4a4_e3m2_wide_tile(const GemmParams& p, int bm, int bn) {
  constexpr int TBM = 256, TBN = 256, KT = 2, GPS = 2, HPS = 8;
  constexpr int PQ = TBM * 16, PP = TBM * 8;             // bytes of one Q / P plane
  constexpr int AQ = 0, AP = AQ + KT * 2 * PQ, BQ = AP + KT * 2 * PP, BP = BQ + KT * 2 * PQ;
  constexpr int XS = TBM + 36;                            // scale words per group (the last 36 zero)
  constexpr int XO = BP + KT * 2 * PP, WO = XO + GPS * XS * 4, BUF = WO + GPS * XS * 4;
  constexpr int NDMA = 8, PER = 2;
  static_assert(TBN == TBM, "scale tiles share one word count");
  __shared__ __attribute__((aligned(1024))) uint8_t sm[2 * BUF];

  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int m0 = bm * TBM, n0 = bn * TBN;
  const int M = p.M, N = p.N, K = p.K, nkt = K / 64, nstages = K / 128;
  const uint32_t lds0 = lds_offset(sm);

  // DMA (M and N multiples of 256: no row is clamped).  Wave w moves plane pa = w >> 1 of the
  // stage's 4 planes (k-step pa >> 1, half pa & 1), rows 128 (w & 1) ..; per-lane offsets are
  // lane x 16 bytes (one Q row, or two 8-byte P rows) and lane x 4 (one scale word), everything
  // else goes into the wave-uniform source and LDS addresses.
  const int pa = wave >> 1, rh = (wave & 1) * 128, sj = wave >> 2, sr = (wave & 3) * 64;
  const uint32_t o16 = (uint32_t)lane * 16u, o4 = (uint32_t)lane * 4u;
  const long aP0 = (long)nkt * 2 * M * 16, bP0 = (long)nkt * 2 * N * 16;   // P region offsets
  const uint32_t lAQ = lds0 + AQ + pa * PQ + rh * 16, lAP = lds0 + AP + pa * PP + rh * 8;
  const uint32_t lBQ = lds0 + BQ + pa * PQ + rh * 16, lBP = lds0 + BP + pa * PP + rh * 8;
  const uint32_t lX = lds0 + XO + 4 * (sj * XS + sr), lW = lds0 + WO + 4 * (sj * XS + sr);
  // sources of stage 0 (advanced one stage at a time)
  const uint8_t* gAQ = p.qa + (long)pa * M * 16 + (long)(m0 + rh) * 16;
  const uint8_t* gAP = p.qa + aP0 + (long)pa * M * 8 + (long)(m0 + rh) * 8;
  const uint8_t* gBQ = p.qwe + (long)pa * N * 16 + (long)(n0 + rh) * 16;
  const uint8_t* gBP = p.qwe + bP0 + (long)pa * N * 8 + (long)(n0 + rh) * 8;
  const uint32_t* gX = p.sxp + (long)sj * M + m0 + sr;
  const uint32_t* gW = p.swp + (long)sj * N + n0 + sr;
  const long stA = 4L * M, stB = 4L * N;   // plane rows per stage
  auto dma_next = [&](int nb, int d) {
    const uint32_t o = (uint32_t)(nb * BUF);
    if (d < 2) dma16(gAQ + 64 * d * 16, o16, lAQ + o + 64 * d * 16);
    else if (d == 2) dma16(gAP, o16, lAP + o);
    else if (d < 5) dma16(gBQ + 64 * (d - 3) * 16, o16, lBQ + o + 64 * (d - 3) * 16);
    else if (d == 5) dma16(gBP, o16, lBP + o);
    else if (d == 6) dma4(gX, o4, lX + o);
    else dma4(gW, o4, lW + o);
  };
  auto advance = [&]() {
    gAQ += stA * 16;
    gAP += stA * 8;
    gBQ += stB * 16;
    gBP += stB * 8;
    gX += (long)GPS * M;
    gW += (long)GPS * N;
  };
  // the zero words after each scale tile, both buffers (2 x 2 x 2 x 36)
  for (int t = tid; t < 2 * 2 * GPS * 36; t += 512) {
    const int b = t / (2 * GPS * 36), r = t % (2 * GPS * 36), w = r / (GPS * 36), g = (r / 36) % GPS, e = r % 36;
    *reinterpret_cast<uint32_t*>(sm + b * BUF + (w ? WO : XO) + 4 * (g * XS + TBM + e)) = 0u;
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  // Per-lane LDS read bases; every read adds a compile-time offset (buffer, plane, sub-tile).
  typedef const __attribute__((address_space(3))) uint8_t* lds_u8;
  typedef const __attribute__((address_space(3))) u32x4* lds_u32x4;
  typedef const __attribute__((address_space(3))) u32x2* lds_u32x2;
  typedef const __attribute__((address_space(3))) uint32_t* lds_u32;
  lds_u8 rAQ = (lds_u8)&sm[AQ + h * PQ + (128 * wm + lr) * 16];
  lds_u8 rAP = (lds_u8)&sm[AP + h * PP + (128 * wm + lr) * 8];
  lds_u8 rBQ = (lds_u8)&sm[BQ + h * PQ + (64 * wn + lr) * 16];
  lds_u8 rBP = (lds_u8)&sm[BP + h * PP + (64 * wn + lr) * 8], rBP1 = rBP + 32 * 8;
  lds_u8 rX = (lds_u8)&sm[XO + 4 * (128 * wm + scale_row_perm(lr))];   // rows permuted: see rescale_acc
  // weight scales: lanes 32-63 read zero words (B rows 8-15 of the scale MFMA)
  lds_u8 rW = (lds_u8)&sm[WO + 4 * (h ? TBN : 64 * wn + lr)];

  // One register set: the next step's A fragments and sx operand are read after this step's
  // MFMAs have taken the current ones, the next group's B fragments and weight-scale operands in
  // the group's last step.  The scale MFMA is the K = 8 bf16 form (two-register operands): word 0
  // loaded from LDS, word 1 stays zero.
  u32x4 faq, fbq[2];
  u32x2 fap, fbp[2], xop = u32x2{}, wop[2] = {u32x2{}, u32x2{}};
  auto read_a = [&](int buf, int gi, int i) {
    faq = *(lds_u32x4)(rAQ + buf * BUF + gi * 2 * PQ + 32 * i * 16);
    fap = *(lds_u32x2)(rAP + buf * BUF + gi * 2 * PP + 32 * i * 8);
    xop[0] = *(lds_u32)(rX + buf * BUF + 4 * gi * XS + 128 * i);
  };
  auto read_b = [&](int buf, int gi) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      fbq[j] = *(lds_u32x4)(rBQ + buf * BUF + gi * 2 * PQ + 32 * j * 16);
      fbp[j] = *(lds_u32x2)((j ? rBP1 : rBP) + buf * BUF + gi * 2 * PP);
      wop[j][0] = *(lds_u32)(rW + buf * BUF + 4 * gi * XS + 128 * j);
    }
  };
  // last stage, RTp == 32: the epilogue's low-rank operands -> the free buffer (256 mid rows of
  // 128 bytes, then 256 l1cat rows of 64 bytes), swizzled for the epilogue's reads
  // CH: chunk cc = ranks 32 cc .. 32 cc + 31, 64 bytes of the hi plane and 64 of the lo plane per
  // mid row (rows of 4 RTp bytes), 64 bytes per l1cat row (2 RTp bytes), in the RTp = 32 layout
  const int nch = p.RTp / 32;
  const bool epi_lds = CH || p.RTp == 32;
  auto epi_prefetch = [&](int fbuf, int cc) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = (4 * wave + c) * 64 + lane, r = idx >> 3, ch = (idx & 7) ^ ((r >> 1) & 7);
      if constexpr (CH) {
        const uint32_t src = (uint32_t)(m0 + r) * (uint32_t)(4 * p.RTp) + (uint32_t)((ch & 4) ? 2 * p.RTp : 0) +
                             64u * cc + 16u * (ch & 3);
        dma16(p.midp, src, lds0 + fbuf * BUF + (4 * wave + c) * 1024);
      } else {
        dma16(p.midp, (uint32_t)(m0 + r) * 128u + 16u * ch, lds0 + fbuf * BUF + (4 * wave + c) * 1024);
      }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int idx = (2 * wave + c) * 64 + lane, r = idx >> 2, ch = (idx & 3) ^ ((r >> 2) & 3);
      if constexpr (CH)
        dma16(p.l1cat, (uint32_t)(n0 + r) * (uint32_t)(2 * p.RTp) + 64u * cc + 16u * ch,
              lds0 + fbuf * BUF + 32768 + (2 * wave + c) * 1024);
      else
        dma16(p.l1cat, (uint32_t)(n0 + r) * 64u + 16u * ch, lds0 + fbuf * BUF + 32768 + (2 * wave + c) * 1024);
    }
  };

  // Stage 0 landed everywhere; stage s + 1 goes out during stage s.
#pragma unroll
  for (int d = 0; d < NDMA; ++d) dma_next(0, d);
  advance();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  read_a(0, 0, 0);
  read_b(0, 0);

  auto stage = [&](auto buf_c, auto last_c) {
    constexpr int buf = decltype(buf_c)::value, nbuf = buf ^ 1;
    constexpr bool LASTST = decltype(last_c)::value;
    asm volatile("" : "+v"(rAQ), "+v"(rAP), "+v"(rBQ), "+v"(rBP), "+v"(rBP1), "+v"(rX), "+v"(rW));
#pragma unroll
    for (int hh = 0; hh < HPS; ++hh) {
      const int gi = hh >> 2, i = hh & 3;
      const bool last = hh == HPS - 1;
      if (LASTST && hh == 0 && epi_lds) epi_prefetch(nbuf, 0);   // ahead of the step's MFMA results
      // this step's fragments in place, the previous step's rescale issued
      asm volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]), "+v"(acc[2][0]),
                   "+v"(acc[2][1]), "+v"(acc[3][0]), "+v"(acc[3][1])::"memory");
      asm volatile("" : "+v"(faq), "+v"(fap), "+v"(xop), "+v"(fbq[0]), "+v"(fbq[1]), "+v"(fbp[0]), "+v"(fbp[1]),
                   "+v"(wop[0]), "+v"(wop[1])::"memory");
      f32x16 P[2], S[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        P[j] = mfma_fp6_32x32x64(faq, fap, fbq[j], fbp[j], f32x16{});
        S[j] = mfma_bf16_32x32x8(xop, wop[j], f32x16{});
      }
      if (!LASTST && hh < NDMA / PER) {
#pragma unroll
        for (int d = hh * PER; d < (hh + 1) * PER; ++d) dma_next(nbuf, d);
      }
      // the MFMAs have their operands; the next fragments go into the same registers
      asm volatile("" : "+v"(P[0]), "+v"(P[1]), "+v"(S[0]), "+v"(S[1])::"memory");
      if (!last) {
        read_a(buf, (hh + 1) >> 2, (hh + 1) & 3);
        if (i == 3) read_b(buf, gi + 1);
      } else if (!LASTST) {
        // stage s + 1 landed everywhere and every wave's reads of this stage are complete
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        asm volatile("s_barrier" ::: "memory");
        read_a(nbuf, 0, 0);
        read_b(nbuf, 0);
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int j = 0; j < 2; ++j) rescale_acc(acc[i][j], P[j], S[j]);
      __builtin_amdgcn_s_setprio(0);
    }
    if (!LASTST) advance();
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using NO = std::integral_constant<bool, false>;
  using YES = std::integral_constant<bool, true>;
  for (int s = 0; s + 2 < nstages; s += 2) {
    stage(B0{}, NO{});
    stage(B1{}, NO{});
  }
  stage(B0{}, NO{});
  stage(B1{}, YES{});
  __builtin_amdgcn_sched_barrier(0);   // nothing of the epilogue moves up into the last steps
  // Only the epilogue operands' DMA can be in flight; once every wave is past its last reads,
  // the last stage's buffer (buffer 1: K / 128 stages, an even count) holds the output staging
  // regions (4 KB per wave).
  if (epi_lds) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  uint8_t* stg = sm + BUF + wave * 4096;
  if constexpr (CH) {
    // chunk cc from buffer cc & 1, chunk cc + 1's DMA into the other while its MFMAs run (buffer 1
    // is free once every wave is past the barrier above); each accumulator takes hi_k then lo_k for
    // k = 0, 16, .. as in epilogue(); then bias, staging (buffer 1) and stores
#pragma unroll
    for (int u = 0; u < 2; ++u) unrotate_acc(*reinterpret_cast<f32x16(*)[2][2]>(&acc[2 * u][0]));
    for (int cc = 0; cc < nch; ++cc) {
      const int cb = cc & 1;
      if (cc + 1 < nch) epi_prefetch(cb ^ 1, cc + 1);
#pragma unroll
      for (int u = 0; u < 2; ++u)
        lowrank_lds(*reinterpret_cast<f32x16(*)[2][2]>(&acc[2 * u][0]), lr, h, sm + cb * BUF, sm + cb * BUF + 32768,
                    128 * wm + 64 * u, 64 * wn);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // chunk cc + 1 landed
      __syncthreads();                                     // and every wave is done with chunk cc
    }
    GemmParams pe = p;
    pe.RTp = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u)
      epilogue<OUT_F32>(pe, *reinterpret_cast<f32x16(*)[2][2]>(&acc[2 * u][0]), m0 + 128 * wm + 64 * u,
                        n0 + 64 * wn, lr, h, stg);
  } else {
    const uint8_t* lmid = epi_lds ? sm : nullptr;
    const uint8_t* ll1 = epi_lds ? sm + 32768 : nullptr;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x16(&a2)[2][2] = *reinterpret_cast<f32x16(*)[2][2]>(&acc[2 * u][0]);
      unrotate_acc(a2);
      epilogue<OUT_F32>(p, a2, m0 + 128 * wm + 64 * u, n0 + 64 * wn, lr, h, stg, lmid, ll1, 128 * wm + 64 * u,
                        64 * wn);
    }
  }
}

// Tile choice for the group-64 e3m2 GEMM.  The wide tiles need M, N multiples of 256 and K of 256,
// and take a shape when their rounds of tiles over the 256 CUs times the tile's work, at the 10%
// lower time per block measured for them (ff.up: 393 against 439 us), is no more than the 256 x
// 128 tiles': ff.up at M = 4096 (4 rounds of 256 x 256 against 8 of 256 x 128) and the config-3
// sibling groups take them, N = 6144 at M = 4096 (2 rounds against 3) does not.
// SVDQ_W4A4_TILES=256x128 or 256x256 in the environment overrides the choice (the second only
// where the wide tiles apply); it exists so that tests can run both tilings on one shape.
int tile_override() {
  const char* e = getenv("SVDQ_W4A4_TILES");
  if (!e) return 0;
  if (!strcmp(e, "256x128")) return 1;
  if (!strcmp(e, "256x256")) return 2;
  return 0;
}
bool wide_tiles_apply(int M, int N, int K) { return K % 256 == 0 && K >= 256 && M % 256 == 0 && N % 256 == 0; }
bool wide_tiles_pay(long tiles_wide, long tiles_narrow) {
  const long wide = (tiles_wide + 255) / 256, narrow = (tiles_narrow + 255) / 256;
  return 2 * wide * 9 <= narrow * 10;
}

template <bool OUT_F32, bool CH = false>
__global__ void __launch_bounds__(512, 1) w4a4_e3m2_wide_kernel(GemmParams p) {
  const int nbm = (p.M + 255) / 256, nbn = (p.N + 255) / 256;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 4, bm, bn);
  w4a4_e3m2_wide_tile<OUT_F32, CH>(p, bm, bn);
}

// Sibling layers on the wide tiles: as w4a4_e3m2_siblings_kernel with 256 x 256 tiles (tile0 counts
// them); every output is bit-identical to a launch per layer.
template <bool OUT_F32, bool CH = false>
__global__ void __launch_bounds__(512, 1) w4a4_e3m2_wide_siblings_kernel(GemmSiblings gs) {
  const int total = gs.tile0[gs.count];
  int lin = blockIdx.x;
  if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
  int i = 0;
#pragma unroll
  for (int c = 1; c < MAX_SIBLINGS; ++c) i += (c < gs.count && lin >= gs.tile0[c]) ? 1 : 0;
  i = __builtin_amdgcn_readfirstlane(i);
  const GemmParams& p = gs.layer[i];
  int bm, bn;
  tile_of_linear(lin - gs.tile0[i], p.M / 256, p.N / 256, 4, bm, bn);
  w4a4_e3m2_wide_tile<OUT_F32, CH>(p, bm, bn);
}

// Weight operand of the W4A4 GEMM, once per layer: each packed dword (8 nibbles, k0 in the
// low nibble) becomes 8 operand bytes [k0 k2 k4 k6 k1 k3 k5 k7].
// The sigmoid gate and SwiGLU product as their own pass over contiguous bf16 tensors (the same op
// code as the GEMM store's): out = op(y, aux) for n elements, 8 per thread and step (16-byte
// loads and stores), the last n % 8 elements by thread 0 of workgroup 0.
template <int E>
__global__ void __launch_bounds__(256) gate_op_kernel(const uint16_t* __restrict__ y, const uint16_t* __restrict__ aux,
                                                      uint16_t* __restrict__ out, long n) {
  const long chunks = n / 8;
  for (long c = (long)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += (long)gridDim.x * blockDim.x) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(y + 8 * c);
    const u32x4 a = *reinterpret_cast<const u32x4*>(aux + 8 * c);
    *reinterpret_cast<u32x4*>(out + 8 * c) = epi_apply_op<E>(v, a, u32x4{});
  }
  if (blockIdx.x == 0 && threadIdx.x == 0 && n % 8) {
    u32x4 v{}, a{};
    for (long e = 8 * chunks; e < n; ++e) {
      v[(e % 8) / 2] |= (uint32_t)y[e] << (16 * (e % 2));
      a[(e % 8) / 2] |= (uint32_t)aux[e] << (16 * (e % 2));
    }
    const u32x4 o = epi_apply_op<E>(v, a, u32x4{});
    for (long e = 8 * chunks; e < n; ++e) out[e] = (uint16_t)(o[(e % 8) / 2] >> (16 * (e % 2)));
  }
}

__global__ void weight_operand_kernel(const uint32_t* __restrict__ qw, u32x2* __restrict__ out, long n, int mode) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    uint32_t lo, hi;
    if (mode == 0) nib8_to_e4m3(qw[i], lo, hi);
    else nib8_to_i8x16(qw[i], lo, hi);
    out[i] = u32x2{lo, hi};
  }
}

// e3m2 (FP6) weight operand, once per layer: thread per (row n, k-step t, half h) turns 32 packed
// codes into their 6-dword field vector (codes_to_e3m2: field f <- k = 64 t + 32 h + f) and writes
// it to the planar layout of the activation pass's e3m2 operand, rows padded to Np (even).
__global__ void weight_operand_e3m2_kernel(const uint8_t* __restrict__ qw, uint8_t* __restrict__ out, int N, int Np,
                                           int K) {
  const int kt_n = K / 64;
  const long total = (long)N * kt_n * 2;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    const int n = (int)(idx % N);
    const long plane = idx / N;                       // t * 2 + h
    const u32x4 w = *reinterpret_cast<const u32x4*>(qw + (long)n * (K / 2) + plane * 16);
    f32x16 x, y;
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t byte = (w[d] >> (8 * e)) & 0xFFu;   // k = 2 (4 d + e) low nibble, + 1 high
        x[4 * d + e] = (float)((int)(byte & 15u) - 8);
        y[4 * d + e] = (float)((int)(byte >> 4) - 8);
      }
    const u32x6 f = codes_to_e3m2(x, y);
    const long row = plane * Np + n;
    *reinterpret_cast<u32x4*>(out + row * 16) = u32x4{f[0], f[1], f[2], f[3]};
    *reinterpret_cast<u32x2*>(out + (long)kt_n * 2 * Np * 16 + row * 8) = u32x2{f[4], f[5]};
  }
}

// Weight-scale operand of the W4A4 scale MFMA, once per layer: (bf16 hi, bf16 lo) of the fp16
// scale, hi + lo == scale exactly; MODE 1 (int8 16*q operands) folds in 1/256.  Written
// group-major, out[g][n] (the GEMM stages one group's scales of consecutive columns).
__global__ void weight_scale_pairs_kernel(const uint16_t* __restrict__ sw, uint32_t* __restrict__ out, int n,
                                          int ngroups, float mult) {
  const long total = (long)n * ngroups;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const long g = i / n, c = i % n;
    const float f = half_bits_to_float(sw[c * ngroups + g]) * mult;
    const uint32_t hi = pack_bf16x2(f, 0.0f) & 0xFFFFu;
    const uint32_t lo = pack_bf16x2(f - bf16lo(hi), 0.0f) & 0xFFFFu;
    out[i] = hi | (lo << 16);
  }
}

// --------------------------------------------------------------------------- W4A16
// The reference pytorch_sim math on the bf16 MFMA: y = x_hat @ W^T with W = bf16(q * bf16(sw))
// (quant/svd.py:119-163, dequantization pack.py:26-44 in bf16), plus the low-rank epilogue.
//
// Block tile (64 WM) x 128: WM x 2 waves, wave tile 64 x 64 = 2 x 2 sub-tiles of 32 x 32 on
// v_mfma_f32_32x32x16_bf16.  A stage is 64 columns of K (one k-group for G = 64, half of one for
// G = 128), double-buffered in LDS: the next stage's x_hat rows (16 bytes per thread and load,
// 8 threads per 128-byte row segment) and packed weight codes (8 bytes = 16 codes per thread)
// are loaded into registers three stages ahead (a ring of three register sets), then written to
// the other buffer one stage ahead -- the weights dequantized on the way (v_cvt_f32_ubyte + one exact FMA per code +
// RNE pack) -- with one barrier per stage.  LDS rows are 64 bf16 plus 16 bytes of padding (144-byte
// pitch): the fragment reads (16 lanes on 16 consecutive rows) and the staging writes hit
// distinct bank groups.
// G = 0: the group size comes at run time (p.group; any multiple of 16): a thread's 16 codes of a
// stage always lie in one group, so each still needs one scale per stage.
template <int G, int WM, bool OUT_F32, bool EPI = false>
__global__ void __launch_bounds__(WM * 128, 1) w4a16_kernel(GemmParams p) {
  constexpr int NT = WM * 128;                // threads
  constexpr int TBM = 64 * WM, TBN = 128, KB = 64;
  constexpr int PITCH = 2 * KB + 16;          // LDS bytes per row
  constexpr int ALD = TBM * 8 / NT;           // 16-byte A loads per thread and stage (= 4)
  constexpr int BROWS = NT / 4;               // weight rows staged per pass (4 threads per row)
  constexpr int BLD = TBN / BROWS;            // weight passes per stage (1 or 2)
  static_assert(ALD * NT == TBM * 8 && BLD * BROWS == TBN, "staging split");
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][TBM * PITCH];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][TBN * PITCH];

  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int nbm = (p.M + TBM - 1) / TBM, nbn = (p.N + TBN - 1) / TBN;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 4, bm, bn);
  const int m0 = bm * TBM, n0 = bn * TBN;
  const int GS = G > 0 ? G : p.group;         // group size
  const int K = p.K, ngroups = K / GS, kp = K / 2, nst = K / KB;

  // staging assignments: A chunk (row, 16-byte chunk) = (idx / 8, idx % 8), idx = tid + NT * i;
  // weights: row tid / 4 (+ BROWS per pass), 16 codes = chunks 2 (tid % 4) and 2 (tid % 4) + 1
  const uint16_t* arow[ALD];
  int aoff[ALD];
#pragma unroll
  for (int i = 0; i < ALD; ++i) {
    const int idx = tid + NT * i, r = idx >> 3, c = idx & 7;
    arow[i] = p.xhat + (long)min(m0 + r, p.M - 1) * p.ldxh + 8 * c;
    aoff[i] = r * PITCH + 16 * c;
  }
  const int bq = tid & 3;
  const uint8_t* brow[BLD];
  const uint16_t* bsc[BLD];
  int boff[BLD];
#pragma unroll
  for (int i = 0; i < BLD; ++i) {
    const int r = (tid >> 2) + BROWS * i, n = min(n0 + r, p.N - 1);
    brow[i] = p.qw + (long)n * kp + 8 * bq;
    bsc[i] = p.sw + (long)n * ngroups;
    boff[i] = r * PITCH + 32 * bq;
  }

  // D register sets: stage s + D is loaded at the start of stage s (three stages of MFMA work
  // cover the load latency); set q holds the stages s with s % D == q.  The loads are issued as
  // inline asm and waited for explicitly: every stage issues the same LPS loads (past the last
  // stage they re-read it), so before stage s + 1 is stored exactly the 2 LPS loads of the two
  // newer sets may still be in flight.  (Left to the compiler, its wait analysis lost track of the
  // sets across the loop and drained every load before each store.)
  constexpr int D = 3;
  constexpr int LPS = ALD + 2 * BLD;          // loads per stage and thread
  u32x4 ra[D][ALD];
  u32x2 rb[D][BLD];
  uint32_t rs[D][BLD];                        // fp16 scale bits
  auto gload_set = [&](int st, u32x4 (&da)[ALD], u32x2 (&db)[BLD], uint32_t (&ds)[BLD]) {
    const int k0 = st * KB;
#pragma unroll
    for (int i = 0; i < ALD; ++i)
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(da[i]) : "v"(arow[i] + k0) : "memory");
#pragma unroll
    for (int i = 0; i < BLD; ++i) {
      asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(db[i]) : "v"(brow[i] + k0 / 2) : "memory");
      asm volatile("global_load_ushort %0, %1, off" : "=v"(ds[i]) : "v"(bsc[i] + (k0 + 16 * bq) / GS) : "memory");
    }
  };
  auto gload = [&](int st, auto q_c) {
    constexpr int q = decltype(q_c)::value;
    gload_set(st, ra[q], rb[q], rs[q]);
  };
  // a set landed: at most the two newer sets' loads (issued after it) still in flight
  auto wait_regs = [&](u32x4 (&da)[ALD], u32x2 (&db)[BLD], uint32_t (&ds)[BLD]) {
    static_assert(2 * LPS < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%c0)" ::"i"(2 * LPS) : "memory");
#pragma unroll
    for (int i = 0; i < ALD; ++i) asm volatile("" : "+v"(da[i]));
#pragma unroll
    for (int i = 0; i < BLD; ++i) asm volatile("" : "+v"(db[i]), "+v"(ds[i]));
  };
  auto wait_set = [&](auto q_c) {
    constexpr int q = decltype(q_c)::value;
    wait_regs(ra[q], rb[q], rs[q]);
  };
  // bf16(q * s), q = nibble - 8: nibble * s and 8 s are exact, so one FMA gives q * s exactly
  auto lstore = [&](int buf, auto q_c) {
    constexpr int q = decltype(q_c)::value;
#pragma unroll
    for (int i = 0; i < ALD; ++i) *reinterpret_cast<u32x4*>(&sA[buf][aoff[i]]) = ra[q][i];
#pragma unroll
    for (int i = 0; i < BLD; ++i) {
      const float sc = round_bf16(half_bits_to_float((uint16_t)rs[q][i])), ns8 = -8.0f * sc;   // bf16 scale, as the sim
      uint32_t o[8];
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const uint32_t v = rb[q][i][d], lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
        o[4 * d + 0] = pack_bf16x2(__builtin_fmaf(ubyte_f32<0>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<0>(hi), sc, ns8));
        o[4 * d + 1] = pack_bf16x2(__builtin_fmaf(ubyte_f32<1>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<1>(hi), sc, ns8));
        o[4 * d + 2] = pack_bf16x2(__builtin_fmaf(ubyte_f32<2>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<2>(hi), sc, ns8));
        o[4 * d + 3] = pack_bf16x2(__builtin_fmaf(ubyte_f32<3>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<3>(hi), sc, ns8));
      }
      *reinterpret_cast<u32x4*>(&sB[buf][boff[i]]) = u32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<u32x4*>(&sB[buf][boff[i] + 16]) = u32x4{o[4], o[5], o[6], o[7]};
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int ra0 = (64 * wm + lr) * PITCH + 16 * h, rb0 = (64 * wn + lr) * PITCH + 16 * h;
  using Q0 = std::integral_constant<int, 0>;
  using Q1 = std::integral_constant<int, 1>;
  using Q2 = std::integral_constant<int, 2>;
  // Loads past the last stage re-read it (clamped index) and the last stage's store fills the
  // unused buffer, so the main loop is branch-free: the compiler then counts exactly which loads
  // are still in flight at each LDS store (a guarded body made it wait for all of them).
  gload(0, Q0{});
  gload(min(1, nst - 1), Q1{});
  gload(min(2, nst - 1), Q2{});
  wait_set(Q0{});
  lstore(0, Q0{});
  __syncthreads();
  // stage st: its data is in LDS buffer st % 2; set q (= st % D) is free, so stage st + D goes
  // out into it; then stage st + 1 moves from its set into the other buffer.  The main loop is
  // branch-free (clamped loads, and the last stage's store fills the unused buffer).
  auto stage = [&](int st, auto q_c) {
    constexpr int q = decltype(q_c)::value;
    using QN = std::integral_constant<int, (q + 1) % D>;
    const int buf = st & 1;
    gload(min(st + D, nst - 1), q_c);
#pragma unroll
    for (int ks = 0; ks < KB / 16; ++ks) {
      u32x4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const u32x4*>(&sA[buf][ra0 + 32 * i * PITCH + 32 * ks]);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const u32x4*>(&sB[buf][rb0 + 32 * j * PITCH + 32 * ks]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16_32x32x16(a[i], b[j], acc[i][j]);
    }
    wait_set(QN{});     // sets q + 2 (stage st + 2) and q (stage st + 3) may still be in flight
    lstore(buf ^ 1, QN{});
    __syncthreads();
  };
  int st = 0;
  for (; st + D <= nst; st += D) {
    stage(st, Q0{});
    stage(st + 1, Q1{});
    stage(st + 2, Q2{});
  }
  if (st < nst) stage(st, Q0{});
  if (st + 1 < nst) stage(st + 1, Q1{});
  // The re-reads past the last stage are never stored: wait for them and mark every set as used
  // after the wait, so that no register of an in-flight load is handed to other values before.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int q = 0; q < D; ++q) {
#pragma unroll
    for (int i = 0; i < ALD; ++i) asm volatile("" ::"v"(ra[q][i]));
#pragma unroll
    for (int i = 0; i < BLD; ++i) asm volatile("" ::"v"(rb[q][i]), "v"(rs[q][i]));
  }
  // the last barrier passed: every wave is done with the A buffers, which now stage the output
  epilogue<OUT_F32, EPI>(p, acc, m0 + 64 * wm, n0 + 64 * wn, lr, h, &sA[0][0] + wave * 4096);
}

// W4A16 on large grids: one wave per SIMD with a TM/2 x 128 register tile (TM/64 x 4 sub-tiles of
// 32 x 32; the accumulators live in AGPRs, only MFMAs touch them before the epilogue), block tile
// TM x 256 on 4 waves, TM = 256 or 192 (launch_w4a16 picks the height that needs the fewest
// rounds of tiles over the CUs).  (Two waves per SIMD with 128 x 64 tiles measured the same or slower.)  Per 64-column stage a wave issues 64 MFMAs (2048 cycles of the SIMD's
// MFMA pipe) and, spread between them, its share of the next stage: 8 x_hat chunks and one weight
// row (64 codes dequantized as in w4a16_kernel) written to the other LDS buffer, so one instruction
// stream keeps the MFMA pipe, the VALU and the LDS busy together.  Loads run two stages ahead with
// the same exact-count asm waits; LDS rows have the 144-byte pitch of w4a16_kernel.
template <int G, bool OUT_F32, bool EPI = false, int TM = 256>
__global__ void __launch_bounds__(256, 1) w4a16_wide_kernel(GemmParams p) {
  constexpr int NT = 256, TBM = TM, TBN = 256, KB = 64;
  constexpr int RI = TBM / 64;                // 32-row sub-tiles per wave (the wave tile is TBM / 2 rows)
  static_assert(TBM == 256 || TBM == 192, "tile height");
  constexpr int PITCH = 2 * KB + 16;
  constexpr int ALD = TBM * 8 / NT;           // x_hat chunks per thread and stage (8 or 6)
  constexpr int LPS = ALD + 3;                // + two 16-byte weight loads + one scale
  constexpr int D = 2;                        // register sets (stages in flight)
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][TBM * PITCH];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][TBN * PITCH];

  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int nbm = (p.M + TBM - 1) / TBM, nbn = (p.N + TBN - 1) / TBN;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 4, bm, bn);
  const int m0 = bm * TBM, n0 = bn * TBN;
  const int K = p.K, ngroups = K / G, kp = K / 2, nst = K / KB;

  const uint16_t* arow[ALD];
  int aoff[ALD];
#pragma unroll
  for (int i = 0; i < ALD; ++i) {
    const int idx = tid + NT * i, r = idx >> 3, c = idx & 7;
    arow[i] = p.xhat + (long)min(m0 + r, p.M - 1) * p.ldxh + 8 * c;
    aoff[i] = r * PITCH + 16 * c;
  }
  const int nrow = min(n0 + tid, p.N - 1);     // weight row of this thread
  const uint8_t* brow = p.qw + (long)nrow * kp;
  const uint16_t* bsc = p.sw + (long)nrow * ngroups;
  const int boff = tid * PITCH;

  u32x4 ra[D][ALD], rb[D][2];
  uint32_t rs[D];
  auto gload_set = [&](int st, u32x4 (&da)[ALD], u32x4 (&db)[2], uint32_t& ds) {
    const int k0 = st * KB;
#pragma unroll
    for (int i = 0; i < ALD; ++i)
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(da[i]) : "v"(arow[i] + k0) : "memory");
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(db[0]) : "v"(brow + k0 / 2) : "memory");
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(db[1]) : "v"(brow + k0 / 2 + 16) : "memory");
    asm volatile("global_load_ushort %0, %1, off" : "=v"(ds) : "v"(bsc + k0 / G) : "memory");
  };
  auto gload = [&](int st, auto q_c) {
    constexpr int q = decltype(q_c)::value;
    gload_set(st, ra[q], rb[q], rs[q]);
  };
  auto wait_regs = [&](u32x4 (&da)[ALD], u32x4 (&db)[2], uint32_t& ds) {
    static_assert((D - 1) * LPS < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%c0)" ::"i"((D - 1) * LPS) : "memory");
#pragma unroll
    for (int i = 0; i < ALD; ++i) asm volatile("" : "+v"(da[i]));
    asm volatile("" : "+v"(db[0]), "+v"(db[1]), "+v"(ds));
  };
  auto wait_set = [&](auto q_c) {
    constexpr int q = decltype(q_c)::value;
    wait_regs(ra[q], rb[q], rs[q]);
  };
  // part `pt` (0..3) of a set's move to LDS buffer buf: the x_hat chunks i with i % 4 == pt (two
  // of 8, or one or two of 6) and the weight row's 16 codes of k 16 pt .. 16 pt + 15
  // (bf16(q * bf16(s)), one exact FMA per code)
  auto lstore_part = [&](int buf, auto q_c, int pt) {
    constexpr int q = decltype(q_c)::value;
#pragma unroll
    for (int i = 0; i < ALD; ++i)
      if (i % 4 == pt) *reinterpret_cast<u32x4*>(&sA[buf][aoff[i]]) = ra[q][i];
    const float sc = round_bf16(half_bits_to_float((uint16_t)rs[q])), ns8 = -8.0f * sc;
    const u32x4 w = rb[q][pt >> 1];
    uint32_t o[8];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const uint32_t v = w[2 * (pt & 1) + d];
      uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
      // opaque to the combiner, which would otherwise fold the masks into one bit-field
      // extract per code: each byte then converts with a single v_cvt_f32_ubyteN
      asm("" : "+v"(lo), "+v"(hi));
      o[4 * d + 0] = pack_bf16x2(__builtin_fmaf(ubyte_f32<0>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<0>(hi), sc, ns8));
      o[4 * d + 1] = pack_bf16x2(__builtin_fmaf(ubyte_f32<1>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<1>(hi), sc, ns8));
      o[4 * d + 2] = pack_bf16x2(__builtin_fmaf(ubyte_f32<2>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<2>(hi), sc, ns8));
      o[4 * d + 3] = pack_bf16x2(__builtin_fmaf(ubyte_f32<3>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<3>(hi), sc, ns8));
    }
    *reinterpret_cast<u32x4*>(&sB[buf][boff + 32 * pt]) = u32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<u32x4*>(&sB[buf][boff + 32 * pt + 16]) = u32x4{o[4], o[5], o[6], o[7]};
  };

  f32x16 acc[RI][4];
#pragma unroll
  for (int i = 0; i < RI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  const int ra0 = ((TBM / 2) * wm + lr) * PITCH + 16 * h, rb0 = (128 * wn + lr) * PITCH + 16 * h;
  using Q0 = std::integral_constant<int, 0>;
  using Q1 = std::integral_constant<int, 1>;
  gload(0, Q0{});
  gload(min(1, nst - 1), Q1{});
  wait_set(Q0{});
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) lstore_part(0, Q0{}, pt);
  __syncthreads();
  // stage st (LDS buffer st % 2, set q = st % D): stage st + D goes out into set q; stage st + 1
  // (set q + 1) moves to the other buffer, a quarter per k-step.
  auto stage = [&](int st, auto q_c) {
    constexpr int q = decltype(q_c)::value;
    using QN = std::integral_constant<int, (q + 1) % D>;
    const int buf = st & 1;
    gload(min(st + D, nst - 1), q_c);   // set q was moved to LDS during the previous stage
    wait_set(QN{});                      // set q + 1 landed; the D - 1 newer sets may be in flight
    // fragments of k-step ks + 1 are read while the MFMAs of k-step ks run (two register sets)
    u32x4 a[2][RI], b[2][4];
    auto read_frags = [&](int ks, u32x4 (&fa)[RI], u32x4 (&fb)[4]) {
#pragma unroll
      for (int i = 0; i < RI; ++i) fa[i] = *reinterpret_cast<const u32x4*>(&sA[buf][ra0 + 32 * i * PITCH + 32 * ks]);
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const u32x4*>(&sB[buf][rb0 + 32 * j * PITCH + 32 * ks]);
    };
    read_frags(0, a[0], b[0]);
#pragma unroll
    for (int ks = 0; ks < KB / 16; ++ks) {
      const int c = ks & 1;
      if (ks + 1 < KB / 16) read_frags(ks + 1, a[c ^ 1], b[c ^ 1]);
#pragma unroll
      for (int i = 0; i < RI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_bf16_32x32x16(a[c][i], b[c][j], acc[i][j]);
      lstore_part(buf ^ 1, QN{}, ks);
    }
    // issue order: k-step 0's reads, then per k-step the next one's reads ahead of its MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, RI + 4, 0);
#pragma unroll
    for (int ks = 0; ks < KB / 16; ++ks) {
      if (ks + 1 < KB / 16) __builtin_amdgcn_sched_group_barrier(0x100, RI + 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, RI * 4, 0);
    }
    __syncthreads();
  };
  int st = 0;
  for (; st + D <= nst; st += D) {
    stage(st, Q0{});
    stage(st + 1, Q1{});
  }
  if (st < nst) stage(st, Q0{});
  // the re-reads past the last stage are never stored: wait for them and mark every set used
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int q = 0; q < D; ++q) {
#pragma unroll
    for (int i = 0; i < ALD; ++i) asm volatile("" ::"v"(ra[q][i]));
    asm volatile("" ::"v"(rb[q][0]), "v"(rb[q][1]), "v"(rs[q]));
  }
  // epilogue per 64 x 64 quadrant of the wave tile (the A buffers stage the output); with three
  // row sub-tiles (TM = 192) the last quadrant holds one, and its other 32 rows (the next wave's)
  // are not stored
  const int wrow = m0 + (TBM / 2) * wm, wend = wrow + TBM / 2;
  if constexpr (EPI) {
    // written out per quadrant: with the fused op the unrolled loop below is too large for the
    // unroller, and a rolled loop would index the accumulators at run time (scratch)
    auto quadrant = [&](auto qi_c, auto qj_c) {
      constexpr int qi = decltype(qi_c)::value, qj = decltype(qj_c)::value;
      constexpr int i1 = 2 * qi + 1 < RI ? 2 * qi + 1 : 2 * qi;
      f32x16 part[2][2] = {{acc[2 * qi][2 * qj], acc[2 * qi][2 * qj + 1]}, {acc[i1][2 * qj], acc[i1][2 * qj + 1]}};
      epilogue<OUT_F32, EPI>(p, part, wrow + 64 * qi, n0 + 128 * wn + 64 * qj, lr, h, &sA[0][0] + wave * 4096,
                             nullptr, nullptr, 0, 0, wend);
    };
    quadrant(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    quadrant(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
    quadrant(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
    quadrant(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
  } else {
#pragma unroll
    for (int qi = 0; qi < (RI + 1) / 2; ++qi)
#pragma unroll
      for (int qj = 0; qj < 2; ++qj) {
        const int i1 = 2 * qi + 1 < RI ? 2 * qi + 1 : 2 * qi;   // the half quadrant repeats its sub-tile
        f32x16 part[2][2] = {{acc[2 * qi][2 * qj], acc[2 * qi][2 * qj + 1]}, {acc[i1][2 * qj], acc[i1][2 * qj + 1]}};
        epilogue<OUT_F32>(p, part, wrow + 64 * qi, n0 + 128 * wn + 64 * qj, lr, h, &sA[0][0] + wave * 4096,
                          nullptr, nullptr, 0, 0, wend);
      }
  }
}

// W4A16 GEMM with specialized waves (group 64 or 128, no fused op; the 192-row tiles of
// w4a16_wide_kernel, with the same per-output arithmetic, so bit-identical outputs).  In one wave
// the dequantization's VALU work and the MFMAs share the issue slots badly; here waves 0-3 only read
// fragments and issue MFMAs (wave tile 96 x 128 of the 192 x 256 block tile, as in
// w4a16_wide_kernel) and waves 4-7 only stage the next k-step block: x_hat by DMA into a swizzled
// A tile (16-byte chunk c of row r at c ^ ((r >> 1) & 7), so a ds_read_b128 phase of 16 rows hits
// 16 distinct bank groups), the weight codes loaded two stages ahead and dequantized into the B
// tile (rows of 144 bytes).  One wave of each kind per SIMD; one barrier per 64-column stage.
// The low-rank term runs as RTp / 32 more stages through the same MFMAs (A = the mid planes
// [hi_2e | lo_2e | hi_2e+1 | lo_2e+1], B = [l1_2e | l1_2e | l1_2e+1 | l1_2e+1]), so each accumulator
// takes hi_k then lo_k as in the epilogue's low-rank MFMAs, and the epilogue only adds the bias and
// stores (the 192 accumulators leave no room for its operands).
template <int G, bool OUT_F32>
__device__ __forceinline__ void w4a16_ws_tile(const GemmParams& p, int bm, int bn) {
  constexpr int NT = 256, TBM = 192, TBN = 256, KB = 64, RI = TBM / 64;
  constexpr int PITCH = 2 * KB + 16;
  constexpr int ALD = TBM * 8 / NT;            // x_hat DMA instructions per producer wave and stage
  constexpr int D = 2;                         // register sets of weight codes (stages in flight)
  constexpr int ABUF = TBM * 128;
  __shared__ __attribute__((aligned(1024))) uint8_t sA[2][ABUF];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][TBN * PITCH];

  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m0 = bm * TBM, n0 = bn * TBN;
  const int K = p.K, ngroups = K / G, kp = K / 2, nst = K / KB;
  // the low-rank term mid @ l1cat^T as RTp / 32 more stages: A rows [hi_2e | lo_2e | hi_2e+1 |
  // lo_2e+1] (16 columns each) of the mid planes, B rows [l1_2e | l1_2e | l1_2e+1 | l1_2e+1], so each
  // accumulator takes hi_k then lo_k for k = 0, 1, .. as in the epilogue's low-rank MFMAs
  const int RTp = p.RTp, nall = nst + RTp / 32;
  using Q0 = std::integral_constant<int, 0>;
  using Q1 = std::integral_constant<int, 1>;

  // The role is wave-uniform, and both roles pass the same barriers: one after the first stage is
  // staged, then one per stage (the staging waves leave after the last; the epilogue has none).
  if (wave >= 4) {
    // ---- producer ----
    const int ptid = tid - NT, pw = wave - 4;
    // x_hat DMA: instruction t (6 per wave: t = 6 pw + i) moves rows 8 t .. 8 t + 7; lane -> row
    // 8 t + lane / 8, LDS position lane % 8 holding chunk (lane % 8) ^ ((row >> 1) & 7).  The
    // per-lane offsets are 32-bit: the launcher takes this kernel only where (M - 1) * ldxh * 2
    // and M * 4 * RTp (the mid planes of the low-rank stages) stay below 2^32.
    const int rr = lane >> 3, jj = lane & 7;
    const long ldb = p.ldxh * 2;
    uint32_t aoffs[ALD];
#pragma unroll
    for (int i = 0; i < ALD; ++i) {
      const int row = 8 * (ALD * pw + i) + rr;
      aoffs[i] = (uint32_t)(min(m0 + row, p.M - 1) * ldb + 16 * (jj ^ ((row >> 1) & 7)));
    }
    const uint32_t ldsA0 = lds_offset(&sA[0][0]);
    const uint8_t* xb = reinterpret_cast<const uint8_t*>(p.xhat);
    auto dma_a = [&](int st, int buf) {
#pragma unroll
      for (int i = 0; i < ALD; ++i) dma16(xb + 2 * st * KB, aoffs[i], ldsA0 + buf * ABUF + (ALD * pw + i) * 1024);
    };
    const int nrow = min(n0 + ptid, p.N - 1);
    const uint8_t* brow = p.qw + (long)nrow * kp;
    const uint16_t* bsc = p.sw + (long)nrow * ngroups;
    const int boff = ptid * PITCH;
    u32x4 rb[D][2];
    uint32_t rs[D];
    constexpr int CL = 3;   // loads per set: two 16-byte code loads and the scale
    auto gload_set = [&](int st, u32x4 (&db)[2], uint32_t& ds) {
      const int k0 = st * KB;
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(db[0]) : "v"(brow + k0 / 2) : "memory");
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(db[1]) : "v"(brow + k0 / 2 + 16) : "memory");
      asm volatile("global_load_ushort %0, %1, off" : "=v"(ds) : "v"(bsc + k0 / G) : "memory");
    };
    auto gload = [&](int st, auto q_c) {
      constexpr int q = decltype(q_c)::value;
      gload_set(st, rb[q], rs[q]);
    };
    auto mark_regs = [&](u32x4 (&db)[2], uint32_t& ds) { asm volatile("" : "+v"(db[0]), "+v"(db[1]), "+v"(ds)); };
    auto mark_set = [&](auto q_c) {
      constexpr int q = decltype(q_c)::value;
      mark_regs(rb[q], rs[q]);
    };
    auto lstore_part = [&](int buf, auto q_c, int pt) {
      constexpr int q = decltype(q_c)::value;
      const float sc = round_bf16(half_bits_to_float((uint16_t)rs[q])), ns8 = -8.0f * sc;
      const u32x4 w = rb[q][pt >> 1];
      uint32_t o[8];
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const uint32_t v = w[2 * (pt & 1) + d];
        uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
        asm("" : "+v"(lo), "+v"(hi));
        o[4 * d + 0] = pack_bf16x2(__builtin_fmaf(ubyte_f32<0>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<0>(hi), sc, ns8));
        o[4 * d + 1] = pack_bf16x2(__builtin_fmaf(ubyte_f32<1>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<1>(hi), sc, ns8));
        o[4 * d + 2] = pack_bf16x2(__builtin_fmaf(ubyte_f32<2>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<2>(hi), sc, ns8));
        o[4 * d + 3] = pack_bf16x2(__builtin_fmaf(ubyte_f32<3>(lo), sc, ns8), __builtin_fmaf(ubyte_f32<3>(hi), sc, ns8));
      }
      *reinterpret_cast<u32x4*>(&sB[buf][boff + 32 * pt]) = u32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<u32x4*>(&sB[buf][boff + 32 * pt + 16]) = u32x4{o[4], o[5], o[6], o[7]};
    };
    dma_a(0, 0);
    gload(0, Q0{});
    gload(min(1, nst - 1), Q1{});
    asm volatile("s_waitcnt vmcnt(%c0)" ::"i"(CL) : "memory");   // x_hat and codes of stage 0
    mark_set(Q0{});
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) lstore_part(0, Q0{}, pt);
    __syncthreads();
    auto xstage = [&](int e, int buf) {
      const uint8_t* mb = reinterpret_cast<const uint8_t*>(p.midp);
#pragma unroll
      for (int i = 0; i < ALD; ++i) {
        const int row = 8 * (ALD * pw + i) + rr, c = jj ^ ((row >> 1) & 7), s4 = c >> 1;
        const int col = 16 * (2 * e + (s4 >> 1)) + 8 * (c & 1);
        const uint32_t off = (uint32_t)((long)min(m0 + row, p.M - 1) * (4 * RTp) + (s4 & 1) * (2 * RTp) + 2 * col);
        dma16(mb, off, ldsA0 + buf * ABUF + (ALD * pw + i) * 1024);
      }
      u32x4 vb[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        vb[q] = *reinterpret_cast<const u32x4*>(p.l1cat + (long)nrow * RTp + 16 * (2 * e + (q >> 1)) + 8 * (q & 1));
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) {
        *reinterpret_cast<u32x4*>(&sB[buf][boff + 32 * pt]) = vb[2 * (pt >> 1)];
        *reinterpret_cast<u32x4*>(&sB[buf][boff + 32 * pt + 16]) = vb[2 * (pt >> 1) + 1];
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    auto pstage = [&](int st, auto q_c) {
      using QN = std::integral_constant<int, (decltype(q_c)::value + 1) % D>;
      const int buf = st & 1;
      if (st + 1 < nst) {
        // stage st + 1: x_hat by DMA, codes from set q + 1 (loaded during stage st - 1); stage
        // st + 2's codes into set q
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        mark_set(QN{});
        dma_a(st + 1, buf ^ 1);
        gload(min(st + D, nst - 1), q_c);
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) lstore_part(buf ^ 1, QN{}, pt);
        asm volatile("s_waitcnt vmcnt(%c0)" ::"i"(CL) : "memory");   // the x_hat DMA landed
      } else if (st + 1 < nall) {
        xstage(st + 1 - nst, buf ^ 1);
      }
      __syncthreads();
    };
    int st = 0;
    for (; st + D <= nall; st += D) {
      pstage(st, Q0{});
      pstage(st + 1, Q1{});
    }
    if (st < nall) pstage(st, Q0{});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int q = 0; q < D; ++q) asm volatile("" ::"v"(rb[q][0]), "v"(rb[q][1]), "v"(rs[q]));
    return;
  }

  // ---- consumer (issues ahead of the producer on its SIMD) ----
  __builtin_amdgcn_s_setprio(1);
  const int wm = wave >> 1, wn = wave & 1;
  f32x16 acc[RI][4];
#pragma unroll
  for (int i = 0; i < RI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  const int r0 = (TBM / 2) * wm + lr, swz = (r0 >> 1) & 7;
  const int rb0 = (128 * wn + lr) * PITCH + 16 * h;
  __syncthreads();
  auto cstage = [&](int st) {
    const int buf = st & 1;
    // units u = 4 ks + j: the 3 MFMAs of B fragment j of k-step ks (one B register set in use, so
    // the 192 accumulators fit); the next unit's B fragment and the next k-step's A fragments are
    // read while a unit's MFMAs run
    u32x4 a[2][RI], b[2];
    auto read_a = [&](int ks, u32x4 (&fa)[RI]) {
#pragma unroll
      for (int i = 0; i < RI; ++i) fa[i] = *reinterpret_cast<const u32x4*>(&sA[buf][r0 * 128 + 4096 * i + 16 * ((2 * ks + h) ^ swz)]);
    };
    auto read_b = [&](int u, u32x4& fb) {
      fb = *reinterpret_cast<const u32x4*>(&sB[buf][rb0 + 32 * (u & 3) * PITCH + 32 * (u >> 2)]);
    };
    read_a(0, a[0]);
    read_b(0, b[0]);
#pragma unroll
    for (int u = 0; u < 4 * (KB / 16); ++u) {
      const int ks = u >> 2, j = u & 3;
      if (u + 1 < 4 * (KB / 16)) read_b(u + 1, b[(u + 1) & 1]);
      if (j == 0 && ks + 1 < KB / 16) read_a(ks + 1, a[(ks + 1) & 1]);
#pragma unroll
      for (int i = 0; i < RI; ++i) acc[i][j] = mfma_bf16_32x32x16(a[ks & 1][i], b[u & 1], acc[i][j]);
    }
    __syncthreads();
  };
  for (int st = 0; st < nall; ++st) cstage(st);
  GemmParams pe = p;   // the low-rank term is in the accumulators: bias and store only
  pe.RTp = 0;
  const int wrow = m0 + (TBM / 2) * wm, wend = wrow + TBM / 2;
#pragma unroll
  for (int qi = 0; qi < (RI + 1) / 2; ++qi)
#pragma unroll
    for (int qj = 0; qj < 2; ++qj) {
      const int i1 = 2 * qi + 1 < RI ? 2 * qi + 1 : 2 * qi;
      f32x16 part[2][2] = {{acc[2 * qi][2 * qj], acc[2 * qi][2 * qj + 1]}, {acc[i1][2 * qj], acc[i1][2 * qj + 1]}};
      epilogue<OUT_F32>(pe, part, wrow + 64 * qi, n0 + 128 * wn + 64 * qj, lr, h, &sA[0][0] + wave * 4096,
                        nullptr, nullptr, 0, 0, wend);
    }
}

template <int G, bool OUT_F32>
__global__ void __launch_bounds__(512, 1) w4a16_ws_kernel(GemmParams p) {
  const int nbm = (p.M + 191) / 192, nbn = (p.N + 255) / 256;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 4, bm, bn);
  w4a16_ws_tile<G, OUT_F32>(p, bm, bn);
}

// Sibling layers (same rows M, same K and group, each with its own x_hat) in one launch on the
// 192 x 256 tiles: numbered back to back (layer i from tile0[i]) and spread over the XCDs as in
// w4a4_e3m2_siblings_kernel; each workgroup runs one tile of one layer, so every output is
// bit-identical to a launch per layer.
template <int G, bool OUT_F32>
__global__ void __launch_bounds__(512, 1) w4a16_ws_siblings_kernel(GemmSiblings gs) {
  const int total = gs.tile0[gs.count];
  int lin = blockIdx.x;
  if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
  int i = 0;
#pragma unroll
  for (int c = 1; c < MAX_SIBLINGS; ++c) i += (c < gs.count && lin >= gs.tile0[c]) ? 1 : 0;
  i = __builtin_amdgcn_readfirstlane(i);
  const GemmParams& p = gs.layer[i];
  int bm, bn;
  tile_of_linear(lin - gs.tile0[i], (p.M + 191) / 192, (p.N + 255) / 256, 4, bm, bn);
  w4a16_ws_tile<G, OUT_F32>(p, bm, bn);
}

// W4A4 GEMM for group sizes other than 64 / 128 (any multiple of 16 dividing K): the generic path.
// Operands are the int8 codes 16 q (SVDQ_OPERAND_I8 layout: within each chunk of 8 columns the even
// columns, then the odd ones, identically for activations and weights, so the order cancels).  K
// advances 16 columns per v_mfma_i32_32x32x16_i8 (lanes 0-31 supply one 8-column chunk of a row,
// lanes 32-63 the next), accumulating the exact group sum P in int32; at every group boundary
// acc += f32(P) * S with S = sx (x) sw on a bf16 MFMA (K = 2: (sx, sx) against (hi, lo) of sw, the
// 1/256 of the int8 operands folded into the weight pair as in the fast kernels) and P is reset.
// Block tile 128 x 128 on 4 waves (wave tile 64 x 64), 64-column stages through LDS (rows padded
// to 80 bytes), one stage at a time.
template <bool OUT_F32>
__global__ void __launch_bounds__(256, 2) w4a4_any_group_kernel(GemmParams p, int G) {
  constexpr int TBM = 128, TBN = 128, KB = 64, PITCH = KB + 16;
  // one buffer: the two operand tiles during the main loop (20 KB), then 4 KB of output staging
  // per wave (16 KB) in the epilogue
  constexpr int LDS_BYTES = (TBM + TBN) * PITCH;
  static_assert(LDS_BYTES >= 4 * 4096, "epilogue staging");
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
  uint8_t* sA = lds;
  uint8_t* sB = lds + TBM * PITCH;
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int nbm = (p.M + TBM - 1) / TBM, nbn = (p.N + TBN - 1) / TBN;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 4, bm, bn);
  const int m0 = bm * TBM, n0 = bn * TBN;
  const int K = p.K;
  f32x16 acc[2][2];
  i32x16 P[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc[i][j] = f32x16{};
      P[i][j] = i32x16{};
    }
  for (int k0 = 0; k0 < K; k0 += KB) {
    // stage: 128 rows x 64 bytes of each operand, 16 bytes per thread and operand, twice
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int idx = tid + 256 * it, r = idx >> 2, c = idx & 3;
      *reinterpret_cast<u32x4*>(&sA[r * PITCH + 16 * c]) =
          ld16(p.qa + (long)min(m0 + r, p.M - 1) * K + k0 + 16 * c);
      *reinterpret_cast<u32x4*>(&sB[r * PITCH + 16 * c]) =
          ld16(p.qwe + (long)min(n0 + r, p.N - 1) * K + k0 + 16 * c);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < KB / 16; ++kk) {
      long a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const long*>(&sA[(64 * wm + 32 * i + lr) * PITCH + 16 * kk + 8 * h]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const long*>(&sB[(64 * wn + 32 * j + lr) * PITCH + 16 * kk + 8 * h]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) P[i][j] = __builtin_amdgcn_mfma_i32_32x32x16_i8(a[i], b[j], P[i][j], 0, 0, 0);
      const int kend = k0 + 16 * kk + 16;
      if (kend % G == 0) {   // group boundary: rescale the exact group sums into acc
        const int g = kend / G - 1;
        u32x4 xop[2], wop[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int m = min(m0 + 64 * wm + 32 * i + lr, p.M - 1);
          xop[i] = u32x4{h ? 0u : p.sxp[(long)g * p.M + m], 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = min(n0 + 64 * wn + 32 * j + lr, p.N - 1);
          wop[j] = u32x4{h ? 0u : p.swp[(long)g * p.N + n], 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const f32x16 S = mfma_bf16_32x32x16(xop[i], wop[j], f32x16{});
            const f32x16 pf = __builtin_convertvector(P[i][j], f32x16);
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(pf[r], S[r], acc[i][j][r]);
            P[i][j] = i32x16{};
          }
      }
    }
    __syncthreads();
  }
  // the operand buffers stage the output (4 KB per wave; the last barrier above ended their use)
  epilogue<OUT_F32>(p, acc, m0 + 64 * wm, n0 + 64 * wn, lr, h, lds + wave * 4096);
}

}  // namespace

bool use_wide_tiles(int M, int N, int K) {
  if (!wide_tiles_apply(M, N, K)) return false;
  const int o = tile_override();
  if (o) return o == 2;
  const long bm = M / 256;
  return wide_tiles_pay(bm * (N / 256), bm * (N / 128));
}

hipError_t launch_w4a4_any_group(const GemmParams& p, int G, bool out_f32, hipStream_t st) {
  if (G <= 0 || G % 16 || p.K % G || p.K % 64) return hipErrorInvalidValue;
  const dim3 grid(((p.M + 127) / 128) * ((p.N + 127) / 128));
  if (out_f32) w4a4_any_group_kernel<true><<<grid, 256, 0, st>>>(p, G);
  else w4a4_any_group_kernel<false><<<grid, 256, 0, st>>>(p, G);
  return hipGetLastError();
}

hipError_t launch_w4a4(const GemmParams& p, int G, int mode, bool out_f32, hipStream_t st) {
  const dim3 grid(((p.M + 255) / 256) * ((p.N + 127) / 128));
#define SVDQ_W4A4_KERNEL w4a4_kernel
#define SVDQ_W4A4(GG, MM)                                                        \
  if (G == GG && mode == MM) {                                                   \
    if (out_f32) SVDQ_W4A4_KERNEL<GG, MM, true><<<grid, 512, 0, st>>>(p);         \
    else if (p.epi) SVDQ_W4A4_KERNEL<GG, MM, false, true><<<grid, 512, 0, st>>>(p); \
    else SVDQ_W4A4_KERNEL<GG, MM, false><<<grid, 512, 0, st>>>(p);                \
    return hipGetLastError();                                                    \
  }
  SVDQ_W4A4(64, 0)
  SVDQ_W4A4(128, 0)
  SVDQ_W4A4(64, 1)
  SVDQ_W4A4(128, 1)
#undef SVDQ_W4A4
  if (mode == 2) {
    if (G == 64 && !p.epi && use_wide_tiles(p.M, p.N, p.K)) {
      const dim3 wgrid((unsigned)(((p.M + 255) / 256) * ((p.N + 255) / 256)));
      // ranks 64 .. 256 (LoRA adapters, larger SVD ranks): the low-rank term in LDS chunks
      const bool ch = p.RTp > 32 && p.RTp <= 256 && p.RTp % 32 == 0;
      if (ch) {
        if (out_f32) w4a4_e3m2_wide_kernel<true, true><<<wgrid, 512, 0, st>>>(p);
        else w4a4_e3m2_wide_kernel<false, true><<<wgrid, 512, 0, st>>>(p);
      } else {
        if (out_f32) w4a4_e3m2_wide_kernel<true><<<wgrid, 512, 0, st>>>(p);
        else w4a4_e3m2_wide_kernel<false><<<wgrid, 512, 0, st>>>(p);
      }
      return hipGetLastError();
    }
    const bool full = p.K % 512 == 0;   // two full 256-column stages per main-loop iteration
    // ranks 64 .. 256 without store ops: the low-rank term in LDS chunks
    const bool ch = !p.epi && p.RTp > 32 && p.RTp <= 256 && p.RTp % 32 == 0;
#define SVDQ_E3M2(GG)                                                                  \
  if (G == GG) {                                                                       \
    if (ch) {                                                                          \
      if (full) {                                                                      \
        if (out_f32) w4a4_e3m2_kernel<GG, true, true, false, true><<<grid, 512, 0, st>>>(p);   \
        else w4a4_e3m2_kernel<GG, false, true, false, true><<<grid, 512, 0, st>>>(p);          \
      } else {                                                                         \
        if (out_f32) w4a4_e3m2_kernel<GG, true, false, false, true><<<grid, 512, 0, st>>>(p);  \
        else w4a4_e3m2_kernel<GG, false, false, false, true><<<grid, 512, 0, st>>>(p);         \
      }                                                                                \
    } else if (full) {                                                                 \
      if (out_f32) w4a4_e3m2_kernel<GG, true, true><<<grid, 512, 0, st>>>(p);           \
      else if (p.epi) w4a4_e3m2_kernel<GG, false, true, true><<<grid, 512, 0, st>>>(p); \
      else w4a4_e3m2_kernel<GG, false, true><<<grid, 512, 0, st>>>(p);                  \
    } else {                                                                           \
      if (out_f32) w4a4_e3m2_kernel<GG, true, false><<<grid, 512, 0, st>>>(p);          \
      else if (p.epi) w4a4_e3m2_kernel<GG, false, false, true><<<grid, 512, 0, st>>>(p); \
      else w4a4_e3m2_kernel<GG, false, false><<<grid, 512, 0, st>>>(p);                 \
    }                                                                                  \
    return hipGetLastError();                                                          \
  }
    SVDQ_E3M2(64)
    SVDQ_E3M2(128)
#undef SVDQ_E3M2
  }
  return hipErrorInvalidValue;
}

hipError_t launch_w4a4_siblings(const GemmSiblings& gs, int G, bool out_f32, hipStream_t st) {
  if (gs.count < 1 || gs.count > MAX_SIBLINGS) return hipErrorInvalidValue;
  const int K = gs.layer[0].K, M = gs.layer[0].M;
  int tiles = 0;
  for (int i = 0; i < gs.count; ++i) {
    const GemmParams& p = gs.layer[i];
    if (p.K != K || p.M != M || p.epi || gs.tile0[i] != tiles) return hipErrorInvalidValue;
    tiles += ((p.M + 255) / 256) * ((p.N + 127) / 128);
  }
  if (gs.tile0[gs.count] != tiles || K % 512) return hipErrorInvalidValue;
  // a layer of rank 64 .. 256: every layer's low-rank term in LDS chunks (rank 32 in one chunk)
  bool ch = false, ch_ok = true;
  for (int i = 0; i < gs.count; ++i) {
    const int r = gs.layer[i].RTp;
    ch = ch || r > 32;
    ch_ok = ch_ok && r > 0 && r <= 256 && r % 32 == 0;
  }
  ch = ch && ch_ok;
  if (G == 64) {
    // the wide tiles when every layer takes them and they pay over the whole launch
    bool apply = true;
    long wide = 0;
    for (int i = 0; i < gs.count; ++i) {
      apply = apply && wide_tiles_apply(M, gs.layer[i].N, K);
      wide += (long)(M / 256) * (gs.layer[i].N / 256);
    }
    const int o = tile_override();
    if (apply && (o ? o == 2 : wide_tiles_pay(wide, tiles))) {
      GemmSiblings w = gs;
      int t = 0;
      for (int i = 0; i < gs.count; ++i) {
        w.tile0[i] = t;
        t += (M / 256) * (gs.layer[i].N / 256);
      }
      w.tile0[gs.count] = t;
      if (ch) {
        if (out_f32) w4a4_e3m2_wide_siblings_kernel<true, true><<<dim3((unsigned)t), 512, 0, st>>>(w);
        else w4a4_e3m2_wide_siblings_kernel<false, true><<<dim3((unsigned)t), 512, 0, st>>>(w);
      } else {
        if (out_f32) w4a4_e3m2_wide_siblings_kernel<true><<<dim3((unsigned)t), 512, 0, st>>>(w);
        else w4a4_e3m2_wide_siblings_kernel<false><<<dim3((unsigned)t), 512, 0, st>>>(w);
      }
      return hipGetLastError();
    }
  }
  const dim3 grid((unsigned)tiles);
  if (G == 64 && ch) {
    if (out_f32) w4a4_e3m2_siblings_kernel<64, true, true><<<grid, 512, 0, st>>>(gs);
    else w4a4_e3m2_siblings_kernel<64, false, true><<<grid, 512, 0, st>>>(gs);
  } else if (G == 64) {
    if (out_f32) w4a4_e3m2_siblings_kernel<64, true><<<grid, 512, 0, st>>>(gs);
    else w4a4_e3m2_siblings_kernel<64, false><<<grid, 512, 0, st>>>(gs);
  } else if (G == 128 && ch) {
    if (out_f32) w4a4_e3m2_siblings_kernel<128, true, true><<<grid, 512, 0, st>>>(gs);
    else w4a4_e3m2_siblings_kernel<128, false, true><<<grid, 512, 0, st>>>(gs);
  } else if (G == 128) {
    if (out_f32) w4a4_e3m2_siblings_kernel<128, true><<<grid, 512, 0, st>>>(gs);
    else w4a4_e3m2_siblings_kernel<128, false><<<grid, 512, 0, st>>>(gs);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gate_op(int op, const uint16_t* y, const uint16_t* aux, uint16_t* out, long n, hipStream_t st) {
  const long blocks = std::max<long>(1, std::min<long>((n / 8 + 255) / 256, 4096));
  if (op == 1) gate_op_kernel<1><<<(unsigned)blocks, 256, 0, st>>>(y, aux, out, n);
  else if (op == 2) gate_op_kernel<2><<<(unsigned)blocks, 256, 0, st>>>(y, aux, out, n);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_weight_scale_pairs(const uint16_t* sw, uint32_t* out, int n, int ngroups, int mode, hipStream_t st) {
  const long blocks = std::min<long>(((long)n * ngroups + 255) / 256, 8192);
  // int8 operands are 16 q on both sides: 1/256 folded into the weight scale
  weight_scale_pairs_kernel<<<(unsigned)blocks, 256, 0, st>>>(sw, out, n, ngroups, mode == 1 ? 1.0f / 256.0f : 1.0f);
  return hipGetLastError();
}

hipError_t launch_weight_operand(const uint8_t* qw, uint8_t* qwe, int N, int K, int mode, hipStream_t st) {
  if (mode == 2) {
    const long total = (long)N * (K / 64) * 2;
    const long blocks = std::min<long>((total + 255) / 256, 8192);
    weight_operand_e3m2_kernel<<<(unsigned)blocks, 256, 0, st>>>(qw, qwe, N, (N + 1) & ~1, K);
    return hipGetLastError();
  }
  const long ndwords = (long)N * (K / 8);
  const long blocks = std::min<long>((ndwords + 255) / 256, 8192);
  weight_operand_kernel<<<(unsigned)blocks, 256, 0, st>>>(reinterpret_cast<const uint32_t*>(qw),
                                                          reinterpret_cast<u32x2*>(qwe), ndwords, mode);
  return hipGetLastError();
}

// The specialized-wave kernel takes a layer without a fused op whose x_hat rows are 16-byte
// aligned and whose DMA offsets fit 32 bits, unless SVDQ_W4A16_KERNEL=wide.
bool w4a16_ws_fits(const GemmParams& p) {
  const char* ke = getenv("SVDQ_W4A16_KERNEL");
  const bool xa = (reinterpret_cast<uintptr_t>(p.xhat) & 15) == 0 && p.ldxh % 8 == 0;
  const bool off32 = ((long)p.M - 1) * p.ldxh * 2 + 128 <= 0xFFFFFFFFL && (long)p.M * 4 * p.RTp <= 0xFFFFFFFFL;
  return !p.epi && xa && off32 && !(ke && !strcmp(ke, "wide"));
}

// Sibling layers on one launch of 192 x 256 tiles pay when their rounds over the 256 CUs cost no
// more than the layers' own launches.  Cost of a round = its tile height in rows (time per tile at
// a given K grows with the rows: 142 / 187 us for 192 / 256 rows at K = 6144); the 128 x 128
// kernel's rounds (one 4-wave workgroup per CU) count 110, its measured 82 us against 142.
bool w4a16_siblings_pay(const GemmSiblings& gs) {
  long own = 0, t192 = 0;
  for (int i = 0; i < gs.count; ++i) {
    const GemmParams& p = gs.layer[i];
    const long nb256 = (p.N + 255) / 256, tw = (long)((p.M + 255) / 256) * nb256;
    const long t = (long)((p.M + 191) / 192) * nb256;
    t192 += t;
    if (tw >= 128) own += std::min((t + 255) / 256 * 192, (tw + 255) / 256 * 256);
    else own += ((long)((p.M + 127) / 128) * ((p.N + 127) / 128) + 255) / 256 * 110;
  }
  return (t192 + 255) / 256 * 192 <= own;
}

hipError_t launch_w4a16_siblings(const GemmSiblings& gs, int G, bool out_f32, hipStream_t st) {
  if (gs.count < 1 || gs.count > MAX_SIBLINGS || (G != 64 && G != 128)) return hipErrorInvalidValue;
  const int M = gs.layer[0].M, K = gs.layer[0].K;
  int tiles = 0;
  for (int i = 0; i < gs.count; ++i) {
    const GemmParams& p = gs.layer[i];
    if (p.M != M || p.K != K || gs.tile0[i] != tiles || !w4a16_ws_fits(p)) return hipErrorInvalidValue;
    tiles += ((M + 191) / 192) * ((p.N + 255) / 256);
  }
  if (gs.tile0[gs.count] != tiles) return hipErrorInvalidValue;
  const dim3 grid((unsigned)tiles);
  if (G == 64) {
    if (out_f32) w4a16_ws_siblings_kernel<64, true><<<grid, 512, 0, st>>>(gs);
    else w4a16_ws_siblings_kernel<64, false><<<grid, 512, 0, st>>>(gs);
  } else {
    if (out_f32) w4a16_ws_siblings_kernel<128, true><<<grid, 512, 0, st>>>(gs);
    else w4a16_ws_siblings_kernel<128, false><<<grid, 512, 0, st>>>(gs);
  }
  return hipGetLastError();
}

hipError_t launch_w4a16(const GemmParams& p, int G, bool out_f32, hipStream_t st) {
  if (G != 64 && G != 128) {
    // other group sizes (multiples of 16 dividing K): the 128 x 128 kernel with a run-time group
    if (G <= 0 || G % 16 || p.K % G || p.K % 64) return hipErrorInvalidValue;
    GemmParams q = p;
    q.group = G;
    const dim3 grid(((p.M + 127) / 128) * ((p.N + 127) / 128));
    if (out_f32) w4a16_kernel<0, 2, true><<<grid, 256, 0, st>>>(q);
    else if (p.epi) w4a16_kernel<0, 2, false, true><<<grid, 256, 0, st>>>(q);
    else w4a16_kernel<0, 2, false><<<grid, 256, 0, st>>>(q);
    return hipGetLastError();
  }
  // 256 x 256 tiles (one wave per SIMD) when they cover the chip at least half, else 128 x 128
  // tiles (two workgroups of 4 waves per CU)
  const long nbn = (p.N + 255) / 256;
  const long tiles_wide = (long)((p.M + 255) / 256) * nbn;
  if (tiles_wide >= 128) {
    // tile height 256 or 192: the one with the least work per CU, rounds of tiles x tile rows (a
    // round = one tile on each of the 256 CUs); e.g. M = 2304, N = 16384: 576 tiles of 256 rows
    // need 3 rounds (the last a quarter full), 768 tiles of 192 rows 3 full rounds
    const long tiles192 = (long)((p.M + 191) / 192) * nbn;
    const bool t192 = ((tiles192 + 255) / 256) * 192 < ((tiles_wide + 255) / 256) * 256;
#define SVDQ_W4A16W(GG, TT)                                                                 \
  if (G == GG) {                                                                            \
    const dim3 grid((unsigned)(TT == 192 ? tiles192 : tiles_wide));                         \
    if (out_f32) w4a16_wide_kernel<GG, true, false, TT><<<grid, 256, 0, st>>>(p);           \
    else if (p.epi) w4a16_wide_kernel<GG, false, true, TT><<<grid, 256, 0, st>>>(p);        \
    else w4a16_wide_kernel<GG, false, false, TT><<<grid, 256, 0, st>>>(p);                  \
    return hipGetLastError();                                                               \
  }
    // the 192-row tiles on specialized waves (w4a16_ws_kernel; its x_hat DMA moves 16-byte chunks:
    // rows 16-byte aligned) unless SVDQ_W4A16_KERNEL=wide.  Its DMA addresses a row by a 32-bit
    // byte offset from the x_hat base (row * ldxh * 2) and from the mid planes' (row * 4 * RTp):
    // larger operands take the register-staged kernel, which addresses rows in 64 bits.
    if (t192 && w4a16_ws_fits(p)) {
      const dim3 grid((unsigned)tiles192);
      if (G == 64) {
        if (out_f32) w4a16_ws_kernel<64, true><<<grid, 512, 0, st>>>(p);
        else w4a16_ws_kernel<64, false><<<grid, 512, 0, st>>>(p);
        return hipGetLastError();
      }
      if (G == 128) {
        if (out_f32) w4a16_ws_kernel<128, true><<<grid, 512, 0, st>>>(p);
        else w4a16_ws_kernel<128, false><<<grid, 512, 0, st>>>(p);
        return hipGetLastError();
      }
    }
    if (t192) {
      SVDQ_W4A16W(64, 192)
      SVDQ_W4A16W(128, 192)
    } else {
      SVDQ_W4A16W(64, 256)
      SVDQ_W4A16W(128, 256)
    }
#undef SVDQ_W4A16W
    return hipErrorInvalidValue;
  }
  const dim3 grid(((p.M + 127) / 128) * ((p.N + 127) / 128));
#define SVDQ_W4A16(GG)                                                                     \
  if (G == GG) {                                                                          \
    if (out_f32) w4a16_kernel<GG, 2, true><<<grid, 256, 0, st>>>(p);                       \
    else if (p.epi) w4a16_kernel<GG, 2, false, true><<<grid, 256, 0, st>>>(p);             \
    else w4a16_kernel<GG, 2, false><<<grid, 256, 0, st>>>(p);                              \
    return hipGetLastError();                                                             \
  }
  SVDQ_W4A16(64)
  SVDQ_W4A16(128)
#undef SVDQ_W4A16
  return hipErrorInvalidValue;
}

}  // namespace svdq
