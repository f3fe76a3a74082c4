// W4A4 and W4A16 SVDQuant GEMMs for gfx950 with the low-rank / LoRA / bias epilogue.
//
// W4A4 (replaces the residual GEMM of quant/svd.py:158 with activation codes, and the
// low-rank add of kernels/triton/generic_int4.py:84-133):
//   y[m,n] = sum_g sx[m,g] sw[n,g] sum_{k in g} qx[m,k] qw[n,k]      (INT8 MFMA, exact int32
//            per group, rescaled into an fp32 accumulator)
//          + mid[m,:] . l1cat[n,:]  + bias[n]                       (bf16 MFMA, mid split
//                                                                    into bf16 hi + lo)
// W4A16 (the pytorch_sim math, quant/svd.py:119-163):
//   y = x_hat @ W^T with W = bf16(q * bf16(sw)) dequantized in registers while staging the
//   tile into LDS (pack.py:26-44 with dtype=bf16), same epilogue.
//
// Tiling: 128x128 block tile, 4 waves in a 2x2 grid, each wave a 64x64 tile = 2x2 MFMA
// 32x32 sub-tiles; one K-group per pipeline stage, LDS double buffered: the next stage's
// global loads are issued before the current stage's MFMAs and written to the other LDS
// buffer afterwards.  Packed INT4 is unpacked to int8 while staging: the nibbles of a dword
// are XORed with 8 (offset binary -> two's complement) and moved to the high half of each
// byte, i.e. the MFMA sees 16*q, and the 1/256 is folded into the weight scale.  This
// also permutes k inside each 8-element chunk (even k first); A and B are permuted alike.
#include "svdq_common.h"
#include "svdq_kernels.h"

namespace svdq {
namespace {

constexpr int BM = 128, BN = 128, NTHR = 256;

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// acc (2x2 sub-tiles of the wave) += mid @ l1cat^T, + bias, then store.
template <bool OUT_F32>
__device__ __forceinline__ void epilogue(const GemmParams& p, f32x16 (&acc)[2][2], int m0, int n0,
                                         int lr, int h) {
  for (int s = 0; s < p.RTp / 16; ++s) {
    u32x4 ahi[2], alo[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int m = m0 + 32 * i + lr;
      float v[8];
      if (m < p.M) {
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(p.mid + (long)m * p.RTp + 16 * s + 8 * h);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(p.mid + (long)m * p.RTp + 16 * s + 8 * h + 4);
        v[0] = v0[0]; v[1] = v0[1]; v[2] = v0[2]; v[3] = v0[3];
        v[4] = v1[0]; v[5] = v1[1]; v[6] = v1[2]; v[7] = v1[3];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
      }
      split_hi_lo(v, ahi[i], alo[i]);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 32 * j + lr;
      b[j] = n < p.N ? ld16(p.l1cat + (long)n * p.RTp + 16 * s + 8 * h) : u32x4{};
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc[i][j] = mfma_bf16_32x32x16(ahi[i], b[j], acc[i][j]);
        acc[i][j] = mfma_bf16_32x32x16(alo[i], b[j], acc[i][j]);
      }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + 32 * j + lr;
    if (n >= p.N) continue;
    const float bv = p.bias ? bf16f(p.bias[n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m >= p.M) continue;
        const float v = acc[i][j][r] + bv;
        if (OUT_F32)
          reinterpret_cast<float*>(p.y)[(long)m * p.ldy + n] = v;
        else
          reinterpret_cast<uint16_t*>(p.y)[(long)m * p.ldy + n] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu);
      }
  }
}

// --------------------------------------------------------------------------- W4A4
template <int G, bool OUT_F32>
__global__ void __launch_bounds__(NTHR) w4a4_kernel(GemmParams p) {
  constexpr int ROWB = G + 16;               // LDS bytes per row of unpacked int8 (padded)
  constexpr int LPR = G / 32;                // 16-byte packed loads per row per stage
  constexpr int LPT = BM * LPR / NTHR;       // packed loads per thread per operand
  constexpr int KS = G / 32;                 // K=32 MFMA steps per group
  __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * ROWB];
  __shared__ __attribute__((aligned(16))) int8_t sB[2][BN * ROWB];
  __shared__ __attribute__((aligned(16))) float sSX[2][BM];
  __shared__ __attribute__((aligned(16))) float sSW[2][BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, h = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  const int nbm = (p.M + BM - 1) / BM, nbn = (p.N + BN - 1) / BN;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 8, bm, bn);
  const int m0 = bm * BM, n0 = bn * BN;
  const int K = p.K, ngroups = K / G, kp = K / 2;

  u32x4 ra[LPT], rb[LPT];
  float xs = 0.0f, ws = 0.0f;

  auto gload = [&](int g) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int idx = tid + NTHR * i, row = idx / LPR, part = idx % LPR;
      const int m = m0 + row, n = n0 + row;
      const u32x4 zero8 = {0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
      ra[i] = m < p.M ? ld16(p.qx + (long)m * kp + g * (G / 2) + 16 * part) : zero8;
      rb[i] = n < p.N ? ld16(p.qw + (long)n * kp + g * (G / 2) + 16 * part) : zero8;
    }
    if (tid < BM) {
      const int m = m0 + tid;
      xs = m < p.M ? bf16f(p.sx[(long)m * ngroups + g]) : 0.0f;
    } else {
      const int n = n0 + tid - BM;
      ws = n < p.N ? half_bits_to_float(p.sw[(long)n * ngroups + g]) * (1.0f / 256.0f) : 0.0f;
    }
  };
  auto unpack16 = [](u32x4 v, u32x4& lo4, u32x4& hi4) {
    // 8 nibbles per dword -> two dwords of int8 (16*q): [k0,k2,k4,k6], [k1,k3,k5,k7]
    uint32_t o[8];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t t = v[d] ^ 0x88888888u;
      o[2 * d] = (t << 4) & 0xF0F0F0F0u;
      o[2 * d + 1] = t & 0xF0F0F0F0u;
    }
    lo4 = u32x4{o[0], o[1], o[2], o[3]};
    hi4 = u32x4{o[4], o[5], o[6], o[7]};
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int idx = tid + NTHR * i, row = idx / LPR, part = idx % LPR;
      u32x4 a0, a1, b0, b1;
      unpack16(ra[i], a0, a1);
      unpack16(rb[i], b0, b1);
      st16(&sA[buf][row * ROWB + 32 * part], a0);
      st16(&sA[buf][row * ROWB + 32 * part + 16], a1);
      st16(&sB[buf][row * ROWB + 32 * part], b0);
      st16(&sB[buf][row * ROWB + 32 * part + 16], b1);
    }
    if (tid < BM) sSX[buf][tid] = xs;
    else sSW[buf][tid - BM] = ws;
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  gload(0);
  lstore(0);
  __syncthreads();

  for (int g = 0; g < ngroups; ++g) {
    const int buf = g & 1;
    if (g + 1 < ngroups) gload(g + 1);

    i32x16 pacc[2][2];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      i32x4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = __builtin_bit_cast(i32x4, ld16(&sA[buf][(64 * wm + 32 * i + lr) * ROWB + 32 * ks + 16 * h]));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = __builtin_bit_cast(i32x4, ld16(&sB[buf][(64 * wn + 32 * j + lr) * ROWB + 32 * ks + 16 * h]));
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          pacc[i][j] = mfma_i8_32x32x32(a[i], b[j], ks == 0 ? i32x16{} : pacc[i][j]);
    }
    f32x4 sxv[2][4];
    float swv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        sxv[i][q] = *reinterpret_cast<const f32x4*>(&sSX[buf][64 * wm + 32 * i + 8 * q + 4 * h]);
#pragma unroll
    for (int j = 0; j < 2; ++j) swv[j] = sSW[buf][64 * wn + 32 * j + lr];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[i][j][r] = __builtin_fmaf((float)pacc[i][j][r], sxv[i][r >> 2][r & 3] * swv[j], acc[i][j][r]);

    if (g + 1 < ngroups) lstore(buf ^ 1);
    __syncthreads();
  }

  epilogue<OUT_F32>(p, acc, m0 + 64 * wm, n0 + 64 * wn, lr, h);
}

// --------------------------------------------------------------------------- W4A16
template <int G, bool OUT_F32>
__global__ void __launch_bounds__(NTHR) w4a16_kernel(GemmParams p) {
  constexpr int ROWH = 2 * G + 16;            // LDS bytes per bf16 row (padded)
  constexpr int ALPR = 2 * G / 16;            // 16-byte loads per A row per stage
  constexpr int ALPT = BM * ALPR / NTHR;      // A loads per thread
  constexpr int BLPR = G / 32;                // 16-byte packed loads per B row
  constexpr int BLPT = BN * BLPR / NTHR;      // B loads per thread
  constexpr int KS = G / 16;                  // K=16 MFMA steps per group
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * ROWH];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][BN * ROWH];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, h = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  const int nbm = (p.M + BM - 1) / BM, nbn = (p.N + BN - 1) / BN;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 8, bm, bn);
  const int m0 = bm * BM, n0 = bn * BN;
  const int K = p.K, ngroups = K / G, kp = K / 2;

  u32x4 ra[ALPT], rb[BLPT];
  float wsc[BLPT];

  auto gload = [&](int g) {
#pragma unroll
    for (int i = 0; i < ALPT; ++i) {
      const int idx = tid + NTHR * i, row = idx / ALPR, part = idx % ALPR;
      const int m = m0 + row;
      ra[i] = m < p.M ? ld16(p.xhat + (long)m * p.ldxh + g * G + 8 * part) : u32x4{};
    }
#pragma unroll
    for (int i = 0; i < BLPT; ++i) {
      const int idx = tid + NTHR * i, row = idx / BLPR, part = idx % BLPR;
      const int n = n0 + row;
      rb[i] = n < p.N ? ld16(p.qw + (long)n * kp + g * (G / 2) + 16 * part) : u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
      wsc[i] = n < p.N ? round_bf16(half_bits_to_float(p.sw[(long)n * ngroups + g])) : 0.0f;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ALPT; ++i) {
      const int idx = tid + NTHR * i, row = idx / ALPR, part = idx % ALPR;
      st16(&sA[buf][row * ROWH + 16 * part], ra[i]);
    }
#pragma unroll
    for (int i = 0; i < BLPT; ++i) {
      const int idx = tid + NTHR * i, row = idx / BLPR, part = idx % BLPR;
      const float s = wsc[i], ns8 = -8.0f * s;
      uint32_t o[16];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t v = rb[i][d];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float w0 = __builtin_fmaf((float)((v >> (8 * e)) & 0xFu), s, ns8);
          const float w1 = __builtin_fmaf((float)((v >> (8 * e + 4)) & 0xFu), s, ns8);
          o[4 * d + e] = pack_bf16x2(w0, w1);
        }
      }
      uint8_t* dst = &sB[buf][row * ROWH + 64 * part];
      st16(dst, u32x4{o[0], o[1], o[2], o[3]});
      st16(dst + 16, u32x4{o[4], o[5], o[6], o[7]});
      st16(dst + 32, u32x4{o[8], o[9], o[10], o[11]});
      st16(dst + 48, u32x4{o[12], o[13], o[14], o[15]});
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  gload(0);
  lstore(0);
  __syncthreads();

  for (int g = 0; g < ngroups; ++g) {
    const int buf = g & 1;
    if (g + 1 < ngroups) gload(g + 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = ld16(&sA[buf][(64 * wm + 32 * i + lr) * ROWH + 32 * ks + 16 * h]);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = ld16(&sB[buf][(64 * wn + 32 * j + lr) * ROWH + 32 * ks + 16 * h]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16_32x32x16(a[i], b[j], acc[i][j]);
    }
    if (g + 1 < ngroups) lstore(buf ^ 1);
    __syncthreads();
  }

  epilogue<OUT_F32>(p, acc, m0 + 64 * wm, n0 + 64 * wn, lr, h);
}

}  // namespace

hipError_t launch_w4a4(const GemmParams& p, int G, bool out_f32, hipStream_t st) {
  const dim3 grid(((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN));
  if (G == 64) {
    if (out_f32) w4a4_kernel<64, true><<<grid, NTHR, 0, st>>>(p);
    else w4a4_kernel<64, false><<<grid, NTHR, 0, st>>>(p);
  } else if (G == 128) {
    if (out_f32) w4a4_kernel<128, true><<<grid, NTHR, 0, st>>>(p);
    else w4a4_kernel<128, false><<<grid, NTHR, 0, st>>>(p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_w4a16(const GemmParams& p, int G, bool out_f32, hipStream_t st) {
  const dim3 grid(((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN));
  if (G == 64) {
    if (out_f32) w4a16_kernel<64, true><<<grid, NTHR, 0, st>>>(p);
    else w4a16_kernel<64, false><<<grid, NTHR, 0, st>>>(p);
  } else if (G == 128) {
    if (out_f32) w4a16_kernel<128, true><<<grid, NTHR, 0, st>>>(p);
    else w4a16_kernel<128, false><<<grid, NTHR, 0, st>>>(p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace svdq
