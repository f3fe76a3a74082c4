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

#include "svdq_common.h"
#include "svdq_kernels.h"

namespace svdq {
namespace {

constexpr int BM = 128, BN = 128, NTHR = 256;

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }



// acc (2x2 sub-tiles of the wave) += mid @ l1cat^T, + bias, then store.  mid holds one
// partial per K split of the activation pass; they are added here in split order.
template <bool OUT_F32>
__device__ __forceinline__ void epilogue(const GemmParams& p, f32x16 (&acc)[2][2], int m0, int n0,
                                         int lr, int h) {
  const long split_stride = (long)p.M * p.RTp;
  for (int s = 0; s < p.RTp / 16; ++s) {
    u32x4 ahi[2], alo[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int m = min(m0 + 32 * i + lr, p.M - 1);
      const float* src = p.mid + (long)m * p.RTp + 16 * s + 8 * h;
      f32x4 v0 = *reinterpret_cast<const f32x4*>(src);
      f32x4 v1 = *reinterpret_cast<const f32x4*>(src + 4);
      for (int sp = 1; sp < p.splits; ++sp) {
        v0 += *reinterpret_cast<const f32x4*>(src + sp * split_stride);
        v1 += *reinterpret_cast<const f32x4*>(src + sp * split_stride + 4);
      }
      const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      split_hi_lo(v, ahi[i], alo[i]);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = min(n0 + 32 * j + lr, p.N - 1);
      b[j] = ld16(p.l1cat + (long)n * p.RTp + 16 * s + 8 * h);
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
// Block tile 256x128, 8 waves in a 4x2 grid (64x64 per wave = 2x2 MFMA 32x32 tiles), one
// K-group per stage.  Per group and output element the accumulator update is one FMA,
// acc += P * S, where P is the exact group dot product from the 8-bit MFMA and S = sx * sw
// comes from a bf16 MFMA whose K=2 operand pairs are (sx, sx) and (bf16 hi, bf16 lo) of the
// fp16 weight scale, i.e. the scale product is exact too.
//   MODE 0: operands e4m3, v_mfma_f32_32x32x64_f8f6f4 (P already float32);
//   MODE 1: operands int8 16*q, 2x v_mfma_i32_32x32x32_i8 (P int32, converted; 1/256 in S).
// Operand A (activation codes, 8-bit) comes from the activation pass; operand B is the
// packed INT4 weight, converted while staging into LDS.  Global loads run two groups ahead
// in two register sets; LDS is double buffered.
// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4): lane L
// of the wave writes LDS bytes [lds + 16 L, lds + 16 L + 16) from base + off.  Issued as
// inline asm so that the compiler does not order every later LDS read after it (it cannot
// tell the two LDS stages apart); the kernel waits for it explicitly before its barrier.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// W4A4 GEMM (FP8 or INT8 MFMA on exact integer codes).
//
// Block tile 256 x 128, 8 waves in a 4 x 2 grid, wave tile 64 x 64 = 2 x 2 sub-tiles of
// 32 x 32.  K advances 128 columns per pipeline stage (two groups of 64 or one of 128), two
// LDS stages.  Both operands are 8-bit codes in HBM (activations from the activation pass,
// weights expanded once per layer) and go global -> LDS by DMA; only the scales pass
// through registers.
//
// LDS operand tiles: rows of 128 bytes = 8 chunks of 16; chunk c of row r sits at chunk
// position c ^ ((r >> 1) & 7).  The 16 lanes of a ds_read_b128 phase read one logical chunk
// of 16 consecutive rows and hit 16 distinct 4-bank groups.
//
// Per group and sub-tile: P = codes_x . codes_w (exact integer sums, fp32) on the FP8 MFMA,
// S = sx (x) sw on a bf16 MFMA with K = 2 ((sx, sx) . (hi(sw), lo(sw)) exact), acc += P * S.
template <int G, int MODE, bool OUT_F32>
__global__ void __launch_bounds__(512, 1) w4a4_kernel(GemmParams p) {
  constexpr int TBM = 256, TBN = 128, NT = 512;
  constexpr int KB = 128;                     // K columns per pipeline stage
  constexpr int GPS = KB / G;                 // groups per stage
  constexpr int KS = G / 64;                  // 64-column MFMA steps per group
  constexpr int ADMA = TBM * KB / (16 * NT);  // A: 16-byte DMA chunks per thread per stage (4)
  constexpr int BDMA = TBN * KB / (16 * NT);  // B: 16-byte DMA chunks per thread per stage (2)
  constexpr int XS = TBM + 1, WS = TBN + 1;   // scale rows per group (+1 zero row)
  static_assert(GPS * TBM <= NT && GPS * TBN <= NT, "one scale of each kind per thread");
  __shared__ __attribute__((aligned(1024))) uint8_t sA[2][TBM * KB];
  __shared__ __attribute__((aligned(1024))) uint8_t sB[2][TBN * KB];
  // Scale-MFMA operands, 4 words per row: (pair, 0, 0, 0); the last row is all zero.
  __shared__ __attribute__((aligned(16))) uint32_t sX[2][GPS][XS * 4];   // pair = (sx, sx)
  __shared__ __attribute__((aligned(16))) uint32_t sW[2][GPS][WS * 4];   // pair = (hi, lo) of sw

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, h = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  const int nbm = (p.M + TBM - 1) / TBM, nbn = (p.N + TBN - 1) / TBN;
  int bm, bn;
  tile_coords(blockIdx.x, nbm, nbn, 4, bm, bn);
  const int m0 = bm * TBM, n0 = bn * TBN;
  const int K = p.K, ngroups = K / G, nstages = (K + KB - 1) / KB;

  // DMA sources: wave w, chunk i covers LDS bytes [(DMA w + i) KB, +1 KB) of a stage tile,
  // i.e. 8 rows; lane L lands at row 8 (DMA w + i) + L / 8, chunk position L % 8.  Columns
  // past K (a last stage holding a single group of 64) are clamped to the row's last chunk;
  // that group's scale is zero.  Offsets are 32-bit (the host bounds the operand sizes).
  uint32_t aoff[ADMA], boff[BDMA];
  int alim[ADMA], blim[BDMA];
#pragma unroll
  for (int i = 0; i < ADMA; ++i) {
    const int row = 8 * (ADMA * wave + i) + lane / 8, c = (lane % 8) ^ ((row >> 1) & 7);
    aoff[i] = (uint32_t)min(m0 + row, p.M - 1) * (uint32_t)K + 16 * c;
    alim[i] = K - 16 - 16 * c;
  }
#pragma unroll
  for (int i = 0; i < BDMA; ++i) {
    const int row = 8 * (BDMA * wave + i) + lane / 8, c = (lane % 8) ^ ((row >> 1) & 7);
    boff[i] = (uint32_t)min(n0 + row, p.N - 1) * (uint32_t)K + 16 * c;
    blim[i] = K - 16 - 16 * c;
  }
  // Scales: thread t stages sx of row t % TBM for group t / TBM of the stage and sw of
  // column t % TBN for group t / TBN (threads past GPS * TBN load a duplicate, not stored).
  const int xj = (tid / TBM) % GPS, xr = tid % TBM, wj = (tid / TBN) % GPS, wr = tid % TBN;
  const uint32_t xoff = (uint32_t)min(m0 + xr, p.M - 1) * (uint32_t)ngroups;
  const uint32_t woff = (uint32_t)min(n0 + wr, p.N - 1) * (uint32_t)ngroups;
  const bool x_live = tid < GPS * TBM, w_live = tid < GPS * TBN;
  // Zero the padding words 1-3 of every row and the whole last row, once (the pair words of
  // rows < TBM / TBN are written every stage, by other threads: never touched here).
  for (int t = tid; t < 2 * GPS * XS; t += NT) {
    uint32_t* r = &sX[t / (GPS * XS)][(t / XS) % GPS][(t % XS) * 4];
    if (t % XS == TBM) r[0] = 0u;
    r[1] = 0u; r[2] = 0u; r[3] = 0u;
  }
  for (int t = tid; t < 2 * GPS * WS; t += NT) {
    uint32_t* r = &sW[t / (GPS * WS)][(t / WS) % GPS][(t % WS) * 4];
    if (t % WS == TBN) r[0] = 0u;
    r[1] = 0u; r[2] = 0u; r[3] = 0u;
  }

  // Fragment addresses (bytes within a stage tile): the lane's row; chunk c at c ^ sw_.
  const int sw_ = (lr >> 1) & 7;
  const int arow = (64 * wm + lr) * 128, brow = (64 * wn + lr) * 128;
  // Scale-MFMA operand rows: lanes 32-63 (the second half of K) read the zero row.
  const int xrow = h ? TBM : 64 * wm + lr, wrow = h ? TBN : 64 * wn + lr;

  uint32_t rx, rw;
  int xg;
  // Issue the loads of stage `s`: scales into registers, then A and B into LDS buffer `buf`.
  // The DMA goes last: the compiler does not count it, so any wait it places for its own
  // loads is ordered before the DMA and never waits for it.
  auto gload = [&](int s, int buf) {
    xg = s * GPS + xj;
    rx = p.sx[xoff + (uint32_t)min(xg, ngroups - 1)];
    rw = p.swp[woff + (uint32_t)min(s * GPS + wj, ngroups - 1)];
#pragma unroll
    for (int i = 0; i < ADMA; ++i)
      dma16(p.qa, aoff[i] + (uint32_t)min(s * KB, alim[i]),
            __builtin_amdgcn_readfirstlane(lds_offset(&sA[buf][(ADMA * wave + i) * 1024])));
#pragma unroll
    for (int i = 0; i < BDMA; ++i)
      dma16(p.qwe, boff[i] + (uint32_t)min(s * KB, blim[i]),
            __builtin_amdgcn_readfirstlane(lds_offset(&sB[buf][(BDMA * wave + i) * 1024])));
  };
  auto lstore = [&](int buf) {
    if (x_live) sX[buf][xj][4 * xr] = xg < ngroups ? rx * 0x10001u : 0u;
    if (w_live) sW[buf][wj][4 * wr] = rw;
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  // Operands of one group: A/B fragments of the wave's 2x2 sub-tiles and the scale-MFMA
  // operands.
  struct Frag {
    u32x4 a[2][KS][2], b[2][KS][2];
    u32x4 x[2], w[2];
  };
  auto read_frag = [&](Frag& f, int buf, int gi) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        // logical chunk c = G/16 gi + 4 ks + 2 h + t of the lane's rows, stored at c ^ sw_
        const int pc = 16 * ((G / 16 * gi + 4 * ks + 2 * h + t) ^ sw_);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          f.a[i][ks][t] = ld16(&sA[buf][arow + 4096 * i + pc]);
          f.b[i][ks][t] = ld16(&sB[buf][brow + 4096 * i + pc]);
        }
      }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      f.x[i] = ld16(&sX[buf][gi][4 * (xrow + (h ? 0 : 32 * i))]);
      f.w[i] = ld16(&sW[buf][gi][4 * (wrow + (h ? 0 : 32 * i))]);
    }
  };
  auto mfma_p = [&](const Frag& f, int i, int j) {
    f32x16 pf;
    if (MODE == 0) {
      pf = mfma_fp8_32x32x64(f.a[i][0], f.b[j][0], f32x16{});
#pragma unroll
      for (int ks = 1; ks < KS; ++ks) pf = mfma_fp8_32x32x64(f.a[i][ks], f.b[j][ks], pf);
    } else {
      i32x16 pi = i32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          pi = mfma_i8_32x32x32(__builtin_bit_cast(i32x4, f.a[i][ks][t]), __builtin_bit_cast(i32x4, f.b[j][ks][t]), pi);
#pragma unroll
      for (int r = 0; r < 16; ++r) pf[r] = (float)pi[r];
    }
    return pf;
  };
  auto fma16 = [&](f32x16& a, const f32x16& pf, const f32x16& sf) {
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = __builtin_fmaf(pf[r], sf[r], a[r]);
  };

  // Issue order per group, sub-tiles t = (0,0) (0,1) (1,0) (1,1):
  //   P_t (product MFMA) | rescale of sub-tile t-1 (16 VALU FMAs) | S_t (scale MFMA)
  // The rescale of t-1 needs S_{t-1}, which completed before P_t could issue, so the FMAs
  // run in the shadow of P_t.  Empty asm statements on the values pin this order (the
  // compiler would otherwise issue all MFMAs of a stage first and run out of registers).
  // Sub-tile (1,1) of a group is rescaled under the next group's first MFMA.
  f32x16 pp = f32x16{}, ps = f32x16{};
  auto group = [&](Frag& f) {
    constexpr int TI[4] = {0, 0, 1, 1}, TJ[4] = {0, 1, 0, 1};
    f32x16 cp[4], cs[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int i = TI[t], j = TJ[t];
      cp[t] = mfma_p(f, i, j);
      f32x16& a = t == 0 ? acc[1][1] : acc[TI[t - 1]][TJ[t - 1]];
      fma16(a, t == 0 ? pp : cp[t - 1], t == 0 ? ps : cs[t - 1]);
      asm volatile("" : "+v"(a), "+v"(f.x[i]), "+v"(f.w[j]));
      cs[t] = mfma_bf16_32x32x16(f.x[i], f.w[j], f32x16{});
      if (t < 3) {
        const int ni = TI[t + 1], nj = TJ[t + 1];
        asm volatile("" : "+v"(f.a[ni][0][0]), "+v"(f.a[ni][0][1]), "+v"(f.b[nj][0][0]), "+v"(f.b[nj][0][1]));
      }
    }
    pp = cp[3];
    ps = cs[3];
  };

  // Two LDS stages: stage s + 1 is loaded while stage s computes.  Loads are unconditional
  // (stage index clamped).
  gload(0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lstore(0);
  __syncthreads();
  for (int s = 0; s < nstages; ++s) {
    const int buf = s & 1;
    gload(min(s + 1, nstages - 1), buf ^ 1);
#pragma unroll
    for (int gi = 0; gi < GPS; ++gi) {
      Frag f;
      read_frag(f, buf, gi);
      group(f);
    }
    // All of stage s + 1 has to land before the barrier.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lstore(buf ^ 1);
    __syncthreads();
  }
  fma16(acc[1][1], pp, ps);

  epilogue<OUT_F32>(p, acc, m0 + 64 * wm, n0 + 64 * wn, lr, h);
}

// Weight operand of the W4A4 GEMM, once per layer: each packed dword (8 nibbles, k0 in the
// low nibble) becomes 8 operand bytes [k0 k2 k4 k6 k1 k3 k5 k7].
__global__ void weight_operand_kernel(const uint32_t* __restrict__ qw, u32x2* __restrict__ out, long n, int mode) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    uint32_t lo, hi;
    if (mode == 0) nib8_to_e4m3(qw[i], lo, hi);
    else nib8_to_i8x16(qw[i], lo, hi);
    out[i] = u32x2{lo, hi};
  }
}

// Weight-scale operand of the W4A4 scale MFMA, once per layer: (bf16 hi, bf16 lo) of the fp16
// scale, hi + lo == scale exactly; MODE 1 (int8 16*q operands) folds in 1/256.
__global__ void weight_scale_pairs_kernel(const uint16_t* __restrict__ sw, uint32_t* __restrict__ out, long n,
                                          float mult) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float f = half_bits_to_float(sw[i]) * mult;
    const uint32_t hi = pack_bf16x2(f, 0.0f) & 0xFFFFu;
    const uint32_t lo = pack_bf16x2(f - bf16lo(hi), 0.0f) & 0xFFFFu;
    out[i] = hi | (lo << 16);
  }
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
      ra[i] = ld16(p.xhat + (long)min(m0 + row, p.M - 1) * p.ldxh + g * G + 8 * part);
    }
#pragma unroll
    for (int i = 0; i < BLPT; ++i) {
      const int idx = tid + NTHR * i, row = idx / BLPR, part = idx % BLPR;
      const int n = min(n0 + row, p.N - 1);
      rb[i] = ld16(p.qw + (long)n * kp + g * (G / 2) + 16 * part);
      wsc[i] = round_bf16(half_bits_to_float(p.sw[(long)n * ngroups + g]));
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

hipError_t launch_w4a4(const GemmParams& p, int G, int mode, bool out_f32, hipStream_t st) {
  const dim3 grid(((p.M + 255) / 256) * ((p.N + 127) / 128));
#define SVDQ_W4A4(GG, MM)                                                        \
  if (G == GG && mode == MM) {                                                   \
    if (out_f32) w4a4_kernel<GG, MM, true><<<grid, 512, 0, st>>>(p);              \
    else w4a4_kernel<GG, MM, false><<<grid, 512, 0, st>>>(p);                     \
    return hipGetLastError();                                                    \
  }
  SVDQ_W4A4(64, 0)
  SVDQ_W4A4(128, 0)
  SVDQ_W4A4(64, 1)
  SVDQ_W4A4(128, 1)
#undef SVDQ_W4A4
  return hipErrorInvalidValue;
}

hipError_t launch_weight_scale_pairs(const uint16_t* sw, uint32_t* out, long n, int mode, hipStream_t st) {
  weight_scale_pairs_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(sw, out, n, mode == 0 ? 1.0f : 1.0f / 256.0f);
  return hipGetLastError();
}

hipError_t launch_weight_operand(const uint8_t* qw, uint8_t* qwe, long ndwords, int mode, hipStream_t st) {
  const long blocks = std::min<long>((ndwords + 255) / 256, 8192);
  weight_operand_kernel<<<(unsigned)blocks, 256, 0, st>>>(reinterpret_cast<const uint32_t*>(qw),
                                                          reinterpret_cast<u32x2*>(qwe), ndwords, mode);
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
