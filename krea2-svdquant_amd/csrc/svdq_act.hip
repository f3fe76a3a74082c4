// Fused activation pass for the SVDQuant linear on gfx950 (one HBM read of x).
//
//   x_hat = bf16(x / s)                                  quant/svd.py:121-122
//   sx    = bf16(max(amax_g |x_hat|, bf16(1e-8)) / 7)    quant/pack.py:20
//   q     = rne(x_hat / sx)  (clamp(-8, 7) never binds)   quant/pack.py:21
//   qa    = 8-bit GEMM operand codes of q;  qx = canonical packed codes, pack.py:53-56
//   mid   = x_hat @ L2^T            (low-rank down)      quant/svd.py:159
//   lmid  = mult * (x @ A^T)        (LoRA down, raw x)    runtime/linear.py:42-45
//
// Layout: a workgroup (4 waves) owns 64 rows and a contiguous range of K-groups (one
// "split"); wave w takes every 4th group of the range.  Lane l of a wave holds row l, so a
// group's smoothing scales are the same for the whole wave (scalar loads, SGPR operands) and
// the group absmax is lane-local.  The 32x32x16 bf16 A operand of the low-rank MFMAs wants
// the two 8-column halves of a 16-column slice of one row in lanes l and l+32; one
// v_permlane32_swap per register turns the lane-per-row data into exactly that for both
// 32-row tiles.  Per-wave partials are summed in a fixed wave order in LDS and each split
// writes its own partial mid[split]; the GEMM epilogue adds the splits in a fixed order
// (deterministic, and no device-scope fences, which cost an L2 write-back each).
//
// Codes never need the reference's clamp: |x_hat| <= amax and sx >= (amax/7)(1 - 2^-9), so
// |x_hat / sx| < 7.02 rounds into [-7, 7].
#include <cstdlib>
#include <cstring>

#include "svdq_common.h"
#include "svdq_kernels.h"

namespace svdq {

namespace {

constexpr float kBf16OneEMinus8 = 1.00117176e-08f;  // bf16(1e-8)
constexpr float kRcp7 = 0.142857149f;               // RN(1/7)

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x2 as_u16x2(uint32_t v) { return __builtin_bit_cast(u16x2, v); }

// The scale vectors are read through the constant address space: they are read-only while
// the kernel runs, the addresses are wave-uniform, so they become scalar loads and SGPR
// operands instead of per-lane vector loads.
typedef const __attribute__((address_space(4))) float* cfloat_ptr;

// x_hat = bf16(RN(x * RN(1/s))) for the lane's row over 64 columns.  This equals the reference's
// bf16(x / s) (float32 division, then bf16) whenever the quotient lies in [2^-90, 2^100] and
// RN(1/s) is finite: x and s carry 8 significant bits, so x / s is never a bf16 rounding midpoint
// and stays at least 2^-17 (relative) away from one, while the product is within 2^-23 of x / s
// (exhaustive check over every bf16 pair: tests/native/smooth_exhaustive.c).  Signed zeros
// come out as IEEE division gives them.
// amx: packed maximum of the |x_hat| bit patterns (inf and NaN compare largest, so a quotient
// the product cannot represent always shows in the group maximum).  XHAT callers also get the
// packed maximum of the |x| bit patterns and the minimum of |x| - 1 (a zero wraps to 0xFFFF and
// drops out), for the range test of every element.
template <bool XHAT>
__device__ __forceinline__ void smooth64_fast(const u32x4 (&xr)[8], cfloat_ptr rv, u32x4 (&xh)[8], u16x2& amx,
                                              u16x2& xmx, u16x2& xmn) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t d = xr[c][e];
      const uint32_t pk = pack_bf16x2(bf16lo(d) * rv[8 * c + 2 * e], bf16hi(d) * rv[8 * c + 2 * e + 1]);
      xh[c][e] = pk;
      amx = __builtin_elementwise_max(amx, as_u16x2(pk & 0x7FFF7FFFu));
      if (XHAT) {
        const u16x2 ax = as_u16x2(d & 0x7FFF7FFFu);
        xmx = __builtin_elementwise_max(xmx, ax);
        xmn = __builtin_elementwise_min(xmn, ax - (u16x2){1, 1});
      }
    }
  }
}

// IEEE division for a group the fast path does not cover (or SVDQ_ACT_EXACT_DIV); am = the
// group's max |x_hat| as a float.
__device__ __forceinline__ void smooth64_exact(const u32x4 (&xr)[8], cfloat_ptr sv, u32x4 (&xh)[8], float& am) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t d = xr[c][e];
      const uint32_t pk = pack_bf16x2(bf16lo(d) / sv[8 * c + 2 * e], bf16hi(d) / sv[8 * c + 2 * e + 1]);
      xh[c][e] = pk;
      am = fmaxf(am, fmaxf(fabsf(bf16lo(pk)), fabsf(bf16hi(pk))));
    }
  }
}

// OPER: GEMM operand codes written (0 none, 1 e4m3, 2 int8 16*q, 3 e3m2 planar).  The e3m2 layout
// of an [R, K] operand, Rp = R rounded up to even: for k-step t (64 columns) and half h (columns
// 64 t + 32 h ..), the first 16 bytes of each row's 24-byte field vector in plane Q[t][h][Rp][16]
// (at byte 0), the last 8 in plane P[t][h][Rp][8] (at byte Rp K / 2) -- rows contiguous, so the
// lanes (rows) of a wave store whole 1 KB / 512 B runs and the GEMM's DMA and LDS reads stream
// whole planes.
// QX: the canonical packed codes may be requested (p.qx checked at run time); without it the
// kernel carries no nibble-packing code at all.
// NT: the MFMA column tiles of the down projections this launch computes, global tiles
// p.t0 .. p.t0 + NT - 1 of [L2 (ceil(r/32) tiles) | LoRA (ceil(rl/32) tiles)].  LX: some of them
// may be LoRA tiles (the raw x is then kept as an MFMA operand too).  Ranks beyond 4 tiles take
// further launches with OPER 0 and no XHAT (down projections only), each writing its own columns
// of the split partials.
// NL > 1: the passes of NL sibling layers over the same x (lp[0 .. NL-1], same M, K, splits; one
// rank tile each, NT = 1, no LoRA): each group of x is loaded once and smoothed, quantized and
// down-projected once per layer, in layer order, so that every layer's codes, scales and split
// partials are bit-identical to its own pass (the same groups per wave, the same MFMA and
// reduction order).
template <int G, int NT, int OPER, bool XHAT, bool QX, bool LX, int NL = 1>
__device__ __forceinline__ void act_tile(const ActParams* lp) {
  constexpr int HB = G / 64;             // 64-column blocks per group
  constexpr bool QUANT = OPER != 0;
  static_assert(NL == 1 || (NT == 1 && !LX && !XHAT && !QX), "shared-x passes: one rank tile, codes only");
  __shared__ __attribute__((aligned(16))) float red[4 * 64 * 32];
  const ActParams& p = lp[0];            // M, K, x and the split are the same for every layer

  const int tid = threadIdx.x;
  const int lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m0 = blockIdx.x * 64;
  const int row = m0 + lane;
  const bool rok = row < p.M;
  const long rowc = min(row, p.M - 1);   // rows past M read row M-1; never stored
  const int K = p.K;
  const int ngroups = K / G;
  const int gb = blockIdx.y * p.gps;
  const int ge = min(ngroups, gb + p.gps);

  f32x16 acc[NL][2][NT];
#pragma unroll
  for (int l = 0; l < NL; ++l)
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[l][a][t] = f32x16{};

  // Without LoRA, x of the wave's next group is loaded into xr as soon as the current group's xr
  // is dead (after the smoothing and its exact fallback): the loads overlap the quantization, the
  // stores and the low-rank MFMAs with no extra registers.  With LoRA the raw x feeds the LoRA
  // down projection, so each group is loaded when it starts.
  constexpr bool LORA = LX;
  u32x4 xr[HB][8];
  auto load_x = [&](int g) {
#pragma unroll
    for (int b = 0; b < HB; ++b)
#pragma unroll
      for (int c = 0; c < 8; ++c) xr[b][c] = ld16(p.x + rowc * p.ldx + g * G + 64 * b + 8 * c);
  };
  if (!LORA && gb + wave < ge) load_x(gb + wave);
  for (int g = gb + wave; g < ge; g += 4) {
    if (LORA) load_x(g);
#pragma unroll
    for (int l = 0; l < NL; ++l) {
    const ActParams& p = lp[l];
    const int TR = (p.r + 31) >> 5;
    const cfloat_ptr sv = (cfloat_ptr)p.srs;
    const cfloat_ptr rv = (cfloat_ptr)(p.srs + K);
    u32x4 xh[HB][8];

    u16x2 amx = {0, 0}, xmx = {0, 0}, xmn = {0xFFFF, 0xFFFF};
#pragma unroll
    for (int b = 0; b < HB; ++b) smooth64_fast<XHAT>(xr[b], rv + g * G + 64 * b, xh[b], amx, xmx, xmn);
    const uint32_t amb = amx[0] > amx[1] ? amx[0] : amx[1];
    float am = bf16f((uint16_t)amb);
    bool bad;
    if (XHAT) {
      // x_hat needs every element exact: every nonzero quotient inside [2^-90, 2^100] (bounded by
      // the row's |x| range over the group's |s| range) and every s normal, so RN(1/s) is finite.
      // The s bit patterns are wave-uniform: scalar minimum / maximum.
      uint32_t smn = 0xFFFFFFFFu, smx = 0u;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const uint32_t sb = __float_as_uint(sv[g * G + j]) & 0x7FFFFFFFu;
        smn = min(smn, sb);
        smx = max(smx, sb);
      }
      const uint32_t xm1 = xmn[0] < xmn[1] ? xmn[0] : xmn[1];   // 0xFFFF: no nonzero element
      const float xmax = bf16f(xmx[0] > xmx[1] ? xmx[0] : xmx[1]), xmin = bf16f((uint16_t)(xm1 + 1));
      bad = smn < 0x00800000u || smx > 0x7F800000u ||
            (xm1 != 0xFFFFu && !(xmin >= 0x1p-90f * __uint_as_float(smx) && xmax <= 0x1p100f * __uint_as_float(smn)));
    } else {
      // Only codes and scales are written: they follow from the group absmax and, per element,
      // from the element's own quotient.  With the absmax inside [2^-90, 2^100] no quotient
      // leaves the range from above, and one below the normal range (< 2^-126, the only inexact
      // case) is under 2^-33 of the scale, so its code is 0 either way.
      bad = amb != 0u && !(am >= 0x1p-90f && am <= 0x1p100f);
    }
    if (p.exact || __any(bad)) {
      am = 0.0f;
#pragma unroll
      for (int b = 0; b < HB; ++b) smooth64_exact(xr[b], sv + g * G + 64 * b, xh[b], am);
    }
    if (l == NL - 1 && !LORA && g + 4 < ge) load_x(g + 4);

    if (QUANT) {
      const float sc = round_bf16(div_rcp(fmaxf(am, kBf16OneEMinus8), 7.0f, kRcp7));
      const float rsc = 1.0f / sc;
#pragma unroll
      for (int b = 0; b < HB; ++b) {
        u32x4 op[4];
        uint32_t nib[8];
        f32x16 ex, ey;                      // OPER 3: the half's even-k and odd-k codes
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float t[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // rint, then +0 turns -0 into +0 (canonical code bytes)
            t[2 * e] = __builtin_rintf(div_rcp(bf16lo(xh[b][c][e]), sc, rsc)) + 0.0f;
            t[2 * e + 1] = __builtin_rintf(div_rcp(bf16hi(xh[b][c][e]), sc, rsc)) + 0.0f;
          }
          if (OPER == 1) {
            const uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
                t[4], t[6], __builtin_amdgcn_cvt_pk_fp8_f32(t[0], t[2], 0, false), true);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
                t[5], t[7], __builtin_amdgcn_cvt_pk_fp8_f32(t[1], t[3], 0, false), true);
            op[c >> 1][2 * (c & 1)] = lo;
            op[c >> 1][2 * (c & 1) + 1] = hi;
          }
          if (OPER == 3) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              ex[4 * (c & 3) + e] = t[2 * e];
              ey[4 * (c & 3) + e] = t[2 * e + 1];
            }
            if ((c & 3) == 3 && rok) {
              // k-step kt, half c / 4: 16 bytes to plane Q, 8 bytes to plane P
              const u32x6 f = codes_to_e3m2(ex, ey);
              const long mp = (p.M + 1) & ~1;      // plane rows, padded to even
              const long plane = (long)((g * HB + b) * 2 + (c >> 2)) * mp + rowc;
              *reinterpret_cast<u32x4*>(p.qa + plane * 16) = u32x4{f[0], f[1], f[2], f[3]};
              *reinterpret_cast<u32x2*>(p.qa + mp * (K / 2) + plane * 8) = u32x2{f[4], f[5]};
            }
          }
          if (OPER == 2 || (QX && p.qx)) {
            uint32_t w = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) w |= (uint32_t)((int)t[e] + 8) << (4 * e);
            nib[c] = w;
            if (OPER == 2) {
              uint32_t lo, hi;
              nib8_to_i8x16(w, lo, hi);
              op[c >> 1][2 * (c & 1)] = lo;
              op[c >> 1][2 * (c & 1) + 1] = hi;
            }
          }
        }
        if (rok) {
          if (OPER != 3) {
            uint8_t* od = p.qa + rowc * K + g * G + 64 * b;
#pragma unroll
            for (int q = 0; q < 4; ++q) *reinterpret_cast<u32x4*>(od + 16 * q) = op[q];
          }
          if (QX && p.qx) {
            uint8_t* dst = p.qx + rowc * (K / 2) + (g * G + 64 * b) / 2;
            *reinterpret_cast<u32x4*>(dst) = u32x4{nib[0], nib[1], nib[2], nib[3]};
            *reinterpret_cast<u32x4*>(dst + 16) = u32x4{nib[4], nib[5], nib[6], nib[7]};
          }
        }
      }
      if (rok) {
        const uint32_t sb = __float_as_uint(sc) >> 16;
        if (p.sx_pairs) reinterpret_cast<uint32_t*>(p.sx)[(long)g * p.M + rowc] = sb * 0x10001u;
        else p.sx[rowc * ngroups + g] = (uint16_t)sb;
      }
    }
    if (XHAT && rok) {
#pragma unroll
      for (int b = 0; b < HB; ++b)
#pragma unroll
        for (int c = 0; c < 8; ++c)
          *reinterpret_cast<u32x4*>(p.xhat + rowc * p.ldxh + g * G + 64 * b + 8 * c) = xh[b][c];
    }

    // ---- low-rank down (x_hat @ L2^T) and LoRA down (x @ A^T) on MFMA, per 64 columns ----
#pragma unroll
    for (int b = 0; b < HB; ++b) {
      // fa[i][c]: A operand of row tile i (rows 32i..32i+31) for the 16-column slice c
      u32x4 fa[2][4], fx[2][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          uint32_t v0 = xh[b][2 * c][d], v1 = xh[b][2 * c + 1][d];
          permlane32_swap(v0, v1);
          fa[0][c][d] = v0;
          fa[1][c][d] = v1;
          if (LX) {
            uint32_t w0 = xr[b][2 * c][d], w1 = xr[b][2 * c + 1][d];
            permlane32_swap(w0, w1);
            fx[0][c][d] = w0;
            fx[1][c][d] = w1;
          }
        }
      }
      const int kb = g * G + 64 * b;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int T = p.t0 + t;   // global tile
        const bool is_l2 = T < TR;
        const int n = is_l2 ? 32 * T + lr : 32 * (T - TR) + lr;
        const int nmax = is_l2 ? p.r : p.rl;
        const uint16_t* bsrc = (is_l2 ? p.l2 : p.lora) + (long)min(n, nmax - 1) * K + kb + 8 * h;
        const bool nok = n < nmax;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          u32x4 bf = ld16(bsrc + 16 * c);
          if (!nok) bf = u32x4{};
#pragma unroll
          for (int i = 0; i < 2; ++i)
            acc[l][i][t] = mfma_bf16_32x32x16(is_l2 ? fa[i][c] : fx[i][c], bf, acc[l][i][t]);
        }
      }
    }
    }   // layers
  }

  // ---- reduce the 4 waves (fixed order) and write this split's partial, layer by layer ----
#pragma unroll
  for (int l = 0; l < NL; ++l) {
  const ActParams& p = lp[l];
  const int TR = (p.r + 31) >> 5;
  const int RTp = p.RTp;
  float* dst = p.mid + (long)blockIdx.y * p.M * RTp;
  const int nval = p.r + p.rl;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        red[wave * 2048 + (32 * a + 8 * (i >> 2) + 4 * h + (i & 3)) * 32 + lr] = acc[l][a][t][i];
    __syncthreads();
    const int T = p.t0 + t;
    const bool is_l2 = T < TR;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int idx = tid + 256 * i;
      const int rr = idx >> 5, cc = idx & 31;
      const int grow = m0 + rr;
      const int j = is_l2 ? 32 * T + cc : 32 * (T - TR) + cc;
      const bool ok = is_l2 ? j < p.r : j < p.rl;
      if (grow < p.M && ok) {
        float v = ((red[idx] + red[2048 + idx]) + red[4096 + idx]) + red[6144 + idx];
        if (!is_l2) v *= p.lora_mult[j];
        dst[(long)grow * RTp + (is_l2 ? j : p.r + j)] = v;
      }
    }
    __syncthreads();
  }
  const int npad = RTp - nval;
  for (int idx = tid; idx < 64 * npad; idx += 256) {
    const int grow = m0 + idx / npad;
    if (grow < p.M) dst[(long)grow * RTp + nval + idx % npad] = 0.0f;
  }
  }   // layers

}

template <int G, int NT, int OPER, bool XHAT, bool QX, bool LX>
__global__ void __launch_bounds__(256) act_kernel(ActParams p) {
  act_tile<G, NT, OPER, XHAT, QX, LX>(&p);
}

// Sibling layers' activation passes over the same x in one launch (blockIdx.z = the layer):
// e3m2 codes, rank tiles of the low-rank down projection only (r <= 32), each layer with its own
// smoothing constants, factors and outputs.
template <int G>
__global__ void __launch_bounds__(256) act_siblings_kernel(ActSiblings s) {
  act_tile<G, 1, 3, false, false, false>(&s.layer[blockIdx.z]);
}

// The same passes with x read once: each workgroup runs all NL layers of its row block and split.
template <int G, int NL>
__global__ void __launch_bounds__(256) act_shared_x_kernel(ActSiblings s) {
  act_tile<G, 1, 3, false, false, false, NL>(s.layer);
}

// Final low-rank operand of the GEMM epilogue: the split partials summed in split order
// (a fixed order, so the result is deterministic), then split into bf16 hi and lo planes
// [M, 2, RTp] (the bf16 MFMA operands of mid @ l1cat^T).  One thread per 8 columns of a row.
__device__ __forceinline__ void mid_finalize_rows(const float* __restrict__ part, int S, int M, int RTp,
                                                  uint16_t* __restrict__ midp) {
  const int chunks = RTp / 8;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)M * chunks) return;
  const long m = idx / chunks;
  const int c = (int)(idx % chunks);
  const long plane = (long)M * RTp;
  const float* src = part + m * RTp + 8 * c;
  // the partials are loaded four splits at a time (past the last split the last one again, not
  // added), then added in split order
  f32x4 v0 = *reinterpret_cast<const f32x4*>(src), v1 = *reinterpret_cast<const f32x4*>(src + 4);
  for (int s0 = 1; s0 < S; s0 += 4) {
    f32x4 a0[4], a1[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long o = (long)min(s0 + j, S - 1) * plane;
      a0[j] = *reinterpret_cast<const f32x4*>(src + o);
      a1[j] = *reinterpret_cast<const f32x4*>(src + o + 4);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (s0 + j < S) {
        v0 += a0[j];
        v1 += a1[j];
      }
  }
  const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
  u32x4 hi, lo;
  split_hi_lo(v, hi, lo);
  uint16_t* dst = midp + m * 2 * RTp + 8 * c;
  *reinterpret_cast<u32x4*>(dst) = hi;
  *reinterpret_cast<u32x4*>(dst + RTp) = lo;
}

__global__ void __launch_bounds__(256) mid_finalize_kernel(const float* __restrict__ part, int S, int M, int RTp,
                                                           uint16_t* __restrict__ midp) {
  mid_finalize_rows(part, S, M, RTp, midp);
}

// The finalize of sibling layers' passes in one launch (blockIdx.y = the layer).
__global__ void __launch_bounds__(256) mid_finalize_siblings_kernel(ActSiblings s, int S) {
  const ActParams& p = s.layer[blockIdx.y];
  mid_finalize_rows(p.mid, S, p.M, p.RTp, s.head[blockIdx.y]);
}

// A4 quantizer for any group size G (a multiple of 16 dividing K), from x_hat (written by the act
// kernel in x_hat mode): the generic path behind group sizes other than 64 and 128.  One thread per
// (row, group), adjacent threads on adjacent groups of a row (contiguous x_hat reads):
//   sx = bf16(max(amax, bf16(1e-8)) / 7), q = clamp(rne(x_hat / sx), -8, 7)   (pack.py:17-21)
// with IEEE float32 division, written as the int8 GEMM operand (16 q, within each chunk of 8
// columns in the order k0 k2 k4 k6 k1 k3 k5 k7), the scales as bf16 [M, K/G] or u32 pairs
// [K/G, M], and optionally the canonical packed codes.
__global__ void quant_any_group_kernel(const uint16_t* __restrict__ xhat, long ldxh, int M, int K, int G,
                                       uint8_t* __restrict__ qa, uint16_t* __restrict__ sx, int sx_pairs,
                                       uint8_t* __restrict__ qx) {
  const int ngroups = K / G;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)M * ngroups) return;
  const long m = idx / ngroups;
  const int g = (int)(idx % ngroups);
  const uint16_t* src = xhat + m * ldxh + (long)g * G;
  uint32_t amb = 0;
  for (int c = 0; c < G; c += 8) {
    const u32x4 v = ld16(src + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      amb = max(amb, v[e] & 0x7FFFu);
      amb = max(amb, (v[e] >> 16) & 0x7FFFu);
    }
  }
  // inf / NaN bit patterns compare largest and propagate through the division as in the reference
  const float sc = round_bf16(fmaxf(bf16f((uint16_t)amb), kBf16OneEMinus8) / 7.0f);
  const uint32_t sb = __float_as_uint(sc) >> 16;
  if (sx_pairs) reinterpret_cast<uint32_t*>(sx)[(long)g * M + m] = sb * 0x10001u;
  else sx[m * ngroups + g] = (uint16_t)sb;
  uint8_t* dst = qa + m * K + (long)g * G;
  uint8_t* pk = qx ? qx + m * (K / 2) + (long)g * G / 2 : nullptr;
  for (int c = 0; c < G; c += 8) {
    const u32x4 v = ld16(src + c);
    int q[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      q[2 * e] = (int)fminf(fmaxf(__builtin_rintf(bf16lo(v[e]) / sc), -8.0f), 7.0f);
      q[2 * e + 1] = (int)fminf(fmaxf(__builtin_rintf(bf16hi(v[e]) / sc), -8.0f), 7.0f);
    }
    // operand bytes: even columns first, then odd (the layout of the fast kernels' int8 operand)
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo |= (uint32_t)(uint8_t)(int8_t)(16 * q[2 * e]) << (8 * e);
      hi |= (uint32_t)(uint8_t)(int8_t)(16 * q[2 * e + 1]) << (8 * e);
    }
    *reinterpret_cast<u32x2*>(dst + c) = u32x2{lo, hi};
    if (pk) {
      uint32_t w = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) w |= (uint32_t)(q[e] + 8) << (4 * e);
      *reinterpret_cast<uint32_t*>(pk + c / 2) = w;
    }
  }
}

// (s, RN(1/s)) in float32 for a bf16 smoothing vector: computed once per layer.
__global__ void prepare_smooth_kernel(const uint16_t* __restrict__ s, float* __restrict__ srs, int K) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < K) {
    const float v = bf16f(s[i]);
    srs[i] = v;
    srs[K + i] = 1.0f / v;
  }
}

template <int G, int OPER, bool XHAT, bool QX, bool MIDONLY = false>
hipError_t launch_act_nt(const ActParams& p, int nt, dim3 grid, hipStream_t st) {
  // the first launch (t0 = 0) may hold LoRA tiles only when it has two or more tiles (tile 0 is
  // L2); a down-projection-only launch may hold any mix
  switch (nt) {
    case 1: act_kernel<G, 1, OPER, XHAT, QX, MIDONLY><<<grid, 256, 0, st>>>(p); break;
    case 2: act_kernel<G, 2, OPER, XHAT, QX, true><<<grid, 256, 0, st>>>(p); break;
    case 3: act_kernel<G, 3, OPER, XHAT, QX, true><<<grid, 256, 0, st>>>(p); break;
    case 4: act_kernel<G, 4, OPER, XHAT, QX, true><<<grid, 256, 0, st>>>(p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int G>
hipError_t launch_act_g(const ActParams& p, int nt, int oper, bool xhat, dim3 grid, hipStream_t st) {
  if (p.t0 > 0) {   // down projections only
    if (oper != 0 || xhat) return hipErrorInvalidValue;
    return launch_act_nt<G, 0, false, false, true>(p, nt, grid, st);
  }
  if (oper == 3 && !xhat && !p.qx) return launch_act_nt<G, 3, false, false>(p, nt, grid, st);
  if (oper == 3 && !xhat) return launch_act_nt<G, 3, false, true>(p, nt, grid, st);
  if (oper == 1 && !xhat) return launch_act_nt<G, 1, false, true>(p, nt, grid, st);
  if (oper == 1 && xhat) return launch_act_nt<G, 1, true, true>(p, nt, grid, st);
  if (oper == 2 && !xhat) return launch_act_nt<G, 2, false, true>(p, nt, grid, st);
  if (oper == 0 && xhat) return launch_act_nt<G, 0, true, true>(p, nt, grid, st);
  return hipErrorInvalidValue;
}

}  // namespace

int act_splits(int M, int K, int G) {
  // 512 workgroups fill the 256 CUs once (two 4-wave workgroups per CU): as many K splits as keep
  // row_tiles * splits within that, so no workgroups are left over for a second round
  const int row_tiles = (M + 63) / 64;
  const int ngroups = K / G;
  int s = 512 / row_tiles;
  const int smax = ngroups / 4 > 0 ? ngroups / 4 : 1;
  if (s > smax) s = smax;
  if (s < 1) s = 1;
  return s;
}

hipError_t launch_act(const ActParams& p, int G, int nt, int oper, bool xhat, int splits, hipStream_t st) {
  dim3 grid((p.M + 63) / 64, splits);
  if (G == 64) return launch_act_g<64>(p, nt, oper, xhat, grid, st);
  if (G == 128) return launch_act_g<128>(p, nt, oper, xhat, grid, st);
  return hipErrorInvalidValue;
}

hipError_t launch_act_siblings(const ActSiblings& s, int G, int splits, hipStream_t st) {
  if (s.count < 1 || s.count > MAX_SIBLINGS) return hipErrorInvalidValue;
  for (int i = 0; i < s.count; ++i)
    if (s.layer[i].M != s.layer[0].M || s.layer[i].K != s.layer[0].K || s.layer[i].r > 32 || s.layer[i].rl ||
        s.layer[i].t0)
      return hipErrorInvalidValue;
  if (G != 64 && G != 128) return hipErrorInvalidValue;
  // One workgroup per layer, row block and split (blockIdx.z = the layer), or with
  // SVDQ_ACT_SIBLINGS=shared_x x read once for all layers (act_shared_x_kernel; same results, but
  // one wave per SIMD and a quarter of the workgroups: 119 against 79 us for the four attention
  // inputs at M = 4352, 60 against 44 us for ff.gate / ff.up).  Group 128 with three or four
  // layers would spill: per layer.
  const char* e = getenv("SVDQ_ACT_SIBLINGS");
  if (s.count >= 2 && (G == 64 || s.count == 2) && e && !strcmp(e, "shared_x")) {
    const dim3 grid((s.layer[0].M + 63) / 64, splits);
#define SVDQ_SHARED_X(NL)                                                            \
  if (s.count == NL) {                                                               \
    if (G == 64) act_shared_x_kernel<64, NL><<<grid, 256, 0, st>>>(s);               \
    else if (NL == 2) act_shared_x_kernel<128, 2><<<grid, 256, 0, st>>>(s);          \
  }
    SVDQ_SHARED_X(2)
    SVDQ_SHARED_X(3)
    SVDQ_SHARED_X(4)
#undef SVDQ_SHARED_X
  } else {
    const dim3 grid((s.layer[0].M + 63) / 64, splits, s.count);
    if (G == 64) act_siblings_kernel<64><<<grid, 256, 0, st>>>(s);
    else act_siblings_kernel<128><<<grid, 256, 0, st>>>(s);
  }
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  const long n = (long)s.layer[0].M * (s.layer[0].RTp / 8);
  mid_finalize_siblings_kernel<<<dim3((unsigned)((n + 255) / 256), s.count), 256, 0, st>>>(s, splits);
  return hipGetLastError();
}

hipError_t launch_mid_finalize(const float* part, int S, int M, int RTp, uint16_t* midp, hipStream_t st) {
  const long n = (long)M * (RTp / 8);
  mid_finalize_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(part, S, M, RTp, midp);
  return hipGetLastError();
}

hipError_t launch_quant_any_group(const uint16_t* xhat, long ldxh, int M, int K, int G, uint8_t* qa, uint16_t* sx,
                                  int sx_pairs, uint8_t* qx, hipStream_t st) {
  const long n = (long)M * (K / G);
  quant_any_group_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(xhat, ldxh, M, K, G, qa, sx, sx_pairs, qx);
  return hipGetLastError();
}

hipError_t launch_prepare_smooth(const uint16_t* s, float* srs, int K, hipStream_t st) {
  prepare_smooth_kernel<<<(K + 255) / 256, 256, 0, st>>>(s, srs, K);
  return hipGetLastError();
}

}  // namespace svdq
