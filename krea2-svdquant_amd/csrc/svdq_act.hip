// Fused activation pass for the SVDQuant linear on gfx950 (one HBM read of x).
//
//   x_hat = bf16(x / s)                                  quant/svd.py:121-122
//   sx    = bf16(max(amax_g |x_hat|, bf16(1e-8)) / 7)    quant/pack.py:20
//   qx    = clamp(rne(x_hat / sx), -8, 7), packed         quant/pack.py:21, :53-56
//   mid   = x_hat @ L2^T            (low-rank down)      quant/svd.py:159
//   lmid  = mult * (x @ A^T)        (LoRA down, raw x)    runtime/linear.py:42-45
//
// Work split: a workgroup (4 waves) owns 64 rows and a contiguous range of K-groups (one
// "split"); wave w takes every 4th group of the range.  Within a wave, lane l handles rows
// l%32 and 32 + l%32 and, of each group, the G/2 contiguous columns of lane-half l/32, which
// is exactly the A-operand layout of the 32x32x16 bf16 MFMA, so mid/lmid accumulate in
// registers without an LDS round trip.  Per-wave partials are summed in a fixed wave order
// in LDS; partials of the splits of a row tile are summed in a fixed split order by the
// last workgroup to finish (atomic arrival counter, reset by that workgroup), so results are
// deterministic.
#include "svdq_common.h"
#include "svdq_kernels.h"

namespace svdq {

namespace {

constexpr float kBf16OneEMinus8 = 1.00117176e-08f;  // bf16(1e-8)
constexpr float kRcp7 = 0.142857149f;               // RN(1/7)
constexpr float kMagic8 = 12582920.0f;              // 1.5 * 2^23 + 8

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ f32x4 ld16f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// Smooth 8 bf16 values (one dword quad) by s with the reciprocal-corrected division;
// exact IEEE division where the caller asks for it (element out of the fast path's range).
template <bool PER_ELEMENT_GUARD>
__device__ __forceinline__ uint32_t smooth_pair(uint32_t d, float s0, float r0, float s1, float r1,
                                                bool exact) {
  const float a = bf16lo(d), b = bf16hi(d);
  float qa, qb;
  if (exact) {
    qa = a / s0;
    qb = b / s1;
  } else {
    qa = div_rcp(a, s0, r0);
    qb = div_rcp(b, s1, r1);
    if (PER_ELEMENT_GUARD) {
      if (!(fabsf(qa) >= 0x1p-90f && fabsf(qa) <= 0x1p100f) && a != 0.0f) qa = a / s0;
      if (!(fabsf(qb) >= 0x1p-90f && fabsf(qb) <= 0x1p100f) && b != 0.0f) qb = b / s1;
      qa = __builtin_copysignf(qa, a * s0);
      qb = __builtin_copysignf(qb, b * s1);
    }
  }
  return pack_bf16x2(qa, qb);
}

template <int G, int NT, bool QUANT, bool XHAT>
__global__ void __launch_bounds__(256) act_kernel(ActParams p) {
  constexpr int HALF = G / 2;   // columns of a group held by one lane
  constexpr int CH = G / 16;    // 8-column chunks per lane per group == MFMA K=16 slices
  __shared__ float red[4][64 * 32];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, h = lane >> 5, lr = lane & 31;
  const int m0 = blockIdx.x * 64;
  const int row[2] = {m0 + lr, m0 + 32 + lr};
  const bool rok[2] = {row[0] < p.M, row[1] < p.M};
  const int K = p.K;
  const int ngroups = K / G;
  const int gb = blockIdx.y * p.gps;
  const int ge = min(ngroups, gb + p.gps);
  const int TR = (p.r + 31) >> 5;
  const float* __restrict__ sv = p.srs;
  const float* __restrict__ rv = p.srs + K;

  f32x16 acc[2][NT];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[a][t] = f32x16{};

  for (int g = gb + wave; g < ge; g += 4) {
    const int kb = g * G + h * HALF;
    u32x4 xr[2][CH], xh[2][CH];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int c = 0; c < CH; ++c)
        xr[a][c] = rok[a] ? ld16(p.x + (long)row[a] * p.ldx + kb + 8 * c) : u32x4{};

    // ---- smoothing: x_hat = bf16(x / s) ----
    auto smooth_all = [&](bool exact) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const f32x4 s0 = ld16f(sv + kb + 8 * c), s1 = ld16f(sv + kb + 8 * c + 4);
        const f32x4 r0 = ld16f(rv + kb + 8 * c), r1 = ld16f(rv + kb + 8 * c + 4);
        const float s8[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        const float r8[8] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            xh[a][c][e] = smooth_pair<XHAT>(xr[a][c][e], s8[2 * e], r8[2 * e], s8[2 * e + 1],
                                            r8[2 * e + 1], exact);
      }
    };
    smooth_all(p.exact != 0);

    if (QUANT) {
      float am[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        float m = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            m = fmaxf(m, fmaxf(fabsf(bf16lo(xh[a][c][e])), fabsf(bf16hi(xh[a][c][e]))));
        am[a] = fmaxf(m, __shfl_xor(m, 32));
      }
      // The reciprocal division is exact while quotients stay normal; a group whose
      // absmax leaves [2^-90, 2^100] is recomputed with IEEE division.
      const bool bad0 = am[0] != 0.0f && !(am[0] >= 0x1p-90f && am[0] <= 0x1p100f);
      const bool bad1 = am[1] != 0.0f && !(am[1] >= 0x1p-90f && am[1] <= 0x1p100f);
      if (!p.exact && (bad0 || bad1)) {
        smooth_all(true);
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          float m = 0.0f;
#pragma unroll
          for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              m = fmaxf(m, fmaxf(fabsf(bf16lo(xh[a][c][e])), fabsf(bf16hi(xh[a][c][e]))));
          am[a] = fmaxf(m, __shfl_xor(m, 32));
        }
      }
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const float sc = round_bf16(div_rcp(fmaxf(am[a], kBf16OneEMinus8), 7.0f, kRcp7));
        const float rsc = 1.0f / sc;
        uint32_t codes[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          uint32_t w = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float ta = div_rcp(bf16lo(xh[a][c][e]), sc, rsc);
            float tb = div_rcp(bf16hi(xh[a][c][e]), sc, rsc);
            ta = fminf(fmaxf(ta, -8.0f), 7.0f) + kMagic8;
            tb = fminf(fmaxf(tb, -8.0f), 7.0f) + kMagic8;
            w |= (__float_as_uint(ta) & 0xFu) << (8 * e);
            w |= (__float_as_uint(tb) & 0xFu) << (8 * e + 4);
          }
          codes[c] = w;
        }
        if (rok[a]) {
          uint8_t* dst = p.qx + (long)row[a] * (K / 2) + kb / 2;
#pragma unroll
          for (int c = 0; c < CH; c += 4)
            *reinterpret_cast<u32x4*>(dst + 4 * c) = u32x4{codes[c], codes[c + 1], codes[c + 2], codes[c + 3]};
          if (h == 0) p.sx[(long)row[a] * ngroups + g] = (uint16_t)(__float_as_uint(sc) >> 16);
        }
      }
    }
    if (XHAT) {
#pragma unroll
      for (int a = 0; a < 2; ++a)
        if (rok[a])
#pragma unroll
          for (int c = 0; c < CH; ++c)
            *reinterpret_cast<u32x4*>(p.xhat + (long)row[a] * p.ldxh + kb + 8 * c) = xh[a][c];
    }

    // ---- low-rank down (x_hat @ L2^T) and LoRA down (x @ A^T) on MFMA ----
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool is_l2 = t < TR;
      const int n = is_l2 ? 32 * t + lr : 32 * (t - TR) + lr;
      const bool nok = is_l2 ? n < p.r : n < p.rl;
      const uint16_t* bsrc = is_l2 ? p.l2 : p.lora;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const u32x4 b = nok ? ld16(bsrc + (long)n * K + kb + 8 * c) : u32x4{};
#pragma unroll
        for (int a = 0; a < 2; ++a) acc[a][t] = mfma_bf16_32x32x16(is_l2 ? xh[a][c] : xr[a][c], b, acc[a][t]);
      }
    }
  }

  // ---- reduce the 4 waves (fixed order) and write this split's partial ----
  const int S = gridDim.y;
  const int RTp = p.RTp;
  float* dst = (S == 1) ? p.mid : p.midp + (long)blockIdx.y * p.M * RTp;
  const int nval = p.r + p.rl;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        red[wave][(32 * a + 8 * (i >> 2) + 4 * h + (i & 3)) * 32 + lr] = acc[a][t][i];
    __syncthreads();
    const bool is_l2 = t < TR;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int idx = tid + 256 * i;
      const int rr = idx >> 5, cc = idx & 31;
      const int grow = m0 + rr;
      const int j = is_l2 ? 32 * t + cc : 32 * (t - TR) + cc;
      const bool ok = is_l2 ? j < p.r : j < p.rl;
      if (grow < p.M && ok) {
        float v = ((red[0][idx] + red[1][idx]) + red[2][idx]) + red[3][idx];
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

  if (S > 1) {
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(p.counters + blockIdx.x, 1) == S - 1);
    __syncthreads();
    if (s_last) {
      __threadfence();
      for (int idx = tid; idx < 64 * RTp; idx += 256) {
        const int grow = m0 + idx / RTp, cc = idx % RTp;
        if (grow >= p.M) continue;
        float v = 0.0f;
        for (int s = 0; s < S; ++s) v += p.midp[((long)s * p.M + grow) * RTp + cc];
        p.mid[(long)grow * RTp + cc] = v;
      }
      if (tid == 0) atomicExch(p.counters + blockIdx.x, 0);
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

template <int G, bool QUANT, bool XHAT>
hipError_t launch_act_nt(const ActParams& p, int nt, dim3 grid, hipStream_t st) {
  switch (nt) {
    case 1: act_kernel<G, 1, QUANT, XHAT><<<grid, 256, 0, st>>>(p); break;
    case 2: act_kernel<G, 2, QUANT, XHAT><<<grid, 256, 0, st>>>(p); break;
    case 3: act_kernel<G, 3, QUANT, XHAT><<<grid, 256, 0, st>>>(p); break;
    case 4: act_kernel<G, 4, QUANT, XHAT><<<grid, 256, 0, st>>>(p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int G>
hipError_t launch_act_g(const ActParams& p, int nt, bool quant, bool xhat, dim3 grid, hipStream_t st) {
  if (quant && xhat) return launch_act_nt<G, true, true>(p, nt, grid, st);
  if (quant) return launch_act_nt<G, true, false>(p, nt, grid, st);
  if (xhat) return launch_act_nt<G, false, true>(p, nt, grid, st);
  return hipErrorInvalidValue;
}

}  // namespace

int act_splits(int M, int K, int G) {
  const int row_tiles = (M + 63) / 64;
  const int ngroups = K / G;
  int s = (512 + row_tiles - 1) / row_tiles;
  const int smax = ngroups / 4 > 0 ? ngroups / 4 : 1;
  if (s > smax) s = smax;
  if (s < 1) s = 1;
  return s;
}

hipError_t launch_act(const ActParams& p, int G, int nt, bool quant, bool xhat, int splits, hipStream_t st) {
  dim3 grid((p.M + 63) / 64, splits);
  if (G == 64) return launch_act_g<64>(p, nt, quant, xhat, grid, st);
  if (G == 128) return launch_act_g<128>(p, nt, quant, xhat, grid, st);
  return hipErrorInvalidValue;
}

hipError_t launch_prepare_smooth(const uint16_t* s, float* srs, int K, hipStream_t st) {
  prepare_smooth_kernel<<<(K + 255) / 256, 256, 0, st>>>(s, srs, K);
  return hipGetLastError();
}

}  // namespace svdq
