// Normalization kernels of the stand-in Krea-2 block, around its quantized linears.
//
// The reference runs its blocks in diffusers (reference src/krea2_svdquant/transformer.py:46-59),
// whose internals it does not contain; the stand-in block of this package normalizes with
//   h = bf16(bf16(x * rsqrt(mean(x^2) + eps) * w) + shift)       (w = 1 + scale: adaptive RMS norm)
// ahead of to_q/to_k/to_v/to_gate and ff.gate/ff.up, and per head of 128 channels of q and k
//   n = bf16(t * rsqrt(mean(t^2) + eps)),  then the rotate-half rotary embedding on pairs
//   (n1, n2) = (n[j], n[j + 64]):  o1 = bf16(fma(-n2, s, bf16(n1 c))),  o2 = bf16(fma(n1, s, bf16(n2 c)))
// with c = cos[tok][j], s = sin[tok][j].  Each rounding sits where the torch ops of the block's
// CPU path round (F.rms_norm, the bf16 add, torch.mul and addcmul), with the mean of squares
// accumulated in float32 (the summation order differs from torch's kernels, so an output can move
// by one bf16 ulp where the float result lies at a rounding boundary).  Both kernels are
// HBM-bound: one read and one write of the activation.
#include "svdq_common.h"
#include "svdq_kernels.h"

namespace svdq {
namespace {

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// The gated residual add bf16(x + g * v) in one rounding (torch.addcmul(x, g, v)) on a chunk of 8.
__device__ __forceinline__ u32x4 addcmul8(u32x4 x, u32x4 g, u32x4 v) {
  u32x4 o;
#pragma unroll
  for (int d = 0; d < 4; ++d)
    o[d] = pack_bf16x2(__builtin_fmaf(bf16lo(g[d]), bf16lo(v[d]), bf16lo(x[d])),
                       __builtin_fmaf(bf16hi(g[d]), bf16hi(v[d]), bf16hi(x[d])));
  return o;
}

// Adaptive RMS norm, one 256-thread workgroup per row.  Pass 1 sums the squares of the row's
// 16-byte chunks (thread t takes chunks t, t + 256, ...; the first NR of them stay in registers),
// pass 2 writes the normalized, weighted and shifted chunks (chunks beyond NR re-read from L2).
// RES: the row is first formed as the gated residual x + g * v (g a vector [H], v the layer output
// [T, ldv]) and written to xo, and that row is normalized (chunks beyond NR re-read from xo).
template <int NR, bool RES = false>
__global__ void __launch_bounds__(256) rms_norm_modulate_kernel(const uint16_t* __restrict__ x, long ldx,
                                                                const uint16_t* __restrict__ w,
                                                                const uint16_t* __restrict__ shift, int H,
                                                                float eps, uint16_t* __restrict__ y, long ldy,
                                                                const uint16_t* __restrict__ v = nullptr,
                                                                long ldv = 0, const uint16_t* __restrict__ g = nullptr,
                                                                uint16_t* __restrict__ xo = nullptr, long ldxo = 0) {
  __shared__ float part[4];
  const int tid = threadIdx.x, nc = H / 8;
  const uint16_t* xr = x + (long)blockIdx.x * ldx;
  uint16_t* xor_ = RES ? xo + (long)blockIdx.x * ldxo : nullptr;
  auto row_chunk = [&](int c) {   // the chunk to normalize (RES: formed and stored first)
    u32x4 r = ld16(xr + 8 * c);
    if (RES) {
      r = addcmul8(r, ld16(g + 8 * c), ld16(v + (long)blockIdx.x * ldv + 8 * c));
      *reinterpret_cast<u32x4*>(xor_ + 8 * c) = r;
    }
    return r;
  };
  u32x4 keep[NR];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int c = tid + 256 * i;
    keep[i] = c < nc ? row_chunk(c) : u32x4{};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float a = bf16lo(keep[i][d]), b = bf16hi(keep[i][d]);
      ss = __builtin_fmaf(a, a, ss);
      ss = __builtin_fmaf(b, b, ss);
    }
  }
  for (int c = tid + 256 * NR; c < nc; c += 256) {
    const u32x4 v = row_chunk(c);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float a = bf16lo(v[d]), b = bf16hi(v[d]);
      ss = __builtin_fmaf(a, a, ss);
      ss = __builtin_fmaf(b, b, ss);
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const float r = rsqrtf((part[0] + part[1] + part[2] + part[3]) / (float)H + eps);
  uint16_t* yr = y + (long)blockIdx.x * ldy;
  auto put = [&](int c, u32x4 v) {
    const u32x4 wv = ld16(w + 8 * c), sv = ld16(shift + 8 * c);
    u32x4 o;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float n0 = round_bf16(bf16lo(v[d]) * r * bf16lo(wv[d]));
      const float n1 = round_bf16(bf16hi(v[d]) * r * bf16hi(wv[d]));
      o[d] = pack_bf16x2(n0 + bf16lo(sv[d]), n1 + bf16hi(sv[d]));
    }
    *reinterpret_cast<u32x4*>(yr + 8 * c) = o;
  };
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int c = tid + 256 * i;
    if (c < nc) put(c, keep[i]);
  }
  for (int c = tid + 256 * NR; c < nc; c += 256) put(c, ld16((RES ? xor_ : xr) + 8 * c));
}

// Per-head RMS norm and rotary embedding, one wave per (token, head) row of 128 channels: lane j
// holds the rotary pair (j, j + 64).  Rows are contiguous (t and out [T, heads, 128]); the
// tables cos / sin are [T, ldcs] bf16, of which the first 64 columns are read.
__global__ void __launch_bounds__(256) head_rms_rope_kernel(const uint16_t* __restrict__ t, long rows, int heads,
                                                            const uint16_t* __restrict__ cs,
                                                            const uint16_t* __restrict__ sn, long ldcs, float eps,
                                                            uint16_t* __restrict__ out) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int j = threadIdx.x & 63;
  const long tok = row / heads;
  const uint16_t* tr = t + row * 128;
  const float x1 = bf16f(tr[j]), x2 = bf16f(tr[j + 64]);
  const float r = rsqrtf(wave_sum(__builtin_fmaf(x1, x1, x2 * x2)) / 128.0f + eps);
  const float n1 = round_bf16(x1 * r), n2 = round_bf16(x2 * r);
  const float c = bf16f(cs[tok * ldcs + j]), s = bf16f(sn[tok * ldcs + j]);
  const float o1 = __builtin_fmaf(-n2, s, round_bf16(n1 * c));
  const float o2 = __builtin_fmaf(n1, s, round_bf16(n2 * c));
  const uint32_t pk = pack_bf16x2(o1, o2);
  uint16_t* orow = out + row * 128;
  orow[j] = (uint16_t)(pk & 0xFFFFu);
  orow[j + 64] = (uint16_t)(pk >> 16);
}

// The same with 16-byte accesses: 8 lanes per row (32 rows per workgroup), lane j holding
// channels 8 j .. 8 j + 7 and their rotary partners 64 + 8 j ..; the mean of squares reduces over
// the 8 lanes.  Needs t, out, cos, sin 16-byte aligned and ldcs % 8 == 0.
__global__ void __launch_bounds__(256) head_rms_rope_vec_kernel(const uint16_t* __restrict__ t, long rows,
                                                                int heads, const uint16_t* __restrict__ cs,
                                                                const uint16_t* __restrict__ sn, long ldcs,
                                                                float eps, uint16_t* __restrict__ out) {
  const long row = (long)blockIdx.x * 32 + (threadIdx.x >> 3);
  if (row >= rows) return;   // a row's 8 lanes leave together: the shuffles stay within live lanes
  const int j = threadIdx.x & 7;
  const long tok = row / heads;
  const u32x4 a = ld16(t + row * 128 + 8 * j), b = ld16(t + row * 128 + 64 + 8 * j);
  float ss = 0.0f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    ss = __builtin_fmaf(bf16lo(a[d]), bf16lo(a[d]), ss);
    ss = __builtin_fmaf(bf16hi(a[d]), bf16hi(a[d]), ss);
    ss = __builtin_fmaf(bf16lo(b[d]), bf16lo(b[d]), ss);
    ss = __builtin_fmaf(bf16hi(b[d]), bf16hi(b[d]), ss);
  }
#pragma unroll
  for (int off = 4; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  const float r = rsqrtf(ss / 128.0f + eps);
  const u32x4 c = ld16(cs + tok * ldcs + 8 * j), sv = ld16(sn + tok * ldcs + 8 * j);
  u32x4 o1, o2;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float p1[2], p2[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float x1 = e ? bf16hi(a[d]) : bf16lo(a[d]), x2 = e ? bf16hi(b[d]) : bf16lo(b[d]);
      const float cc = e ? bf16hi(c[d]) : bf16lo(c[d]), ssn = e ? bf16hi(sv[d]) : bf16lo(sv[d]);
      const float n1 = round_bf16(x1 * r), n2 = round_bf16(x2 * r);
      p1[e] = __builtin_fmaf(-n2, ssn, round_bf16(n1 * cc));
      p2[e] = __builtin_fmaf(n1, ssn, round_bf16(n2 * cc));
    }
    o1[d] = pack_bf16x2(p1[0], p1[1]);
    o2[d] = pack_bf16x2(p2[0], p2[1]);
  }
  *reinterpret_cast<u32x4*>(out + row * 128 + 8 * j) = o1;
  *reinterpret_cast<u32x4*>(out + row * 128 + 64 + 8 * j) = o2;
}

}  // namespace

hipError_t launch_rms_norm_modulate(const uint16_t* x, long ldx, const uint16_t* w, const uint16_t* shift, int T,
                                    int H, float eps, uint16_t* y, long ldy, hipStream_t st) {
  // rows of up to 4 * 256 chunks (H <= 8192) stay in registers between the passes
  rms_norm_modulate_kernel<4><<<T, 256, 0, st>>>(x, ldx, w, shift, H, eps, y, ldy);
  return hipGetLastError();
}

hipError_t launch_residual_rms_norm_modulate(const uint16_t* x, long ldx, const uint16_t* v, long ldv,
                                             const uint16_t* g, const uint16_t* w, const uint16_t* shift, int T, int H,
                                             float eps, uint16_t* xo, long ldxo, uint16_t* y, long ldy,
                                             hipStream_t st) {
  rms_norm_modulate_kernel<4, true><<<T, 256, 0, st>>>(x, ldx, w, shift, H, eps, y, ldy, v, ldv, g, xo, ldxo);
  return hipGetLastError();
}

hipError_t launch_head_rms_rope(const uint16_t* t, int T, int heads, const uint16_t* cs, const uint16_t* sn,
                                long ldcs, float eps, uint16_t* out, hipStream_t st) {
  const long rows = (long)T * heads;
  const bool vec = ((reinterpret_cast<uintptr_t>(t) | reinterpret_cast<uintptr_t>(out) |
                     reinterpret_cast<uintptr_t>(cs) | reinterpret_cast<uintptr_t>(sn)) & 15) == 0 && ldcs % 8 == 0;
  if (vec)
    head_rms_rope_vec_kernel<<<(unsigned)((rows + 31) / 32), 256, 0, st>>>(t, rows, heads, cs, sn, ldcs, eps, out);
  else
    head_rms_rope_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, st>>>(t, rows, heads, cs, sn, ldcs, eps, out);
  return hipGetLastError();
}

}  // namespace svdq
