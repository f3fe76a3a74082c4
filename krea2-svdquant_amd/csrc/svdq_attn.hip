// Softmax attention of the stand-in Krea-2 block on gfx950 (flash-attention forward, bf16).
//
//   o[t, h, :] = sum_u softmax_u(scale * q[t, h, :] . k[u, h / G, :]) v[u, h / G, :]
//
// with G = heads / kv_heads query heads per KV head (grouped-query attention), no mask, head
// dimension 128: the attention of the block the reference runs through diffusers
// (src/krea2_svdquant/transformer.py:46-59), which the stand-in computes with PyTorch's
// scaled_dot_product_attention.  Scores and the softmax statistics are float32, the
// probabilities enter the P V product as bf16 (as in the fused SDPA kernels), o is float32 until
// the final bf16 rounding.
//
// Key / value tiles of 64 rows stream through LDS, double-buffered (the next tile's global loads
// are in flight while the current one is used, one barrier per tile); a wave takes 32 QB queries
// and works through each tile in two halves of 32 keys:
//   S^T = K Q^T    (A = K rows from LDS, B = the wave's Q in VGPRs; one K fragment read serves the
//                  QB query blocks)
//   softmax on S^T: a lane holds one query (column) and 16 of the half's 32 keys, so the maximum
//                  is lane-local plus one exchange between the lane halves; the row sum (of the
//                  bf16 probabilities the product uses) stays per lane until the end
//   O^T += V^T P^T (A = V^T from LDS, B = P^T straight from the softmax registers)
// P^T's registers hold, for lane half h and element e of a 16-key slice, the key
// 8 (e / 4) + 4 h + e % 4 (the accumulator layout of S^T); V is written to LDS transposed with
// each slice's keys permuted to that order, so one 16-byte read gives the matching A operand.
//
// Two kernels, one launch after the other on the same stream:
//  * attn_fast_kernel (QB = 2, one wave per SIMD, O in AGPRs).  Each query's exponent offset is
//    its maximum over the first 32 keys and never moves, so the output accumulators are touched
//    by MFMAs only (an offset that follows the running maximum needs the output rescaled on the
//    VALU, which makes the compiler shuttle the 128 accumulators between AGPRs and VGPRs every
//    tile).  Later probabilities may exceed 1; up to 2^64 they are exact in bf16 / float32.  A
//    wave whose scores rise further above the offset, or whose output is not finite, marks
//    itself in the flag workspace (every wave writes its entry, so it needs no clearing) and
//    stores nothing.
//  * attn_safe_kernel (QB = 1, two waves per SIMD): the running-maximum formulation, output
//    rescaled every tile.  A workgroup runs only if a fast wave of its queries was marked, and
//    then writes those queries.
#include "svdq_common.h"
#include "svdq_kernels.h"

namespace svdq {
namespace {

constexpr int AD = 128;               // head dimension
constexpr int ABN = 64;               // keys per tile
constexpr int KPITCH = AD * 2 + 16;   // LDS bytes per K row (272: 16 rows of a read hit distinct banks)
constexpr int VPITCH = ABN * 2 + 16;  // LDS bytes per V^T row (144)
constexpr float OFFSET_LIMIT = 64.0f; // log2 units above the fixed offset the fast kernel accepts

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// position of key kk (0..15 within a 16-key slice) in the V^T row: lane half (kk >> 2) & 1,
// element (kk & 3) + 4 ((kk >> 3) & 1)
__device__ __forceinline__ int slice_pos(int kk) { return 8 * ((kk >> 2) & 1) + 4 * ((kk >> 3) & 1) + (kk & 3); }

// max / sum over the two lane halves (lanes l and l ^ 32)
__device__ __forceinline__ float half_max(float v) {
  uint32_t a = __float_as_uint(v), b = a;
  permlane32_swap(a, b);
  return fmaxf(__uint_as_float(a), __uint_as_float(b));
}
__device__ __forceinline__ float half_sum(float v) {
  uint32_t a = __float_as_uint(v), b = a;
  permlane32_swap(a, b);
  return __uint_as_float(a) + __uint_as_float(b);
}

// The fast kernel's MFMAs as inline asm, so that the register classes are fixed: the scores in
// VGPRs (read by the softmax), the output accumulators in AGPRs (read only at the end).  The
// compiler does not see their hazards:
//  * an accumulator is only ever its own srcC (full overlap: no wait states);
//  * k-step 0 of the scores uses a zero srcC, so no VALU-written zeros feed an MFMA;
//  * the scores are read by VALU after score_fence (an 8-pass MFMA's result: 11 wait states);
//  * the probabilities (VALU-written B operands) are read after 5 wait states;
//  * the output is read after out_fence (2 x 16 wait states).
__device__ __forceinline__ void mfma_score0(f32x16& acc, u32x4 a, u32x4 b) {
  asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_score(f32x16& acc, u32x4 a, u32x4 b) {
  asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_out(f32x16& acc, u32x4 a, u32x4 b) {
  asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Work of the fast kernel: items (head, block of 256 queries), item = head * nq + block.  The
// items that fill whole rounds over the CUs run one workgroup each; the rest (a last, partly
// filled round) are cut into `split` pieces along the keys -- `per` key tiles each -- whose
// partial outputs attn_combine_kernel merges, so that the last round takes about 1 / split of
// a full item's time.
struct AttnPlan {
  int nq, items, nmain, tail, split, per;
};
__host__ __device__ inline AttnPlan attn_plan(int T, int H, int cus) {
  AttnPlan pl;
  pl.nq = (T + 255) / 256;
  pl.items = pl.nq * H;
  pl.nmain = pl.items / cus * cus;
  pl.tail = pl.items - pl.nmain;
  const int nt = (T + ABN - 1) / ABN;
  int split = pl.tail ? cus / pl.tail : 1;
  split = split < 1 ? 1 : split > 8 ? 8 : split > nt ? nt : split;
  pl.per = (nt + split - 1) / split;
  pl.split = (nt + pl.per - 1) / pl.per;   // no empty piece
  return pl;
}
constexpr int ATTN_CUS = 256;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int* flags;        // [H, nflag], one per fast wave (64 queries): 1 = written by the safe kernel
  int nflag;
  int T, H, Hkv;
  long ldq, ldkv, ldo;
  float scale_log2;
  AttnPlan plan;
  float* part_o;     // [tail * split, 256, 128] unnormalized partial outputs of the pieces
  float* part_ml;    // [tail * split, 256, 2]: exponent offset (log2 units), row sum
  int* part_flag;    // [tail * split, 4]: a piece's wave past the offset limit
};

template <bool FAST>
__device__ __forceinline__ void attn_body(const AttnArgs& p) {
  constexpr int QB = FAST ? 2 : 1;            // 32-query blocks per wave
  constexpr int ABM = 4 * 32 * QB;            // queries per workgroup (4 waves)
  __shared__ __attribute__((aligned(16))) uint8_t sK[2][ABN * KPITCH];
  __shared__ __attribute__((aligned(16))) uint8_t sV[2][AD * VPITCH];
  const int T = p.T;
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // fast kernel: item (or piece of one) -> head, query block, key tiles [j0, j1); safe kernel: the
  // grid (query blocks of 128, heads)
  const int nt = (T + ABN - 1) / ABN;
  int head, q0, j0 = 0, j1 = nt, piece = -1;
  if constexpr (FAST) {
    const AttnPlan& pl = p.plan;
    int item = blockIdx.x;
    if (item >= pl.nmain) {
      piece = item - pl.nmain;                       // tail piece index
      item = pl.nmain + piece / pl.split;
      j0 = (piece % pl.split) * pl.per;
      j1 = min(nt, j0 + pl.per);
    }
    head = item / pl.nq;
    q0 = (item % pl.nq) * ABM;
  } else {
    head = blockIdx.y;
    q0 = blockIdx.x * ABM;
  }
  const int kvh = head / (p.H / p.Hkv);
  const int qbase = q0 + wave * (32 * QB);   // the wave's first query
  if constexpr (!FAST) {
    // the two fast waves (64 queries each) that covered this workgroup's 128 queries
    const int* fl = p.flags + (long)head * p.nflag + q0 / 64;
    if (fl[0] == 0 && fl[1] == 0) return;   // workgroup-uniform
  }

  // Q^T fragments (B operand) of query block qb (queries qbase + 32 qb + lr): k-step s covers
  // d = 16 s .. 16 s + 15, lane half h d 16 s + 8 h ..  (rows past T read row T - 1, never stored)
  u32x4 qf[QB][AD / 16];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const long qc = min(qbase + 32 * qb + lr, T - 1);
#pragma unroll
    for (int s = 0; s < AD / 16; ++s) qf[qb][s] = ld16(p.q + qc * p.ldq + (long)head * AD + 16 * s + 8 * h);
  }

  // staging.  K: chunk idx = tid + 256 i (i = 0..3) is key row idx / 16, 16-byte d chunk idx % 16,
  // stored as is.  V: thread t takes keys 4 (t % 16) .. 4 (t % 16) + 3 -- four keys whose V^T
  // positions are adjacent -- at d chunk t / 16, and stores each of its 8 d rows' four values as
  // one 8-byte write: a wave's 64 lanes then cover all 64 keys of 4 d rows (at most a 2-way bank
  // conflict), where scattered 2-byte writes conflicted 8 ways.
  const uint16_t* kbase = p.k + (long)kvh * AD;
  const uint16_t* vbase = p.v + (long)kvh * AD;
  const int vkg = tid & 15, vc = tid >> 4;   // V key group, d chunk
  u32x4 kr[4], vr[4];
  auto gload = [&](int j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i, row = idx >> 4, c = idx & 15;
      // keys past T read key T - 1 and are masked
      kr[i] = ld16(kbase + (long)min(j * ABN + row, T - 1) * p.ldkv + 8 * c);
      vr[i] = ld16(vbase + (long)min(j * ABN + 4 * vkg + i, T - 1) * p.ldkv + 8 * vc);
    }
  };
  // V^T byte column of key 4 vkg: slice vkg / 4, first position of keys 4 (vkg % 4) .. + 3
  const int vcol = 2 * (16 * (vkg >> 2) + slice_pos(4 * (vkg & 3)));
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i, row = idx >> 4, c = idx & 15;
      *reinterpret_cast<u32x4*>(&sK[buf][row * KPITCH + 16 * c]) = kr[i];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {   // d = 8 vc + 2 e (low halves) and 8 vc + 2 e + 1 (high halves)
      const u32x2 lo = {__builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x05040100u),
                        __builtin_amdgcn_perm(vr[3][e], vr[2][e], 0x05040100u)};
      const u32x2 hi = {__builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x07060302u),
                        __builtin_amdgcn_perm(vr[3][e], vr[2][e], 0x07060302u)};
      *reinterpret_cast<u32x2*>(&sV[buf][(8 * vc + 2 * e) * VPITCH + vcol]) = lo;
      *reinterpret_cast<u32x2*>(&sV[buf][(8 * vc + 2 * e + 1) * VPITCH + vcol]) = hi;
    }
  };

  // O^T accumulators: register r of d block db holds d = 32 db + 8 (r / 4) + 4 h + r % 4
  f32x16 O[QB][AD / 32];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int db = 0; db < AD / 32; ++db) O[qb][db] = f32x16{};
  float m_use[QB], l_lane[QB];   // exponent offset, the lane's share of the row sum
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_use[qb] = -INFINITY;
    l_lane[qb] = 0.0f;
  }
  bool over = false;   // fast kernel: a score beyond the offset limit

  gload(j0);
  lstore(0);
  __syncthreads();
  for (int j = j0; j < j1; ++j) {
    const int buf = (j - j0) & 1;
    if (j + 1 < j1) gload(j + 1);
    const int kvalid = T - j * ABN;   // keys of this tile below T (>= 1)
#pragma unroll
    for (int hk = 0; hk < 2; ++hk) {
      // S^T = K Q^T for keys 32 hk .. 32 hk + 31
      f32x16 S[QB];
      const uint8_t* ka = &sK[buf][(32 * hk + lr) * KPITCH + 16 * h];
#pragma unroll
      for (int s = 0; s < AD / 16; ++s) {
        const u32x4 a = ld16(ka + 32 * s);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if constexpr (FAST) {
            if (s == 0) mfma_score0(S[qb], a, qf[qb][s]);
            else mfma_score(S[qb], a, qf[qb][s]);
          } else {
            S[qb] = mfma_bf16_32x32x16(a, qf[qb][s], s == 0 ? f32x16{} : S[qb]);
          }
        }
      }
      if constexpr (FAST) asm volatile("s_nop 10" : "+v"(S[0]), "+v"(S[1]));   // score_fence (QB = 2)
      // softmax in log2 units, p = exp2(scale_log2 s - m) (the scale is positive, so the maximum
      // is taken over the raw scores); register r holds key 32 hk + 8 (r / 4) + 4 h + r % 4.
      // Keys past T (last tile only) get a score of -inf.
      if (kvalid < 32 * hk + 32) {   // wave-uniform
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (32 * hk + 8 * (r >> 2) + 4 * h + (r & 3) >= kvalid) S[qb][r] = -INFINITY;
      }
      float mt[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float m = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, S[qb][r]);
        mt[qb] = half_max(m) * p.scale_log2;
      }
      if constexpr (FAST) {
        if (j == j0 && hk == 0) {
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) m_use[qb] = mt[qb];   // key 0 is valid: finite
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) over |= mt[qb] > m_use[qb] + OFFSET_LIMIT;
      } else {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float m_new = fmaxf(m_use[qb], mt[qb]);
          const float alpha = __builtin_amdgcn_exp2f(m_use[qb] - m_new);
          m_use[qb] = m_new;
          l_lane[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < AD / 32; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) O[qb][db][r] *= alpha;
        }
      }
      // probabilities rounded to bf16: the B operands of P^T, one per 16-key slice
      u32x4 pf[QB][2];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int r = 0; r < 16; ++r)   // (a fast wave past the offset limit may overflow: it is marked)
          S[qb][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[qb][r], p.scale_log2, -m_use[qb]));
        // the row sum over the bf16 probabilities the P V product uses, two per v_dot2
        float ls = l_lane[qb];
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // (the packed word goes through a scalar: bit-casting the vector element itself
            // compiles to a read of element 0)
            const uint32_t w = pack_bf16x2(S[qb][8 * sl + 2 * e], S[qb][8 * sl + 2 * e + 1]);
            pf[qb][sl][e] = w;
            ls = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, 0x3F803F80u),
                                                 ls, false);
          }
        l_lane[qb] = ls;
      }
      if constexpr (FAST)   // the B operands were written by VALU
        asm volatile("s_nop 4" : "+v"(pf[0][0]), "+v"(pf[0][1]), "+v"(pf[1][0]), "+v"(pf[1][1]));
      // O^T += V^T P^T over the half's two 16-key slices
#pragma unroll
      for (int db = 0; db < AD / 32; ++db) {
        const uint8_t* va = &sV[buf][(32 * db + lr) * VPITCH + 16 * h + 64 * hk];
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {
          const u32x4 a = ld16(va + 32 * sl);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            if constexpr (FAST) mfma_out(O[qb][db], a, pf[qb][sl]);
            else O[qb][db] = mfma_bf16_32x32x16(a, pf[qb][sl], O[qb][db]);
          }
        }
      }
    }
    if (j + 1 < j1) lstore(buf ^ 1);   // the buffer every wave finished reading before the last barrier
    __syncthreads();
  }
  if constexpr (FAST) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)   // out_fence
      asm volatile("s_nop 15\n\ts_nop 15" : "+a"(O[qb][0]), "+a"(O[qb][1]), "+a"(O[qb][2]), "+a"(O[qb][3]));
  }
  if (FAST && piece >= 0) {
    // a piece: its unnormalized output, offset and row sum for the combine (rows past T too)
    const bool mark = __any(over);
    if (lane == 0) p.part_flag[piece * 4 + wave] = mark ? 1 : 0;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const long row = (long)piece * 256 + wave * (32 * QB) + 32 * qb + lr;
      const float l = half_sum(l_lane[qb]);
      if (h == 0) *reinterpret_cast<f32x2*>(p.part_ml + 2 * row) = f32x2{m_use[qb], l};
      float* orow = p.part_o + row * AD;
#pragma unroll
      for (int db = 0; db < AD / 32; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4*>(orow + 32 * db + 8 * g + 4 * h) =
              f32x4{O[qb][db][4 * g], O[qb][db][4 * g + 1], O[qb][db][4 * g + 2], O[qb][db][4 * g + 3]};
    }
    return;
  }
  // normalize (lanes l and l ^ 32 hold the same query); the fast kernel checks every value first
  uint32_t pk[QB][AD / 32][8];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float inv = 1.0f / half_sum(l_lane[qb]);
    const bool live = qbase + 32 * qb + lr < T;
#pragma unroll
    for (int db = 0; db < AD / 32; ++db)
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const float a = O[qb][db][2 * g] * inv, b = O[qb][db][2 * g + 1] * inv;
        if (FAST) over |= live && !(__builtin_isfinite(a) && __builtin_isfinite(b));
        pk[qb][db][g] = pack_bf16x2(a, b);
      }
  }
  const bool mark = FAST && __any(over);   // wave-uniform
  if constexpr (FAST) {
    if (lane == 0) p.flags[(long)head * p.nflag + qbase / 64] = mark ? 1 : 0;
  }
  if (!mark) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qrow = qbase + 32 * qb + lr;
      if (qrow < T) {
        uint16_t* orow = p.o + (long)qrow * p.ldo + (long)head * AD;
#pragma unroll
        for (int db = 0; db < AD / 32; ++db)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * g + 4 * h) = u32x2{pk[qb][db][2 * g], pk[qb][db][2 * g + 1]};
      }
    }
  }
}

__global__ void __launch_bounds__(256, 1) attn_fast_kernel(AttnArgs p) { attn_body<true>(p); }
__global__ void __launch_bounds__(256, 2) attn_safe_kernel(AttnArgs p) { attn_body<false>(p); }

// Merges the pieces of a tail item, 16 threads per query (one 8-column chunk each, so that a
// wave reads 4 whole 512-byte rows of a piece): workgroup g takes queries 16 (g % 16) ...
// of tail item g / 16,
//   o = sum_i 2^(m_i - m) O_i / sum_i 2^(m_i - m) l_i,   m = max_i m_i,
// and writes the item's flags (a wave of the item is marked if any piece's wave was).
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs p) {
  const AttnPlan& pl = p.plan;
  const int gid = blockIdx.x * 256 + threadIdx.x;
  const int c = gid & 15, qi = (gid >> 4) & 255, tail_item = gid >> 12;
  const int item = pl.nmain + tail_item, wave = qi >> 6;
  const int head = item / pl.nq, qrow = (item % pl.nq) * 256 + qi;
  const int s = pl.split;
  bool mark = false;
  for (int i = 0; i < s; ++i) mark |= p.part_flag[(tail_item * s + i) * 4 + wave] != 0;
  if ((qi & 63) == 0 && c == 0) p.flags[(long)head * p.nflag + (item % pl.nq) * 4 + wave] = mark ? 1 : 0;
  if (mark || qrow >= p.T) return;
  const long row0 = (long)tail_item * s * 256 + qi;
  float m = -INFINITY;
  for (int i = 0; i < s; ++i) m = fmaxf(m, p.part_ml[2 * (row0 + i * 256)]);
  float l = 0.0f;
  for (int i = 0; i < s; ++i) {
    const f32x2 ml = *reinterpret_cast<const f32x2*>(p.part_ml + 2 * (row0 + i * 256));
    l += __builtin_amdgcn_exp2f(ml[0] - m) * ml[1];
  }
  const float inv = 1.0f / l;
  f32x4 a0 = {}, a1 = {};
  for (int i = 0; i < s; ++i) {
    const long row = row0 + i * 256;
    const float w = __builtin_amdgcn_exp2f(p.part_ml[2 * row] - m) * inv;
    const f32x4* src = reinterpret_cast<const f32x4*>(p.part_o + row * AD + 8 * c);
    a0 += w * src[0];
    a1 += w * src[1];
  }
  uint16_t* orow = p.o + (long)qrow * p.ldo + (long)head * AD;
  *reinterpret_cast<u32x4*>(orow + 8 * c) =
      u32x4{pack_bf16x2(a0[0], a0[1]), pack_bf16x2(a0[2], a0[3]), pack_bf16x2(a1[0], a1[1]), pack_bf16x2(a1[2], a1[3])};
}

// workspace layout (bytes, each part 16-byte aligned): flags, part_flag, part_ml, part_o
struct AttnWs {
  long flags, part_flag, part_ml, part_o, total;
};
AttnWs attn_ws(int T, int H) {
  const AttnPlan pl = attn_plan(T, H, ATTN_CUS);
  const long pieces = (long)pl.tail * pl.split;
  auto up = [](long b) { return (b + 15) / 16 * 16; };
  AttnWs w;
  w.flags = 0;
  w.part_flag = up(4L * pl.items * 4);
  w.part_ml = w.part_flag + up(4L * pieces * 4);
  w.part_o = w.part_ml + up(8L * pieces * 256);
  w.total = w.part_o + 4L * pieces * 256 * AD;
  return w;
}

}  // namespace

long attention_workspace_bytes(int T, int H) { return attn_ws(T, H).total; }

hipError_t launch_attention_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int T, int H,
                                int Hkv, long ldq, long ldkv, long ldo, float scale, void* workspace, hipStream_t st) {
  const AttnWs w = attn_ws(T, H);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const AttnPlan pl = attn_plan(T, H, ATTN_CUS);
  AttnArgs a{q, k, v, o, reinterpret_cast<int*>(ws + w.flags), pl.nq * 4, T, H, Hkv, ldq, ldkv, ldo,
             scale * 1.4426950408889634f, pl, reinterpret_cast<float*>(ws + w.part_o),
             reinterpret_cast<float*>(ws + w.part_ml), reinterpret_cast<int*>(ws + w.part_flag)};
  attn_fast_kernel<<<(unsigned)(pl.nmain + pl.tail * pl.split), 256, 0, st>>>(a);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  if (pl.tail) {
    attn_combine_kernel<<<(unsigned)pl.tail * 16, 256, 0, st>>>(a);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  }
  attn_safe_kernel<<<dim3((unsigned)((T + 127) / 128), (unsigned)H), 256, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace svdq
