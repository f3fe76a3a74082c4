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
//  * attn_fast_kernel (QB = 2, one wave per SIMD, O in AGPRs), software-pipelined so that the
//    softmax of one half runs on the VALU between the MFMAs of the next half's scores and the
//    previous half's output.  Each query's exponent offset is its maximum over the first 32 keys
//    of its range and never moves, so the output accumulators are touched by MFMAs only (an offset
//    that follows the running maximum needs the output rescaled on the VALU, which makes the
//    compiler shuttle the 128 accumulators between AGPRs and VGPRs every tile).  Later
//    probabilities may exceed 1; f32 and bf16 hold them exactly in range.  A wave whose row sum
//    passes 2^64, or whose output is not finite, marks itself in the flag workspace (every wave
//    writes its entry, so it needs no clearing) and stores nothing.
//  * attn_safe_kernel (QB = 1, two waves per SIMD): the running-maximum formulation, output
//    rescaled every tile.  A workgroup runs only if a fast wave of its queries was marked, and
//    then writes those queries.
// The items of the last, partly filled round over the CUs are cut along the keys into pieces whose
// partial results attn_combine_kernel merges.
#include "svdq_common.h"
#include "svdq_kernels.h"

namespace svdq {
namespace {

constexpr int AD = 128;               // head dimension
constexpr int ABN = 64;               // keys per tile
constexpr int KPITCH = AD * 2 + 16;   // LDS bytes per K row (272: 16 rows of a read hit distinct banks)
constexpr int VPITCH = ABN * 2 + 16;  // LDS bytes per V^T row (144)
constexpr float ROWSUM_LIMIT = 18446744073709551616.0f;   // 2^64: the fast kernel's largest accepted row sum

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

// The fast kernel's MFMAs as volatile inline asm: the register classes are fixed (the scores in
// VGPRs, read by the softmax; the output accumulators in AGPRs, read only at the end) and the
// MFMAs keep their program order (and the LDS reads theirs around them).  The compiler does not
// see their hazards, so the fast kernel keeps them itself:
//  * an accumulator is only ever its own srcC (full overlap: no wait states);
//  * k-step 0 of the scores uses a zero srcC, so no VALU-written zeros feed an MFMA;
//  * VALU reads a score at least 16 MFMAs after it was written, or behind a 32-wait-state fence;
//  * the probabilities (VALU-written B operands) are read at least one phase later, behind such a
//    fence;
//  * a source fragment's registers are not rewritten until two more MFMAs have issued;
//  * no VALU work sits between two adjacent MFMAs that read the same fragment;
//  * the output is read after out_fence (2 x 16 wait states);
//  * a VALU write of an MFMA's source register (A, B or C) comes at least 2 wait states before the
//    MFMA (the ISA's VALU-write -> MFMA-read rule).  The compiler moves the output accumulators
//    between AGPRs and VGPRs around the rescale with v_accvgpr_write, and may place the last of
//    those writes right before an output MFMA, which then reads the old value of that register:
//    mfma_out starts with s_nop 1.  (A layout with softmax work between the two MFMAs of a fragment
//    gave wrong results for the second MFMA of every pair; its build has v_accvgpr_write of that
//    MFMA's srcC 0 and 1 wait states before it.)
// (tests/test_attn_mfma_order.py checks the last four rules on the built library.)
__device__ __forceinline__ void mfma_score0(f32x16& acc, u32x4 a, u32x4 b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_score(f32x16& acc, u32x4 a, u32x4 b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_out(f32x16& acc, u32x4 a, u32x4 b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
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
  // optional per-head RMS norm + rotary embedding of q on load (null qcos: q is used as given)
  const uint16_t* qcos;
  const uint16_t* qsin;
  long ldcs;
  float qeps;
};

// Q^T fragments of query row qc for lane half h: fragment s holds d = 16 s + 8 h .. + 7.  With
// rotary tables, the row is first normalized per head and rotated as the block's head norm does
//   n = bf16(q * rsqrt(mean(q^2) + eps));  (n1, n2) = (n[j], n[j + 64]):
//   o1 = bf16(fma(-n2, sin, bf16(n1 cos))),  o2 = bf16(fma(n1, sin, bf16(n2 cos)))
// (j < 64, cos / sin of the query's position): the lane holds both members of its pairs
// (fragments s and s + 4), and the mean of squares adds the other half's lane (lane ^ 32).  All 64
// lanes must be active.
__device__ __forceinline__ void load_q(const AttnArgs& p, long qc, int head, int h, u32x4 (&qf)[AD / 16]) {
  const uint16_t* qr = p.q + qc * p.ldq + (long)head * AD + 8 * h;
#pragma unroll
  for (int s = 0; s < AD / 16; ++s) qf[s] = ld16(qr + 16 * s);
  if (!p.qcos) return;   // uniform
  float ss = 0.0f;
#pragma unroll
  for (int s = 0; s < AD / 16; ++s)
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      ss = __builtin_fmaf(bf16lo(qf[s][d]), bf16lo(qf[s][d]), ss);
      ss = __builtin_fmaf(bf16hi(qf[s][d]), bf16hi(qf[s][d]), ss);
    }
  ss += __shfl_xor(ss, 32, 64);
  const float r = rsqrtf(ss / 128.0f + p.qeps);
#pragma unroll
  for (int s = 0; s < AD / 32; ++s) {
    const u32x4 c = ld16(p.qcos + qc * p.ldcs + 16 * s + 8 * h), sn = ld16(p.qsin + qc * p.ldcs + 16 * s + 8 * h);
    u32x4 o1, o2;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      float a1[2], a2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float x1 = e ? bf16hi(qf[s][d]) : bf16lo(qf[s][d]);
        const float x2 = e ? bf16hi(qf[s + 4][d]) : bf16lo(qf[s + 4][d]);
        const float cc = e ? bf16hi(c[d]) : bf16lo(c[d]), sv = e ? bf16hi(sn[d]) : bf16lo(sn[d]);
        const float n1 = round_bf16(x1 * r), n2 = round_bf16(x2 * r);
        a1[e] = __builtin_fmaf(-n2, sv, round_bf16(n1 * cc));
        a2[e] = __builtin_fmaf(n1, sv, round_bf16(n2 * cc));
      }
      o1[d] = pack_bf16x2(a1[0], a1[1]);
      o2[d] = pack_bf16x2(a2[0], a2[1]);
    }
    qf[s] = o1;
    qf[s + 4] = o2;
  }
}

// Global -> register -> LDS staging of a 64-key tile.  K: chunk idx = tid + 256 i (i = 0..3) is key
// row tid / 16 + 16 i, 16-byte d chunk tid % 16, stored as is.  V: thread t takes keys
// 4 (t % 16) .. + 3 -- four keys whose V^T positions are adjacent -- at d chunk t / 16, and stores
// each of its 8 d rows' four values as one 8-byte write: a wave's 64 lanes then cover all 64 keys
// of 4 d rows (at most a 2-way bank conflict), where scattered 2-byte writes conflicted 8 ways.
// Loads are buffer loads whose resource starts at the tile's first key and holds the keys up to
// T: the byte offsets of a thread's rows are the same for every tile (no address arithmetic per
// tile on the VALU), and keys past T read 0 (the hardware's range check); the scores mask them.
struct TileStaging {
  const uint16_t* k;
  const uint16_t* v;
  long ld;
  int T, rowb;          // rowb: bytes per key row
  int kvo, vvo;         // byte offsets of this thread's first K chunk and V chunk within a tile
  int kst, vst;
  u32x4 kr[4], vr[4];
  __device__ __forceinline__ TileStaging(const AttnArgs& p, int kvh, int tid) {
    const int vkg = tid & 15, vc = tid >> 4;
    const int krow = tid >> 4, vkey = 4 * vkg;
    k = p.k;
    v = p.v;
    ld = p.ldkv;
    T = p.T;
    rowb = 2 * (int)p.ldkv;
    kvo = 2 * (krow * (int)p.ldkv + kvh * AD + 8 * (tid & 15));
    vvo = 2 * (vkey * (int)p.ldkv + kvh * AD + 8 * vc);
    kst = krow * KPITCH + 16 * (tid & 15);
    // V^T byte column of key 4 vkg: slice vkg / 4, first position of keys 4 (vkg % 4) .. + 3
    vst = 8 * vc * VPITCH + 2 * (16 * (vkg >> 2) + slice_pos(4 * (vkg & 3)));
  }
  // the keys j * ABN .. T - 1 of a tensor as a raw buffer (stride 0, T * ldkv * 2 < 2^31 bytes)
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t keys_from(const uint16_t* base, int j) const {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base) + (long)j * ABN * ld, (short)0,
                                             (T - j * ABN) * rowb, 0x00020000);
  }
  __device__ __forceinline__ void load_k(int j) {
    const __amdgpu_buffer_rsrc_t r = keys_from(k, j);
#pragma unroll
    for (int i = 0; i < 4; ++i) kr[i] = __builtin_amdgcn_raw_buffer_load_b128(r, kvo + 16 * i * rowb, 0, 0);
  }
  __device__ __forceinline__ void load_v(int j) {
    const __amdgpu_buffer_rsrc_t r = keys_from(v, j);
#pragma unroll
    for (int i = 0; i < 4; ++i) vr[i] = __builtin_amdgcn_raw_buffer_load_b128(r, vvo + i * rowb, 0, 0);
  }
  __device__ __forceinline__ void store_k(uint8_t* sk) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(sk + kst + 16 * i * KPITCH) = kr[i];
  }
  __device__ __forceinline__ void store_v(uint8_t* sv) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {   // d = 8 vc + 2 e (low halves) and 8 vc + 2 e + 1 (high halves)
      const u32x2 lo = {__builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x05040100u),
                        __builtin_amdgcn_perm(vr[3][e], vr[2][e], 0x05040100u)};
      const u32x2 hi = {__builtin_amdgcn_perm(vr[1][e], vr[0][e], 0x07060302u),
                        __builtin_amdgcn_perm(vr[3][e], vr[2][e], 0x07060302u)};
      *reinterpret_cast<u32x2*>(sv + vst + 2 * e * VPITCH) = lo;
      *reinterpret_cast<u32x2*>(sv + vst + (2 * e + 1) * VPITCH) = hi;
    }
  }
};

// The safe kernel: one query block of 32 per wave, 128 queries per workgroup, the running-maximum
// formulation (the output rescaled on the VALU whenever the maximum grows).  A workgroup runs only
// if a fast wave of its queries was marked, and then writes all of its queries.
__global__ void __launch_bounds__(256, 2) attn_safe_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t sK[2][ABN * KPITCH];
  __shared__ __attribute__((aligned(16))) uint8_t sV[2][AD * VPITCH];
  const int T = p.T;
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = (T + ABN - 1) / ABN;
  const int head = blockIdx.y, q0 = blockIdx.x * 128;
  // the two fast waves (64 queries each) that covered these 128 queries
  const int* fl = p.flags + (long)head * p.nflag + q0 / 64;
  if (fl[0] == 0 && fl[1] == 0) return;   // workgroup-uniform
  const int kvh = head / (p.H / p.Hkv);
  const int qrow = q0 + 32 * wave + lr;
  // Q^T fragments (B operand): k-step s covers d = 16 s .. 16 s + 15, lane half h d 16 s + 8 h ..
  // (rows past T read row T - 1, never stored)
  u32x4 qf[AD / 16];
  load_q(p, min(qrow, T - 1), head, h, qf);
  TileStaging st(p, kvh, tid);

  // O^T accumulators: register r of d block db holds d = 32 db + 8 (r / 4) + 4 h + r % 4
  f32x16 O[AD / 32];
#pragma unroll
  for (int db = 0; db < AD / 32; ++db) O[db] = f32x16{};
  float m_run = -INFINITY, l_lane = 0.0f;   // running maximum (log2 units), the lane's row sum

  st.load_k(0);
  st.load_v(0);
  st.store_k(sK[0]);
  st.store_v(sV[0]);
  __syncthreads();
  for (int j = 0; j < nt; ++j) {
    const int buf = j & 1;
    if (j + 1 < nt) {
      st.load_k(j + 1);
      st.load_v(j + 1);
    }
    const int kvalid = T - j * ABN;   // keys of this tile below T (>= 1)
#pragma unroll
    for (int hk = 0; hk < 2; ++hk) {
      // S^T = K Q^T for keys 32 hk .. 32 hk + 31; register r holds key 32 hk + 8 (r / 4) + 4 h + r % 4
      f32x16 S = {};
      const uint8_t* ka = &sK[buf][(32 * hk + lr) * KPITCH + 16 * h];
#pragma unroll
      for (int s = 0; s < AD / 16; ++s) S = mfma_bf16_32x32x16(ld16(ka + 32 * s), qf[s], S);
      if (kvalid < 32 * hk + 32) {   // keys past T: -inf (wave-uniform)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (32 * hk + 8 * (r >> 2) + 4 * h + (r & 3) >= kvalid) S[r] = -INFINITY;
      }
      float m = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) m = fmaxf(m, S[r]);
      // the scale is positive, so the maximum is taken over the raw scores
      const float m_new = fmaxf(m_run, half_max(m) * p.scale_log2);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_lane *= alpha;
#pragma unroll
      for (int db = 0; db < AD / 32; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) O[db][r] *= alpha;
      // probabilities rounded to bf16 (the B operands of P^T, one per 16-key slice); the row sum
      // over the same bf16 values, two per v_dot2
      u32x4 pf[2];
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = __builtin_amdgcn_exp2f(__builtin_fmaf(S[8 * sl + 2 * e], p.scale_log2, -m_run));
          const float b = __builtin_amdgcn_exp2f(__builtin_fmaf(S[8 * sl + 2 * e + 1], p.scale_log2, -m_run));
          const uint32_t w = pack_bf16x2(a, b);
          pf[sl][e] = w;
          l_lane = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                                   __builtin_bit_cast(bf16x2, 0x3F803F80u), l_lane, false);
        }
      // O^T += V^T P^T over the half's two 16-key slices
#pragma unroll
      for (int db = 0; db < AD / 32; ++db) {
        const uint8_t* va = &sV[buf][(32 * db + lr) * VPITCH + 16 * h + 64 * hk];
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) O[db] = mfma_bf16_32x32x16(ld16(va + 32 * sl), pf[sl], O[db]);
      }
    }
    if (j + 1 < nt) {   // the buffer every wave finished reading before the last barrier
      st.store_k(sK[buf ^ 1]);
      st.store_v(sV[buf ^ 1]);
    }
    __syncthreads();
  }
  if (qrow < T) {
    const float inv = 1.0f / half_sum(l_lane);
    uint16_t* orow = p.o + (long)qrow * p.ldo + (long)head * AD;
#pragma unroll
    for (int db = 0; db < AD / 32; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * g + 4 * h) =
            u32x2{pack_bf16x2(O[db][4 * g] * inv, O[db][4 * g + 1] * inv),
                  pack_bf16x2(O[db][4 * g + 2] * inv, O[db][4 * g + 3] * inv)};
  }
}

template <bool B> struct Flag { static constexpr bool value = B; };

// pin(x): an empty asm that claims to rewrite x.  VALU work that reads x cannot move above it and
// work that produces x cannot move below it; with the MFMAs as volatile asm (kept in program
// order, and LDS reads with them) this fixes the interleaving of the fast kernel's phases.
template <typename V> __device__ __forceinline__ void pin(V& x) { asm volatile("" : "+v"(x)); }
// hold(x): an empty asm that reads x, so its registers stay allocated up to this point
template <typename V> __device__ __forceinline__ void hold(const V& x) { asm volatile("" ::"v"(x)); }

// The fast kernel: 64 queries per wave (two blocks of 32), 256 per workgroup, one wave per SIMD,
// software-pipelined over half tiles of 32 keys.  Stage t holds K tile t and V tile t - 1 in one
// LDS buffer and runs two phases; a phase issues
//   the score MFMAs of the next half (16: S^T = K Q^T),
//   the output MFMAs of the previous half (16: O^T += V^T P^T, P from the phase before),
//   the softmax of the current half (its scores from the phase before),
// interleaved one VALU part per MFMA, so the VALU work runs while the matrix cores are busy (a
// wave's MFMAs and its own independent VALU work overlap when interleaved; phases of MFMAs only
// and VALU only do not).  The exponent offset is fixed per query (its maximum over the range's
// first 32 keys), so the output accumulators are touched by MFMAs only and stay in AGPRs; a wave
// whose row sum passes 2^64, or whose output is not finite, is marked for the safe kernel.
//
// Hazards the compiler cannot see (MFMAs in asm): every score read by VALU was written at least 16
// MFMAs earlier or behind a score fence (11 wait states), every probability read by an MFMA was
// written by VALU at least one phase earlier and behind a 5-wait-state fence, accumulators are
// only their own srcC, and the output is read after 2 x 16 wait states.
__global__ void __launch_bounds__(256, 1) attn_fast_kernel(AttnArgs p) {
  constexpr int QB = 2;
  __shared__ __attribute__((aligned(16))) uint8_t sK[2][ABN * KPITCH];
  __shared__ __attribute__((aligned(16))) uint8_t sV[2][AD * VPITCH];
  const int T = p.T;
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = (T + ABN - 1) / ABN;
  // item (or piece of one) -> head, query block, key tiles [j0, j1)
  const AttnPlan& pl = p.plan;
  int item = blockIdx.x, j0 = 0, j1 = nt, piece = -1;
  if (item >= pl.nmain) {
    piece = item - pl.nmain;
    item = pl.nmain + piece / pl.split;
    j0 = (piece % pl.split) * pl.per;
    j1 = min(nt, j0 + pl.per);
  }
  const int head = item / pl.nq, q0 = (item % pl.nq) * 256;
  const int kvh = head / (p.H / p.Hkv);
  const int qbase = q0 + 64 * wave;   // the wave's first query

  u32x4 qf[QB][AD / 16];   // Q^T fragments of query block qb (queries qbase + 32 qb + lr)
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) load_q(p, min(qbase + 32 * qb + lr, T - 1), head, h, qf[qb]);
  TileStaging st(p, kvh, tid);

  f32x16 O[QB][AD / 32];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int db = 0; db < AD / 32; ++db) O[qb][db] = f32x16{};
  f32x16 Sn[QB];              // scores of the next half (written by this phase's MFMAs)
  float sc[QB][16];           // scores of the current half (register r: key 8 (r / 4) + 4 h + r % 4)
  u32x4 pp[QB][2], pc[QB][2]; // bf16 probabilities of the previous / current half, per 16-key slice
  float m_use[QB], ls[QB] = {0.0f, 0.0f};   // exponent offset, the lane's share of the row sum
  const float sl2 = p.scale_log2;
  const int klane = lr * KPITCH + 16 * h, vlane = lr * VPITCH + 16 * h;

  // A fragments of a phase: id < 8 the K rows of k-step id (if the phase has score MFMAs), then
  // V^T (d block, slice).  A phase issues its MFMAs in slots:
  //  * with both kinds, S_g q0, PV_g q0, S_g q1, PV_g q1 for g = 0..7 (32 slots): no two adjacent
  //    MFMAs read the same fragment, so one softmax part goes before every MFMA;
  //  * with one kind, the two MFMAs of a fragment back to back (16 slots), the softmax parts
  //    before the first of each pair.
  // (An earlier layout that put softmax work between the two adjacent MFMAs of a fragment gave
  // wrong results for the second of every pair, deterministically: rebuilt, its code writes the
  // last accumulator AGPRs of that MFMA (v_accvgpr_write after the rescale) 0 and 1 wait states
  // before it, under the ISA's 2 -- see mfma_out.  The kernel keeps the layouts that test exact:
  // no VALU work between two adjacent MFMAs that read the same fragment.  One wave per SIMD stalls
  // in order behind an MFMA that waits for the matrix pipe, so VALU work placed between MFMAs of
  // different fragments hides under twice as much MFMA time as work placed only between pairs.)
  // A fragment is read from LDS LEAD slots before its first use; the ones used earlier than that
  // come from pre, read during the phase before (or by prefetch after a barrier).
  constexpr int LEAD = 6;
  u32x4 pre[4];
  auto slot_id = [](bool both, int i) { return both ? ((i & 1) ? 8 + (i >> 2) : (i >> 2)) : (i >> 1); };
  auto slot_qb = [](bool both, int i) { return both ? (i >> 1) & 1 : i & 1; };
  auto first_use = [](bool both, int id) { return both ? (id < 8 ? 4 * id : 4 * (id - 8) + 1) : 2 * id; };
  auto last_use = [](bool both, int id) { return both ? (id < 8 ? 4 * id + 2 : 4 * (id - 8) + 3) : 2 * id + 1; };
  auto npre = [](bool both) { return both ? 4 : 3; };                         // first use < LEAD
  auto pre_id = [](bool both, int r) { return both ? ((r & 1) ? 8 + (r >> 1) : (r >> 1)) : r; };
  auto frag_at = [](bool ds, const uint8_t* ka, const uint8_t* va, int id) {
    const int g = id - 8 * ds;
    return ds && id < 8 ? ld16(ka + 32 * id) : ld16(va + (g >> 1) * (32 * VPITCH) + 32 * (g & 1));
  };
  auto prefetch = [&](auto s_, auto pv_, const uint8_t* ka, const uint8_t* va) {
    constexpr bool DS = decltype(s_)::value, BOTH = DS && decltype(pv_)::value;
#pragma unroll
    for (int r = 0; r < npre(BOTH); ++r) pre[r] = frag_at(DS, ka, va, pre_id(BOTH, r));
  };
  // nx_: the next phase, whose first fragments are read during this one's last slots (0: none, it
  // follows a barrier; 1: score MFMAs only, K rows nka; 2: output MFMAs only, V^T rows nva; 3: both)
  auto phase = [&](auto s_, auto pv_, auto soft_, const uint8_t* ka, const uint8_t* va, auto nx_,
                   const uint8_t* nka, const uint8_t* nva) {
    constexpr bool DS = decltype(s_)::value, DPV = decltype(pv_)::value, DSOFT = decltype(soft_)::value;
    constexpr int NX = decltype(nx_)::value;
    constexpr bool NDS = NX & 1, NBOTH = NX == 3;
    constexpr bool BOTH = DS && DPV;
    constexpr int NS = BOTH ? 32 : 16;   // slots (MFMAs)
    constexpr int NF = BOTH ? 16 : 8;    // fragments
    u32x4 fr[16];                        // by fragment id
#pragma unroll
    for (int r = 0; r < npre(BOTH); ++r) fr[pre_id(BOTH, r)] = pre[r];
    float xs[16][2];
    uint32_t pw[QB][2][4];
    // softmax part i: pair k = i / 2 (query block qb, slice sl, word e: scores r, r + 1); even
    // parts take exp2, odd parts pack the bf16 word and add it to the row sum
    auto part = [&](int i) {
      const int k = i >> 1, qb = k >> 3, sl = (k >> 2) & 1, e = k & 3, r = 8 * sl + 2 * e;
      if ((i & 1) == 0) {
        pin(sc[qb][r]);
        pin(sc[qb][r + 1]);
        xs[k][0] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[qb][r], sl2, -m_use[qb]));
        xs[k][1] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[qb][r + 1], sl2, -m_use[qb]));
        pin(xs[k][0]);
        pin(xs[k][1]);
      } else {
        // (the packed word goes through a scalar: bit-casting a vector element compiles to a
        // read of element 0)
        pin(xs[k][0]);
        pin(xs[k][1]);
        const uint32_t w = pack_bf16x2(xs[k][0], xs[k][1]);
        pw[qb][sl][e] = w;
        ls[qb] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                                 __builtin_bit_cast(bf16x2, 0x3F803F80u), ls[qb], false);
        pin(pw[qb][sl][e]);
        pin(ls[qb]);
      }
    };
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      // LDS reads LEAD slots ahead: this phase's fragments, then the next phase's first ones
#pragma unroll
      for (int id = 0; id < NF; ++id)
        if (first_use(BOTH, id) - LEAD == i) fr[id] = frag_at(DS, ka, va, id);
      if constexpr (NX != 0) {
#pragma unroll
        for (int r = 0; r < npre(NBOTH); ++r)
          if (NS + first_use(NBOTH, pre_id(NBOTH, r)) - LEAD == i) pre[r] = frag_at(NDS, nka, nva, pre_id(NBOTH, r));
      }
      // softmax parts, software-pipelined: a pair's pack + sum comes well after its exp2
      if constexpr (DSOFT) {
        if (BOTH) {
          if ((i & 1) == 0) part(2 * (i >> 1));
          else if (i >= 3) part(2 * ((i - 3) >> 1) + 1);
        } else if ((i & 1) == 0) {
          const int m = i >> 1;   // fragment m: exp2 of pairs 2m, 2m + 1, pack + sum of 2m - 2, 2m - 1
          part(4 * m);
          part(4 * m + 2);
          if (m > 0) {
            part(4 * m - 3);
            part(4 * m - 1);
          }
        }
      }
      const int id = slot_id(BOTH, i), qb = slot_qb(BOTH, i);
      if (DS && id < 8) {
        if (id == 0) mfma_score0(Sn[qb], fr[id], qf[qb][0]);
        else mfma_score(Sn[qb], fr[id], qf[qb][id & 7]);
      } else {
        const int g = max(id - 8 * DS, 0);
        mfma_out(O[qb][g >> 1], fr[id], pp[qb][g & 1]);
      }
      // operand hold: a fragment last read two slots ago keeps its registers until here (no
      // VALU or LDS write reaches them earlier)
#pragma unroll
      for (int id2 = 0; id2 < NF; ++id2)
        if (last_use(BOTH, id2) == i - 2) hold(fr[id2]);
    }
    if constexpr (DSOFT) {
      if (BOTH) {
        part(31);
      } else {
        part(29);
        part(31);
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) pc[qb][sl] = u32x4{pw[qb][sl][0], pw[qb][sl][1], pw[qb][sl][2], pw[qb][sl][3]};
    }
    // phase fence (32 wait states: a whole 8-pass MFMA) before the registers of the phase's last
    // operands -- the fragments read in its last two slots, the previous probabilities -- are
    // released, and before VALU reads scores written by this phase
    constexpr int LA = BOTH ? 7 : NF - 1, LB = BOTH ? 15 : NF - 1;
    if constexpr (DPV)
      asm volatile("s_nop 15\n\ts_nop 15" ::"v"(fr[LA]), "v"(fr[LB]), "v"(pp[0][0]), "v"(pp[0][1]), "v"(pp[1][0]),
                   "v"(pp[1][1]));
    else
      asm volatile("s_nop 15\n\ts_nop 15" ::"v"(fr[LA]), "v"(fr[LB]));
    if constexpr (DS) {   // (pins after the fence: the scores' readers stay below it)
      pin(Sn[0]);
      pin(Sn[1]);
    }
    if constexpr (DSOFT) {
      pin(pc[0][0]);
      pin(pc[0][1]);
      pin(pc[1][0]);
      pin(pc[1][1]);
    }
  };
  auto take_scores = [&]() {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[qb][r] = Sn[qb][r];
  };
  auto take_probs = [&]() {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) pp[qb][sl] = pc[qb][sl];
  };
  // keys past T (last tile only) get a score of -inf
  auto mask = [&](int j, int hk) {
    const int kvalid = T - j * ABN;
    if (kvalid < 32 * hk + 32) {   // wave-uniform
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (32 * hk + 8 * (r >> 2) + 4 * h + (r & 3) >= kvalid) sc[qb][r] = -INFINITY;
    }
  };
  using Y = Flag<true>;
  using N = Flag<false>;
  using NONE = std::integral_constant<int, 0>;
  using NEXT_S = std::integral_constant<int, 1>;
  using NEXT_PV = std::integral_constant<int, 2>;
  using NEXT_BOTH = std::integral_constant<int, 3>;

  // stage j0: K tile j0 only
  st.load_k(j0);
  st.store_k(sK[0]);
  __syncthreads();
  prefetch(Y{}, N{}, &sK[0][klane], nullptr);
  if (j0 + 1 < j1) st.load_k(j0 + 1);
  st.load_v(j0);
  phase(Y{}, N{}, N{}, &sK[0][klane], nullptr, NEXT_S{}, &sK[0][32 * KPITCH + klane], nullptr);
  take_scores();
  mask(j0, 0);
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {   // the offsets: the first 32 keys' maximum (key 64 j0 < T: finite)
    float m = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) m = fmaxf(m, sc[qb][r]);
    m_use[qb] = half_max(m) * sl2;   // the scale is positive: the maximum of the raw scores
  }
  phase(Y{}, N{}, Y{}, &sK[0][32 * KPITCH + klane], nullptr, NONE{}, nullptr, nullptr);
  take_probs();
  take_scores();
  if (j0 + 1 < j1) st.store_k(sK[1]);
  st.store_v(sV[1]);
  __syncthreads();
  // stages j0 + 1 .. j1 - 1: K tile t, V tile t - 1
  for (int t = j0 + 1; t < j1; ++t) {
    const int b = (t - j0) & 1;
    prefetch(Y{}, Y{}, &sK[b][klane], &sV[b][vlane]);
    if (t + 1 < j1) st.load_k(t + 1);
    st.load_v(t);
    // softmax of tile t - 1's second half (not the range's last tile: no mask)
    phase(Y{}, Y{}, Y{}, &sK[b][klane], &sV[b][vlane], NEXT_BOTH{}, &sK[b][32 * KPITCH + klane], &sV[b][64 + vlane]);
    take_probs();
    take_scores();
    mask(t, 0);
    phase(Y{}, Y{}, Y{}, &sK[b][32 * KPITCH + klane], &sV[b][64 + vlane], NONE{}, nullptr, nullptr);
    take_probs();
    take_scores();
    if (t + 1 < j1) st.store_k(sK[b ^ 1]);
    st.store_v(sV[b ^ 1]);
    __syncthreads();
  }
  // stage j1: V tile j1 - 1 only
  {
    const int b = (j1 - j0) & 1;
    prefetch(N{}, Y{}, nullptr, &sV[b][vlane]);
    mask(j1 - 1, 1);
    phase(N{}, Y{}, Y{}, nullptr, &sV[b][vlane], NEXT_PV{}, nullptr, &sV[b][64 + vlane]);
    take_probs();
    phase(N{}, Y{}, N{}, nullptr, &sV[b][64 + vlane], NONE{}, nullptr, nullptr);
  }
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)   // output fence
    asm volatile("s_nop 15\n\ts_nop 15" : "+a"(O[qb][0]), "+a"(O[qb][1]), "+a"(O[qb][2]), "+a"(O[qb][3]));

  bool over = false;
  float l[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    l[qb] = half_sum(ls[qb]);
    over |= !(l[qb] <= ROWSUM_LIMIT);   // also catches inf / NaN
  }
  if (piece >= 0) {
    // a piece: its unnormalized output, offset and row sum for the combine (rows past T too).  Its
    // wave is also marked when an accumulator is not finite (p v past the f32 range: |v| above
    // about 2^64 with the fixed offset), as a whole item's normalized output is; the values are
    // checked as they go out (0 x inf and 0 x NaN are NaN, 0 x finite is 0).  Rows past T (q read
    // as 0) are checked too: a mark there only sends the wave to the running-maximum kernel.
    float nf = 0.0f;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const long row = (long)piece * 256 + 64 * wave + 32 * qb + lr;
      if (h == 0) *reinterpret_cast<f32x2*>(p.part_ml + 2 * row) = f32x2{m_use[qb], l[qb]};
      float* orow = p.part_o + row * AD;
#pragma unroll
      for (int db = 0; db < AD / 32; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 o4 = {O[qb][db][4 * g], O[qb][db][4 * g + 1], O[qb][db][4 * g + 2], O[qb][db][4 * g + 3]};
          *reinterpret_cast<f32x4*>(orow + 32 * db + 8 * g + 4 * h) = o4;
#pragma unroll
          for (int e = 0; e < 4; ++e) nf = __builtin_fmaf(o4[e], 0.0f, nf);
        }
    }
    const bool mark = __any(over || nf != 0.0f);   // NaN != 0
    if (lane == 0) p.part_flag[piece * 4 + wave] = mark ? 1 : 0;
    return;
  }
  // normalize (lanes l and l ^ 32 hold the same query), checking every value first
  uint32_t pk[QB][AD / 32][8];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float inv = 1.0f / l[qb];
    const bool live = qbase + 32 * qb + lr < T;
#pragma unroll
    for (int db = 0; db < AD / 32; ++db)
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const float a = O[qb][db][2 * g] * inv, b = O[qb][db][2 * g + 1] * inv;
        over |= live && !(__builtin_isfinite(a) && __builtin_isfinite(b));
        pk[qb][db][g] = pack_bf16x2(a, b);
      }
  }
  const bool mark = __any(over);   // wave-uniform
  if (lane == 0) p.flags[(long)head * p.nflag + qbase / 64] = mark ? 1 : 0;
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
                                int Hkv, long ldq, long ldkv, long ldo, float scale, void* workspace, hipStream_t st,
                                const uint16_t* qcos, const uint16_t* qsin, long ldcs, float qeps) {
  const AttnWs w = attn_ws(T, H);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const AttnPlan pl = attn_plan(T, H, ATTN_CUS);
  AttnArgs a{q, k, v, o, reinterpret_cast<int*>(ws + w.flags), pl.nq * 4, T, H, Hkv, ldq, ldkv, ldo,
             scale * 1.4426950408889634f, pl, reinterpret_cast<float*>(ws + w.part_o),
             reinterpret_cast<float*>(ws + w.part_ml), reinterpret_cast<int*>(ws + w.part_flag), qcos, qsin, ldcs,
             qeps};
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
