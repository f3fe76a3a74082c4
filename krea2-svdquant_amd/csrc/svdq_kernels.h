// Internal kernel parameter blocks and launchers (host side).  Not part of the C-ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svdq {

struct ActParams {
  const uint16_t* x;        // [M, ldx] bf16
  long ldx;
  const float* srs;         // [2K] f32: s, then RN(1/s)
  const uint16_t* l2;       // [r, K] bf16
  const uint16_t* lora;     // [rl, K] bf16 (null when rl == 0)
  const float* lora_mult;   // [rl]
  int r, rl;
  int M, K, RTp;            // RTp: row stride of mid (>= r + rl, multiple of 32)
  int t0;                   // first MFMA column tile of the down projections in this launch
  uint8_t* qx;              // [M, K/2] canonical packed codes (optional)
  uint8_t* qa;              // [M, K] 8-bit GEMM operand codes (quantizing modes)
  uint16_t* sx;             // [M, K/G] bf16, or [K/G, M] u32 (sx, sx) pairs when sx_pairs
  uint16_t* xhat;           // [M, ldxh] bf16 (null unless requested)
  long ldxh;
  float* mid;               // [S, M, RTp]: one partial per K split (summed by launch_mid_finalize)
  int gps;                  // K-groups per split
  int exact;                // 1: IEEE division for x / s everywhere
  int sx_pairs;             // 1: sx as u32 bf16 pairs
};

struct GemmParams {
  const uint8_t* qa;        // W4A4: [M, K] 8-bit activation operand codes
  const uint32_t* sxp;      // W4A4: [K/G, M] activation scales as u32 bf16 pairs (sx, sx)
  const uint16_t* xhat;     // W4A16: [M, ldxh] bf16 smoothed activations
  long ldxh;
  const uint8_t* qw;        // [N, K/2] packed weight codes (W4A16)
  const uint8_t* qwe;       // [N, K] 8-bit weight operand codes (W4A4)
  const uint16_t* sw;       // [N, K/G] fp16 weight scales (W4A16)
  const uint32_t* swp;      // [K/G, N] (bf16 hi, bf16 lo) pairs of the weight scales (W4A4)
  const uint16_t* midp;     // [M, 2, RTp] bf16 low-rank/LoRA down projections: hi plane, lo plane
  const uint16_t* l1cat;    // [N, RTp] bf16 up projections (zero padded)
  int RTp;
  const uint16_t* bias;     // [N] bf16 or null
  void* y;                  // [M, ldy] bf16 or f32
  long ldy;
  int M, N, K;
  int group;                // run-time group size (the kernels templated on G = 0)
  // Elementwise op on the bf16-rounded output (bf16 output only): 0 none, 1 aux * sigmoid(y),
  // 2 silu(aux) * y, 3 aux + evec[n] * y, each intermediate rounded to bf16 as torch does.
  int epi;
  const uint16_t* aux;      // [M, ldaux] bf16 (epi != 0)
  long ldaux;
  const uint16_t* evec;     // [N] bf16 (epi == 3)
  int aux_vec;              // 1: aux (and evec) take 16-byte loads (aligned, ldaux % 8 == 0)
};

// Up to MAX_SIBLINGS W4A4 layers over the same activation rows (same M, K and group size), run
// as one launch of the e3m2 kernel; tile0[i] = the first tile of layer i (256 x 128 tiles,
// prefix sums, tile0[count] = all tiles).  No fused store ops.
constexpr int MAX_SIBLINGS = 4;
struct GemmSiblings {
  GemmParams layer[MAX_SIBLINGS];
  int count;
  int tile0[MAX_SIBLINGS + 1];
};

// Activation passes of up to MAX_SIBLINGS layers over the same x (same M, K, group, RTp and
// splits; e3m2 codes with sx pairs, rank r <= 32, no LoRA tiles) as one launch, then one finalize
// launch: layer[i] as for launch_act (mid = the split partials), head[i] = its finalized operand.
struct ActSiblings {
  ActParams layer[MAX_SIBLINGS];
  uint16_t* head[MAX_SIBLINGS];
  int count;
};
hipError_t launch_act_siblings(const ActSiblings& s, int G, int splits, hipStream_t st);

int act_splits(int M, int K, int G);
// oper: 0 = no codes (x_hat only), 1 = e4m3 operand codes, 2 = int8 16*q operand codes, 3 = e3m2;
// nt: column tiles of the down projections from p.t0 (at most 4); with p.t0 > 0 the launch computes
// down projections only (oper 0, no x_hat)
hipError_t launch_act(const ActParams& p, int G, int nt, int oper, bool xhat, int splits, hipStream_t st);
// Sums the S split partials `part` [S, M, RTp] in split order and writes the GEMM epilogue's
// operand midp [M, 2, RTp] (bf16 hi plane, then bf16 lo plane, hi + lo within 2^-18 of the f32 sum, relative).
hipError_t launch_mid_finalize(const float* part, int S, int M, int RTp, uint16_t* midp, hipStream_t st);
hipError_t launch_prepare_smooth(const uint16_t* s, float* srs, int K, hipStream_t st);
// A4 codes and scales for any group size G (multiple of 16 dividing K) from x_hat: int8 operand
// (16 q) [M, K], scales bf16 [M, K/G] or u32 pairs [K/G, M], packed codes [M, K/2] if qx
hipError_t launch_quant_any_group(const uint16_t* xhat, long ldxh, int M, int K, int G, uint8_t* qa, uint16_t* sx,
                                  int sx_pairs, uint8_t* qx, hipStream_t st);
// mode: 0 = e4m3 operands on the FP8 MFMA, 1 = int8 operands on the INT8 MFMA, 2 = e3m2 planar
// operands on the FP6 MFMA
hipError_t launch_w4a4(const GemmParams& p, int G, int mode, bool out_f32, hipStream_t st);
// whether launch_w4a4 (e3m2, group 64, no fused op) runs the 256 x 256 tiles for this shape
bool use_wide_tiles(int M, int N, int K);
// e3m2 operands, G = 64 or 128, K % 512 == 0, every layer without fused store ops
hipError_t launch_w4a4_siblings(const GemmSiblings& gs, int G, bool out_f32, hipStream_t st);
// out = op(y, aux) elementwise over n contiguous bf16 values (op 1 mul_sigmoid, 2 silu_mul; the
// GEMM store's op code), pointers 16-byte aligned
hipError_t launch_gate_op(int op, const uint16_t* y, const uint16_t* aux, uint16_t* out, long n, hipStream_t st);
hipError_t launch_weight_scale_pairs(const uint16_t* sw, uint32_t* out, int n, int ngroups, int mode, hipStream_t st);
// mode: 0 = e4m3, 1 = int8 16*q (both [N, K] bytes), 2 = e3m2 planar ((N + 1) & ~1 rows, K * 3 / 4
// bytes per row)
hipError_t launch_weight_operand(const uint8_t* qw, uint8_t* qwe, int N, int K, int mode, hipStream_t st);
hipError_t launch_w4a16(const GemmParams& p, int G, bool out_f32, hipStream_t st);
// W4A16 sibling layers (same M, K and group; tile0 counting 192 x 256 tiles) in one launch of the
// specialized-wave kernel; hipErrorInvalidValue when a layer cannot take it (w4a16_ws_fits).
// w4a16_siblings_pay: whether that launch beats the layers' own launches (their tile rounds).
bool w4a16_ws_fits(const GemmParams& p);
bool w4a16_siblings_pay(const GemmSiblings& gs);
hipError_t launch_w4a16_siblings(const GemmSiblings& gs, int G, bool out_f32, hipStream_t st);
// W4A4 GEMM for any group size G (multiple of 16 dividing K): int8 operands (SVDQ_OPERAND_I8 layout)
hipError_t launch_w4a4_any_group(const GemmParams& p, int G, bool out_f32, hipStream_t st);
// Stand-in block normalizations (svdq_block.hip): adaptive RMS norm of rows [T, H] (H % 8 == 0),
// per-head RMS norm + rotary embedding of contiguous [T, heads, 128]
hipError_t launch_rms_norm_modulate(const uint16_t* x, long ldx, const uint16_t* w, const uint16_t* shift, int T,
                                    int H, float eps, uint16_t* y, long ldy, hipStream_t st);
// xo = bf16(x + g * v) (torch.addcmul, g a vector [H]), then y = the adaptive RMS norm of xo
hipError_t launch_residual_rms_norm_modulate(const uint16_t* x, long ldx, const uint16_t* v, long ldv,
                                             const uint16_t* g, const uint16_t* w, const uint16_t* shift, int T, int H,
                                             float eps, uint16_t* xo, long ldxo, uint16_t* y, long ldy,
                                             hipStream_t st);
hipError_t launch_head_rms_rope(const uint16_t* t, int T, int heads, const uint16_t* cs, const uint16_t* sn,
                                long ldcs, float eps, uint16_t* out, hipStream_t st);
// Stand-in block attention (svdq_attn.hip): softmax(scale q k^T) v, head dimension 128, H query heads
// over Hkv key / value heads (H % Hkv == 0); rows of q / o hold H heads, rows of k / v Hkv heads
// qcos / qsin (optional, [T, ldcs] bf16): q is normalized per head and rotated on load (the
// block's head norm + rotary of q), eps qeps
hipError_t launch_attention_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int T, int H,
                                int Hkv, long ldq, long ldkv, long ldo, float scale, void* workspace, hipStream_t st,
                                const uint16_t* qcos = nullptr, const uint16_t* qsin = nullptr, long ldcs = 0,
                                float qeps = 0.0f);
long attention_workspace_bytes(int T, int H);

}  // namespace svdq
