/* C-ABI of the MI355X (gfx950) SVDQuantLinear backend.
 *
 * Plain pointers, sizes and a hipStream_t; no torch types.  Every buffer is device memory on
 * the current HIP device, 16-byte aligned, row-major.  Every entry point enqueues work on
 * `stream` and returns immediately (no host synchronisation); it returns SVDQ_OK (0) or a
 * negative svdq_status, and svdq_last_error() then describes the failure (per host thread).
 *
 * Storage dtypes follow the reference checkpoint layout (reference runtime/load.py:90-126,
 * scripts/convert_simulated.py:201-208):
 *   bf16  : smooth_scale [K], l1 [N, r], l2 [r, K], bias [N], activations
 *   fp16  : weight_scales [N, K/G]
 *   uint8 : qweight_packed [N, K/2], byte j = (q[2j] + 8) | (q[2j+1] + 8) << 4
 *
 * A layer forward (reference runtime/linear.py:156-161 -> SVDQuantLinear.forward) is
 *   svdq_act_quant  (smoothing, A4 quantization + packing, low-rank and LoRA down)
 *   svdq_w4a4_gemm  (W4A4 GEMM + low-rank up + LoRA up + bias)
 * or, for the W4A16 variant,
 *   svdq_act_quant with SVDQ_ACT_XHAT only, then svdq_w4a16_gemm.
 */
#ifndef SVDQ_GFX950_H
#define SVDQ_GFX950_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum svdq_status {
  SVDQ_OK = 0,
  SVDQ_ERR_ARG = -1,         /* null pointer, non-positive size, bad flag            */
  SVDQ_ERR_SHAPE = -2,       /* K % group, rank limits, leading dimensions            */
  SVDQ_ERR_ALIGN = -3,       /* pointer or leading dimension not 16-byte aligned      */
  SVDQ_ERR_UNSUPPORTED = -4, /* group size or rank combination without a kernel       */
  SVDQ_ERR_LAUNCH = -5       /* the HIP runtime rejected the launch                   */
} svdq_status;

/* flags of svdq_act_quant */
#define SVDQ_ACT_PACKED 1u        /* also write the canonical packed A4 codes qx (pack.py layout) */
#define SVDQ_ACT_XHAT 2u          /* write the smoothed bf16 activation x_hat                   */
#define SVDQ_ACT_EXACT_DIV 4u     /* IEEE division for x / s everywhere (slow reference mode)   */
#define SVDQ_ACT_OPERAND_E4M3 8u  /* quantize: write scales sx and e4m3 operand codes qa        */
#define SVDQ_ACT_OPERAND_I8 16u   /* quantize: write scales sx and int8 (16*q) operand codes qa */
#define SVDQ_ACT_SX_PAIRS 32u     /* quantize: write sx as u32 bf16 pairs (sx | sx << 16), the
                                     form svdq_w4a4_gemm takes (its scale-MFMA operand)        */
#define SVDQ_ACT_OPERAND_E3M2 64u /* quantize: write scales sx and e3m2 (FP6) operand codes qa in
                                     the planar layout (see svdq_act_quant)                       */

/* Operand formats of svdq_w4a4_gemm (must match the SVDQ_ACT_OPERAND_* flag used). */
#define SVDQ_OPERAND_E4M3 0    /* FP8 MFMA (v_mfma_f32_32x32x64_f8f6f4): every INT4 code is exact */
#define SVDQ_OPERAND_I8 1      /* INT8 MFMA (v_mfma_i32_32x32x32_i8) on 16*q                     */
#define SVDQ_OPERAND_E3M2 2    /* FP6 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4, e3m2 x e3m2), twice the
                                  FP8 rate: every INT4 code is an exact e3m2 value; planar layout */

/* Library version string. */
const char* svdq_version(void);

/* Message for the most recent failing call on this host thread ("" if none). */
const char* svdq_last_error(void);

/* Most layers of one sibling call (svdq_act_quant_siblings, svdq_w4a4_gemm_siblings). */
#define SVDQ_MAX_SIBLINGS 4

/* Group sizes with kernels in this build; returns 1 if `group` is supported: any positive
 * multiple of 16 (the reference quantizer takes any group, quant/pack.py:6-23; its own test uses
 * 16, tests/test_svd_linear_cpu.py:10).  64 and 128 have the tuned kernels and every operand
 * format.  Every other group size takes the generic kernels: K % 64 == 0, the int8 operand only
 * (SVDQ_ACT_OPERAND_I8 / SVDQ_OPERAND_I8), quantized from x_hat (svdq_act_quant needs
 * SVDQ_ACT_XHAT and an xhat buffer with it), no fused epilogue op on svdq_w4a4_gemm_epi, and no
 * 2^31 limit on M*K or N*K. */
int svdq_group_supported(int group);

/* Per-layer constant of the activation pass: srs[0:K] = float(smooth), srs[K:2K] =
 * RN(1 / float(smooth)).  Replaces the per-call `x / smooth` set-up of reference
 * quant/svd.py:121-122 and kernels/triton/generic_int4.py:167-171.
 *   smooth : bf16 [K]      srs : f32 [2K] (output) */
int svdq_prepare_smooth(const void* smooth, float* srs, int K, hipStream_t stream);

/* Output sizing of svdq_act_quant for (M, K, group, RTp): the number S of K splits the
 * activation pass uses and the floats of its `mid` workspace, (S + 1) * M * RTp: the
 * finalized GEMM operand (M * RTp floats' worth of bytes) followed by one partial per split. */
int svdq_act_quant_workspace(int M, int K, int group, int RTp, int* splits, int64_t* mid_floats);

/* Fused activation pass.  Replaces reference quant/svd.py:121-122 (x_hat = x / smooth),
 * quant/pack.py:6-23 + 47-56 applied per group to x_hat (the A4 step of README.md:188-195),
 * quant/svd.py:159 / kernels/triton/generic_int4.py:238-241 (mid = x_hat @ l2^T) and
 * runtime/linear.py:42-45 (LoRA down x @ A^T on the raw x, times the multiplier).
 *   x        : bf16 [M, ldx]          srs : f32 [2K] from svdq_prepare_smooth
 *   l2       : bf16 [r, K]            lora_down : bf16 [rl, K] or NULL (rl = 0)
 *   lora_mult: f32 [rl]: per-column multiplier scale * alpha / rank of the owning adapter
 *   Quantizing (one SVDQ_ACT_OPERAND_* flag):
 *     sx : bf16 [M, K/group] scales, bit-exact bf16(max(amax, bf16(1e-8)) / 7); with
 *          SVDQ_ACT_SX_PAIRS u32 [K/group, M] (group-major) holding (bits | bits << 16)
 *     qa : u8 [M, K] operand codes of the W4A4 GEMM: the code of k sits at byte
 *          8*(k/8) + perm(k%8), perm = {0,4,1,5,2,6,3,7} (even k of a chunk of 8, then odd k);
 *          e4m3(q) or int8 16*q.  SVDQ_ACT_OPERAND_E3M2: u8 [Mp * K * 3/4], Mp = M rounded up to
 *          even, planar: for k-step t = k / 64 and half h = (k / 32) % 2 the row's 32 e3m2
 *          codes are contiguous 6-bit fields (field f = code of k = 64 t + 32 h + f) in 24 bytes,
 *          bytes 0-15 at Q[t][h][Mp][16] (offset 0), bytes 16-23 at P[t][h][Mp][8] (offset
 *          Mp * K / 2); rows of the padding are not written
 *     qx : u8 [M, K/2] canonical packed codes (pack.py:47-56), if SVDQ_ACT_PACKED
 *   xhat     : bf16 [M, ldxh] (SVDQ_ACT_XHAT; with a quantizing flag: e4m3 at group 64 / 128, and
 *              required with I8 at any other group size, whose codes are quantized from it)
 *   E3M2 needs K % 64 == 0 (always true at group 64 or 128) and a 16-byte aligned qa.
 *   mid      : workspace of svdq_act_quant_workspace's mid_floats floats.  Output at its head:
 *              bf16 [M, 2, RTp], per row the hi plane then the lo plane of the f32 low-rank
 *              activations (hi + lo within 2^-18 relative), whose columns are [0, r) = x_hat @ l2^T,
 *              [r, r+rl) = mult * (x @ A^T), [r+rl, RTp) = 0; the split partials behind it are
 *              summed in split order.  RTp % 32 == 0, RTp >= r + rl (any rank: the down
 *              projections run in launches of 4 MFMA column tiles, 32 columns each);
 *              S (`splits`) from svdq_act_quant_workspace. */
int svdq_act_quant(const void* x, int64_t ldx, const float* srs, const void* l2, int r,
                   const void* lora_down, int rl, const float* lora_mult, int M, int K, int group,
                   int RTp, unsigned flags, void* qa, void* sx, void* qx, void* xhat, int64_t ldxh,
                   float* mid, int splits, hipStream_t stream);

/* The activation passes of sibling layers over the same x (e.g. attn.to_q / to_k / to_v / to_gate,
 * whose smoothing vectors differ, so each has its own codes): each layer's output equals
 * svdq_act_quant(x, ..., layer's srs, l2, r, no LoRA, ...) bit for bit.  With flags =
 * SVDQ_ACT_OPERAND_E3M2 | SVDQ_ACT_SX_PAIRS, group 64 or 128 and every r <= 32 the layers run as
 * one launch and their finalize as one more; otherwise svdq_act_quant per layer, in order.  The
 * reference quantizes each layer's input in its own forward (quant/svd.py:121-122,
 * quant/pack.py:6-23 through runtime/linear.py:156-161).
 *   layers[i]: srs, l2 [r, K] and r of the layer; its qa, sx (as in svdq_act_quant) and mid
 *              workspace of svdq_act_quant_workspace(M, K, group, RTp) floats
 *   RTp, splits: shared (one svdq_act_quant_workspace query) */
typedef struct svdq_act_sibling {
  const float* srs;
  const void* l2;
  int r;
  void* qa;
  void* sx;
  float* mid;
} svdq_act_sibling;
int svdq_act_quant_siblings(const void* x, int64_t ldx, const svdq_act_sibling* layers, int count, int M, int K,
                            int group, int RTp, unsigned flags, int splits, hipStream_t stream);

/* Largest split-partial buffer of svdq_act_quant_noalloc, in floats (16 MiB): S * M * RTp must
 * not exceed it (S from svdq_act_quant_workspace). */
#define SVDQ_ACT_NOALLOC_MAX_FLOATS (4 << 20)

/* svdq_act_quant without any allocation or caller workspace.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, flags, arithmetic and
 * outputs as svdq_act_quant, except that `midp` is only the finalized GEMM operand (bf16
 * [M, 2, RTp], i.e. the head of svdq_act_quant's workspace, M * RTp floats' worth of bytes);
 * the S split partials live in a file-scope device array of SVDQ_ACT_NOALLOC_MAX_FLOATS floats
 * that each GPU holds until the process ends.  Calls whose partials do not fit return
 * SVDQ_ERR_SHAPE.  Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, or threads) race and must be serialized by the caller.  The array of the
 * calling thread's current device is used, so that device must own `stream` and the buffers.
 * The entry point calls no hipMalloc / hipFree; its first call on a device looks the array up
 * (hipGetSymbolAddress). */
int svdq_act_quant_noalloc(const void* x, int64_t ldx, const float* srs, const void* l2, int r,
                           const void* lora_down, int rl, const float* lora_mult, int M, int K, int group,
                           int RTp, unsigned flags, void* qa, void* sx, void* qx, void* xhat, int64_t ldxh,
                           float* midp, hipStream_t stream);

/* Per-layer weight-scale operand of svdq_w4a4_gemm: swp[g][n] = bf16 hi | bf16 lo << 16 with
 * hi + lo == float(sw[n][g]) exactly (times 1/256 for SVDQ_OPERAND_I8), group-major.  No
 * reference counterpart: it splits the checkpoint's fp16 weight_scales (runtime/load.py:116)
 * for the bf16 MFMA that forms the per-group scale products.
 *   sw : fp16 [N, ngroups]      swp : u32 [ngroups, N] (output) */
int svdq_prepare_weight_scales(const void* sw, void* swp, int N, int ngroups, int operand, hipStream_t stream);

/* Per-layer weight operand of svdq_w4a4_gemm: the packed INT4 codes of the checkpoint
 * (runtime/load.py:90-126, pack.py:47-56) expanded to one 8-bit MFMA operand code per weight,
 * in the byte order and `operand` format of svdq_act_quant's qa.  No reference counterpart:
 * the GEMM streams both operands into LDS without unpacking, trading N*K bytes of HBM for
 * the per-tile conversion work.
 *   qw : u8 [N, K/2]      qwe : u8 [N, K] (output);  K % 16 == 0
 *   SVDQ_OPERAND_E3M2: qwe u8 [Np * K * 3/4], Np = N rounded up to even, in the planar layout
 *   of svdq_act_quant's e3m2 qa (rows n); K % 64 == 0 */
int svdq_prepare_weight_operand(const void* qw, void* qwe, int N, int K, int operand, hipStream_t stream);

/* W4A4 GEMM with fused epilogue.  Replaces the residual product of reference
 * quant/svd.py:158 / kernels/triton/generic_int4.py:18-82 (with INT4 activations), the
 * low-rank add + bias of generic_int4.py:84-133 / svd.py:159-163 and the LoRA add of
 * runtime/linear.py:158-160:
 *   y = sum_g sx sw (qa . qw)_g + mid @ l1cat^T + bias
 *   qa : u8 [M, K] operand codes (svdq_act_quant) in `operand` format (SVDQ_OPERAND_*); the
 *        planar [Mp * K * 3/4] bytes for SVDQ_OPERAND_E3M2
 *   sxp: u32 [K/group, M] bf16 pairs (svdq_act_quant with SVDQ_ACT_SX_PAIRS)
 *   qwe: u8 [N, K] from svdq_prepare_weight_operand (same format; planar for E3M2)
 *   swp: u32 [K/group, N] from svdq_prepare_weight_scales (same operand format)
 *   E4M3 / I8 at group 64 / 128: M*K and N*K below 2^31 (larger problems are split over rows
 *   by the caller).  Other group sizes (see svdq_group_supported): SVDQ_OPERAND_I8 and
 *   SVDQ_EPI_NONE only.
 *   mid: bf16 [M, 2, RTp] (hi, lo planes) = the head of svdq_act_quant's mid workspace
 *   l1cat : bf16 [N, RTp] = [l1 | up_1 | ... | 0]
 *   bias: bf16 [N] or NULL     y : [M, ldy], bf16 (out_f32 = 0) or f32 (out_f32 = 1) */
int svdq_w4a4_gemm(const void* qa, int operand, const void* sxp, const void* qwe, const void* swp,
                   const void* mid, const void* l1cat, int RTp, const void* bias, int M, int N, int K, int group,
                   void* y, int64_t ldy, int out_f32, hipStream_t stream);

/* Block tile of the W4A4 GEMM svdq_w4a4_gemm runs for a shape (no fused op): returns the tile's
 * column count, 256 (256 x 256 tiles, wave tile 128 x 64) or 128 (256 x 128 tiles), or 0 when the
 * shape takes another kernel (other operand formats and group sizes).  Both tilings give
 * bit-identical outputs; the environment variable SVDQ_W4A4_TILES=256x128 or 256x256 overrides
 * the choice (the second only where M, N and K are multiples of 256).  No reference counterpart:
 * a host-side query for callers that report which kernel ran (bench.py, tests). */
int svdq_w4a4_gemm_tile_cols(int M, int N, int K, int group, int operand);

/* W4A16 GEMM with fused epilogue: the reference pytorch_sim math (quant/svd.py:119-163;
 * dequantization pack.py:26-44 in bf16) and kernels/triton/generic_int4.py:18-133.
 *   xhat : bf16 [M, ldxh] (from svdq_act_quant with SVDQ_ACT_XHAT); other arguments as in
 *   svdq_w4a4_gemm. */
int svdq_w4a16_gemm(const void* xhat, int64_t ldxh, const void* qw, const void* sw, const void* mid,
                    const void* l1cat, int RTp, const void* bias, int M, int N, int K, int group, void* y,
                    int64_t ldy, int out_f32, hipStream_t stream);

/* Elementwise ops the GEMMs can apply to their bf16 output before the store (the `_epi` entry
 * points).  With o = the bf16 layer output (the y above), a = aux[m][n] (bf16) and g = vec[n] (bf16);
 * every step rounds to bf16 as the unfused torch op on bf16 tensors does. */
#define SVDQ_EPI_NONE 0           /* y                                                      */
#define SVDQ_EPI_MUL_SIGMOID 1    /* bf16(a * bf16(sigmoid(o)))   gated attention output    */
#define SVDQ_EPI_SILU_MUL 2       /* bf16(bf16(silu(a)) * o)      SwiGLU, a = the gate      */
#define SVDQ_EPI_RESIDUAL_GATE 3  /* bf16(a + g * o), one rounding (torch.addcmul): gated residual */

/* svdq_w4a4_gemm / svdq_w4a16_gemm with an elementwise op fused into the store.  No reference
 * counterpart inside the reference: they fold the elementwise torch ops that a DiT block applies
 * to a quantized linear's output (SwiGLU of ff.gate / ff.up, the sigmoid output gate of
 * attention, the gated residual of to_out.0 and ff.down) into the GEMM's one bf16 store, for
 * the callers around Krea2Transformer2DModel's linears (reference README.md:41-51 names them).
 *   epi  : SVDQ_EPI_*; out_f32 must be 0 when epi != SVDQ_EPI_NONE
 *   aux  : bf16 [M, ldaux], ldaux >= N (may not alias y); read by 16-byte loads when it is
 *          16-byte aligned with ldaux % 8 == 0 (and vec 16-byte aligned), else per element
 *   vec  : bf16 [N] (SVDQ_EPI_RESIDUAL_GATE only)
 *   other arguments as in svdq_w4a4_gemm / svdq_w4a16_gemm. */
int svdq_w4a4_gemm_epi(const void* qa, int operand, const void* sxp, const void* qwe, const void* swp,
                       const void* mid, const void* l1cat, int RTp, const void* bias, int M, int N, int K, int group,
                       void* y, int64_t ldy, int out_f32, int epi, const void* aux, int64_t ldaux, const void* vec,
                       hipStream_t stream);
int svdq_w4a16_gemm_epi(const void* xhat, int64_t ldxh, const void* qw, const void* sw, const void* mid,
                        const void* l1cat, int RTp, const void* bias, int M, int N, int K, int group, void* y,
                        int64_t ldy, int out_f32, int epi, const void* aux, int64_t ldaux, const void* vec,
                        hipStream_t stream);

/* Sibling linears in one launch: up to SVDQ_MAX_SIBLINGS W4A4 GEMMs over the same activation rows
 * (same M, K and group; each layer with its own operands, scales, low-rank factors, bias and
 * output), e.g. attn.to_q / to_k / to_v / to_gate or ff.gate / ff.up of one block.  The reference
 * calls such layers one after another, each through SVDQuantLinear.forward (reference
 * runtime/linear.py:156-161; the layer names: reference README.md:41-51); each output here
 * equals svdq_w4a4_gemm's for that layer bit for bit.  With SVDQ_OPERAND_E3M2, group 64 or 128 and
 * K % 512 == 0 the layers' output tiles run in one launch, so that the tiles of small layers
 * and the last partial round of workgroups of each layer share the CUs; otherwise the layers are
 * launched one after another on `stream`.
 *   layers[i]: the per-layer arguments of svdq_w4a4_gemm (qa and sxp from that layer's own
 *              svdq_act_quant: the smoothing differs per layer), with out_f32 = 0 or 1 for all. */
typedef struct svdq_w4a4_sibling {
  const void* qa;
  const void* sxp;
  const void* qwe;
  const void* swp;
  const void* mid;
  const void* l1cat;
  int RTp;
  const void* bias;
  int N;
  void* y;
  int64_t ldy;
} svdq_w4a4_sibling;
int svdq_w4a4_gemm_siblings(const svdq_w4a4_sibling* layers, int count, int operand, int M, int K, int group,
                            int out_f32, hipStream_t stream);

/* The same for W4A16 layers: up to SVDQ_MAX_SIBLINGS svdq_w4a16_gemm calls over the same rows (same
 * M, K and group; each layer with its own x_hat from its own svdq_act_quant, since the smoothing
 * differs per layer), e.g. attn.to_q / to_gate / to_k / to_v.  The reference calls them one after
 * another through SVDQuantLinear.forward (reference runtime/linear.py:156-161); each output here
 * equals svdq_w4a16_gemm's for that layer bit for bit.  With group 64 or 128 and every layer fit
 * for the specialized-wave kernel (no fused op; x_hat 16-byte aligned rows) the layers' 192 x 256
 * output tiles run in one launch when their rounds over the CUs cost no more than the layers'
 * own launches (the attention inputs at M = 2304: 720 tiles in 3 rounds against 2 rounds of
 * 256 x 256 tiles and 2 of 128 x 128 tiles); otherwise the layers run one after another on
 * `stream`.
 *   layers[i]: the per-layer arguments of svdq_w4a16_gemm, with out_f32 = 0 or 1 for all. */
typedef struct svdq_w4a16_sibling {
  const void* xhat;
  int64_t ldxh;
  const void* qw;
  const void* sw;
  const void* mid;
  const void* l1cat;
  int RTp;
  const void* bias;
  int N;
  void* y;
  int64_t ldy;
} svdq_w4a16_sibling;
int svdq_w4a16_gemm_siblings(const svdq_w4a16_sibling* layers, int count, int M, int K, int group, int out_f32,
                             hipStream_t stream);

/* The sigmoid output gate and the SwiGLU product of a DiT block as one pass each over contiguous
 * bf16 tensors: out[i] = op(y[i], aux[i]) with op SVDQ_EPI_MUL_SIGMOID (aux * sigmoid(y)) or
 * SVDQ_EPI_SILU_MUL (silu(aux) * y), rounded as the fused store ops above (and as the torch ops on
 * bf16 tensors).  No counterpart inside the reference (its blocks run these ops in diffusers); for
 * the callers of svdq_w4a4_gemm_siblings, whose grouped layers cannot carry a fused op.
 *   y, aux, out: 16-byte aligned, n elements each (out may equal y or aux) */
int svdq_gate_op(int op, const void* y, const void* aux, void* out, int64_t n, hipStream_t stream);

/* Normalizations of the stand-in Krea-2 block around its quantized linears.  No counterpart in
 * the reference: its blocks run in diffusers (reference src/krea2_svdquant/transformer.py:46-59),
 * whose internals it does not contain.  bf16 in and out, float32 math, one pass over the rows.
 *
 * Adaptive RMS norm, per row of H (H % 8 == 0; x, w, shift, y 16-byte aligned, ldx, ldy
 * multiples of 8, y may not overlap x):
 *   y = bf16(bf16(x * rsqrt(mean(x^2) + eps) * w) + shift)     w = 1 + scale, shift: bf16 [H] */
int svdq_rms_norm_modulate(const void* x, int64_t ldx, const void* w, const void* shift, int T, int H, float eps,
                           void* y, int64_t ldy, hipStream_t stream);

/* The gated residual add that precedes the norm, in the same pass:
 *   xo = bf16(x + g * v)   (torch.addcmul(x, g, v): one rounding; g: bf16 [H], v: bf16 [T, ldv])
 *   y  = the adaptive RMS norm above of xo
 * All pointers 16-byte aligned, leading dimensions multiples of 8; xo may equal x, y overlaps
 * neither. */
int svdq_residual_rms_norm_modulate(const void* x, int64_t ldx, const void* v, int64_t ldv, const void* g,
                                    const void* w, const void* shift, int T, int H, float eps, void* xo, int64_t ldxo,
                                    void* y, int64_t ldy, hipStream_t stream);

/* Per-head RMS norm and rotate-half rotary embedding of t, contiguous bf16 [T, heads, 128] (q or
 * k), into out (same layout, may not overlap t).  cos / sin: bf16 [T, ldcs] position tables, of
 * which columns 0..63 are read (the rotate-half tables repeat their first half).  Per head:
 *   n = bf16(t * rsqrt(mean(t^2) + eps));  for j < 64, (n1, n2) = (n[j], n[j + 64]):
 *   out[j] = bf16(fma(-n2, sin, bf16(n1 * cos))),  out[j + 64] = bf16(fma(n1, sin, bf16(n2 * cos))) */
int svdq_head_rms_rope(const void* t, int T, int heads, const void* cos, const void* sin, int64_t ldcs, float eps,
                       void* out, hipStream_t stream);

/* Softmax attention of the stand-in block (no mask), head dimension 128, grouped-query:
 *   o[t, h, :] = sum_u softmax_u(scale * q[t, h, :] . k[u, h / (H / Hkv), :]) v[u, h / (H / Hkv), :]
 * q, o: bf16 rows of H heads x 128 with row strides ldq, ldo; k, v: bf16 rows of Hkv heads x 128
 * with row stride ldkv (elements; multiples of 8, pointers 16-byte aligned, o not overlapping the
 * inputs; T * ldkv * 2 below 2^31 bytes).  Scores and softmax statistics float32, probabilities rounded to bf16 for the product
 * with v, o rounded to bf16 once.  workspace: svdq_attention_workspace(T, H) bytes of device memory,
 * 16-byte aligned, no initial contents (the call's kernels share it on the stream; overlapping
 * calls need separate workspaces).  No counterpart in the reference: its blocks run in diffusers
 * (reference src/krea2_svdquant/transformer.py:46-59), whose attention is PyTorch's
 * scaled_dot_product_attention. */
int64_t svdq_attention_workspace(int T, int H);
int svdq_attention_fwd(const void* q, int64_t ldq, const void* k, const void* v, int64_t ldkv, int T, int H,
                       int Hkv, float scale, void* o, int64_t ldo, void* workspace, hipStream_t stream);

/* svdq_attention_fwd with the block's per-head RMS norm and rotary embedding of q applied on load
 * (as svdq_head_rms_rope(q, ...) followed by svdq_attention_fwd, without the normalized copy of q;
 * a normalized value can differ by one bf16 ulp where the float32 mean of squares, summed in
 * another order, sits at a rounding boundary).  cos / sin: bf16 [T, ldcs] position tables
 * (columns 0..63 read), 16-byte aligned, ldcs % 8 == 0; eps >= 0.  No counterpart in the
 * reference (its blocks run in diffusers). */
int svdq_attention_fwd_qnorm(const void* q, int64_t ldq, const void* k, const void* v, int64_t ldkv, int T, int H,
                             int Hkv, float scale, const void* cos, const void* sin, int64_t ldcs, float eps, void* o,
                             int64_t ldo, void* workspace, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SVDQ_GFX950_H */
