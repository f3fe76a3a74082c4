// extern "C" entry points of libsvdq_gfx950.so: argument validation and kernel launch.
#include <stdarg.h>
#include <stdio.h>
#include <mutex>
#include <string>

#include "../../include/svdq_gfx950.h"
#include "svdq_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return SVDQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(SVDQ_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

bool fast_group(int group) { return group == 64 || group == 128; }

// The group size the activation kernel runs with: the layer's own for 64 / 128; 64 for the generic
// path (the kernel then writes x_hat and the down projections only, which do not depend on the
// group, and the generic quantizer reads x_hat).
int kernel_group(int group) { return fast_group(group) ? group : 64; }

int check_group(int group, int K) {
  if (!svdq_group_supported(group))
    return fail(SVDQ_ERR_UNSUPPORTED, "group size %d has no kernel (64, 128, or a multiple of 16)", group);
  if (K <= 0 || K % group != 0) return fail(SVDQ_ERR_SHAPE, "K=%d must be a positive multiple of group=%d", K, group);
  if (!fast_group(group) && K % 64 != 0)
    return fail(SVDQ_ERR_SHAPE, "K=%d: group size %d needs K %% 64 == 0", K, group);
  return SVDQ_OK;
}

int mid_tiles(int r, int rl) { return (r + 31) / 32 + (rl + 31) / 32; }

}  // namespace

extern "C" {

const char* svdq_version(void) { return "svdq_gfx950 0.1.0"; }

const char* svdq_last_error(void) { return g_last_error.c_str(); }

int svdq_group_supported(int group) { return group > 0 && group % 16 == 0; }

int svdq_prepare_smooth(const void* smooth, float* srs, int K, hipStream_t stream) {
  if (!smooth || !srs) return fail(SVDQ_ERR_ARG, "prepare_smooth: null pointer");
  if (K <= 0) return fail(SVDQ_ERR_ARG, "prepare_smooth: K=%d", K);
  return launched(svdq::launch_prepare_smooth(static_cast<const uint16_t*>(smooth), srs, K, stream),
                  "prepare_smooth");
}

int svdq_act_quant_workspace(int M, int K, int group, int RTp, int* splits, int64_t* mid_floats) {
  if (M <= 0) return fail(SVDQ_ERR_ARG, "act_quant_workspace: M=%d", M);
  if (int e = check_group(group, K)) return e;
  if (RTp <= 0 || RTp % 32) return fail(SVDQ_ERR_SHAPE, "RTp=%d must be a positive multiple of 32", RTp);
  const int s = svdq::act_splits(M, K, kernel_group(group));
  if (splits) *splits = s;
  if (mid_floats) *mid_floats = (int64_t)(s + 1) * M * RTp;
  return ok();
}

}  // extern "C"

namespace {

// The activation pass behind svdq_act_quant and svdq_act_quant_noalloc: `head` receives the
// finalized GEMM operand [M, 2, RTp] bf16, `part` holds the `splits` f32 partials [splits, M, RTp]
// (every entry of rows < M written by the act kernel before the finalize kernel reads it).
int act_quant_run(const void* x, int64_t ldx, const float* srs, const void* l2, int r, const void* lora_down,
                  int rl, const float* lora_mult, int M, int K, int group, int RTp, unsigned flags, void* qa,
                  void* sx, void* qx, void* xhat, int64_t ldxh, float* head, float* part, int splits,
                  hipStream_t stream, svdq::ActParams* checked = nullptr) {
  // checked: validate only, and return the launch parameters of the first launch instead
  const unsigned known = SVDQ_ACT_PACKED | SVDQ_ACT_XHAT | SVDQ_ACT_EXACT_DIV | SVDQ_ACT_OPERAND_E4M3 |
                         SVDQ_ACT_OPERAND_I8 | SVDQ_ACT_SX_PAIRS | SVDQ_ACT_OPERAND_E3M2;
  if (flags & ~known) return fail(SVDQ_ERR_ARG, "act_quant: unknown flags 0x%x", flags);
  const bool e4m3 = flags & SVDQ_ACT_OPERAND_E4M3, i8 = flags & SVDQ_ACT_OPERAND_I8;
  const bool e3m2 = flags & SVDQ_ACT_OPERAND_E3M2;
  const bool quant = e4m3 || i8 || e3m2, want_xhat = flags & SVDQ_ACT_XHAT, packed = flags & SVDQ_ACT_PACKED;
  if ((int)e4m3 + (int)i8 + (int)e3m2 > 1) return fail(SVDQ_ERR_ARG, "act_quant: two operand formats requested");
  if (!quant && !want_xhat) return fail(SVDQ_ERR_ARG, "act_quant: neither an operand format nor XHAT requested");
  if (packed && !quant) return fail(SVDQ_ERR_ARG, "act_quant: PACKED needs an operand format");
  const bool pairs = flags & SVDQ_ACT_SX_PAIRS;
  if (pairs && !quant) return fail(SVDQ_ERR_ARG, "act_quant: SX_PAIRS needs an operand format");
  if (M <= 0) return fail(SVDQ_ERR_ARG, "act_quant: M=%d", M);
  if (int e = check_group(group, K)) return e;
  const bool generic = !fast_group(group);
  if (generic) {
    // the generic path: int8 operand codes, quantized from the x_hat the caller's buffer receives
    if (e4m3 || e3m2)
      return fail(SVDQ_ERR_UNSUPPORTED, "act_quant: group size %d has int8 operands only (SVDQ_ACT_OPERAND_I8)", group);
    if (i8 && !want_xhat)
      return fail(SVDQ_ERR_ARG, "act_quant: group size %d quantizes from x_hat: add SVDQ_ACT_XHAT and an xhat buffer",
                  group);
  } else if ((i8 || e3m2) && want_xhat) {
    return fail(SVDQ_ERR_UNSUPPORTED, "act_quant: XHAT with int8 or e3m2 operands has no kernel");
  }
  if (r < 1 || rl < 0) return fail(SVDQ_ERR_SHAPE, "act_quant: rank r=%d rl=%d", r, rl);
  if (RTp % 32 || RTp < r + rl) return fail(SVDQ_ERR_SHAPE, "act_quant: RTp=%d (r=%d rl=%d)", RTp, r, rl);
  const int nt = mid_tiles(r, rl);   // MFMA column tiles of the down projections (any number)
  if (!x || !srs || !l2 || !head || !part || (rl > 0 && (!lora_down || !lora_mult)) || (quant && (!qa || !sx)) ||
      (packed && !qx) || (want_xhat && !xhat))
    return fail(SVDQ_ERR_ARG, "act_quant: null pointer");
  if (ldx < K || ldx % 8 || (want_xhat && (ldxh < K || ldxh % 8)))
    return fail(SVDQ_ERR_ALIGN, "act_quant: ldx=%lld ldxh=%lld must be >= K and multiples of 8",
                (long long)ldx, (long long)ldxh);
  if (!aligned16(x) || !aligned16(srs) || !aligned16(l2) || !aligned16(head) || !aligned16(part) ||
      (rl > 0 && !aligned16(lora_down)) || (quant && !aligned16(qa)) || (packed && !aligned16(qx)) ||
      (pairs && reinterpret_cast<uintptr_t>(sx) % 4) ||
      (want_xhat && !aligned16(xhat)))
    return fail(SVDQ_ERR_ALIGN, "act_quant: device pointers must be 16-byte aligned");
  svdq::ActParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.srs = srs;
  p.l2 = static_cast<const uint16_t*>(l2);
  p.lora = static_cast<const uint16_t*>(lora_down);
  p.lora_mult = lora_mult;
  p.r = r;
  p.rl = rl;
  p.M = M;
  p.K = K;
  p.RTp = RTp;
  p.qx = packed ? static_cast<uint8_t*>(qx) : nullptr;
  p.qa = static_cast<uint8_t*>(qa);
  p.sx = static_cast<uint16_t*>(sx);
  p.xhat = static_cast<uint16_t*>(xhat);
  p.ldxh = ldxh;
  p.mid = part;
  const int ngroups = K / kernel_group(group);   // the act kernel's groups
  p.gps = (ngroups + splits - 1) / splits;
  p.exact = (flags & SVDQ_ACT_EXACT_DIV) ? 1 : 0;
  p.sx_pairs = pairs ? 1 : 0;
  if (checked) {
    p.t0 = 0;
    *checked = p;
    return SVDQ_OK;
  }
  // The first launch quantizes and computes the first 4 column tiles; each further launch adds 4
  // more tiles of the down projections (rank + LoRA rank beyond 128), into their own columns of
  // the split partials.
  p.t0 = 0;
  if (generic) {   // x_hat and the first tiles, then the group-size-generic quantizer from x_hat
    svdq::ActParams q = p;
    q.qa = nullptr;
    q.sx = nullptr;
    q.qx = nullptr;
    if (int e = launched(svdq::launch_act(q, kernel_group(group), nt < 4 ? nt : 4, 0, true, splits, stream),
                         "act_quant"))
      return e;
    if (i8) {
      if (int e = launched(svdq::launch_quant_any_group(p.xhat, ldxh, M, K, group, p.qa, p.sx, pairs ? 1 : 0, p.qx,
                                                        stream),
                           "act_quant (any-group quantizer)"))
        return e;
    }
  } else if (int e = launched(svdq::launch_act(p, group, nt < 4 ? nt : 4, e4m3 ? 1 : (i8 ? 2 : (e3m2 ? 3 : 0)),
                                               want_xhat, splits, stream),
                              "act_quant")) {
    return e;
  }
  for (int t0 = 4; t0 < nt; t0 += 4) {
    svdq::ActParams q = p;
    q.t0 = t0;
    q.qa = nullptr;
    q.sx = nullptr;
    q.qx = nullptr;
    q.xhat = nullptr;
    if (int e = launched(svdq::launch_act(q, kernel_group(group), nt - t0 < 4 ? nt - t0 : 4, 0, false, splits, stream),
                         "act_quant (down projections)"))
      return e;
  }
  return launched(svdq::launch_mid_finalize(p.mid, splits, M, RTp, reinterpret_cast<uint16_t*>(head), stream),
                  "act_quant (mid)");
}

// Device scratch of svdq_act_quant_noalloc: the activation pass's split partials.  Each GPU holds
// its own copy from code-object load until the process ends; the host side reaches it only
// through the per-device address hipGetSymbolAddress returns (the array's name is a host-side
// stand-in, not a device address).
constexpr int64_t kScratchFloats = SVDQ_ACT_NOALLOC_MAX_FLOATS;   // 16 MiB
__device__ __align__(256) float scratch[kScratchFloats];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch[kMaxDevices] = {};

// The scratch address on the calling thread's current device, looked up once per device.
int device_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SVDQ_ERR_LAUNCH, "act_quant_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(SVDQ_ERR_UNSUPPORTED, "act_quant_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(SVDQ_ERR_LAUNCH, "act_quant_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch[dev];
  return SVDQ_OK;
}

}  // namespace

extern "C" {

int svdq_act_quant(const void* x, int64_t ldx, const float* srs, const void* l2, int r,
                   const void* lora_down, int rl, const float* lora_mult, int M, int K, int group,
                   int RTp, unsigned flags, void* qa, void* sx, void* qx, void* xhat, int64_t ldxh,
                   float* mid, int splits, hipStream_t stream) {
  if (M > 0 && group > 0 && K > 0 && K % group == 0) {
    const int expect = svdq::act_splits(M, K, kernel_group(group));
    if (splits != expect) return fail(SVDQ_ERR_ARG, "act_quant: splits=%d, workspace says %d", splits, expect);
  }
  float* part = mid ? mid + (int64_t)(M > 0 ? M : 0) * (RTp > 0 ? RTp : 0) : nullptr;   // partials after the head
  return act_quant_run(x, ldx, srs, l2, r, lora_down, rl, lora_mult, M, K, group, RTp, flags, qa, sx, qx, xhat,
                       ldxh, mid, part, splits, stream);
}

int svdq_act_quant_siblings(const void* x, int64_t ldx, const svdq_act_sibling* layers, int count, int M, int K,
                            int group, int RTp, unsigned flags, int splits, hipStream_t stream) {
  if (!layers) return fail(SVDQ_ERR_ARG, "act_quant_siblings: null layer array");
  if (count < 1 || count > SVDQ_MAX_SIBLINGS)
    return fail(SVDQ_ERR_ARG, "act_quant_siblings: count=%d, must be 1..%d", count, SVDQ_MAX_SIBLINGS);
  bool one = fast_group(group) && flags == (SVDQ_ACT_OPERAND_E3M2 | SVDQ_ACT_SX_PAIRS);
  for (int i = 0; i < count; ++i) one = one && layers[i].r >= 1 && layers[i].r <= 32;
  if (!one) {   // other formats, flags, groups or ranks: one svdq_act_quant per layer, in order
    for (int i = 0; i < count; ++i) {
      const svdq_act_sibling& l = layers[i];
      if (int e = svdq_act_quant(x, ldx, l.srs, l.l2, l.r, nullptr, 0, nullptr, M, K, group, RTp, flags, l.qa, l.sx,
                                 nullptr, nullptr, 0, l.mid, splits, stream))
        return e;
    }
    return SVDQ_OK;
  }
  const int expect = svdq::act_splits(M, K, group);
  if (M > 0 && splits != expect)
    return fail(SVDQ_ERR_ARG, "act_quant_siblings: splits=%d, workspace says %d", splits, expect);
  svdq::ActSiblings s{};
  s.count = count;
  for (int i = 0; i < count; ++i) {
    const svdq_act_sibling& l = layers[i];
    float* part = l.mid ? l.mid + (int64_t)(M > 0 ? M : 0) * (RTp > 0 ? RTp : 0) : nullptr;
    if (int e = act_quant_run(x, ldx, l.srs, l.l2, l.r, nullptr, 0, nullptr, M, K, group, RTp, flags, l.qa, l.sx,
                              nullptr, nullptr, 0, l.mid, part, splits, stream, &s.layer[i]))
      return e;
    s.head[i] = reinterpret_cast<uint16_t*>(l.mid);
  }
  return launched(svdq::launch_act_siblings(s, group, splits, stream), "act_quant_siblings");
}

int svdq_act_quant_noalloc(const void* x, int64_t ldx, const float* srs, const void* l2, int r,
                           const void* lora_down, int rl, const float* lora_mult, int M, int K, int group,
                           int RTp, unsigned flags, void* qa, void* sx, void* qx, void* xhat, int64_t ldxh,
                           float* midp, hipStream_t stream) {
  if (M <= 0) return fail(SVDQ_ERR_ARG, "act_quant_noalloc: M=%d", M);
  if (int e = check_group(group, K)) return e;
  if (RTp <= 0 || RTp % 32) return fail(SVDQ_ERR_SHAPE, "act_quant_noalloc: RTp=%d must be a positive multiple of 32", RTp);
  const int splits = svdq::act_splits(M, K, kernel_group(group));
  const int64_t need = (int64_t)splits * M * RTp;
  if (need > kScratchFloats)
    return fail(SVDQ_ERR_SHAPE,
                "act_quant_noalloc: the split partials need %lld floats (%d splits x M=%d x RTp=%d), more than the "
                "%lld-float device scratch; use svdq_act_quant with a workspace",
                (long long)need, splits, M, RTp, (long long)kScratchFloats);
  float* part = nullptr;
  if (int e = device_scratch(&part)) return e;
  return act_quant_run(x, ldx, srs, l2, r, lora_down, rl, lora_mult, M, K, group, RTp, flags, qa, sx, qx, xhat,
                       ldxh, midp, part, splits, stream);
}

static int gemm_common_checks(const char* who, const void* qw, const void* sw, const void* mid,
                              const void* l1cat, int RTp, int M, int N, int K, int group, void* y, int64_t ldy,
                              int out_f32) {
  if (M <= 0 || N <= 0) return fail(SVDQ_ERR_ARG, "%s: M=%d N=%d", who, M, N);
  if (int e = check_group(group, K)) return e;
  if (!qw || !sw || !mid || !l1cat || !y) return fail(SVDQ_ERR_ARG, "%s: null pointer", who);
  if (RTp <= 0 || RTp % 32) return fail(SVDQ_ERR_SHAPE, "%s: RTp=%d must be a positive multiple of 32", who, RTp);
  if (out_f32 != 0 && out_f32 != 1) return fail(SVDQ_ERR_ARG, "%s: out_f32=%d", who, out_f32);
  if (ldy < N) return fail(SVDQ_ERR_SHAPE, "%s: ldy=%lld < N=%d", who, (long long)ldy, N);
  if (!aligned16(qw) || !aligned16(mid) || !aligned16(l1cat) || (K / 2) % 8)
    return fail(SVDQ_ERR_ALIGN, "%s: device pointers must be 16-byte aligned", who);
  return SVDQ_OK;
}

static svdq::GemmParams gemm_params(const void* qw, const void* sw, const void* mid, const void* l1cat, int RTp,
                                    const void* bias, int M, int N, int K, void* y, int64_t ldy) {
  svdq::GemmParams p{};
  p.qw = static_cast<const uint8_t*>(qw);
  p.sw = static_cast<const uint16_t*>(sw);
  p.midp = static_cast<const uint16_t*>(mid);
  p.l1cat = static_cast<const uint16_t*>(l1cat);
  p.RTp = RTp;
  p.bias = static_cast<const uint16_t*>(bias);
  p.y = y;
  p.ldy = ldy;
  p.M = M;
  p.N = N;
  p.K = K;
  return p;
}

int svdq_prepare_weight_scales(const void* sw, void* swp, int N, int ngroups, int operand, hipStream_t stream) {
  if (!sw || !swp) return fail(SVDQ_ERR_ARG, "prepare_weight_scales: null pointer");
  if (N <= 0 || ngroups <= 0) return fail(SVDQ_ERR_ARG, "prepare_weight_scales: N=%d ngroups=%d", N, ngroups);
  if (operand != SVDQ_OPERAND_E4M3 && operand != SVDQ_OPERAND_I8 && operand != SVDQ_OPERAND_E3M2)
    return fail(SVDQ_ERR_ARG, "prepare_weight_scales: operand format %d", operand);
  return launched(svdq::launch_weight_scale_pairs(static_cast<const uint16_t*>(sw), static_cast<uint32_t*>(swp), N,
                                                  ngroups, operand, stream),
                  "prepare_weight_scales");
}

int svdq_prepare_weight_operand(const void* qw, void* qwe, int N, int K, int operand, hipStream_t stream) {
  if (!qw || !qwe) return fail(SVDQ_ERR_ARG, "prepare_weight_operand: null pointer");
  if (N <= 0 || K <= 0 || K % 16) return fail(SVDQ_ERR_SHAPE, "prepare_weight_operand: N=%d K=%d (K %% 16 == 0)", N, K);
  if (operand != SVDQ_OPERAND_E4M3 && operand != SVDQ_OPERAND_I8 && operand != SVDQ_OPERAND_E3M2)
    return fail(SVDQ_ERR_ARG, "prepare_weight_operand: operand format %d", operand);
  if (operand == SVDQ_OPERAND_E3M2 && K % 64)
    return fail(SVDQ_ERR_SHAPE, "prepare_weight_operand: K=%d (e3m2 needs K %% 64 == 0)", K);
  if (!aligned16(qw) || !aligned16(qwe)) return fail(SVDQ_ERR_ALIGN, "prepare_weight_operand: pointers must be 16-byte aligned");
  return launched(svdq::launch_weight_operand(static_cast<const uint8_t*>(qw), static_cast<uint8_t*>(qwe), N, K,
                                              operand, stream),
                  "prepare_weight_operand");
}

static int epi_checks(const char* who, int epi, const void* aux, int64_t ldaux, const void* vec, int N,
                      int out_f32) {
  if (epi == SVDQ_EPI_NONE) return SVDQ_OK;
  if (epi != SVDQ_EPI_MUL_SIGMOID && epi != SVDQ_EPI_SILU_MUL && epi != SVDQ_EPI_RESIDUAL_GATE)
    return fail(SVDQ_ERR_ARG, "%s: epilogue op %d", who, epi);
  if (out_f32) return fail(SVDQ_ERR_ARG, "%s: epilogue ops need bf16 output (out_f32 = 0)", who);
  if (!aux || (epi == SVDQ_EPI_RESIDUAL_GATE && !vec)) return fail(SVDQ_ERR_ARG, "%s: null epilogue operand", who);
  if (ldaux < N) return fail(SVDQ_ERR_SHAPE, "%s: ldaux=%lld < N=%d", who, (long long)ldaux, N);
  if (reinterpret_cast<uintptr_t>(aux) % 2 || reinterpret_cast<uintptr_t>(vec) % 2)
    return fail(SVDQ_ERR_ALIGN, "%s: aux and vec must be 2-byte aligned (bf16)", who);
  return SVDQ_OK;
}

static void set_epi(svdq::GemmParams& p, int epi, const void* aux, int64_t ldaux, const void* vec) {
  p.epi = epi;
  p.aux = static_cast<const uint16_t*>(aux);
  p.ldaux = ldaux;
  p.evec = static_cast<const uint16_t*>(vec);
  p.aux_vec = aligned16(aux) && ldaux % 8 == 0 && (vec == nullptr || aligned16(vec));
}

int svdq_w4a4_gemm(const void* qa, int operand, const void* sxp, const void* qwe, const void* swp,
                   const void* mid, const void* l1cat, int RTp, const void* bias, int M, int N, int K, int group,
                   void* y, int64_t ldy, int out_f32, hipStream_t stream) {
  return svdq_w4a4_gemm_epi(qa, operand, sxp, qwe, swp, mid, l1cat, RTp, bias, M, N, K, group, y, ldy, out_f32,
                            SVDQ_EPI_NONE, nullptr, 0, nullptr, stream);
}

int svdq_w4a4_gemm_tile_cols(int M, int N, int K, int group, int operand) {
  if (operand != SVDQ_OPERAND_E3M2 || !fast_group(group) || M <= 0 || N <= 0 || K <= 0 || K % group) return 0;
  return group == 64 && svdq::use_wide_tiles(M, N, K) ? 256 : 128;
}

// Checks of one W4A4 layer's arguments and its kernel parameters (no fused op yet).
static int w4a4_layer(const char* who, const void* qa, int operand, const void* sxp, const void* qwe, const void* swp,
                      const void* mid, const void* l1cat, int RTp, const void* bias, int M, int N, int K, int group,
                      void* y, int64_t ldy, int out_f32, svdq::GemmParams& p) {
  if (int e = gemm_common_checks(who, qwe, swp, mid, l1cat, RTp, M, N, K, group, y, ldy, out_f32)) return e;
  if (!qa || !sxp) return fail(SVDQ_ERR_ARG, "%s: null pointer", who);
  if (operand != SVDQ_OPERAND_E4M3 && operand != SVDQ_OPERAND_I8 && operand != SVDQ_OPERAND_E3M2)
    return fail(SVDQ_ERR_ARG, "%s: operand format %d", who, operand);
  if (!aligned16(qa) || !aligned16(qwe) || reinterpret_cast<uintptr_t>(sxp) % 4 || reinterpret_cast<uintptr_t>(swp) % 4)
    return fail(SVDQ_ERR_ALIGN, "%s: qa, qwe must be 16-byte aligned, sxp, swp 4-byte aligned", who);
  // The 8-bit kernels address qa and qwe with 32-bit byte offsets (the e3m2 kernel with 64-bit
  // plane bases and 32-bit row offsets).
  if (operand != SVDQ_OPERAND_E3M2 && fast_group(group) &&
      ((int64_t)M * K > INT32_MAX || (int64_t)N * K > INT32_MAX || (int64_t)M * (K / group) * 4 > INT32_MAX ||
       (int64_t)N * (K / group) * 4 > INT32_MAX))
    return fail(SVDQ_ERR_SHAPE, "%s: M*K=%lld or N*K=%lld exceeds 2^31-1 bytes; split the call", who,
                (long long)M * K, (long long)N * K);
  if (!fast_group(group) && operand != SVDQ_OPERAND_I8)
    return fail(SVDQ_ERR_UNSUPPORTED, "%s: group size %d has int8 operands only (SVDQ_OPERAND_I8)", who, group);
  p = gemm_params(nullptr, swp, mid, l1cat, RTp, bias, M, N, K, y, ldy);
  p.qwe = static_cast<const uint8_t*>(qwe);
  p.qa = static_cast<const uint8_t*>(qa);
  p.sxp = static_cast<const uint32_t*>(sxp);
  p.swp = static_cast<const uint32_t*>(swp);
  return SVDQ_OK;
}

static hipError_t launch_w4a4_layer(const svdq::GemmParams& p, int group, int operand, int out_f32, hipStream_t stream) {
  if (!fast_group(group)) return svdq::launch_w4a4_any_group(p, group, out_f32 == 1, stream);
  return svdq::launch_w4a4(p, group, operand, out_f32 == 1, stream);
}

int svdq_w4a4_gemm_epi(const void* qa, int operand, const void* sxp, const void* qwe, const void* swp,
                       const void* mid, const void* l1cat, int RTp, const void* bias, int M, int N, int K, int group,
                       void* y, int64_t ldy, int out_f32, int epi, const void* aux, int64_t ldaux, const void* vec,
                       hipStream_t stream) {
  svdq::GemmParams p;
  if (int e = w4a4_layer("w4a4_gemm", qa, operand, sxp, qwe, swp, mid, l1cat, RTp, bias, M, N, K, group, y, ldy,
                         out_f32, p))
    return e;
  if (int e = epi_checks("w4a4_gemm", epi, aux, ldaux, vec, N, out_f32)) return e;
  set_epi(p, epi, aux, ldaux, vec);
  if (!fast_group(group) && epi != SVDQ_EPI_NONE)
    return fail(SVDQ_ERR_UNSUPPORTED, "w4a4_gemm: group size %d has no fused epilogue ops", group);
  return launched(launch_w4a4_layer(p, group, operand, out_f32, stream),
                  fast_group(group) ? "w4a4_gemm" : "w4a4_gemm (any group)");
}

int svdq_w4a4_gemm_siblings(const svdq_w4a4_sibling* layers, int count, int operand, int M, int K, int group,
                            int out_f32, hipStream_t stream) {
  if (!layers) return fail(SVDQ_ERR_ARG, "w4a4_gemm_siblings: null layer array");
  if (count < 1 || count > SVDQ_MAX_SIBLINGS)
    return fail(SVDQ_ERR_ARG, "w4a4_gemm_siblings: count=%d, must be 1..%d", count, SVDQ_MAX_SIBLINGS);
  svdq::GemmSiblings gs{};
  gs.count = count;
  int tiles = 0;
  for (int i = 0; i < count; ++i) {
    const svdq_w4a4_sibling& l = layers[i];
    if (int e = w4a4_layer("w4a4_gemm_siblings", l.qa, operand, l.sxp, l.qwe, l.swp, l.mid, l.l1cat, l.RTp, l.bias,
                           M, l.N, K, group, l.y, l.ldy, out_f32, gs.layer[i]))
      return e;
    gs.tile0[i] = tiles;
    tiles += ((M + 255) / 256) * ((l.N + 127) / 128);
  }
  gs.tile0[count] = tiles;
  if (operand == SVDQ_OPERAND_E3M2 && fast_group(group) && K % 512 == 0)
    return launched(svdq::launch_w4a4_siblings(gs, group, out_f32 == 1, stream), "w4a4_gemm_siblings");
  // other formats, groups and K: one launch per layer, in order
  for (int i = 0; i < count; ++i)
    if (int e = launched(launch_w4a4_layer(gs.layer[i], group, operand, out_f32, stream), "w4a4_gemm_siblings"))
      return e;
  return SVDQ_OK;
}

int svdq_gate_op(int op, const void* y, const void* aux, void* out, int64_t n, hipStream_t stream) {
  if (op != SVDQ_EPI_MUL_SIGMOID && op != SVDQ_EPI_SILU_MUL)
    return fail(SVDQ_ERR_ARG, "gate_op: op=%d (SVDQ_EPI_MUL_SIGMOID or SVDQ_EPI_SILU_MUL)", op);
  if (!y || !aux || !out) return fail(SVDQ_ERR_ARG, "gate_op: null pointer");
  if (n < 0) return fail(SVDQ_ERR_SHAPE, "gate_op: n=%lld", (long long)n);
  if (!aligned16(y) || !aligned16(aux) || !aligned16(out))
    return fail(SVDQ_ERR_ALIGN, "gate_op: y, aux, out must be 16-byte aligned");
  if (n == 0) return SVDQ_OK;
  return launched(svdq::launch_gate_op(op, static_cast<const uint16_t*>(y), static_cast<const uint16_t*>(aux),
                                       static_cast<uint16_t*>(out), n, stream),
                  "gate_op");
}

int svdq_rms_norm_modulate(const void* x, int64_t ldx, const void* w, const void* shift, int T, int H, float eps,
                           void* y, int64_t ldy, hipStream_t stream) {
  if (!x || !w || !shift || !y) return fail(SVDQ_ERR_ARG, "rms_norm_modulate: null pointer");
  if (T <= 0 || H <= 0 || H % 8) return fail(SVDQ_ERR_SHAPE, "rms_norm_modulate: T=%d, H=%d (H %% 8 == 0)", T, H);
  if (!(eps >= 0.0f)) return fail(SVDQ_ERR_ARG, "rms_norm_modulate: eps must be >= 0");
  if (ldx < H || ldy < H || ldx % 8 || ldy % 8 || !aligned16(x) || !aligned16(w) || !aligned16(shift) ||
      !aligned16(y))
    return fail(SVDQ_ERR_ALIGN, "rms_norm_modulate: 16-byte aligned pointers, ldx, ldy >= H and multiples of 8");
  return launched(svdq::launch_rms_norm_modulate(static_cast<const uint16_t*>(x), ldx, static_cast<const uint16_t*>(w),
                                                 static_cast<const uint16_t*>(shift), T, H, eps,
                                                 static_cast<uint16_t*>(y), ldy, stream),
                  "rms_norm_modulate");
}

int svdq_residual_rms_norm_modulate(const void* x, int64_t ldx, const void* v, int64_t ldv, const void* g,
                                    const void* w, const void* shift, int T, int H, float eps, void* xo, int64_t ldxo,
                                    void* y, int64_t ldy, hipStream_t stream) {
  if (!x || !v || !g || !w || !shift || !xo || !y) return fail(SVDQ_ERR_ARG, "residual_rms_norm_modulate: null pointer");
  if (T <= 0 || H <= 0 || H % 8)
    return fail(SVDQ_ERR_SHAPE, "residual_rms_norm_modulate: T=%d, H=%d (H %% 8 == 0)", T, H);
  if (!(eps >= 0.0f)) return fail(SVDQ_ERR_ARG, "residual_rms_norm_modulate: eps must be >= 0");
  if (ldx < H || ldv < H || ldxo < H || ldy < H || ldx % 8 || ldv % 8 || ldxo % 8 || ldy % 8 || !aligned16(x) ||
      !aligned16(v) || !aligned16(g) || !aligned16(w) || !aligned16(shift) || !aligned16(xo) || !aligned16(y))
    return fail(SVDQ_ERR_ALIGN,
                "residual_rms_norm_modulate: 16-byte aligned pointers, leading dimensions >= H and multiples of 8");
  return launched(svdq::launch_residual_rms_norm_modulate(
                      static_cast<const uint16_t*>(x), ldx, static_cast<const uint16_t*>(v), ldv,
                      static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(w),
                      static_cast<const uint16_t*>(shift), T, H, eps, static_cast<uint16_t*>(xo), ldxo,
                      static_cast<uint16_t*>(y), ldy, stream),
                  "residual_rms_norm_modulate");
}

int svdq_head_rms_rope(const void* t, int T, int heads, const void* cos, const void* sin, int64_t ldcs, float eps,
                       void* out, hipStream_t stream) {
  if (!t || !cos || !sin || !out) return fail(SVDQ_ERR_ARG, "head_rms_rope: null pointer");
  if (T <= 0 || heads <= 0 || ldcs < 64) return fail(SVDQ_ERR_SHAPE, "head_rms_rope: T=%d heads=%d ldcs=%lld",
                                                     T, heads, (long long)ldcs);
  if (!(eps >= 0.0f)) return fail(SVDQ_ERR_ARG, "head_rms_rope: eps must be >= 0");
  if (reinterpret_cast<uintptr_t>(t) % 2 || reinterpret_cast<uintptr_t>(out) % 2 ||
      reinterpret_cast<uintptr_t>(cos) % 2 || reinterpret_cast<uintptr_t>(sin) % 2)
    return fail(SVDQ_ERR_ALIGN, "head_rms_rope: bf16 pointers must be 2-byte aligned");
  return launched(svdq::launch_head_rms_rope(static_cast<const uint16_t*>(t), T, heads,
                                             static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin),
                                             ldcs, eps, static_cast<uint16_t*>(out), stream),
                  "head_rms_rope");
}

int64_t svdq_attention_workspace(int T, int H) {
  return T > 0 && H > 0 ? (int64_t)svdq::attention_workspace_bytes(T, H) : 0;
}

static int attention_checks(const void* q, int64_t ldq, const void* k, const void* v, int64_t ldkv, int T, int H,
                            int Hkv, float scale, const void* o, int64_t ldo, const void* workspace) {
  if (!q || !k || !v || !o || !workspace) return fail(SVDQ_ERR_ARG, "attention_fwd: null pointer");
  if (!aligned16(workspace)) return fail(SVDQ_ERR_ALIGN, "attention_fwd: workspace must be 16-byte aligned");
  if (T <= 0 || H <= 0 || Hkv <= 0 || H % Hkv)
    return fail(SVDQ_ERR_SHAPE, "attention_fwd: T=%d H=%d Hkv=%d (H must be a multiple of Hkv)", T, H, Hkv);
  if (ldq < 128LL * H || ldo < 128LL * H || ldkv < 128LL * Hkv)
    return fail(SVDQ_ERR_SHAPE, "attention_fwd: row strides ldq=%lld ldkv=%lld ldo=%lld below the heads' width",
                (long long)ldq, (long long)ldkv, (long long)ldo);
  if (!(scale > 0.0f) || !(scale < 1e30f)) return fail(SVDQ_ERR_ARG, "attention_fwd: scale must be positive and finite");
  if ((int64_t)T * ldkv * 2 > INT32_MAX)   // the kernels address K and V as buffers of 32-bit byte offsets
    return fail(SVDQ_ERR_SHAPE, "attention_fwd: T * ldkv * 2 = %lld bytes of K or V exceed 2^31 - 1",
                (long long)T * ldkv * 2);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || ldq % 8 || ldkv % 8 || ldo % 8)
    return fail(SVDQ_ERR_ALIGN, "attention_fwd: pointers must be 16-byte aligned and row strides multiples of 8");
  return SVDQ_OK;
}

int svdq_attention_fwd(const void* q, int64_t ldq, const void* k, const void* v, int64_t ldkv, int T, int H,
                       int Hkv, float scale, void* o, int64_t ldo, void* workspace, hipStream_t stream) {
  if (int e = attention_checks(q, ldq, k, v, ldkv, T, H, Hkv, scale, o, ldo, workspace)) return e;
  return launched(svdq::launch_attention_fwd(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                             static_cast<const uint16_t*>(v), static_cast<uint16_t*>(o), T, H, Hkv,
                                             ldq, ldkv, ldo, scale, workspace, stream),
                  "attention_fwd");
}

int svdq_attention_fwd_qnorm(const void* q, int64_t ldq, const void* k, const void* v, int64_t ldkv, int T, int H,
                             int Hkv, float scale, const void* cos, const void* sin, int64_t ldcs, float eps, void* o,
                             int64_t ldo, void* workspace, hipStream_t stream) {
  if (!cos || !sin) return fail(SVDQ_ERR_ARG, "attention_fwd_qnorm: null pointer");
  if (ldcs < 64 || ldcs % 8 || !aligned16(cos) || !aligned16(sin))
    return fail(SVDQ_ERR_ALIGN, "attention_fwd_qnorm: cos, sin 16-byte aligned, ldcs >= 64 and a multiple of 8");
  if (!(eps >= 0.0f)) return fail(SVDQ_ERR_ARG, "attention_fwd_qnorm: eps must be >= 0");
  if (!q || !k || !v || !o || !workspace) return fail(SVDQ_ERR_ARG, "attention_fwd_qnorm: null pointer");
  // the remaining checks and the launch as svdq_attention_fwd, with the tables
  if (int e = attention_checks(q, ldq, k, v, ldkv, T, H, Hkv, scale, o, ldo, workspace)) return e;
  return launched(svdq::launch_attention_fwd(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                             static_cast<const uint16_t*>(v), static_cast<uint16_t*>(o), T, H, Hkv,
                                             ldq, ldkv, ldo, scale, workspace, stream,
                                             static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin),
                                             ldcs, eps),
                  "attention_fwd_qnorm");
}

int svdq_w4a16_gemm(const void* xhat, int64_t ldxh, const void* qw, const void* sw, const void* mid,
                    const void* l1cat, int RTp, const void* bias, int M, int N, int K, int group, void* y,
                    int64_t ldy, int out_f32, hipStream_t stream) {
  return svdq_w4a16_gemm_epi(xhat, ldxh, qw, sw, mid, l1cat, RTp, bias, M, N, K, group, y, ldy, out_f32,
                             SVDQ_EPI_NONE, nullptr, 0, nullptr, stream);
}

int svdq_w4a16_gemm_epi(const void* xhat, int64_t ldxh, const void* qw, const void* sw, const void* mid,
                        const void* l1cat, int RTp, const void* bias, int M, int N, int K, int group, void* y,
                        int64_t ldy, int out_f32, int epi, const void* aux, int64_t ldaux, const void* vec,
                        hipStream_t stream) {
  if (int e = gemm_common_checks("w4a16_gemm", qw, sw, mid, l1cat, RTp, M, N, K, group, y, ldy, out_f32))
    return e;
  if (int e = epi_checks("w4a16_gemm", epi, aux, ldaux, vec, N, out_f32)) return e;
  if (!xhat) return fail(SVDQ_ERR_ARG, "w4a16_gemm: null pointer");
  if (ldxh < K || ldxh % 8 || !aligned16(xhat))
    return fail(SVDQ_ERR_ALIGN, "w4a16_gemm: xhat must be 16-byte aligned with ldxh >= K, ldxh %% 8 == 0");
  svdq::GemmParams p = gemm_params(qw, sw, mid, l1cat, RTp, bias, M, N, K, y, ldy);
  p.xhat = static_cast<const uint16_t*>(xhat);
  p.ldxh = ldxh;
  set_epi(p, epi, aux, ldaux, vec);
  return launched(svdq::launch_w4a16(p, group, out_f32 == 1, stream), "w4a16_gemm");
}

int svdq_w4a16_gemm_siblings(const svdq_w4a16_sibling* layers, int count, int M, int K, int group, int out_f32,
                             hipStream_t stream) {
  if (!layers) return fail(SVDQ_ERR_ARG, "w4a16_gemm_siblings: null layer array");
  if (count < 1 || count > SVDQ_MAX_SIBLINGS)
    return fail(SVDQ_ERR_ARG, "w4a16_gemm_siblings: count=%d, must be 1..%d", count, SVDQ_MAX_SIBLINGS);
  svdq::GemmSiblings gs{};
  gs.count = count;
  int tiles = 0;
  bool fits = fast_group(group);
  for (int i = 0; i < count; ++i) {
    const svdq_w4a16_sibling& l = layers[i];
    if (int e = gemm_common_checks("w4a16_gemm_siblings", l.qw, l.sw, l.mid, l.l1cat, l.RTp, M, l.N, K, group, l.y,
                                   l.ldy, out_f32))
      return e;
    if (!l.xhat) return fail(SVDQ_ERR_ARG, "w4a16_gemm_siblings: layer %d: null xhat", i);
    if (l.ldxh < K || l.ldxh % 8 || !aligned16(l.xhat))
      return fail(SVDQ_ERR_ALIGN, "w4a16_gemm_siblings: layer %d: xhat must be 16-byte aligned with ldxh >= K, "
                  "ldxh %% 8 == 0", i);
    svdq::GemmParams& p = gs.layer[i];
    p = gemm_params(l.qw, l.sw, l.mid, l.l1cat, l.RTp, l.bias, M, l.N, K, l.y, l.ldy);
    p.xhat = static_cast<const uint16_t*>(l.xhat);
    p.ldxh = l.ldxh;
    fits = fits && svdq::w4a16_ws_fits(p);
    gs.tile0[i] = tiles;
    tiles += ((M + 191) / 192) * ((l.N + 255) / 256);
  }
  gs.tile0[count] = tiles;
  if (fits && svdq::w4a16_siblings_pay(gs))
    return launched(svdq::launch_w4a16_siblings(gs, group, out_f32 == 1, stream), "w4a16_gemm_siblings");
  // otherwise one launch per layer, in order, each with its own tile choice
  for (int i = 0; i < count; ++i)
    if (int e = launched(svdq::launch_w4a16(gs.layer[i], group, out_f32 == 1, stream), "w4a16_gemm_siblings"))
      return e;
  return SVDQ_OK;
}

}  // extern "C"
