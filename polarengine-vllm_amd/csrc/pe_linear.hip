// Dispatch of the quantized linear forward (PolarQuantLinearMethod.apply,
// polarengine_vllm/linear_method.py:157-222) and of the batched reference API
// (polar_matmul, kernels/polar_gemm.py:425-534).
//
// Routing by M (rows of the activation):
//   M <= 16 (when x, or one K group of it, fits in LDS beside the codebook
//   table), or 17 <= M <= 32 when one K group fits
//                     -> gemv_mfma: decode GEMV on 16x16x32 MFMA, FWHT fused
//                        into its prologue (one launch per linear, also with
//                        the K split over workgroups: the last workgroup of
//                        each row group adds the partial sums; M > 16 with
//                        two m-tiles per weight lookup);
//   M == 1 otherwise  -> gemv1 (register-resident dot2 GEMV, LDS activations)
//                        for row-major weights with K within its LDS budget;
//   M <= 64 else      -> FWHT-128 to pair-f16 x_tf, then the small-M MFMA
//                        kernel (16x16x32 f16, K split across waves); at
//                        M = 33..64 with fp16 out, the prefill GEMM instead
//                        when its K split over workgroups applies;
//   M > 64            -> FWHT-128 to pair-f16 x_tf, then the prefill GEMM
//                        (32x32x16 f16 MFMA, dequantized B; K split over
//                        workgroups when the output tiles are few).
// The reference routes M = 1 to split-K GEMV and every M > 1 to its Triton
// GEMM; results are the same function either way.

#include <mutex>

#include "pe_internal.h"

namespace pe {

// `packed` flags: PE_PACK_NIBBLE (bit 0, bits <= 4), PE_LAYOUT_TILE16 (bit 1).
static int check_format(int bits, int packed, int n_levels, bool* nibble, bool* tiled) {
  if (bits < 2 || bits > 8) return PE_ERR_BITS;
  if (packed & ~(PE_PACK_NIBBLE | PE_LAYOUT_TILE16)) return PE_ERR_BITS;
  if ((packed & PE_PACK_NIBBLE) && bits > 4) return PE_ERR_BITS;
  if (n_levels != (1 << bits)) return PE_ERR_BITS;
  *nibble = (packed & PE_PACK_NIBBLE) != 0;
  *tiled = (packed & PE_LAYOUT_TILE16) != 0;
  return PE_OK;
}


// The path one call of the linear forward takes, and the workspace it needs.
// Both the size queries and the entry points use this, so a query can never
// disagree with the path the call runs.
enum LinearRoute {
  LR_DECODE = 0,  // gemv_mfma: FWHT fused (raw x) or pair-f16 x_tf; partial sums when K-split
  LR_GEMV1 = 1,   // M = 1, row-major weights, K within the gemv1 LDS budget (raw x only)
  LR_MM = 2       // [FWHT-128 into the workspace], then the small-M / prefill matmul
};
// Workspace layout: [kWsCounterBytes of counters][pair-f16 x_tf (raw-x MM
// route)][fp32 partial sums of a K split]; no workspace at all when the path
// needs neither x_tf nor partials.
struct LinearPlan {
  int route;
  size_t xtf_bytes;  // pair-f16 x_tf after the counters (raw-x MM route only)
  size_t ws_bytes;   // total workspace
};

static LinearPlan plan_linear(bool raw_x, int64_t M, int kp, int out_f, int bits, int packed) {
  const bool nib = (packed & PE_PACK_NIBBLE) != 0 && bits <= 4;
  const bool tiled = (packed & PE_LAYOUT_TILE16) != 0;
  const int nb = kp / kBlock, n_levels = 1 << bits;
  auto with_counters = [](size_t data) { return data ? kWsCounterBytes + data : 0; };
  if (M >= 1 && M <= kDecMaxRows && gemv_mfma_fits(nib, (int)M, out_f, nb, n_levels))
    return LinearPlan{LR_DECODE, 0, with_counters(round_up(
                                        gemv_mfma_workspace(nib, (int)M, out_f, nb, n_levels), 256))};
  if (raw_x && M == 1 && !tiled && kp <= gemv1_max_kp(nib)) return LinearPlan{LR_GEMV1, 0, 0};
  const size_t xtf = raw_x ? round_up((size_t)M * kp * 2, 256) : 0;
  return LinearPlan{LR_MM, xtf,
                    with_counters(xtf + round_up(mm_xtf_workspace(nib, M, out_f, nb), 256))};
}

static bool plan_args_ok(int64_t M, int kp, int out_f, int bits) {
  return M >= 1 && kp > 0 && kp % kBlock == 0 && out_f > 0 && bits >= 2 && bits <= 8;
}

}  // namespace pe

using namespace pe;

extern "C" size_t pe_linear_xtf_workspace_size(int64_t M, int in_f_padded, int out_f, int bits,
                                               int packed) {
  if (!plan_args_ok(M, in_f_padded, out_f, bits)) return 0;
  return plan_linear(false, M, in_f_padded, out_f, bits, packed).ws_bytes;
}

extern "C" size_t pe_linear_workspace_size(int64_t M, int in_f, int out_f, int bits, int packed) {
  if (in_f <= 0) return 0;
  const int kp = (in_f + kBlock - 1) / kBlock * kBlock;
  if (!plan_args_ok(M, kp, out_f, bits)) return 0;
  return plan_linear(true, M, kp, out_f, bits, packed).ws_bytes;
}

extern "C" int pe_linear_forward_xtf(const void* x_tf_pair, int64_t M, int in_f_padded,
                                     const void* codes, int bits, int packed,
                                     const uint16_t* norms_f16, const float* ct_scaled,
                                     const float* ct_host, int n_levels, const void* bias,
                                     int out_dtype, void* y, int out_f, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!x_tf_pair || !codes || !norms_f16 || !ct_scaled || !y) return PE_ERR_NULL;
  if (M < 0 || out_f <= 0 || in_f_padded <= 0 || in_f_padded % kBlock) return PE_ERR_DIMS;
  const int ybf = bf16_flag(out_dtype);
  if (ybf < 0) return PE_ERR_DTYPE;
  bool nib = false, tiled = false;
  if (int rc = check_format(bits, packed, n_levels, &nib, &tiled)) return rc;
  if (!aligned16(x_tf_pair) || !aligned16(codes)) return PE_ERR_ALIGN;
  if (M == 0) return PE_OK;
  const int nb = in_f_padded / kBlock;
  const LinearPlan plan = plan_linear(false, M, in_f_padded, out_f, bits, packed);
  if (plan.ws_bytes && (!workspace || workspace_bytes < plan.ws_bytes)) return PE_ERR_WORKSPACE;
  if (workspace && !aligned16(workspace)) return PE_ERR_ALIGN;
  uint32_t* cnt = reinterpret_cast<uint32_t*>(workspace);
  char* data = plan.ws_bytes ? reinterpret_cast<char*>(workspace) + kWsCounterBytes : nullptr;
  const size_t data_bytes = plan.ws_bytes ? workspace_bytes - kWsCounterBytes : 0;
  if (plan.route == LR_DECODE) {
    DecArgs a{reinterpret_cast<const uint8_t*>(codes), norms_f16, ct_scaled, n_levels,
              x_tf_pair, (int64_t)in_f_padded, y, out_f, reinterpret_cast<const uint16_t*>(bias),
              (int)M, out_f, nb, wlayout(nib, tiled, nb), ct_host, data, data_bytes,
              0, ybf, cnt};
    return gemv_mfma(nib, false, a, st);
  }
  return mm_xtf(nib, tiled, codes, norms_f16, ct_scaled, n_levels, x_tf_pair, M, out_f, nb, y,
                OM_F16, out_f, reinterpret_cast<const uint16_t*>(bias), data, data_bytes, st,
                ybf != 0);
}

extern "C" int pe_linear_forward(const void* x, int x_dtype, int64_t M, int in_f, int64_t ldx,
                                 const void* codes, int bits, int packed,
                                 const uint16_t* norms_f16, const float* ct_scaled,
                                 const float* ct_host, int n_levels, const void* bias, void* y,
                                 int out_f, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!x || !codes || !norms_f16 || !ct_scaled || !y) return PE_ERR_NULL;
  if (M < 0 || in_f <= 0 || out_f <= 0 || ldx < in_f) return PE_ERR_DIMS;
  // x, bias and y share one 16-bit dtype (fp16 or bf16)
  const int xbf = bf16_flag(x_dtype);
  if (xbf < 0) return PE_ERR_DTYPE;
  // The kernels read 128-wide blocks of x: in_f must already be a multiple of
  // 128 (the Python layer pads otherwise, as linear_method.py:194-195 does).
  if (in_f % kBlock) return PE_ERR_DIMS;
  bool nib = false, tiled = false;
  if (int rc = check_format(bits, packed, n_levels, &nib, &tiled)) return rc;
  if (!aligned16(x) || !aligned16(codes) || (ldx * 2) % 16) return PE_ERR_ALIGN;
  if (M == 0) return PE_OK;
  const int nb = in_f / kBlock;
  const LinearPlan plan = plan_linear(true, M, in_f, out_f, bits, packed);
  if (plan.ws_bytes && (!workspace || workspace_bytes < plan.ws_bytes)) return PE_ERR_WORKSPACE;
  if (workspace && !aligned16(workspace)) return PE_ERR_ALIGN;
  const uint16_t* b16 = reinterpret_cast<const uint16_t*>(bias);
  uint32_t* cnt = reinterpret_cast<uint32_t*>(workspace);
  char* data = plan.ws_bytes ? reinterpret_cast<char*>(workspace) + kWsCounterBytes : nullptr;
  const size_t data_bytes = plan.ws_bytes ? workspace_bytes - kWsCounterBytes : 0;
  if (plan.route == LR_DECODE) {
    DecArgs a{reinterpret_cast<const uint8_t*>(codes), norms_f16, ct_scaled, n_levels, x, ldx, y,
              out_f, b16, (int)M, out_f, nb, wlayout(nib, tiled, nb), ct_host, data, data_bytes,
              xbf, xbf, cnt};
    return gemv_mfma(nib, true, a, st);
  }
  if (plan.route == LR_GEMV1) {
    Gemv1Args a{reinterpret_cast<const uint8_t*>(codes), norms_f16, ct_scaled, n_levels, x, y,
                b16, out_f, nb, xbf, xbf};
    return gemv1(nib, XM_RAW_F16, OM_F16, a, st);
  }
  if (int rc = fwht128(x, x_dtype, M, in_f, ldx, data, PE_XTF_PAIR_F16, st)) return rc;
  return mm_xtf(nib, tiled, codes, norms_f16, ct_scaled, n_levels, data, M, out_f, nb, y, OM_F16,
                out_f, b16, data + plan.xtf_bytes, data_bytes - plan.xtf_bytes, st, xbf != 0);
}

// Workspace of pe_polar_matmul: the counter block, then the fp32 x_tf
// repacked to pair f16; none at M = 1 when the GEMV takes x_tf directly (K
// within its LDS budget for either code format: int8 is the smaller bound).
extern "C" size_t pe_polar_matmul_workspace_size(int64_t M, int in_f_padded) {
  if (M <= 0 || in_f_padded <= 0) return 0;
  if (M == 1 && in_f_padded <= gemv1_max_kp(false)) return 0;
  return kWsCounterBytes + round_up((size_t)M * in_f_padded * 2, 256);
}

extern "C" int pe_polar_matmul(const void* codes, int packed, const float* x_tf, int64_t M,
                               const uint16_t* norms_f16, const float* ct_scaled, int n_levels,
                               float* out, int out_f, int in_f_padded, void* workspace,
                               size_t workspace_bytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!codes || !x_tf || !norms_f16 || !ct_scaled || !out) return PE_ERR_NULL;
  if (M < 0 || out_f <= 0 || in_f_padded <= 0 || in_f_padded % kBlock) return PE_ERR_DIMS;
  if (packed & ~PE_PACK_NIBBLE) return PE_ERR_BITS;  // reference layout only
  const bool nib = packed != 0;
  if (n_levels < 2 || n_levels > (nib ? 16 : 256) || (n_levels & (n_levels - 1))) return PE_ERR_BITS;
  if (!aligned16(codes) || !aligned16(x_tf)) return PE_ERR_ALIGN;
  if (M == 0) return PE_OK;
  const int nb = in_f_padded / kBlock;
  if (M == 1 && in_f_padded <= gemv1_max_kp(nib)) {
    Gemv1Args a{reinterpret_cast<const uint8_t*>(codes), norms_f16, ct_scaled, n_levels, x_tf,
                out, nullptr, out_f, nb};
    return gemv1(nib, XM_XTF_F32, OM_F32, a, st);
  }
  const size_t need = round_up((size_t)M * in_f_padded * 2, 256);
  if (!workspace || workspace_bytes < kWsCounterBytes + need) return PE_ERR_WORKSPACE;
  if (!aligned16(workspace)) return PE_ERR_ALIGN;
  char* ws = reinterpret_cast<char*>(workspace) + kWsCounterBytes;
  if (int rc = repack_pair(x_tf, M, in_f_padded, ws, st)) return rc;
  return mm_xtf(nib, false, codes, norms_f16, ct_scaled, n_levels, ws, M, out_f, nb, out, OM_F32,
                out_f, nullptr, ws + need, workspace_bytes - kWsCounterBytes - need, st);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of pe_linear_forward (no counterpart in the
// reference): the workspace is a static device array, one per GPU, that the
// code object reserves when it loads. Its first kWsCounterBytes are the
// completion counters (zero when the module loads; every call leaves them
// zero), the rest holds whatever the call's path needs (pair-f16 x_tf, fp32
// partial sums). Calls on one GPU share it, so calls that overlap on one GPU
// (concurrent streams, threads) race.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace pe {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device

// The scratch array's device address on the current device, looked up once
// per device (the array's name is a host-side stand-in, never an address).
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return PE_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return PE_ERR_DEVICE;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return PE_OK;
}
}  // namespace
}  // namespace pe

extern "C" size_t pe_linear_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int pe_linear_forward_noalloc(const void* x, int x_dtype, int64_t M, int in_f,
                                         int64_t ldx, const void* codes, int bits, int packed,
                                         const uint16_t* norms_f16, const float* ct_scaled,
                                         const float* ct_host, int n_levels, const void* bias,
                                         void* y, int out_f, void* stream) {
  // the path's workspace, by the rule pe_linear_forward applies (0 for
  // arguments it rejects: the call below then returns that error)
  const size_t need = pe_linear_workspace_size(M, in_f, out_f, bits, packed);
  if (need > kScratchBytes) return PE_ERR_SCRATCH;
  void* ws = nullptr;
  if (need) {
    if (int rc = scratch_address(&ws)) return rc;
  }
  return pe_linear_forward(x, x_dtype, M, in_f, ldx, codes, bits, packed, norms_f16, ct_scaled,
                           ct_host, n_levels, bias, y, out_f, ws, need ? kScratchBytes : 0,
                           stream);
}
