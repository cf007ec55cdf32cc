/*
 * polarengine_amd.h -- C ABI of the MI355X (gfx950) PolarEngine quantized-linear
 * library, libpolarengine_amd.so.
 *
 * Every entry point takes raw device pointers, sizes and a HIP stream
 * (hipStream_t passed as void*, NULL = the null stream), launches
 * asynchronously on that stream, allocates nothing, never synchronises the
 * host, and returns an int status (PE_OK = 0). Outputs and workspaces are
 * owned by the caller. Entry points are re-entrant; concurrent calls on one
 * workspace race.
 *
 * Workspaces: a workspace (any size query's bytes, 16-byte aligned) must be
 * zero-filled once before its first use. Its first 4096 bytes hold
 * completion counters of kernels whose workgroups hand work to one another
 * within one launch (the K split's partial sums, added up by the last
 * workgroup of a group; the MoE routing, bucketed by the last routing
 * workgroup), so no second kernel is launched; every call leaves them zero
 * again and no entry point writes anything else there, so one zeroed buffer,
 * sized for the largest query, can serve every entry point in turn.
 *
 * Runtime weight layout (one quantized linear, N = out_f, Kp = in_f padded to
 * a multiple of 128, nb = Kp / 128), as registered by the reference's
 * PolarQuantLinearMethod.create_weights / process_weights_after_loading
 * (polarengine_vllm/linear_method.py:119-135, 243-248):
 *   bits 5..8 : codes int8  [N, Kp]         one code per byte (unsigned value)
 *   bits 2..4 : codes uint8 [N, Kp/2]       half-block nibbles,
 *               byte[n, 64*b + i] = code[n, 128*b + 64 + i] << 4 | code[n, 128*b + i]
 *               (polarengine_vllm/packing.py:22-60)
 *   norms     : float16 [N, nb]             per-block L2 norms
 *   ct_scaled : float32 [2**bits]           Lloyd-Max centroids / sqrt(128)
 *
 * Transformed-activation layout "pair f16" (PE_XTF_PAIR_F16), produced by
 * pe_fwht128 and consumed by the *_xtf entry points:
 *   half2 xtf[M][nb][64], xtf[m][b][i] = (H x_m,b)[i], (H x_m,b)[i + 64]
 * i.e. the two activations that one nibble byte multiplies sit in one dword.
 */
#ifndef POLARENGINE_AMD_H
#define POLARENGINE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
enum {
  PE_OK = 0,
  PE_ERR_NULL = 1,      /* a required pointer is NULL                         */
  PE_ERR_DIMS = 2,      /* bad size (K % 128, <= 0, above a kernel limit)     */
  PE_ERR_BITS = 3,      /* unsupported bit width / n_levels / packing combo   */
  PE_ERR_ALIGN = 4,     /* pointer not 16-byte aligned                        */
  PE_ERR_DTYPE = 5,     /* unsupported dtype or layout code                   */
  PE_ERR_WORKSPACE = 6, /* workspace NULL or smaller than the size query      */
  PE_ERR_LAUNCH = 7,    /* hipGetLastError reported a launch failure          */
  PE_ERR_DEVICE = 8,    /* device query failed                                */
  PE_ERR_SCRATCH = 9    /* call larger than the allocation-free entry point's
                           static scratch (pe_linear_noalloc_max_bytes)       */
};

/* ---- weight format flags (the `packed` argument of the linear entry points) */
enum {
  PE_PACK_NIBBLE = 1,  /* half-block nibble codes (bits 2..4), else int8         */
  PE_LAYOUT_TILE16 = 2 /* tiled-16 runtime layout from pe_tile_weights, else the
                          reference's row-major [N, row_bytes] / [N, nb]         */
};

/* ---- dtype / layout codes ---------------------------------------------- */
enum { PE_DTYPE_F16 = 0, PE_DTYPE_BF16 = 1, PE_DTYPE_F32 = 2 };
enum {
  PE_XTF_F32 = 0,      /* natural layout, float32 [rows, cols]              */
  PE_XTF_F16 = 1,      /* natural layout, float16 [rows, cols]              */
  PE_XTF_PAIR_F16 = 2, /* pair layout, see header comment                  */
  PE_XTF_BF16 = 3      /* natural layout, bfloat16 [rows, cols]             */
};

/* Human-readable text for a status code (static storage). */
const char* pe_status_string(int status);

/* ABI version of this header; bumps on any signature change. */
int pe_abi_version(void);

/*
 * Blockwise normalised Walsh-Hadamard transform over contiguous 128-blocks of
 * each row: y[r, 128b:128b+128] = x[r, 128b:128b+128] @ H128.
 * Replaces kernels/fwht.py:77-108 (fwht_matmul, x.reshape(-1,128) @ H) and the
 * pybind fwht / fwht_ of kernels/cuda/fwht_cuda.cu:93-141. x_dtype is
 * PE_DTYPE_F16/BF16/F32 with row stride ldx (elements); y_layout is a
 * PE_XTF_* code (row stride = cols for the natural layouts). x == y is
 * allowed for F32 -> PE_XTF_F32 (the in-place fwht_).
 */
int pe_fwht128(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx,
               void* y, int y_layout, void* stream);

/*
 * Normalised Walsh-Hadamard transform over the WHOLE last dimension of each
 * row, n a power of two (1 <= n <= 32768): stages h = 1, 2, 4, ..., n/2 pair
 * (a, b) -> (a + b, a - b), then y = result / sqrt(n). fp32 arithmetic, one
 * rounding to y_dtype. Replaces fwht_butterfly (kernels/fwht.py:160-190) and
 * the CUDA fwht_butterfly_kernel (kernels/cuda/fwht_cuda.cu:35-86). x has
 * x_dtype (PE_DTYPE_F16/BF16/F32) and row stride ldx >= n (elements); y is
 * [rows, n] of y_dtype, contiguous. x == y is allowed when ldx == n and the
 * dtypes match. PE_ERR_DIMS for n not a power of two or above 32768.
 */
int pe_fwht_pow2(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t ldx,
                 void* y, int y_dtype, void* stream);

/*
 * Reference native GEMV on int8 codes (bits 5..8, or unpacked 2..4):
 * out[n] = sum_b norms[n,b] * sum_k ct_scaled[codes[n,128b+k]] * x_tf[128b+k].
 * Replaces polar_gemv (kernels/polar_gemv.py:181-216; pybind
 * kernels/cuda/polar_gemv_cuda.cu:261-307). x_tf is float32 [in_f_padded]
 * (already transformed), out is float32 [out_f]. block_size must be 128;
 * n_levels = len(ct_scaled) in [4, 256].
 */
int pe_polar_gemv(const int8_t* codes, const float* x_tf, const uint16_t* norms_f16,
                  const float* ct_scaled, int n_levels, float* out, int out_f,
                  int in_f_padded, int n_blocks, int block_size, void* stream);

/*
 * Same on half-block nibble codes (bits 2..4). Replaces polar_gemv_packed
 * (kernels/polar_gemv.py:219-256; polar_gemv_cuda.cu:309-349) and the split-K
 * variants polar_gemv[_packed]_splitk (kernels/polar_gemv_splitk.py:421-569),
 * which compute the same function. in_f_half = n_blocks * 64.
 */
int pe_polar_gemv_packed(const uint8_t* packed, const float* x_tf, const uint16_t* norms_f16,
                         const float* ct_scaled, int n_levels, float* out, int out_f,
                         int in_f_half, int n_blocks, int block_size, void* stream);

/*
 * Batched form: out[M, out_f] (float32) = x_tf[M, in_f_padded] (float32,
 * transformed) against the codes. packed = 1 for nibble codes. Replaces
 * polar_matmul / polar_gemm[_packed] (kernels/polar_gemm.py:311-534).
 * Needs a workspace of pe_polar_matmul_workspace_size(M, in_f_padded) bytes.
 */
size_t pe_polar_matmul_workspace_size(int64_t M, int in_f_padded);
int pe_polar_matmul(const void* codes, int packed, const float* x_tf, int64_t M,
                    const uint16_t* norms_f16, const float* ct_scaled, int n_levels,
                    float* out, int out_f, int in_f_padded, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * The quantized linear forward of PolarQuantLinearMethod.apply
 * (polarengine_vllm/linear_method.py:157-222): pad -> FWHT -> quantized
 * GEMV/GEMM (fp32 accumulate) -> cast -> + bias.
 *   x      : [M, in_f] in x_dtype (PE_DTYPE_F16 or PE_DTYPE_BF16), row stride
 *            ldx; the transformed activation enters the matrix cores as fp16
 *   codes  : runtime layout for (bits, packed); packed = PE_PACK_NIBBLE for
 *            nibble codes, | PE_LAYOUT_TILE16 for the tiled-16 layout
 *   ct_host: NULL, or a host copy of ct_scaled (n_levels floats, equal to the
 *            device values); the decode kernel then takes the codebook by
 *            value in its kernel arguments instead of reading ct_scaled
 *   bias   : NULL or [out_f] in x_dtype
 *   y      : [M, out_f] in x_dtype, row stride out_f. The reference always
 *            returns fp16 (linear_method.py:219); here a bf16 activation gets
 *            a bf16 result (rounded once, then + bias, rounded again).
 * Needs at least pe_linear_workspace_size(...) bytes of workspace (NULL is
 * valid when the query returns 0): the pair-f16 x_tf wherever the transform
 * is not fused into the decode kernel (M > 32, and any M whose shape exceeds
 * the decode kernel's LDS or addressing limits, M = 1 included), and the
 * fp32 partial sums of a K split over workgroups (decode at 2 <= M <= 32
 * when the activations do not fit one workgroup; prefill when the output
 * tiles are too few for the CUs). The query and the call choose the path by
 * the same rule from the same arguments.
 */
size_t pe_linear_workspace_size(int64_t M, int in_f, int out_f, int bits, int packed);
int pe_linear_forward(const void* x, int x_dtype, int64_t M, int in_f, int64_t ldx,
                      const void* codes, int bits, int packed, const uint16_t* norms_f16,
                      const float* ct_scaled, const float* ct_host, int n_levels,
                      const void* bias, void* y, int out_f, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * Allocation-free form of pe_linear_forward. No counterpart in the reference:
 * it is for callers that cannot allocate or own a workspace (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments and results as pe_linear_forward without the workspace; the
 * library uses a static device array of pe_linear_noalloc_max_bytes() bytes
 * (32 MiB) per GPU instead, reserved when the library's code object loads on
 * that GPU and held until the process ends. A call whose path needs more
 * (pe_linear_workspace_size above that limit, e.g. a long prefill) returns
 * PE_ERR_SCRATCH and launches nothing. Every call on one GPU uses the same
 * array: calls that overlap on one GPU (other streams, other threads) race;
 * calls ordered on one stream do not. The array keeps the last call's
 * contents; the counters it needs at zero start at zero and every call
 * leaves them zero.
 */
size_t pe_linear_noalloc_max_bytes(void);
int pe_linear_forward_noalloc(const void* x, int x_dtype, int64_t M, int in_f, int64_t ldx,
                              const void* codes, int bits, int packed, const uint16_t* norms_f16,
                              const float* ct_scaled, const float* ct_host, int n_levels,
                              const void* bias, void* y, int out_f, void* stream);

/*
 * Same, starting from an already-transformed activation in the pair-f16
 * layout (the FWHTCache hit of linear_method.py:190-197, shared by Q/K/V).
 * in_f_padded = 128 * nb of x_tf; ct_host as for pe_linear_forward;
 * out_dtype PE_DTYPE_F16 or PE_DTYPE_BF16 for y and bias.
 */
size_t pe_linear_xtf_workspace_size(int64_t M, int in_f_padded, int out_f, int bits, int packed);
int pe_linear_forward_xtf(const void* x_tf_pair, int64_t M, int in_f_padded,
                          const void* codes, int bits, int packed, const uint16_t* norms_f16,
                          const float* ct_scaled, const float* ct_host, int n_levels,
                          const void* bias, int out_dtype, void* y, int out_f, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * Nibble packing of int8 codes in [0, 15] (bit-exact): replaces
 * pack_codes_int4 (kernels/polar_gemv.py:263-283), called by
 * process_weights_after_loading (linear_method.py:243-248).
 * codes int8 [rows, K] -> packed uint8 [rows, K/2]; K % 128 == 0.
 */
int pe_pack_nibble(const int8_t* codes, uint8_t* packed, int64_t rows, int64_t K, void* stream);

/*
 * Tiled-16 runtime layout (PE_LAYOUT_TILE16) of one quantized matrix, bit-exact
 * rearrangement: codes [N, row_bytes] (row_bytes = nb * bpb, bpb = 64 nibble /
 * 128 int8 bytes per 128-block) -> codes_t [ceil(N/16)][nb][16][bpb], norms
 * [N, nb] -> norms_t [ceil(N/16)][nb][16]; rows past N are zero. One (16-row
 * tile, block) is then one contiguous 1-2 KB read for the decode and GEMM
 * kernels. No reference counterpart: like the nibble packing of
 * process_weights_after_loading (linear_method.py:243-248), it is a one-time
 * runtime re-layout of the registered buffers.
 */
int pe_tile_weights(const void* codes, const uint16_t* norms, int64_t N, int row_bytes, int nb,
                    void* codes_t, uint16_t* norms_t, void* stream);

/*
 * On-disk Q5 (LSB-first, 8 codes in 5 bytes) to int8 codes, bit-exact:
 * replaces unpack_codes_q5 (packing.py:163-209) as used by the loader
 * (loader.py:412-417). packed uint8 [rows, K*5/8] -> codes int8 [rows, K].
 */
int pe_unpack_q5(const uint8_t* packed, int8_t* codes, int64_t rows, int64_t K, void* stream);

/*
 * PolarQuant quantizer: weight [N, K] (w_dtype PE_DTYPE_F16 / BF16 / F32, row
 * stride ldw elements) -> codes and fp16 block norms [N, nb], nb = ceil(K/128).
 * Replaces PolarQuantizer.quantize_tensor (quantizer.py:206-257): zero-pad K,
 * per-block L2 norm clamped at 1e-10, unit block times the unnormalised
 * Hadamard transform, code = first index of the nearest of ct[0..n_levels)
 * (the raw Lloyd-Max centroids, device float32). pack = 0: int8 codes
 * [N, nb*128]; pack = 1 (n_levels <= 16): half-block nibbles uint8 [N, nb*64].
 * codes must be 8-byte aligned.
 */
int pe_quantize(const void* w, int w_dtype, int64_t N, int K, int64_t ldw, const float* ct,
                int n_levels, int pack, void* codes, uint16_t* norms_f16, void* stream);

/*
 * KV-cache compression (replaces PolarKVQuantizer.quantize / dequantize,
 * kv_cache/cache.py:201-256, and the hybrid ops of kv_cache/triton_kernels.py:
 * 139-228). head_dim 64, 128 or 256, nbits 2..4, ct = the 2^nbits KV centroids
 * (device float32, kv_cache/cache.py:27-54).
 *   pe_kv_quantize:   x [n_vec, head_dim] (x_dtype BF16 / F16 / F32, row
 *                     stride ldx elements) -> packed uint8 [n_vec,
 *                     head_dim*nbits/8] in BitPacker order + norms bf16 [n_vec]
 *   pe_kv_dequantize: packed + norms -> out bf16 [n_vec, head_dim], row stride
 *                     ldo elements (16-byte aligned rows)
 */
int pe_kv_quantize(const void* x, int x_dtype, int64_t n_vec, int head_dim, int64_t ldx,
                   const float* ct, int nbits, uint8_t* packed, uint16_t* norms_bf16,
                   void* stream);
int pe_kv_dequantize(const uint8_t* packed, const uint16_t* norms_bf16, int64_t n_vec,
                     int head_dim, const float* ct, int nbits, uint16_t* out_bf16, int64_t ldo,
                     void* stream);

/*
 * HLWQ bit-packed codes (bitpack_5, MSB-first: 8 codes in 5 bytes) to int8
 * codes, bit-exact: replaces unpack_codes_q5_hlwq (packing.py:229-271) as the
 * loader uses it for the "hlwq-q5" format (loader.py:332-360). packed is the
 * flat byte stream (packed_bytes a multiple of 5); the first `total` codes are
 * written to codes int8 [total].
 */
int pe_unpack_q5_hlwq(const uint8_t* packed, int64_t packed_bytes, int8_t* codes, int64_t total,
                      void* stream);

/*
 * MoE routing: scores (softmax or sigmoid of logits + optional correction
 * bias) -> top-k (ties to the lower expert id) -> optional renormalise.
 * Semantics of the routing in nemotron_offload.py:172-189 with the argument
 * list of PolarPassthroughMoEMethod.apply (moe_method.py:74-78).
 *   logits float32 [T, E]; topk_w float32 [T, top_k]; topk_ids int32 [T, top_k]
 *   scoring: 0 = softmax, 1 = sigmoid. E <= 256, top_k <= 16.
 */
int pe_moe_route(const float* logits, int64_t T, int E, int top_k, int renormalize,
                 int scoring, const float* correction_bias, float* topk_w,
                 int32_t* topk_ids, void* stream);

/*
 * Grouped top-k routing (vLLM's grouped_topk, which the reference reaches by
 * passing use_grouped_topk / num_expert_group / topk_group through
 * PolarPassthroughMoEMethod.apply, moe_method.py:74-89): scores = softmax or
 * sigmoid of the logits; the E experts form num_expert_group contiguous groups
 * (E % num_expert_group == 0, at most 64 groups); a group's score is its best
 * expert score, or, with correction_bias, the sum of its two best scores +
 * bias; the topk_group best groups (ties: lower group) are kept, top_k of
 * their experts are taken by (biased) score (ties: lower id), and the
 * weights are the unbiased scores, optionally renormalised. top_k must not
 * exceed the kept experts; E, top_k limits as pe_moe_route.
 */
int pe_moe_route_grouped(const float* logits, int64_t T, int E, int top_k, int renormalize,
                         int scoring, const float* correction_bias, int num_expert_group,
                         int topk_group, float* topk_w, int32_t* topk_ids, void* stream);

/*
 * Quantized SwiGLU MoE forward over resident experts (the grouped-expert
 * path). The reference forwards MoE layers to vLLM's bf16 fused MoE
 * (moe_method.py:74-92); the per-expert math is that of
 * nemotron_offload.py:203-226.
 *   x       : [T, H] in x_dtype (PE_DTYPE_F16 or PE_DTYPE_BF16), H % 128 == 0
 *   topk_w / topk_ids : routing (pe_moe_route or the caller's own)
 *   w13     : codes [E, 2I, ...] in the runtime layout for (bits13, packed13),
 *             norms float16 [E, 2I, H/128], ct13 float32 [2**bits13];
 *             rows [0, I) are gate, rows [I, 2I) are up
 *   packed13 / packed2: 1 = nibble codes (bits <= 4), | PE_LAYOUT_TILE16 = each
 *             expert's codes and norms in the tiled-16 layout (pe_tile_weights
 *             over the [E * rows, row_bytes] matrix; rows per expert, 2I and H,
 *             must then be multiples of 16)
 *   w2      : codes [E, H, ...] over in_f = I padded to Ip = ceil(I/128)*128,
 *             norms float16 [E, H, Ip/128], ct2 float32 [2**bits2]
 *   out     : [T, H] in x_dtype = sum_k topk_w[t,k] * expert_{ids[t,k]}(x_t),
 *             the terms added in slot order k = 0, 1, .. in fp32 (slots whose
 *             id is outside 0..E-1 are skipped; a token with none is zero)
 * Four launches: x transform with the bucketing of the pairs by expert;
 * gate/up with SwiGLU; down; the weighted combine.
 * Workspace: pe_moe_workspace_size(T, top_k, E, H, I) bytes.
 */
size_t pe_moe_workspace_size(int64_t T, int top_k, int E, int H, int I);
int pe_moe_forward(const void* x, int x_dtype, int64_t T, int H, int I, int E, int top_k,
                   const float* topk_w, const int32_t* topk_ids,
                   const void* w13_codes, int bits13, int packed13,
                   const uint16_t* w13_norms, const float* ct13, int n_levels13,
                   const void* w2_codes, int bits2, int packed2,
                   const uint16_t* w2_norms, const float* ct2, int n_levels2,
                   void* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Routing and experts in one call: replaces PolarPassthroughMoEMethod.apply
 * (moe_method.py:74-92), which takes the router logits and hands routing and
 * experts to vLLM's fused MoE. Routing as pe_moe_route (num_expert_group = 0)
 * or pe_moe_route_grouped (num_expert_group > 0), with the same limits; the
 * rest as pe_moe_forward. The routing shares the first launch with the x
 * transform (its last workgroup buckets the pairs), so the call is four
 * launches, as pe_moe_forward's. The routing results stay in the workspace.
 *   logits : float32 [T, E]
 * Workspace: pe_moe_workspace_size(T, top_k, E, H, I) bytes.
 */
int pe_moe_forward_routed(const void* x, int x_dtype, int64_t T, int H, int I, int E, int top_k,
                          const float* logits, int renormalize, int scoring,
                          const float* correction_bias, int num_expert_group, int topk_group,
                          const void* w13_codes, int bits13, int packed13,
                          const uint16_t* w13_norms, const float* ct13, int n_levels13,
                          const void* w2_codes, int bits2, int packed2,
                          const uint16_t* w2_norms, const float* ct2, int n_levels2,
                          void* out, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* POLARENGINE_AMD_H */
