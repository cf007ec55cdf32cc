// Quantized grouped-expert MoE for gfx950.
//
// The reference has no quantized MoE compute: PolarPassthroughMoEMethod
// forwards experts to vLLM's bf16 fused MoE (moe_method.py:74-92). The
// per-expert math followed here is the reference's in-repo MoE forward
// (nemotron_offload.py:172-226): scores = softmax|sigmoid(logits + bias),
// top-k, renormalise, gate = x W13[:I]^T, up = x W13[I:]^T,
// h = silu(gate) * up, y = h W2^T, out = sum_k w_k y_k.
//
// Launch sequence of pe_moe_forward (no host synchronisation):
//   1. moe_align: bucket the T*top_k (token, slot) pairs by expert (one
//      workgroup; LDS histogram + scan + scatter) -> per-expert offsets,
//      token of each sorted pair, sorted position of each pair;
//   2. FWHT-128 of x into pair-f16 (shared by every expert);
//   3. grouped small-M MFMA over (n-tile, expert): gate and up tiles of W13
//      with the SwiGLU epilogue -> h [pairs, I] fp16 (A rows gathered by
//      token id);
//   4. FWHT-128 of h (zero-padded to a multiple of 128) into pair-f16;
//   5. grouped small-M MFMA with W2 -> y2 [pairs, H] fp32;
//   6. combine: out[t] = sum_k w[t, k] * y2[pos(t, k)] in fixed k order, fp16.
// Each output row depends only on its own inputs, so bucket order inside an
// expert (set by LDS atomics) does not change any result bit.

#include "pe_internal.h"

namespace pe {

// ---------------------------------------------------------------------------
// routing: one wave per token, up to 256 experts (4 per lane)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits, int64_t T,
                                                        int E, int top_k, int renormalize,
                                                        int scoring, const float* __restrict__ bias,
                                                        float* __restrict__ topk_w,
                                                        int32_t* __restrict__ topk_ids) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole wave
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    float l = -INFINITY;
    if (e < E) {
      l = logits[t * E + e];
      if (bias) l += bias[e];
    }
    v[i] = l;
  }
  if (scoring == 0) {  // softmax over E
    float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = (lane + 64 * i) < E ? expf(v[i] - mx) : 0.f;
      sum += v[i];
    }
    sum = wave_sum(sum);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = v[i] / sum;
  } else {  // sigmoid
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (lane + 64 * i) < E ? 1.f / (1.f + expf(-v[i])) : -1.f;
  }
  // top-k by repeated arg-max; ties go to the lower expert id
  float wsum = 0.f;
  float sel_w[16];
  int sel_e[16];
  for (int k = 0; k < top_k; ++k) {
    float best = -2.f;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane + 64 * i;
      if (e < E && (v[i] > best || (v[i] == best && e < be))) { best = v[i]; be = e; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ob = __shfl_xor(best, off, 64);
      const int oe = __shfl_xor(be, off, 64);
      if (ob > best || (ob == best && oe < be)) { best = ob; be = oe; }
    }
    sel_w[k] = best;
    sel_e[k] = be;
    wsum += best;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (lane + 64 * i == be) v[i] = -3.f;  // remove from the candidates
  }
  if (lane == 0) {
    for (int k = 0; k < top_k; ++k) {
      topk_w[t * top_k + k] = renormalize ? sel_w[k] / wsum : sel_w[k];
      topk_ids[t * top_k + k] = sel_e[k];
    }
  }
}

// ---------------------------------------------------------------------------
// bucket pairs by expert (single workgroup)
// ---------------------------------------------------------------------------
constexpr int kAlignThreads = 1024;

__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(
    const int32_t* __restrict__ topk_ids, int64_t P, int top_k, int E,
    int32_t* __restrict__ offsets /* [E+1] */, int32_t* __restrict__ sorted_token /* [P] */,
    int32_t* __restrict__ pair_pos /* [P] */) {
  __shared__ int cnt[256];
  __shared__ int base[257];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += kAlignThreads) cnt[e] = 0;
  __syncthreads();
  for (int64_t p = tid; p < P; p += kAlignThreads) {
    const int e = topk_ids[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int e = 0; e < E; ++e) {
      base[e] = acc;
      acc += cnt[e];
    }
    base[E] = acc;
  }
  __syncthreads();
  for (int e = tid; e <= E; e += kAlignThreads) offsets[e] = base[e];
  for (int e = tid; e < E; e += kAlignThreads) cnt[e] = 0;
  __syncthreads();
  for (int64_t p = tid; p < P; p += kAlignThreads) {
    const int e = topk_ids[p];
    int pos = -1;
    if (e >= 0 && e < E) {
      pos = base[e] + atomicAdd(&cnt[e], 1);
      sorted_token[pos] = (int32_t)(p / top_k);
    }
    pair_pos[p] = pos;
  }
}

// out[t, h] = sum_k w[t, k] * y2[pos(t, k), h], k in order; 8 columns per lane
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y2,
                                                          const float* __restrict__ topk_w,
                                                          const int32_t* __restrict__ pair_pos,
                                                          int64_t T, int top_k, int H,
                                                          uint16_t* __restrict__ out) {
  const int per_row = H / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= T * per_row) return;
  const int64_t t = i / per_row;
  const int c = (int)(i - t * per_row) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < top_k; ++k) {
    const int pos = pair_pos[t * top_k + k];
    if (pos < 0) continue;
    const float w = topk_w[t * top_k + k];
    const float4* src = reinterpret_cast<const float4*>(y2 + (int64_t)pos * H + c);
    const float4 a = src[0], b = src[1];
    acc[0] += w * a.x; acc[1] += w * a.y; acc[2] += w * a.z; acc[3] += w * a.w;
    acc[4] += w * b.x; acc[5] += w * b.y; acc[6] += w * b.z; acc[7] += w * b.w;
  }
  uint4 o;
  o.x = pack_h2(acc[0], acc[1]);
  o.y = pack_h2(acc[2], acc[3]);
  o.z = pack_h2(acc[4], acc[5]);
  o.w = pack_h2(acc[6], acc[7]);
  *reinterpret_cast<uint4*>(out + t * H + c) = o;
}

struct MoeWs {
  size_t offsets, sorted_token, pair_pos, xtf, htf, y2, total;
};

static MoeWs moe_ws_layout(int64_t T, int top_k, int E, int H, int I) {
  const int64_t P = T * top_k;
  const int64_t Ip = (I + kBlock - 1) / kBlock * kBlock;
  MoeWs w{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += round_up(bytes, 256);
    return at;
  };
  w.offsets = take((size_t)(E + 1) * 4);
  w.sorted_token = take((size_t)P * 4);
  w.pair_pos = take((size_t)P * 4);
  w.xtf = take((size_t)T * H * 2);
  w.htf = take((size_t)P * Ip * 2);
  w.y2 = take((size_t)P * H * 4);
  w.total = o;
  return w;
}

}  // namespace pe

using namespace pe;

extern "C" int pe_moe_route(const float* logits, int64_t T, int E, int top_k, int renormalize,
                            int scoring, const float* correction_bias, float* topk_w,
                            int32_t* topk_ids, void* stream) {
  if (!logits || !topk_w || !topk_ids) return PE_ERR_NULL;
  if (T < 0 || E <= 0 || E > 256 || top_k <= 0 || top_k > 16 || top_k > E) return PE_ERR_DIMS;
  if (scoring != 0 && scoring != 1) return PE_ERR_DTYPE;
  if (T == 0) return PE_OK;
  if ((T + 3) / 4 > INT32_MAX) return PE_ERR_DIMS;
  moe_route_kernel<<<dim3((unsigned)((T + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream)>>>(logits, T, E, top_k, renormalize,
                                                              scoring, correction_bias, topk_w,
                                                              topk_ids);
  return launch_status();
}

extern "C" size_t pe_moe_workspace_size(int64_t T, int top_k, int E, int H, int I) {
  if (T <= 0 || top_k <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
  return moe_ws_layout(T, top_k, E, H, I).total;
}

extern "C" int pe_moe_forward(const void* x, int64_t T, int H, int I, int E, int top_k,
                              const float* topk_w, const int32_t* topk_ids,
                              const void* w13_codes, int bits13, int packed13,
                              const uint16_t* w13_norms, const float* ct13, int n_levels13,
                              const void* w2_codes, int bits2, int packed2,
                              const uint16_t* w2_norms, const float* ct2, int n_levels2,
                              void* out, void* workspace, size_t workspace_bytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!x || !topk_w || !topk_ids || !w13_codes || !w13_norms || !ct13 || !w2_codes ||
      !w2_norms || !ct2 || !out)
    return PE_ERR_NULL;
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || E > 256 || top_k <= 0 || top_k > E) return PE_ERR_DIMS;
  if (H % kBlock) return PE_ERR_DIMS;
  for (int which = 0; which < 2; ++which) {
    const int bits = which ? bits2 : bits13, packed = which ? packed2 : packed13;
    const int nl = which ? n_levels2 : n_levels13;
    if (bits < 2 || bits > 8 || (packed & ~(1 | PE_LAYOUT_TILE16)) || ((packed & 1) && bits > 4) ||
        nl != (1 << bits))
      return PE_ERR_BITS;
  }
  // tiled-16 experts: every expert's rows are whole 16-row tiles
  if (((packed13 & PE_LAYOUT_TILE16) && (2 * I) % 16) || ((packed2 & PE_LAYOUT_TILE16) && H % 16))
    return PE_ERR_DIMS;
  if (!aligned16(x) || !aligned16(w13_codes) || !aligned16(w2_codes) || !aligned16(out))
    return PE_ERR_ALIGN;
  if (T == 0) return PE_OK;
  const int64_t P = T * top_k;
  if (P > INT32_MAX / 2) return PE_ERR_DIMS;
  const MoeWs L = moe_ws_layout(T, top_k, E, H, I);
  if (!workspace || workspace_bytes < L.total) return PE_ERR_WORKSPACE;
  if (!aligned16(workspace)) return PE_ERR_ALIGN;
  char* ws = reinterpret_cast<char*>(workspace);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* sorted_token = reinterpret_cast<int32_t*>(ws + L.sorted_token);
  int32_t* pair_pos = reinterpret_cast<int32_t*>(ws + L.pair_pos);
  const int Ip = (I + kBlock - 1) / kBlock * kBlock;
  const int nb13 = H / kBlock, nb2 = Ip / kBlock;
  const bool nib13 = (packed13 & 1) != 0, nib2 = (packed2 & 1) != 0;
  const bool tiled13 = (packed13 & PE_LAYOUT_TILE16) != 0, tiled2 = (packed2 & PE_LAYOUT_TILE16) != 0;
  const int64_t row13 = nib13 ? (int64_t)nb13 * 64 : (int64_t)nb13 * kBlock;
  const int64_t row2 = nib2 ? (int64_t)nb2 * 64 : (int64_t)nb2 * kBlock;

  // 1. bucket pairs by expert
  moe_align_kernel<<<dim3(1), dim3(kAlignThreads), 0, st>>>(topk_ids, P, top_k, E, offsets,
                                                             sorted_token, pair_pos);
  if (int rc = launch_status()) return rc;
  // 2. x -> pair f16
  if (int rc = fwht128(x, PE_DTYPE_F16, T, H, H, ws + L.xtf, PE_XTF_PAIR_F16, st)) return rc;
  // 3. gate/up + SwiGLU, each 128-column block of h transformed in the same
  // kernel -> htf [P, Ip] pair f16 (columns past I are zero)
  {
    SmallArgs a{reinterpret_cast<const uint8_t*>(w13_codes), w13_norms, ct13, n_levels13,
                reinterpret_cast<const uint32_t*>(ws + L.xtf), sorted_token, offsets,
                2 * (int64_t)I * row13, 2 * (int64_t)I * nb13, ws + L.htf, Ip, nullptr, 0, I,
                nb13, wlayout(nib13, tiled13, nb13)};
    if (int rc = moe_grouped(nib13, SE_SWIGLU_XTF, a, E, st)) return rc;
  }
  // 5. down -> y2 [P, H] fp32
  {
    SmallArgs a{reinterpret_cast<const uint8_t*>(w2_codes), w2_norms, ct2, n_levels2,
                reinterpret_cast<const uint32_t*>(ws + L.htf), nullptr, offsets,
                (int64_t)H * row2, (int64_t)H * nb2, ws + L.y2, H, nullptr, 0, H, nb2,
                wlayout(nib2, tiled2, nb2)};
    if (int rc = moe_grouped(nib2, SE_F32, a, E, st)) return rc;
  }
  // 6. weighted combine -> out fp16
  const int64_t work = T * (H / 8);
  moe_combine_kernel<<<dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st>>>(
      reinterpret_cast<const float*>(ws + L.y2), topk_w, pair_pos, T, top_k, H,
      reinterpret_cast<uint16_t*>(out));
  return launch_status();
}
