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
//   1. moe_prep: FWHT-128 of x into pair f16 (shared by every expert) and, in
//      the grid's last workgroup, the bucketing of the T*top_k (token, slot)
//      pairs by expert (LDS histogram + scan + scatter) -> per-expert offsets,
//      token of each sorted pair, sorted position of each pair;
//   2. grouped experts, W13: gate and up tiles with SwiGLU; each 128-column
//      block of h goes through the FWHT in the same kernel -> pair-f16 h
//      [pairs, Ip] (A rows gathered by token id; columns past I are zero);
//   3. grouped experts, W2 -> y2 [pairs, H] fp32;
//   4. combine: out[t] = sum_k w[t, k] * y2[pos(t, k)] in fixed k order, fp16.
// Each output row depends only on its own inputs, so bucket order inside an
// expert (set by LDS atomics) does not change any result bit.

#include "pe_internal.h"

namespace pe {

// ---------------------------------------------------------------------------
// routing: one wave per token, up to 256 experts (expert e = lane + 64 i).
// Each expert gets a 64-bit key: the score's bits mapped to an unsigned order
// above, the inverted expert id below, so a larger key is a higher score and
// equal scores rank the lower id first. The keys go to LDS; each lane counts
// the keys above its own (its rank), and ranks 0..top_k-1 are the selection
// in descending order, the order of the reference's repeated arg-max / topk.
//
// Grouped top-k (n_group > 0; the use_grouped_topk / num_expert_group /
// topk_group arguments moe_method.py:74-78 passes on to vLLM's fused MoE,
// whose grouped_topk is restated here): the E experts form n_group
// contiguous groups; a group's score is its best expert score, or with a
// correction bias the sum of its two best biased scores; the topk_group best
// groups (ties: lower group) stay, every other expert is masked, and top_k is
// taken over the rest by biased score. The weights are the unbiased scores.
// ---------------------------------------------------------------------------
constexpr int kRouteWaves = 4;
constexpr int kRouteMaxGroups = 64;

__device__ __forceinline__ uint64_t route_key(float s, int e) {
  const uint32_t b = __builtin_bit_cast(uint32_t, s + 0.f);  // -0 -> +0
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}

__global__ __launch_bounds__(64 * kRouteWaves) void moe_route_kernel(
    const float* __restrict__ logits, int64_t T, int E, int top_k, int renormalize, int scoring,
    const float* __restrict__ bias, float* __restrict__ topk_w, int32_t* __restrict__ topk_ids,
    int n_group, int topk_group) {
  __shared__ uint64_t keys[kRouteWaves][256];
  __shared__ float sel_w[kRouteWaves][16];
  __shared__ int sel_e[kRouteWaves][16];
  __shared__ float gsc[kRouteWaves][256];            // grouped: biased expert scores
  __shared__ float grp[kRouteWaves][kRouteMaxGroups];  // grouped: group scores
  __shared__ int gkeep[kRouteWaves][kRouteMaxGroups];  // grouped: group selected
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * kRouteWaves + wave;
  const bool live = t < T;
  const int64_t tr = live ? t : T - 1;  // idle waves recompute a live row: barriers are per workgroup
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    float l = -INFINITY;
    if (e < E) {
      l = logits[tr * E + e];
      if (bias && n_group == 0) l += bias[e];  // ungrouped: bias on the logits
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
    for (int i = 0; i < 4; ++i) v[i] = (lane + 64 * i) < E ? 1.f / (1.f + expf(-v[i])) : 0.f;
  }
  const int Ep = (E + 1) & ~1;  // keys read in pairs; a padding key is 0, below every real key
  // ranking score of each expert: the score, or (grouped, with a bias) the
  // biased score; masked experts (grouped: outside the kept groups) get the
  // padding key 0 and rank below every live one
  float rs[4];
  bool live_e[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    if (v[i] != v[i]) v[i] = -1.f;  // NaN scores rank last
    rs[i] = v[i];
    if (n_group > 0 && bias && e < E) rs[i] = v[i] + bias[e];
    if (rs[i] != rs[i]) rs[i] = -1.f;
    live_e[i] = e < E;
  }
  if (n_group > 0) {  // uniform
    const int epg = E / n_group;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane + 64 * i;
      if (e < E) gsc[wave][e] = rs[i];
    }
    __syncthreads();
    if (lane < n_group) {
      float m1 = -INFINITY, m2 = -INFINITY;  // two best of the group, duplicates kept
      for (int j = 0; j < epg; ++j) {
        const float s = gsc[wave][lane * epg + j];
        if (s > m1) {
          m2 = m1;
          m1 = s;
        } else if (s > m2) {
          m2 = s;
        }
      }
      grp[wave][lane] = bias ? m1 + m2 : m1;
    }
    __syncthreads();
    if (lane < n_group) {
      const float mine_g = grp[wave][lane];
      int r = 0;
      for (int h = 0; h < n_group; ++h) {
        const float o = grp[wave][h];
        r += (o > mine_g || (o == mine_g && h < lane)) ? 1 : 0;
      }
      gkeep[wave][lane] = r < topk_group;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane + 64 * i;
      if (e < E) live_e[i] = gkeep[wave][e / epg] != 0;
    }
  }
  uint64_t mine[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    mine[i] = live_e[i] ? route_key(rs[i], e) : 0;
    if (e < Ep) keys[wave][e] = mine[i];
  }
  __syncthreads();
  int rank[4] = {0, 0, 0, 0};
  for (int j = 0; j < Ep; j += 2) {
    const uint64_t k0 = keys[wave][j], k1 = keys[wave][j + 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (64 * i < E) {  // uniform
        rank[i] += k0 > mine[i] ? 1 : 0;
        rank[i] += k1 > mine[i] ? 1 : 0;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    if (live_e[i] && rank[i] < top_k) {
      sel_w[wave][rank[i]] = v[i];  // the unbiased score (grouped) or the score
      sel_e[wave][rank[i]] = e;
    }
  }
  __syncthreads();
  if (live && lane < top_k) {
    float wsum = 0.f;
    for (int k = 0; k < top_k; ++k) wsum += sel_w[wave][k];  // selection order
    const float w = sel_w[wave][lane];
    topk_w[t * top_k + lane] = renormalize ? w / wsum : w;
    topk_ids[t * top_k + lane] = sel_e[wave][lane];
  }
}

// ---------------------------------------------------------------------------
// moe_prep: workgroups 0..fwht_wgs-1 transform x (one 128-block per 16-lane
// group) into pair f16; workgroup fwht_wgs buckets the pairs by expert.
// ---------------------------------------------------------------------------
constexpr int kPrepThreads = 256;

__device__ void moe_align_block(const int32_t* __restrict__ topk_ids, int64_t P, int top_k, int E,
                                int32_t* __restrict__ offsets /* [E+1] */,
                                int32_t* __restrict__ sorted_token /* [P] */,
                                int32_t* __restrict__ pair_pos /* [P] */) {
  __shared__ int cnt[256];
  __shared__ int base[257];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += kPrepThreads) cnt[e] = 0;
  __syncthreads();
  for (int64_t p = tid; p < P; p += kPrepThreads) {
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
  for (int e = tid; e <= E; e += kPrepThreads) offsets[e] = base[e];
  for (int e = tid; e < E; e += kPrepThreads) cnt[e] = 0;
  __syncthreads();
  for (int64_t p = tid; p < P; p += kPrepThreads) {
    const int e = topk_ids[p];
    int pos = -1;
    if (e >= 0 && e < E) {
      pos = base[e] + atomicAdd(&cnt[e], 1);
      sorted_token[pos] = (int32_t)(p / top_k);
    }
    pair_pos[p] = pos;
  }
}

__global__ __launch_bounds__(kPrepThreads) void moe_prep_kernel(
    const uint16_t* __restrict__ x, int64_t T, int nbc, uint32_t* __restrict__ xtf, int fwht_wgs,
    const int32_t* __restrict__ topk_ids, int64_t P, int top_k, int E, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_token, int32_t* __restrict__ pair_pos, int xbf) {
  if ((int)blockIdx.x == fwht_wgs) {  // whole workgroup
    moe_align_block(topk_ids, P, top_k, E, offsets, sorted_token, pair_pos);
    return;
  }
  const int64_t total = T * (int64_t)nbc;
  int64_t bid = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int q = threadIdx.x & 15;
  const bool live = bid < total;
  if (!live) bid = total - 1;  // the group stays converged; its store is masked
  const int64_t r = bid / nbc;
  const int cb = (int)(bid - r * nbc);
  float v[8];
  if (xbf) load8<PE_DTYPE_BF16>(x + (r * nbc + cb) * kBlock + q * 8, v);
  else load8<PE_DTYPE_F16>(x + (r * nbc + cb) * kBlock + q * 8, v);
  fwht128_group16(v, q);
  store_pair_block(v, q, xtf + bid * 64, live);
}

// out[t, c..c+3] = sum_k w[t, k] * y2[pos(t, k), c..c+3], k in order; 4
// columns per lane, the loads of four slots issued before their sums
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y2,
                                                          const float* __restrict__ topk_w,
                                                          const int32_t* __restrict__ pair_pos,
                                                          int64_t T, int top_k, int H,
                                                          uint16_t* __restrict__ out, int ybf) {
  const int per_row = H / 4;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= T * per_row) return;
  const int64_t t = i / per_row;
  const int c = (int)(i - t * per_row) * 4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < top_k; k0 += 4) {
    int pos[4];
    float w[4];
    float4 yv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = k0 + u;
      pos[u] = k < top_k ? pair_pos[t * top_k + k] : -1;
      w[u] = pos[u] >= 0 ? topk_w[t * top_k + k] : 0.f;
      yv[u] = pos[u] >= 0 ? *reinterpret_cast<const float4*>(y2 + (int64_t)pos[u] * H + c)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (pos[u] < 0) continue;
      acc[0] += w[u] * yv[u].x;
      acc[1] += w[u] * yv[u].y;
      acc[2] += w[u] * yv[u].z;
      acc[3] += w[u] * yv[u].w;
    }
  }
  uint2 o;
  o.x = pack16x2(acc[0], acc[1], ybf != 0);
  o.y = pack16x2(acc[2], acc[3], ybf != 0);
  *reinterpret_cast<uint2*>(out + t * H + c) = o;
}

struct MoeWs {
  size_t offsets, sorted_token, pair_pos, xtf, htf, y2, total;
};

static MoeWs moe_ws_layout(int64_t T, int top_k, int E, int H, int I) {
  const int64_t P = T * top_k;
  const int64_t Ip = (I + kBlock - 1) / kBlock * kBlock;
  MoeWs w{};
  size_t o = kWsCounterBytes;  // the library-wide counter block stays untouched
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

static int route(const float* logits, int64_t T, int E, int top_k, int renormalize, int scoring,
                 const float* correction_bias, int n_group, int topk_group, float* topk_w,
                 int32_t* topk_ids, hipStream_t st) {
  if (!logits || !topk_w || !topk_ids) return PE_ERR_NULL;
  if (T < 0 || E <= 0 || E > 256 || top_k <= 0 || top_k > 16 || top_k > E) return PE_ERR_DIMS;
  if (scoring != 0 && scoring != 1) return PE_ERR_DTYPE;
  if (T == 0) return PE_OK;
  const int64_t wgs = (T + kRouteWaves - 1) / kRouteWaves;
  if (wgs > INT32_MAX) return PE_ERR_DIMS;
  moe_route_kernel<<<dim3((unsigned)wgs), dim3(64 * kRouteWaves), 0, st>>>(
      logits, T, E, top_k, renormalize, scoring, correction_bias, topk_w, topk_ids, n_group,
      topk_group);
  return launch_status();
}

extern "C" int pe_moe_route(const float* logits, int64_t T, int E, int top_k, int renormalize,
                            int scoring, const float* correction_bias, float* topk_w,
                            int32_t* topk_ids, void* stream) {
  return route(logits, T, E, top_k, renormalize, scoring, correction_bias, 0, 0, topk_w, topk_ids,
               reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pe_moe_route_grouped(const float* logits, int64_t T, int E, int top_k,
                                    int renormalize, int scoring, const float* correction_bias,
                                    int num_expert_group, int topk_group, float* topk_w,
                                    int32_t* topk_ids, void* stream) {
  // whole groups, at most 64 of them; the kept groups must hold top_k experts;
  // a bias ranks groups by their two best experts
  if (num_expert_group <= 0 || num_expert_group > kRouteMaxGroups || E % num_expert_group ||
      topk_group <= 0 || topk_group > num_expert_group ||
      top_k > topk_group * (E / num_expert_group) ||
      (correction_bias && E / num_expert_group < 2))
    return PE_ERR_DIMS;
  return route(logits, T, E, top_k, renormalize, scoring, correction_bias, num_expert_group,
               topk_group, topk_w, topk_ids, reinterpret_cast<hipStream_t>(stream));
}

extern "C" size_t pe_moe_workspace_size(int64_t T, int top_k, int E, int H, int I) {
  if (T <= 0 || top_k <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
  return moe_ws_layout(T, top_k, E, H, I).total;
}

extern "C" int pe_moe_forward(const void* x, int x_dtype, int64_t T, int H, int I, int E, int top_k,
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
  const int xbf = bf16_flag(x_dtype);  // x and out: fp16 or bf16
  if (xbf < 0) return PE_ERR_DTYPE;
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

  // 1. x -> pair f16, and the pairs bucketed by expert (last workgroup)
  {
    const int nbc = H / kBlock;
    const int64_t fwht_wgs = (T * nbc + 15) / 16;
    if (fwht_wgs + 1 > INT32_MAX) return PE_ERR_DIMS;
    moe_prep_kernel<<<dim3((unsigned)(fwht_wgs + 1)), dim3(kPrepThreads), 0, st>>>(
        reinterpret_cast<const uint16_t*>(x), T, nbc, reinterpret_cast<uint32_t*>(ws + L.xtf),
        (int)fwht_wgs, topk_ids, P, top_k, E, offsets, sorted_token, pair_pos, xbf);
    if (int rc = launch_status()) return rc;
  }
  // 2. gate/up + SwiGLU, each 128-column block of h transformed in the same
  // kernel -> htf [P, Ip] pair f16 (columns past I are zero)
  {
    SmallArgs a{reinterpret_cast<const uint8_t*>(w13_codes), w13_norms, ct13, n_levels13,
                reinterpret_cast<const uint32_t*>(ws + L.xtf), sorted_token, offsets,
                2 * (int64_t)I * row13, 2 * (int64_t)I * nb13, ws + L.htf, Ip, nullptr, 0, I,
                nb13, wlayout(nib13, tiled13, nb13)};
    if (int rc = moe_grouped(nib13, SE_SWIGLU_XTF, a, E, st)) return rc;
  }
  // 3. down -> y2 [P, H] fp32
  {
    SmallArgs a{reinterpret_cast<const uint8_t*>(w2_codes), w2_norms, ct2, n_levels2,
                reinterpret_cast<const uint32_t*>(ws + L.htf), nullptr, offsets,
                (int64_t)H * row2, (int64_t)H * nb2, ws + L.y2, H, nullptr, 0, H, nb2,
                wlayout(nib2, tiled2, nb2)};
    if (int rc = moe_grouped(nib2, SE_F32, a, E, st)) return rc;
  }
  // 4. weighted combine -> out (x's dtype)
  const int64_t work = T * (H / 4);
  moe_combine_kernel<<<dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st>>>(
      reinterpret_cast<const float*>(ws + L.y2), topk_w, pair_pos, T, top_k, H,
      reinterpret_cast<uint16_t*>(out), xbf);
  return launch_status();
}
