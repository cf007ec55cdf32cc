// Quantized grouped-expert MoE for gfx950.
//
// The reference has no quantized MoE compute: PolarPassthroughMoEMethod
// forwards experts to vLLM's bf16 fused MoE (moe_method.py:74-92). The
// per-expert math followed here is the reference's in-repo MoE forward
// (nemotron_offload.py:172-226): scores = softmax|sigmoid(logits + bias),
// top-k, renormalise, gate = x W13[:I]^T, up = x W13[I:]^T,
// h = silu(gate) * up, y = h W2^T, out = sum_k w_k y_k.
//
// Launch sequence of pe_moe_forward / pe_moe_forward_routed (no host
// synchronisation):
//   1. moe_front_kernel: the routing of pe_moe_forward_routed (the ids are
//      given to pe_moe_forward), the FWHT-128 of x into pair f16 (shared by
//      every expert), and the bucketing of the T*top_k (token, slot) pairs by
//      expert -> per-expert offsets, token of each sorted pair, sorted
//      position of each pair;
//   2. grouped experts, W13: gate and up tiles with SwiGLU; each 128-column
//      block of h goes through the FWHT in the same kernel -> pair-f16 h
//      [pairs, Ip] (A rows gathered by token id; columns past I are zero);
//   3. grouped experts, W2 -> y2 [pairs, H] fp32 (prefill regime: x's 16-bit type);
//   4. combine: out[t] = sum_k w[t, k] * y2[pos(t, k)] in fixed k order.
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

struct RouteParams {
  const float* logits;  // [T, E] fp32
  int64_t T;
  int E, top_k, renormalize, scoring;
  const float* bias;    // nullable correction bias [E]
  float* topk_w;        // [T, top_k]
  int32_t* topk_ids;    // [T, top_k]
  int n_group, topk_group;
};

// Routes tokens t0 + wave (wave = 0..kRouteWaves-1) of this workgroup. COH:
// the ids are stored device-coherently, for a workgroup of the same launch
// that buckets them.
template <bool COH>
__device__ void route_tokens(const RouteParams& p, int64_t t0) {
  const float* __restrict__ logits = p.logits;
  const float* __restrict__ bias = p.bias;
  const int64_t T = p.T;
  const int E = p.E, top_k = p.top_k, scoring = p.scoring, n_group = p.n_group;
  __shared__ uint64_t keys[kRouteWaves][256];
  __shared__ float sel_w[kRouteWaves][16];
  __shared__ int sel_e[kRouteWaves][16];
  __shared__ float gsc[kRouteWaves][256];            // grouped: biased expert scores
  __shared__ float grp[kRouteWaves][kRouteMaxGroups];  // grouped: group scores
  __shared__ int gkeep[kRouteWaves][kRouteMaxGroups];  // grouped: group selected
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t = t0 + wave;
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
      gkeep[wave][lane] = r < p.topk_group;
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
    p.topk_w[t * top_k + lane] = p.renormalize ? w / wsum : w;
    if constexpr (COH)
      st_dev32(reinterpret_cast<uint32_t*>(p.topk_ids) + t * top_k + lane, (uint32_t)sel_e[wave][lane]);
    else
      p.topk_ids[t * top_k + lane] = sel_e[wave][lane];
  }
}

__global__ __launch_bounds__(64 * kRouteWaves) void moe_route_kernel(RouteParams p) {
  route_tokens<false>(p, (int64_t)blockIdx.x * kRouteWaves);
}

// ---------------------------------------------------------------------------
// moe_front_kernel: what the expert products need, in one launch.
//  * routing workgroups (route_wgs > 0): kRouteWaves tokens each; the last of
//    them to finish (a device-scope counter in the workspace's counter block,
//    which it resets) buckets the pairs;
//  * transform workgroups: FWHT-128 of x into pair f16, one 128-block per
//    16-lane group;
//  * with the ids given (route_wgs == 0), one more workgroup buckets them.
// With more than kFrontBucketMaxPairs pairs the bucketing is left to
// moe_bucket_kernel, launched next (bucket_here == 0).
// Bucketing (one workgroup): LDS histogram of the T*top_k (token, slot) pairs
// by expert, exclusive scan, scatter -> per-expert offsets, the token of each
// sorted pair, the sorted position of each pair (-1 for an id outside
// 0..E-1). Given ids may hold such slots: the output rows of tokens without
// one valid slot are zeroed here, as no other kernel writes them.
// ---------------------------------------------------------------------------
constexpr int kFrontThreads = 64 * kRouteWaves;

struct FrontArgs {
  RouteParams r;          // r.logits null: the ids are given
  int route_wgs, fwht_wgs;
  const uint16_t* x;      // [T, H] fp16 or bf16
  int nbc, xbf;           // 128-blocks per row; x is bfloat16
  uint32_t* xtf;          // [T, H/2] pair f16
  int32_t* offsets;       // [E + 1]
  int32_t* sorted_token;  // [P]
  int32_t* pair_pos;      // [P]
  uint32_t* done;         // routing completion counter (zero; left zero)
  int bucket_here;        // 0: moe_bucket_kernel buckets the pairs after this launch
  uint16_t* out;          // [T, H]
};

constexpr int kAlignBatch = 8;  // ids per thread loaded before their use

// COH: the ids were written by other workgroups of this launch (routing; all
// valid by construction) and are read device-coherently; else they are the
// caller's, read plainly, and may hold ids outside 0..E-1.
template <bool COH>
__device__ void moe_align_block(const FrontArgs& a) {
  __shared__ int cnt[256];
  __shared__ int base[257];
  __shared__ int wtot[kFrontThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = a.r.E, top_k = a.r.top_k;
  const int64_t P = a.r.T * top_k;
  const uint32_t* ids = reinterpret_cast<const uint32_t*>(a.r.topk_ids);
  // the ids of pairs p0 + tid + kFrontThreads * u, all loads issued first
  auto load_ids = [&](int64_t p0, int (&e)[kAlignBatch]) {
#pragma unroll
    for (int u = 0; u < kAlignBatch; ++u) {
      const int64_t p = p0 + tid + (int64_t)kFrontThreads * u;
      const int64_t pc = p < P ? p : P - 1;
      e[u] = COH ? (int)ld_dev32(ids + pc) : (int)ids[pc];
    }
  };
  constexpr int64_t kChunk = (int64_t)kFrontThreads * kAlignBatch;
  // one chunk (P <= 2048: T * top_k of a decode batch): the ids stay in
  // registers for the scatter pass, one memory round trip fewer
  const bool one = P <= kChunk;
  int e1[kAlignBatch];
  for (int e = tid; e < E; e += kFrontThreads) cnt[e] = 0;
  __syncthreads();
  for (int64_t p0 = 0; p0 < P; p0 += kChunk) {
    int e[kAlignBatch];
    load_ids(p0, e);
#pragma unroll
    for (int u = 0; u < kAlignBatch; ++u) e1[u] = e[u];
#pragma unroll
    for (int u = 0; u < kAlignBatch; ++u)
      if (p0 + tid + (int64_t)kFrontThreads * u < P && e[u] >= 0 && e[u] < E) atomicAdd(&cnt[e[u]], 1);
  }
  __syncthreads();
  // exclusive scan over the experts, thread e holding cnt[e] (E <= 256)
  const int v = tid < E ? cnt[tid] : 0;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += wtot[w];
  if (tid < E) {
    base[tid] = before + incl - v;
    cnt[tid] = 0;  // this thread's count, read above
  }
  if (tid == E - 1) base[E] = before + incl;
  __syncthreads();
  for (int e = tid; e <= E; e += kFrontThreads) a.offsets[e] = base[e];
  for (int64_t p0 = 0; p0 < P; p0 += kChunk) {
    int e[kAlignBatch];
    if (one) {  // uniform
#pragma unroll
      for (int u = 0; u < kAlignBatch; ++u) e[u] = e1[u];
    } else {
      load_ids(p0, e);
    }
#pragma unroll
    for (int u = 0; u < kAlignBatch; ++u) {
      const int64_t p = p0 + tid + (int64_t)kFrontThreads * u;
      if (p >= P) continue;
      int pos = -1;
      if (e[u] >= 0 && e[u] < E) {
        pos = base[e[u]] + atomicAdd(&cnt[e[u]], 1);
        a.sorted_token[pos] = (int32_t)(p / top_k);
      }
      a.pair_pos[p] = pos;
    }
  }
  if constexpr (!COH) {
    const int64_t H = (int64_t)a.nbc * kBlock;
    for (int64_t t = tid; t < a.r.T; t += kFrontThreads) {
      bool any = false;
      for (int k = 0; k < top_k; ++k) {
        const int e = a.r.topk_ids[t * top_k + k];
        any = any || (e >= 0 && e < E);
      }
      if (!any)
        for (int64_t c = 0; c < H; ++c) a.out[t * H + c] = 0;
    }
  }
}

__global__ __launch_bounds__(kFrontThreads) void moe_front_kernel(FrontArgs a) {
  int bid = blockIdx.x;
  if (bid < a.route_wgs) {
    route_tokens<true>(a.r, (int64_t)bid * kRouteWaves);
    if (!a.bucket_here) return;  // uniform: the next launch buckets the ids
    // this workgroup's ids are stored once every thread's vmcnt drains
    // (stores count there on this architecture); then it is counted in
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ uint32_t last;
    if (threadIdx.x == 0) last = atomicAdd(a.done, 1u) + 1 == (uint32_t)a.route_wgs ? 1u : 0u;
    __syncthreads();
    if (!last) return;  // uniform
    moe_align_block<true>(a);
    if (threadIdx.x == 0) __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  bid -= a.route_wgs;
  if (bid == a.fwht_wgs) {  // ids given: the bucketing workgroup (whole workgroup)
    moe_align_block<false>(a);
    return;
  }
  const int64_t total = a.r.T * (int64_t)a.nbc;
  int64_t blk = (int64_t)bid * 16 + (threadIdx.x >> 4);
  const int q = threadIdx.x & 15;
  const bool live = blk < total;
  if (!live) blk = total - 1;  // the group stays converged; its store is masked
  float v[8];
  if (a.xbf) load8<PE_DTYPE_BF16>(a.x + blk * kBlock + q * 8, v);
  else load8<PE_DTYPE_F16>(a.x + blk * kBlock + q * 8, v);
  fwht128_group16(v, q);
  store_pair_block(v, q, a.xtf + blk * 64, live);
}

// moe_bucket_kernel: the bucketing of moe_align_block for many pairs (P >
// kFrontBucketMaxPairs), as a launch of its own after the routing: one
// workgroup of 1024 threads; every pair takes its slot in its expert with an
// LDS atomic as its id is read, the sorted token list is built in LDS
// (dynamic, 4 bytes per pair) and written out in order, so no store is
// scattered over memory (from one CU, the scattered stores of 16384 pairs
// took about 8 us of the front launch's 24 at 2048 tokens). Ids outside
// 0..E-1 (given ids only) get position -1, and the output rows of tokens
// without one valid slot are zeroed here, as in moe_align_block.
constexpr int kBucketThreads = 1024;
constexpr int kBucketPerThread = 32;  // pairs per thread in registers: P <= 32768
constexpr int kFrontBucketMaxPairs = 2048;

__global__ __launch_bounds__(kBucketThreads) void moe_bucket_kernel(FrontArgs a) {
  extern __shared__ int32_t sorted_lds[];
  __shared__ int cnt[256];
  __shared__ int base[257];
  __shared__ int wtot[kBucketThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = a.r.E, top_k = a.r.top_k;
  const int P = (int)(a.r.T * top_k);
  for (int e = tid; e < E; e += kBucketThreads) cnt[e] = 0;
  __syncthreads();
  int ids[kBucketPerThread], rank[kBucketPerThread];
#pragma unroll
  for (int u = 0; u < kBucketPerThread; ++u) {
    const int p = tid + kBucketThreads * u;
    ids[u] = p < P ? a.r.topk_ids[p] : -1;
  }
#pragma unroll
  for (int u = 0; u < kBucketPerThread; ++u) {
    const bool ok = ids[u] >= 0 && ids[u] < E;
    rank[u] = ok ? atomicAdd(&cnt[ids[u]], 1) : -1;
  }
  __syncthreads();
  // exclusive scan over the experts, thread e holding cnt[e] (E <= 256: four waves)
  const int v = tid < E ? cnt[tid] : 0;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += wtot[w];
  if (tid < E) base[tid] = before + incl - v;
  if (tid == E - 1) base[E] = before + incl;
  __syncthreads();
  for (int e = tid; e <= E; e += kBucketThreads) a.offsets[e] = base[e];
#pragma unroll
  for (int u = 0; u < kBucketPerThread; ++u) {
    const int p = tid + kBucketThreads * u;
    if (p >= P) continue;
    int pos = -1;
    if (rank[u] >= 0) {
      pos = base[ids[u]] + rank[u];
      sorted_lds[pos] = p / top_k;
    }
    a.pair_pos[p] = pos;
  }
  __syncthreads();
  const int valid = base[E];
  for (int i = tid; i < valid; i += kBucketThreads) a.sorted_token[i] = sorted_lds[i];
  if (a.route_wgs == 0) {  // given ids: tokens without a valid slot
    const int64_t H = (int64_t)a.nbc * kBlock;
    for (int64_t t = tid; t < a.r.T; t += kBucketThreads) {
      bool any = false;
      for (int k = 0; k < top_k; ++k) {
        const int e = a.r.topk_ids[t * top_k + k];
        any = any || (e >= 0 && e < E);
      }
      if (!any)
        for (int64_t c = 0; c < H; ++c) a.out[t * H + c] = 0;
    }
  }
}

// out[t, c..] = sum_k w[t, k] * y2[pos(t, k), c..], k in order; 4 (fp32
// rows) or 8 (16-bit rows) columns per lane, the loads of eight slots issued
// before their sums (top-8 in one memory round trip). y2 rows are fp32 (YT =
// float) or 16-bit (YT = uint16_t: bfloat16 if y2bf, else fp16).
constexpr int kCombineBatch = 8;

template <typename YT>
__global__ __launch_bounds__(256) void moe_combine_kernel(const YT* __restrict__ y2, int y2bf,
                                                          const float* __restrict__ topk_w,
                                                          const int32_t* __restrict__ pair_pos,
                                                          int64_t T, int top_k, int H,
                                                          uint16_t* __restrict__ out, int ybf) {
  // columns per lane: one 16-byte load of each slot's row
  constexpr int CPL = 16 / sizeof(YT);
  const int per_row = H / CPL;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= T * per_row) return;
  const int64_t t = i / per_row;
  const int c = (int)(i - t * per_row) * CPL;
  float acc[CPL];
#pragma unroll
  for (int q = 0; q < CPL; ++q) acc[q] = 0.f;
  for (int k0 = 0; k0 < top_k; k0 += kCombineBatch) {
    int pos[kCombineBatch];
    float w[kCombineBatch];
    uint4 yv[kCombineBatch];
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      const int k = k0 + u;
      pos[u] = k < top_k ? pair_pos[t * top_k + k] : -1;
      w[u] = pos[u] >= 0 ? topk_w[t * top_k + k] : 0.f;
      yv[u] = pos[u] >= 0 ? *reinterpret_cast<const uint4*>(y2 + (int64_t)pos[u] * H + c) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      if (pos[u] < 0) continue;
      const uint32_t d[4] = {yv[u].x, yv[u].y, yv[u].z, yv[u].w};
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        float v;
        if constexpr (sizeof(YT) == 4) {
          v = __builtin_bit_cast(float, d[q]);
        } else {
          const uint16_t h = (uint16_t)(d[q >> 1] >> (16 * (q & 1)));
          v = y2bf ? bf2f(h) : h2f(h);
        }
        acc[q] += w[u] * v;
      }
    }
  }
  uint32_t o[CPL / 2];
#pragma unroll
  for (int q = 0; q < CPL / 2; ++q) o[q] = pack16x2(acc[2 * q], acc[2 * q + 1], ybf != 0);
  if constexpr (CPL == 8) {
    *reinterpret_cast<uint4*>(out + t * H + c) = make_uint4(o[0], o[1], o[2], o[3]);
  } else {
    *reinterpret_cast<uint2*>(out + t * H + c) = make_uint2(o[0], o[1]);
  }
}

struct MoeWs {
  size_t offsets, sorted_token, pair_pos, topk_w, topk_ids, xtf, htf, y2, total;
};

static MoeWs moe_ws_layout(int64_t T, int top_k, int E, int H, int I) {
  const int64_t P = T * top_k;
  const int64_t Ip = (I + kBlock - 1) / kBlock * kBlock;
  MoeWs w{};
  size_t o = kWsCounterBytes;  // the library-wide counter block comes first
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += round_up(bytes, 256);
    return at;
  };
  w.offsets = take((size_t)(E + 1) * 4);
  w.sorted_token = take((size_t)P * 4);
  w.pair_pos = take((size_t)P * 4);
  w.topk_w = take((size_t)P * 4);
  w.topk_ids = take((size_t)P * 4);
  w.xtf = take((size_t)T * H * 2);
  w.htf = take((size_t)P * Ip * 2);
  w.y2 = take((size_t)P * H * 4);
  w.total = o;
  return w;
}

// Checks of the routing arguments (n_group 0: plain top-k).
static int route_check(int64_t T, int E, int top_k, int scoring, const float* bias, int n_group,
                       int topk_group) {
  if (T < 0 || E <= 0 || E > 256 || top_k <= 0 || top_k > 16 || top_k > E) return PE_ERR_DIMS;
  if (scoring != 0 && scoring != 1) return PE_ERR_DTYPE;
  // grouped: whole groups, at most 64 of them; the kept groups must hold
  // top_k experts; a bias ranks groups by their two best experts
  if (n_group != 0 &&
      (n_group < 0 || n_group > kRouteMaxGroups || E % n_group || topk_group <= 0 ||
       topk_group > n_group || top_k > topk_group * (E / n_group) || (bias && E / n_group < 2)))
    return PE_ERR_DIMS;
  return PE_OK;
}

// Experts with at least this many rows on average (the prefill regime) run
// on the grouped four-wave prefill kernel: 128-row tiles of 32x32x16 MFMAs,
// each expert's weights read once per 128 rows, instead of the expert
// kernel's passes of 64 rows on 16x16x32 MFMAs (64 experts, top-8: 1024
// tokens 351 -> 313 us, 2048 tokens 603 -> 487; at 96 rows level).
constexpr int kMoeGemmMinRows = 128;

struct MoeWeights {
  const void* w13_codes;
  int bits13, packed13;
  const uint16_t* w13_norms;
  const float* ct13;
  int n_levels13;
  const void* w2_codes;
  int bits2, packed2;
  const uint16_t* w2_norms;
  const float* ct2;
  int n_levels2;
};

// The launches of one MoE call. route: routing parameters (logits given) or
// null (topk_w / topk_ids given).
static int moe_run(const void* x, int x_dtype, int64_t T, int H, int I, int E, int top_k,
                   const RouteParams* route, const float* topk_w, const int32_t* topk_ids,
                   const MoeWeights& W, void* out, void* workspace, size_t workspace_bytes,
                   hipStream_t st) {
  if (!x || !W.w13_codes || !W.w13_norms || !W.ct13 || !W.w2_codes || !W.w2_norms || !W.ct2 || !out)
    return PE_ERR_NULL;
  if (!route && (!topk_w || !topk_ids)) return PE_ERR_NULL;
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || E > 256 || top_k <= 0 || top_k > E) return PE_ERR_DIMS;
  if (H % kBlock) return PE_ERR_DIMS;
  const int xbf = bf16_flag(x_dtype);  // x and out: fp16 or bf16
  if (xbf < 0) return PE_ERR_DTYPE;
  for (int which = 0; which < 2; ++which) {
    const int bits = which ? W.bits2 : W.bits13, packed = which ? W.packed2 : W.packed13;
    const int nl = which ? W.n_levels2 : W.n_levels13;
    if (bits < 2 || bits > 8 || (packed & ~(1 | PE_LAYOUT_TILE16)) || ((packed & 1) && bits > 4) ||
        nl != (1 << bits))
      return PE_ERR_BITS;
  }
  // tiled-16 experts: every expert's rows are whole 16-row tiles
  if (((W.packed13 & PE_LAYOUT_TILE16) && (2 * I) % 16) || ((W.packed2 & PE_LAYOUT_TILE16) && H % 16))
    return PE_ERR_DIMS;
  if (!aligned16(x) || !aligned16(W.w13_codes) || !aligned16(W.w2_codes) || !aligned16(out))
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
  const bool nib13 = (W.packed13 & 1) != 0, nib2 = (W.packed2 & 1) != 0;
  const bool tiled13 = (W.packed13 & PE_LAYOUT_TILE16) != 0, tiled2 = (W.packed2 & PE_LAYOUT_TILE16) != 0;
  const int64_t row13 = nib13 ? (int64_t)nb13 * 64 : (int64_t)nb13 * kBlock;
  const int64_t row2 = nib2 ? (int64_t)nb2 * 64 : (int64_t)nb2 * kBlock;

  // 1. routing (or the given ids), x -> pair f16, the pairs bucketed by expert
  {
    FrontArgs f{};
    if (route) {
      f.r = *route;
      f.r.topk_w = reinterpret_cast<float*>(ws + L.topk_w);
      f.r.topk_ids = reinterpret_cast<int32_t*>(ws + L.topk_ids);
      f.route_wgs = (int)((T + kRouteWaves - 1) / kRouteWaves);
    } else {
      f.r.T = T;
      f.r.E = E;
      f.r.top_k = top_k;
      f.r.topk_w = const_cast<float*>(topk_w);
      f.r.topk_ids = const_cast<int32_t*>(topk_ids);
      f.route_wgs = 0;
    }
    const int64_t fwht_wgs = (T * (H / kBlock) + 15) / 16;
    if (fwht_wgs + f.route_wgs + 1 > INT32_MAX) return PE_ERR_DIMS;
    f.fwht_wgs = (int)fwht_wgs;
    f.x = reinterpret_cast<const uint16_t*>(x);
    f.nbc = H / kBlock;
    f.xbf = xbf;
    f.xtf = reinterpret_cast<uint32_t*>(ws + L.xtf);
    f.offsets = offsets;
    f.sorted_token = sorted_token;
    f.pair_pos = pair_pos;
    f.done = reinterpret_cast<uint32_t*>(ws);  // counter block word 0
    f.out = reinterpret_cast<uint16_t*>(out);
    // many pairs: the bucketing in a launch of its own (moe_bucket_kernel)
    const bool bucket_apart = P > kFrontBucketMaxPairs && P <= (int64_t)kBucketThreads * kBucketPerThread;
    f.bucket_here = bucket_apart ? 0 : 1;
    const int grid = f.route_wgs + f.fwht_wgs + (route || bucket_apart ? 0 : 1);
    moe_front_kernel<<<dim3((unsigned)grid), dim3(kFrontThreads), 0, st>>>(f);
    if (int rc = launch_status()) return rc;
    if (bucket_apart) {
      const size_t lds = (size_t)P * 4;
      static const bool attr_ok = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(moe_bucket_kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024) == hipSuccess;
      }();
      (void)attr_ok;
      moe_bucket_kernel<<<dim3(1), dim3(kBucketThreads), lds, st>>>(f);
      if (int rc = launch_status()) return rc;
    }
  }
  const float* wts = route ? reinterpret_cast<const float*>(ws + L.topk_w) : topk_w;
  // 2. gate/up + SwiGLU, each 128-column block of h transformed in the same
  // kernel -> htf [P, Ip] pair f16 (columns past I are zero)
  // 3. down -> y2 [P, H] fp32
  const MoeGemmArgs g13{reinterpret_cast<const uint8_t*>(W.w13_codes), W.w13_norms, W.ct13, W.n_levels13,
                        wlayout(nib13, tiled13, nb13), nb13, ws + L.xtf, ws + L.htf, Ip, 2 * I, P,
                        GemmGroup{offsets, sorted_token, 2 * (int64_t)I * row13, 2 * (int64_t)I * nb13, T, E, I}};
  const MoeGemmArgs g2{reinterpret_cast<const uint8_t*>(W.w2_codes), W.w2_norms, W.ct2, W.n_levels2,
                       wlayout(nib2, tiled2, nb2), nb2, ws + L.htf, ws + L.y2, H, H, P,
                       GemmGroup{offsets, nullptr, (int64_t)H * row2, (int64_t)H * nb2, P, E, 0}};
  // the prefill regime writes y2 in x's 16-bit type (as vLLM's fused MoE
  // keeps its intermediate rows): half the bytes for w2 to store and the
  // combine to read (2048 tokens 467.2 -> 455.5 us, 4096 925 -> 882)
  bool y2_16 = false;
  if (P >= (int64_t)kMoeGemmMinRows * E && moe_gemm4_fits(g13, SE_SWIGLU_XTF) && moe_gemm4_fits(g2, SE_F16)) {
    if (int rc = moe_gemm4(nib13, SE_SWIGLU_XTF, g13, st)) return rc;
    MoeGemmArgs g2h = g2;
    g2h.ybf = xbf;
    if (int rc = moe_gemm4(nib2, SE_F16, g2h, st)) return rc;
    y2_16 = true;
  } else {
    {
      SmallArgs a{reinterpret_cast<const uint8_t*>(W.w13_codes), W.w13_norms, W.ct13, W.n_levels13,
                  reinterpret_cast<const uint32_t*>(ws + L.xtf), sorted_token, offsets,
                  2 * (int64_t)I * row13, 2 * (int64_t)I * nb13, ws + L.htf, Ip, nullptr, (int)P, I,
                  nb13, wlayout(nib13, tiled13, nb13)};  // M: all pairs (rows per pass)
      if (int rc = moe_grouped(nib13, SE_SWIGLU_XTF, a, E, st)) return rc;
    }
    {
      SmallArgs a{reinterpret_cast<const uint8_t*>(W.w2_codes), W.w2_norms, W.ct2, W.n_levels2,
                  reinterpret_cast<const uint32_t*>(ws + L.htf), nullptr, offsets,
                  (int64_t)H * row2, (int64_t)H * nb2, ws + L.y2, H, nullptr, (int)P, H, nb2,
                  wlayout(nib2, tiled2, nb2)};
      if (int rc = moe_grouped(nib2, SE_F32, a, E, st)) return rc;
    }
  }
  // 4. weighted combine -> out (x's dtype)
  const int64_t work = T * (H / (y2_16 ? 8 : 4));
  if (y2_16)
    moe_combine_kernel<uint16_t><<<dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st>>>(
        reinterpret_cast<const uint16_t*>(ws + L.y2), xbf, wts, pair_pos, T, top_k, H,
        reinterpret_cast<uint16_t*>(out), xbf);
  else
    moe_combine_kernel<float><<<dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st>>>(
        reinterpret_cast<const float*>(ws + L.y2), 0, wts, pair_pos, T, top_k, H,
        reinterpret_cast<uint16_t*>(out), xbf);
  return launch_status();
}

}  // namespace pe

using namespace pe;

static int route(const float* logits, int64_t T, int E, int top_k, int renormalize, int scoring,
                 const float* correction_bias, int n_group, int topk_group, float* topk_w,
                 int32_t* topk_ids, hipStream_t st) {
  if (!logits || !topk_w || !topk_ids) return PE_ERR_NULL;
  if (int rc = route_check(T, E, top_k, scoring, correction_bias, n_group, topk_group)) return rc;
  if (T == 0) return PE_OK;
  const int64_t wgs = (T + kRouteWaves - 1) / kRouteWaves;
  if (wgs > INT32_MAX) return PE_ERR_DIMS;
  const RouteParams p{logits, T, E, top_k, renormalize, scoring, correction_bias, topk_w, topk_ids,
                      n_group, topk_group};
  moe_route_kernel<<<dim3((unsigned)wgs), dim3(64 * kRouteWaves), 0, st>>>(p);
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
  if (num_expert_group <= 0) return PE_ERR_DIMS;
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
  const MoeWeights W{w13_codes, bits13, packed13, w13_norms, ct13, n_levels13,
                     w2_codes,  bits2,  packed2,  w2_norms,  ct2,  n_levels2};
  return moe_run(x, x_dtype, T, H, I, E, top_k, nullptr, topk_w, topk_ids, W, out, workspace,
                 workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pe_moe_forward_routed(const void* x, int x_dtype, int64_t T, int H, int I, int E,
                                     int top_k, const float* logits, int renormalize, int scoring,
                                     const float* correction_bias, int num_expert_group,
                                     int topk_group, const void* w13_codes, int bits13,
                                     int packed13, const uint16_t* w13_norms, const float* ct13,
                                     int n_levels13, const void* w2_codes, int bits2, int packed2,
                                     const uint16_t* w2_norms, const float* ct2, int n_levels2,
                                     void* out, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (!logits) return PE_ERR_NULL;
  if (int rc = route_check(T, E, top_k, scoring, correction_bias, num_expert_group, topk_group))
    return rc;
  if ((T + kRouteWaves - 1) / kRouteWaves > INT32_MAX / 2) return PE_ERR_DIMS;
  const RouteParams r{logits, T, E, top_k, renormalize, scoring, correction_bias, nullptr, nullptr,
                      num_expert_group, topk_group};
  const MoeWeights W{w13_codes, bits13, packed13, w13_norms, ct13, n_levels13,
                     w2_codes,  bits2,  packed2,  w2_norms,  ct2,  n_levels2};
  return moe_run(x, x_dtype, T, H, I, E, top_k, &r, nullptr, nullptr, W, out, workspace,
                 workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}
