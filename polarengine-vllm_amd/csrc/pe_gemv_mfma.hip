// Decode GEMV for M <= 16 on MFMA with the FWHT fused: y[m, n] =
// sum_b norm[n, b] * <ct[codes[n, b, :]], (H x_m)[b, :]>, fp16 out.
//
// This is the M = 1..16 decode path of the quantized linear (the reference
// routes M = 1 to polar_gemv[_packed]_splitk and M > 1 to polar_gemm[_packed],
// kernels/polar_gemm.py:485-534; linear_method.py:184-221 does the FWHT).
//
// Why this shape (gfx950): the codebook lookup costs one v_perm + one
// ds_read_b32 per code byte no matter what; doing the multiply-adds on the
// matrix core (v_mfma_f32_16x16x32_f16, activations as A, dequantized weights
// as B) instead of v_dot2 cuts the VALU work per byte by ~2.5x, and the
// weight rows then need no cross-lane reduction.
//
//  * one workgroup of NW = TN x KS waves per CU-sized share of rows: TN
//    n-tiles of 16 weight rows (TN chosen so the grid covers the CUs once),
//    KS K-slices of 128-blocks per tile, interleaved (slice s takes blocks
//    s, s + KS, ..: the KS waves of a tile read neighbouring blocks at each
//    step); the slices combine through LDS at the end;
//  * the prologue never waits behind the weight stream: each wave first
//    issues its activation loads and takes the codebook (kernel arguments,
//    or scalar loads of ct that do not queue behind the vector weight
//    stream), then issues its first D weight blocks, writes its share of
//    the codebook table, transforms its activations, and streams the rest D
//    deep. D stays small: the CU's memory pipeline is full at about three
//    1 KB blocks per wave, and a deeper ring only stalls the issuing wave
//    (its prologue finishes later); a workgroup barrier before the first
//    weight block (every activation load queued first) measured 3% slower;
//  * fused FWHT: each 16-lane group transforms one (row, block) of x (DPP
//    butterflies) into pair-f16 in LDS;
//  * A = activation pairs (row m = lane % 16; rows >= M repeat row M - 1 and
//    are discarded), B = table lookups half2(ct[lo], ct[hi]); block norms
//    scale the fp32 block partial.

#include "pe_internal.h"

namespace pe {

template <bool NIB, int TN>
struct DecBlk {
  u32x4v lo[TN];
  u32x4v hi[TN];
  uint16_t nb[TN];
};

// Weight source of one lane: buffer resources for codes and norms (a real one
// and a zero-length one), the lane's row offsets in VGPRs. The block offset
// goes in the scalar offset, so a block's loads cost no VALU; a block past the
// wave's range reads through the zero-length resource, which returns zeros
// without touching memory -- the load count stays the same on every path
// (exact vmcnt waits).
struct DecSrc {
  __amdgpu_buffer_rsrc_t codes, codes_none, norms, norms_none;
  uint32_t voff_codes, voff_norms;
};

constexpr int kBufNT = 2;              // cache policy: non-temporal (weights are read once)
constexpr int kBufSC1 = 16;            // cache policy: device-coherent (sc1)
constexpr int kBufFlags = 0x00020000;  // raw buffer, 32-bit data format (dword 3 of the resource)

template <bool NIB, int TN>
__device__ __forceinline__ void dec_load(DecBlk<NIB, TN>& k, const DecSrc& src, int b, bool valid,
                                         int c_blk, int n_blk2) {
  static_assert(TN == 1, "one 16-row tile per wave");
  const __amdgpu_buffer_rsrc_t rc = valid ? src.codes : src.codes_none;
  const __amdgpu_buffer_rsrc_t rn = valid ? src.norms : src.norms_none;
  k.lo[0] = __builtin_bit_cast(
      u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rc, src.voff_codes, b * c_blk, kBufNT));
  if constexpr (!NIB)
    k.hi[0] = __builtin_bit_cast(
        u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rc, src.voff_codes, b * c_blk + 64, kBufNT));
  k.nb[0] = __builtin_amdgcn_raw_buffer_load_b16(rn, src.voff_norms, b * n_blk2, kBufNT);
}

template <bool NIB>
__device__ __forceinline__ half8v dec_dequant(uint32_t wl, uint32_t wh, uint32_t lane4) {
  uint32_t p[4];
  if constexpr (NIB) {
    p[0] = lds_ld32(tbl_addr<0>(wl, lane4));
    p[1] = lds_ld32(tbl_addr<1>(wl, lane4));
    p[2] = lds_ld32(tbl_addr<2>(wl, lane4));
    p[3] = lds_ld32(tbl_addr<3>(wl, lane4));
  } else {
    const uint32_t a0 = lds_ld32(tbl_addr<0>(wl, lane4)), b0 = lds_ld32(tbl_addr<0>(wh, lane4));
    const uint32_t a1 = lds_ld32(tbl_addr<1>(wl, lane4)), b1 = lds_ld32(tbl_addr<1>(wh, lane4));
    const uint32_t a2 = lds_ld32(tbl_addr<2>(wl, lane4)), b2 = lds_ld32(tbl_addr<2>(wh, lane4));
    const uint32_t a3 = lds_ld32(tbl_addr<3>(wl, lane4)), b3 = lds_ld32(tbl_addr<3>(wh, lane4));
    p[0] = __builtin_amdgcn_perm(b0, a0, 0x05040100u);
    p[1] = __builtin_amdgcn_perm(b1, a1, 0x05040100u);
    p[2] = __builtin_amdgcn_perm(b2, a2, 0x05040100u);
    p[3] = __builtin_amdgcn_perm(b3, a3, 0x05040100u);
  }
  return __builtin_bit_cast(half8v, u32x4v{p[0], p[1], p[2], p[3]});
}

// Codebook table. The values come either by value in the kernel arguments,
// already as fp16 (the host converted its copy of ct: no dependent memory
// read, no conversion), or from wave-uniform scalar loads of the device ct
// (which at least do not queue behind the vector weight stream). Every lane
// then writes its own copy of each entry.
// Nibble: entry (hi << 4) | lo = half2(ct[lo], ct[hi]) (the 16 values are the
// whole codebook), wave w takes hi = w and w + NW; int8: entry e = fp16(ct[e])
// in the low half, wave w takes e = 16 w .. 16 w + 15 and 16 (w + NW) .. + 15.
// NW >= 8 covers 256 entries.

// Codebook by value: fp16 bits, two per dword (v[i] = ct[2 i] | ct[2 i + 1] << 16);
// entries past n_levels repeat the last one.
template <bool NIB>
struct DecCtArg {
  uint32_t v[NIB ? 8 : 128];
};

template <bool NIB>
struct DecTable {
  uint32_t h[NIB ? 16 : 32];  // fp16 bits: nibble ct[0..15]; int8 the wave's two 16-entry chunks
};

template <bool NIB, int NW, bool CTV>
__device__ __forceinline__ void dec_table_load(DecTable<NIB>& t, const float* __restrict__ ct,
                                               const DecCtArg<NIB>& ctv, int n_levels, int wave) {
  const int last = n_levels - 1;
  auto half_of = [&](int e) -> uint32_t {  // fp16 bits of entry e (uniform)
    const uint32_t w = ctv.v[e >> 1];
    return (e & 1) ? (w >> 16) : (w & 0xffffu);
  };
  if constexpr (NIB) {
#pragma unroll
    for (int lo = 0; lo < 16; ++lo)
      t.h[lo] = CTV ? half_of(lo) : (uint32_t)f2h_bits(ct[lo < n_levels ? lo : last]);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int e = (wave + h * NW) * 16 + k;
        const int ec = e < n_levels ? e : last;
        t.h[h * 16 + k] = CTV ? half_of(ec < 255 ? ec : 255) : (uint32_t)f2h_bits(ct[ec]);
      }
  }
}

// FULL: n_levels is the whole code range (16 or 256): every entry of a
// chunk exists, no per-entry test
template <bool NIB, int NW, bool FULL>
__device__ __forceinline__ void dec_table_write(const DecTable<NIB>& t, int n_levels, int wave,
                                                uint32_t lane4) {
  if constexpr (NIB) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int hi = wave + h * NW;
      if (hi < n_levels) {
        uint32_t chi = t.h[0];  // ct[hi] by a uniform select (no further load)
#pragma unroll
        for (int k = 1; k < 16; ++k) chi = hi == k ? t.h[k] : chi;
        const uint32_t base = ((uint32_t)hi << 12) | lane4;
#pragma unroll
        for (int lo = 0; lo < 16; ++lo)
          if (FULL || lo < n_levels) lds_st32(base + ((uint32_t)lo << 8), t.h[lo] | (chi << 16));
      }
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int chunk = wave + h * NW;  // entries 16 chunk .. 16 chunk + 15 (uniform)
      if (chunk < 16) {                 // never past entry 255: the activations follow
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const int e = chunk * 16 + k;
          if (FULL || e < n_levels) lds_st32((uint32_t)e << 8 | lane4, t.h[h * 16 + k]);
        }
      }
    }
  }
}

// partial-sum slabs the last group loads at once
constexpr int kSplitBatch = 16;

// FWHT-128 of the wave's 32 items on the matrix cores, stored as pair f16
// into each item's 256-byte LDS slot: pair p = 32 mp + 8 q + 4 h + r holds
// positions p (m-block mp) and p + 64 (m-block mp + 2), so each lane writes
// four 16-byte runs per m-block pair (16-byte chunk c of the slot stored at
// chunk c ^ sw). Every lane takes part; only live lanes store.
template <bool BF>
__device__ __forceinline__ void dec_xform_mfma(const u32x4v (&xq)[8], uint32_t slot, bool live,
                                               int lane, uint32_t sw) {
  const H128Signs sg = h128_signs<BF ? 0x3F803F80u : 0x3C003C00u>(lane);
  const uint32_t h = (uint32_t)lane >> 5;
#pragma unroll
  for (int mp = 0; mp < 2; ++mp) {
    float16v a0, a1;
    h128_mfma_pair<BF>(sg, xq, mp, mp + 2, a0, a1);
    if (live) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        u32x4v w;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          w[r] = pack_h2(a0[4 * q + r] * kInvSqrt128, a1[4 * q + r] * kInvSqrt128);
        lds_st128(slot + 16u * ((8u * mp + 2u * q + h) ^ sw), w);
      }
    }
  }
}

// x: raw fp16 activations [M, K] (XRAW) or pair-f16 x_tf [M][nb][64] (else),
// row stride ldx fp16 elements. The workgroup covers TN 16-row tiles with
// NW = TN * KS waves: wave w works on tile w / KS over the K-slice w % KS
// (blocks w % KS, w % KS + KS, ..), streaming it D blocks deep; a tile's KS
// waves are neighbours, so they issue their first loads together (1-1.5%
// over slices of one tile spread across the workgroup). XC: activation
// registers per lane. SPLIT: the K blocks are divided into gridDim.y groups,
// blockIdx.y's group only (its activations alone in LDS); each workgroup
// writes fp32 partial sums part[blockIdx.y][M][N], and the last of the
// gridDim.y workgroups of a row group to finish (counted in cnt[blockIdx.x])
// adds the groups' partials in group order, writes y and resets its counter.
// XMF (raw x, at most 32 items per wave): the activations' FWHT runs on the
// matrix cores, 32 (row, block) items per wave (dec_xform_mfma), instead of
// one item per 16-lane group on the VALU.
template <bool NIB, int TN, int KS, bool XRAW, bool MASK, int XC, int D, bool CTV, bool SPLIT,
          int MTD = 1, bool XMF = false, bool SWZ = false>
__global__ __launch_bounds__(TN * KS * 64) void gemv_mfma_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ norms,
    const float* __restrict__ ct, int n_levels, uint32_t code_mask,
    const void* __restrict__ x, int64_t ldx, void* __restrict__ y, int64_t ldy,
    const uint16_t* __restrict__ bias, int M, int N, int nb, uint32_t xs_addr, WLayout lay,
    DecCtArg<NIB> ctv, int io, float* __restrict__ part, uint32_t* __restrict__ cnt) {
  constexpr int NW = TN * KS;
  const bool xbf = (io & 1) != 0, ybf = (io & 2) != 0;  // raw x / y and bias are bfloat16
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar loads, branches
  const int l16 = lane & 15, g = lane >> 4;
  const uint32_t lane4 = (uint32_t)lane << 2;
  // LDS: [codebook table][activations, 256 B per (row, block) from xs_addr];
  // after the K loop the reduction buffer reuses the start of LDS.

  const int jt = wave / KS, ks = wave % KS;
  // K blocks of this workgroup: [kb0, kb0 + nbr)
  const int kb0 = SPLIT ? (int)((int64_t)nb * blockIdx.y / gridDim.y) : 0;
  const int nbr = SPLIT ? (int)((int64_t)nb * (blockIdx.y + 1) / gridDim.y) - kb0 : nb;
  // interleaved slices: block i of this wave is kb0 + ks + KS i
  const int b_begin = kb0 + ks;
  const int nbw = nbr > ks ? (nbr - ks + KS - 1) / KS : 0;  // blocks of this wave (uniform)

  // weight row of this lane (clamped; clamped rows are never stored)
  DecSrc src;
  const int c_blk = (int)lay.c_blk, n_blk2 = (int)lay.n_blk * 2;  // block strides in bytes
  {
    int n = (blockIdx.x * TN + jt) * 16 + l16;
    n = n < N ? n : N - 1;
    // extents up to the last row's end (< 2 GiB: host check)
    const int codes_bytes =
        (int)(lay.codes_off(N - 1) + (int64_t)(nb - 1) * lay.c_blk + (NIB ? 64 : kBlock));
    const int norms_bytes = (int)(lay.norms_off(N - 1) + (int64_t)(nb - 1) * lay.n_blk + 1) * 2;
    src.codes = __builtin_amdgcn_make_buffer_rsrc((void*)codes, (short)0, codes_bytes, kBufFlags);
    src.codes_none = __builtin_amdgcn_make_buffer_rsrc((void*)codes, (short)0, 0, kBufFlags);
    src.norms = __builtin_amdgcn_make_buffer_rsrc((void*)norms, (short)0, norms_bytes, kBufFlags);
    src.norms_none = __builtin_amdgcn_make_buffer_rsrc((void*)norms, (short)0, 0, kBufFlags);
    src.voff_codes = (uint32_t)(lay.codes_off(n) + 16 * g);
    src.voff_norms = (uint32_t)(lay.norms_off(n) * 2);
  }

  // ---- 0. activations: the workgroup's M x nb (row, block) items are spread
  // over its 4 NW 16-lane groups: group gi = 4 wave + g takes items
  // gi + 4 NW i (i < XC), lane l16 holding elements 8 l16 .. 8 l16 + 7.
  // Unconditional (clamped) loads, queued on the CU before any weight load
  // (the activations are on the critical path of the prologue; the weight
  // blocks are not needed before the K loop).
  const int nitems = M * nbr;
  // LDS bytes per activation row: 256 per block plus 16, so that the 16 rows
  // one ds_read_b128 phase reads (lanes l16 = rows) start in 16 different
  // bank groups; without the pad every row began in the same bank (row sizes
  // are multiples of 256 B) and M > 1 reads conflicted 16 ways. SWZ (where
  // the padded rows do not fit, e.g. M = 4 at K = 12288 beside the 64 KB
  // table): no pad, 16-byte chunk c of row m stored at chunk c ^ (m & 15) of
  // its block, which spreads a phase's rows over the banks the same way.
  const uint32_t xrow_b = (uint32_t)nbr * 256u + (SWZ ? 0u : 16u);
  const int gi = wave * 4 + g;
  int it_m, it_b;
  {
    const int it = gi < nitems ? gi : 0;
    it_m = it / nbr;
    it_b = it - it_m * nbr;
  }
  constexpr bool XM = XMF && XRAW;
  // XM: wave w transforms items 32 w .. 32 w + 31, rows fastest (item i is
  // row i % M of block i / M, so the 16 lanes of one LDS write phase cover
  // up to 16 rows, whose padded slots start in different banks); lane l
  // loads positions 16 kt + 8 (l / 32) .. + 7 of item 32 w + l % 32
  u32x4v xq[XM ? 8 : 1];
  int q_m = 0, q_b = 0;
  bool q_live = false;
  if constexpr (XM) {
    const int i = 32 * wave + (lane & 31);
    q_live = i < nitems;
    const int ic = q_live ? i : nitems - 1;
    q_m = ic % M;
    q_b = ic / M;
    if (32 * wave < nitems) {  // uniform
      const char* src = reinterpret_cast<const char*>(x) +
                        ((int64_t)q_m * ldx + (int64_t)(kb0 + q_b) * kBlock + 8 * (lane >> 5)) * 2;
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) xq[kt] = *reinterpret_cast<const u32x4v*>(src + kt * 32);
    }
  }
  u32x4v xr[XC];
  if constexpr (!XM) {
    const char* xb = reinterpret_cast<const char*>(x);
    int m = it_m, b = it_b;
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      const bool ok = gi + 4 * NW * i < nitems;
      const int64_t off = ok ? ((int64_t)m * ldx + (int64_t)(kb0 + b) * kBlock) * 2 + l16 * 16 : 0;
      xr[i] = *reinterpret_cast<const u32x4v*>(xb + off);
      b += 4 * NW;
      while (b >= nbr) {
        b -= nbr;
        ++m;
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // codebook values (scalar loads: they do not queue behind the weight stream)
  DecTable<NIB> tab;
  dec_table_load<NIB, NW, CTV>(tab, ct, ctv, n_levels, wave);
  __builtin_amdgcn_sched_barrier(0);

  // ---- first D blocks of weights: the stream starts before the rest of the
  // prologue
  DecBlk<NIB, 1> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    dec_load<NIB, 1>(ring[d], src, b_begin + KS * d, d < nbw, c_blk, n_blk2);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- 1. codebook table (all waves)
  dec_table_write<NIB, NW, !MASK>(tab, n_levels, wave, lane4);

  // ---- 2. activations into LDS as pair f16: 256 B per (row, block), pair p
  // = (x_tf[128 b + p], x_tf[128 b + 64 + p]) at byte 4 p. XRAW: FWHT of the
  // item by its 16-lane group first (XM: by the wave's MFMAs).
  if constexpr (XM) {
    if (32 * wave < nitems) {  // uniform
      const uint32_t slot = xs_addr + (uint32_t)q_m * xrow_b + (uint32_t)q_b * 256u;
      const uint32_t sw = SWZ ? (uint32_t)q_m & 15u : 0u;
      if (xbf) dec_xform_mfma<true>(xq, slot, q_live, lane, sw);
      else dec_xform_mfma<false>(xq, slot, q_live, lane, sw);
    }
  } else {
    int m = it_m, b = it_b;
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      if (gi + 4 * NW * i < nitems) {  // uniform inside the group
        const uint32_t blk = xs_addr + (uint32_t)m * xrow_b + (uint32_t)b * 256u;
        if constexpr (XRAW) {
          const int q = l16;
          float v[8];
          if (xbf) {  // uniform
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              v[2 * k] = bf2f((uint16_t)(xr[i][k] & 0xffff));
              v[2 * k + 1] = bf2f((uint16_t)(xr[i][k] >> 16));
            }
          } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              v[2 * k] = h2f((uint16_t)(xr[i][k] & 0xffff));
              v[2 * k + 1] = h2f((uint16_t)(xr[i][k] >> 16));
            }
          }
          fwht128_group16(v, q);
          float o[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) o[k] = lane_xor<8>(v[k]);
          // lanes q < 8 own pairs 8q..8q+3, lanes q >= 8 pairs 8(q-8)+4..+7
          u32x4v w;
          uint32_t p0;
          if (q < 8) {
            p0 = 8u * q;
            w = u32x4v{pack_h2(v[0], o[0]), pack_h2(v[1], o[1]), pack_h2(v[2], o[2]),
                       pack_h2(v[3], o[3])};
          } else {
            p0 = 8u * (q - 8) + 4u;
            w = u32x4v{pack_h2(o[4], v[4]), pack_h2(o[5], v[5]), pack_h2(o[6], v[6]),
                       pack_h2(o[7], v[7])};
          }
          lds_st128(blk + 16u * ((p0 >> 2) ^ (SWZ ? (uint32_t)m & 15u : 0u)), w);
        } else {
          lds_st128(blk + 16u * ((uint32_t)l16 ^ (SWZ ? (uint32_t)m & 15u : 0u)), xr[i]);
        }
      }
      b += 4 * NW;
      while (b >= nbr) {
        b -= nbr;
        ++m;
      }
    }
  }
  __syncthreads();

  // ---- 3. K loop, D blocks in flight: A (row m = l16) from
  // LDS, B dequantized from the code registers; a block's lookups are issued
  // before its MFMAs.
  // MTD m-tiles of 16 rows share every weight lookup
  float4v acc[MTD];
#pragma unroll
  for (int i = 0; i < MTD; ++i) acc[i] = float4v{0.f, 0.f, 0.f, 0.f};
  // A row of this lane in m-tile i: row 16 i + l16; rows past M repeat row
  // M-1; they only feed D rows >= M, which are never stored
  // (item (m, b) of the group sits at m * xrow_b + (b - kb0) * 256: the base
  // wraps below zero and comes back with b >= kb0)
  uint32_t arow[MTD], achk[MTD][4];  // SWZ: byte offset of chunk 4 g + t in the row's blocks
#pragma unroll
  for (int i = 0; i < MTD; ++i) {
    const int r = 16 * i + l16;
    const uint32_t rr = (uint32_t)(r < M ? r : M - 1);
    arow[i] = xs_addr + rr * xrow_b - (uint32_t)kb0 * 256u + (SWZ ? 0u : 64u * g);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      achk[i][t] = SWZ ? 16u * ((4u * (uint32_t)g + t) ^ (rr & 15u)) : 16u * t;
  }
  auto do_block = [&](const DecBlk<NIB, 1>& k, int b) {
    u32x4v af[MTD][4];
#pragma unroll
    for (int i = 0; i < MTD; ++i)
#pragma unroll
      for (int t = 0; t < 4; ++t) af[i][t] = lds_ld128(arow[i] + (uint32_t)b * 256u + achk[i][t]);
    half8v bf[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t wl = k.lo[0][t], wh = NIB ? 0u : k.hi[0][t];
      if constexpr (MASK) {
        wl &= code_mask;
        wh &= code_mask;
      }
      bf[t] = dec_dequant<NIB>(wl, wh, lane4);
    }
    float4v blk[MTD];
#pragma unroll
    for (int i = 0; i < MTD; ++i) blk[i] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < MTD; ++i)
        blk[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, af[i][t]), bf[t],
                                                        blk[i], 0, 0, 0);
    const float nrm = h2f(k.nb[0]);
#pragma unroll
    for (int i = 0; i < MTD; ++i) acc[i] += blk[i] * nrm;
  };
  for (int i = 0; i < nbw; i += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (i + d < nbw) do_block(ring[d], b_begin + KS * (i + d));
      dec_load<NIB, 1>(ring[d], src, b_begin + KS * (i + d + D), i + d + D < nbw, c_blk, n_blk2);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- 4. combine the KS K-slices of each tile through LDS:
  // red[ks][jt][i][lane][4]
  __syncthreads();
#pragma unroll
  for (int i = 0; i < MTD; ++i)
    lds_st128((uint32_t)((((ks * TN + jt) * MTD + i) * 64 + lane) * 16), __builtin_bit_cast(u32x4v, acc[i]));
  __syncthreads();
  // outputs: rows m < M (D element e of lane l in m-tile i: row 16 i +
  // 4 (l / 16) + e), 16 TN columns
  if constexpr (!SPLIT) {
    for (int o = tid; o < TN * MTD * 256; o += NW * 64) {
      const int ji = o >> 8, le = o & 255, ln = le >> 2, e = le & 3;  // ji = j * MTD + i
      const int j = ji / MTD, i = ji - j * MTD;
      const int m = 16 * i + 4 * (ln >> 4) + e;
      const int n = (blockIdx.x * TN + j) * 16 + (ln & 15);
      if (m >= M || n >= N) continue;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < KS; ++w)
        s += __builtin_bit_cast(float, lds_ld32((uint32_t)(((((w * TN + j) * MTD + i) * 64) * 4 + le) * 4)));
      reinterpret_cast<uint16_t*>(y)[(int64_t)m * ldy + n] = out16(s, bias, n, ybf);
    }
  } else {
    // Partial sums of this K group, four consecutive columns per thread, as
    // device-coherent stores (cache policy sc1: written through to the level
    // every XCD reads); part[g][m][n] addressed through a buffer resource.
    const int nq = 4 * TN;  // column quads of this workgroup
    const bool vec = (N & 3) == 0;
    const int64_t slab = (int64_t)M * N;
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)part, (short)0, (int)(gridDim.y * slab * 4), kBufFlags);
    for (int o = tid; o < M * nq; o += NW * 64) {
      const int m = o / nq, q = o - m * nq;
      const int j = q >> 2, c0 = (q & 3) * 4, i = m >> 4, r = m & 15;
      const int n = (blockIdx.x * TN + j) * 16 + c0;
      if (n >= N) continue;
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int ln = c0 + u + 16 * (r >> 2);
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < KS; ++w)
          sum += __builtin_bit_cast(
              float, lds_ld32((uint32_t)(((((w * TN + j) * MTD + i) * 64 + ln) * 4 + (r & 3)) * 4)));
        v[u] = sum;
      }
      const uint32_t off = (uint32_t)((((int64_t)blockIdx.y * M + m) * N + n) * 4);
      if (vec) {
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4v{__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                   __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])},
            prs, off, 0, kBufSC1);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (n + u < N)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v[u]), prs,
                                                  off + 4u * u, 0, kBufSC1);
      }
    }
    // Once the stores have completed (vmcnt(0) counts stores on this
    // architecture) the group is counted in; the workgroup that brings the
    // count to gridDim.y adds all the groups. (A device-scope fence instead
    // writes back and invalidates the whole XCD's L2 once per wave: 6x slower
    // at M = 16.)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const uint32_t flag = (uint32_t)(NW * MTD * 64 * 16);  // LDS word past the reduction buffer
    if (tid == 0) {
      const uint32_t done = atomicAdd(&cnt[blockIdx.x], 1u);
      lds_st32(flag, done + 1 == gridDim.y ? 1u : 0u);
    }
    __syncthreads();
    if (lds_ld32(flag) == 0) return;  // uniform: not the last group
    const int G = gridDim.y;
    for (int o = tid; o < M * nq; o += NW * 64) {
      const int m = o / nq, q = o - m * nq;
      const int n = (blockIdx.x * TN + (q >> 2)) * 16 + (q & 3) * 4;
      if (n >= N) continue;
      const uint32_t off0 = (uint32_t)(((int64_t)m * N + n) * 4);
      const uint32_t gstep = (uint32_t)(slab * 4);
      // groups in order 0, 1, .., sixteen loads in flight (coherent sc1
      // reads: the other groups' partials, never a stale line of this XCD's
      // L2); G <= 16 (on 256 CUs every N >= 3072) takes one round trip
      float a[4] = {0.f, 0.f, 0.f, 0.f};
      for (int g0 = 0; g0 < G; g0 += kSplitBatch) {
        u32x4v t[kSplitBatch];
#pragma unroll
        for (int k = 0; k < kSplitBatch; ++k) {
          if (g0 + k < G) {
            const uint32_t off = off0 + (uint32_t)(g0 + k) * gstep;
            if (vec) {
              t[k] = __builtin_bit_cast(u32x4v,
                                        __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, kBufSC1));
            } else {
#pragma unroll
              for (int u = 0; u < 4; ++u)
                t[k][u] = n + u < N ? __builtin_amdgcn_raw_buffer_load_b32(prs, off + 4u * u, 0, kBufSC1)
                                    : 0u;
            }
          }
        }
        // (bit_cast of a whole vector: this compiler reads element 0 when a
        // bit_cast is applied to a vector element)
#pragma unroll
        for (int k = 0; k < kSplitBatch; ++k)
          if (g0 + k < G) {
            const float4v tf = __builtin_bit_cast(float4v, t[k]);
#pragma unroll
            for (int u = 0; u < 4; ++u) a[u] += tf[u];
          }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (n + u < N)
          reinterpret_cast<uint16_t*>(y)[(int64_t)m * ldy + n + u] = out16(a[u], bias, n + u, ybf);
    }
    if (tid == 0) __hip_atomic_store(&cnt[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// y[m, n] = fp16(sum over the groups g = 0.. in order of part[g][m][n]) (+ bias
// as the direct epilogue adds it)
__global__ __launch_bounds__(256) void dec_split_reduce_kernel(const float* __restrict__ part,
                                                               int G, int M, int N,
                                                               const uint16_t* __restrict__ bias,
                                                               uint16_t* __restrict__ y,
                                                               int64_t ldy, int ybf) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int m = (int)(i / N), n = (int)(i - (int64_t)m * N);
  const int64_t slab = (int64_t)M * N;
  const float* p = part + (int64_t)m * N + n;
  // the loads of four groups are issued together, then added in group order
  float s = 0.f;
  int g = 0;
  for (; g + 4 <= G; g += 4) {
    const float v0 = p[g * slab], v1 = p[(g + 1) * slab], v2 = p[(g + 2) * slab], v3 = p[(g + 3) * slab];
    s += v0;
    s += v1;
    s += v2;
    s += v3;
  }
  for (; g < G; ++g) s += p[g * slab];
  y[(int64_t)m * ldy + n] = out16(s, bias, n, ybf != 0);
}

// ---------------------------------------------------------------------------
// host launch
// ---------------------------------------------------------------------------

int split_reduce(const float* part, int G, int M, int N, const uint16_t* bias, void* y, int64_t ldy,
                 hipStream_t st, bool ybf) {
  const int64_t total = (int64_t)M * N;
  if (total <= 0 || (total + 255) / 256 > INT32_MAX) return PE_ERR_DIMS;
  dec_split_reduce_kernel<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st>>>(
      part, G, M, N, bias, reinterpret_cast<uint16_t*>(y), ldy, (int)ybf);
  return launch_status();
}

// waves per workgroup: TN tiles x KS K-slices = 12 (one workgroup per CU;
// measured better than 15-16 waves: fewer competing streams per CU); at least
// 8 so that the table fill covers 256 entries with two per wave
constexpr int kDecW = 12;
template <int TN>
constexpr int dec_ks() { return kDecW / TN; }

// activation registers per lane: M * nb items of 16 x 16 B over the 4 NW
// 16-lane groups of the workgroup
static int dec_xc(int M, int nb, int nw) { return (M * nb + 4 * nw - 1) / (4 * nw); }

// 16-row m-tiles per MFMA pass: 1 (M <= 16) or 2 (M <= 32 = kDecMaxRows)
static int dec_mtd(int M) { return M <= 16 ? 1 : 2; }

// LDS bytes: the table and M activation rows of nb blocks, 16 bytes of pad per
// row unless the rows are swizzled (pad = false, the smaller layout, which
// the fit checks assume; the launch pads where that fits)
static size_t dec_lds(bool nibble, int M, int nb, int n_levels, int nw, bool pad = false) {
  size_t lds = (size_t)table_entries(nibble, n_levels) * 256 + (size_t)M * (nb * 256 + (pad ? 16 : 0));
  const size_t red = (size_t)nw * dec_mtd(M) * 64 * 16 + 16;  // + the K split's last-group flag
  return lds < red ? red : lds;
}

template <bool NIB, int TN, bool XRAW, bool MASK, int XC, bool CTV, bool SPLIT, int MTD, bool XMF,
          bool SWZ>
static int launch_dec_k(const DecArgs& a, hipStream_t st, int groups) {
  constexpr int KS = dec_ks<TN>(), NW = TN * KS;
  // blocks in flight per wave (nibble 1 KB, int8 2 KB each); deeper rings
  // measured slower (3 -> 8: 7.6 -> 8.8 us on Q4 12288 x 4096)
  constexpr int D = NIB ? 3 : 2;
  auto kern = gemv_mfma_kernel<NIB, TN, KS, XRAW, MASK, XC, D, CTV, SPLIT, MTD, XMF, SWZ>;
  if (dec_mtd(a.M) != MTD) return PE_ERR_DIMS;
  const int nbg = (a.nb + groups - 1) / groups;  // most blocks of one group
  const size_t lds = dec_lds(NIB, a.M, nbg, a.n_levels, NW, !SWZ);
  // XMF: 32 items per wave (the same capacity as XC = 8: 8 per 16-lane group)
  if (lds > 160 * 1024 || dec_xc(a.M, nbg, NW) > (XMF ? 8 : XC)) return PE_ERR_DIMS;
  static const bool attr_ok = [&] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  }();
  (void)attr_ok;
  const int tiles = (a.N + TN * 16 - 1) / (TN * 16);
  const uint8_t mb = NIB ? (uint8_t)((a.n_levels - 1) * 0x11) : (uint8_t)(a.n_levels - 1);
  const uint32_t xs_addr = (uint32_t)table_entries(NIB, a.n_levels) * 256u;
  DecCtArg<NIB> ctv;
  constexpr int kCtv = (int)(sizeof(ctv.v) / sizeof(uint32_t));
  for (int i = 0; i < kCtv; ++i) {
    uint32_t w = 0;
    if (CTV)
      for (int q = 0; q < 2; ++q) {
        const int e = 2 * i + q;
        w |= (uint32_t)host_f2h(a.ct_host[e < a.n_levels ? e : a.n_levels - 1]) << (16 * q);
      }
    ctv.v[i] = w;
  }
  kern<<<dim3(tiles, groups), dim3(NW * 64), lds, st>>>(
      a.codes, a.norms, a.ct, a.n_levels, 0x01010101u * mb, a.x, a.ldx, a.y, a.ldy, a.bias, a.M,
      a.N, a.nb, xs_addr, a.lay, ctv, (a.xbf ? 1 : 0) | (a.ybf ? 2 : 0),
      SPLIT ? reinterpret_cast<float*>(a.ws) : nullptr, SPLIT ? a.cnt : nullptr);
  return launch_status();
}

// Padded activation rows where they fit; swizzled ones otherwise (only the
// forms holding up to 8 items per 16-lane group can need it: 384 items of
// 256 B beside a 64 KB table fill the LDS exactly)
template <bool NIB, int TN, bool XRAW, bool MASK, int XC, bool CTV, bool SPLIT = false, int MTD = 1,
          bool XMF = false>
static int launch_dec(const DecArgs& a, hipStream_t st, int groups = 1) {
  if constexpr (XC == 8 || XMF) {
    constexpr int NW = TN * dec_ks<TN>();
    const int nbg = (a.nb + groups - 1) / groups;
    if (dec_lds(NIB, a.M, nbg, a.n_levels, NW, true) > 160 * 1024)
      return launch_dec_k<NIB, TN, XRAW, MASK, XC, CTV, SPLIT, MTD, XMF, true>(a, st, groups);
  }
  return launch_dec_k<NIB, TN, XRAW, MASK, XC, CTV, SPLIT, MTD, XMF, false>(a, st, groups);
}

// activation registers per lane from which the transform moves to the
// matrix cores (32 items per wave): at one item per 16-lane group (M = 1 at
// K <= 6144) the VALU butterfly is cheaper; from two on the MFMAs are
// (down projection 4096 x 12288 at M = 1: 7.89 -> 7.57 us)
constexpr int kDecXformMfmaXc = 2;

template <bool NIB, int TN, bool XRAW, bool MASK>
static int launch_dec_xc(const DecArgs& a, hipStream_t st) {
  const int xc = dec_xc(a.M, a.nb, TN * dec_ks<TN>());
  if (XRAW && xc >= kDecXformMfmaXc)
    return a.ct_host ? launch_dec<NIB, TN, XRAW, MASK, 1, true, false, 1, XRAW>(a, st)
                     : launch_dec<NIB, TN, XRAW, MASK, 1, false, false, 1, XRAW>(a, st);
  if (a.ct_host) {
    if (xc <= 1) return launch_dec<NIB, TN, XRAW, MASK, 1, true>(a, st);
    if (xc <= 2) return launch_dec<NIB, TN, XRAW, MASK, 2, true>(a, st);
    if (xc <= 4) return launch_dec<NIB, TN, XRAW, MASK, 4, true>(a, st);
    return launch_dec<NIB, TN, XRAW, MASK, 8, true>(a, st);
  }
  if (xc <= 1) return launch_dec<NIB, TN, XRAW, MASK, 1, false>(a, st);
  if (xc <= 2) return launch_dec<NIB, TN, XRAW, MASK, 2, false>(a, st);
  if (xc <= 4) return launch_dec<NIB, TN, XRAW, MASK, 4, false>(a, st);
  return launch_dec<NIB, TN, XRAW, MASK, 8, false>(a, st);
}

// n-tiles per workgroup: the fewest rounds of one workgroup per CU, each
// CU's share as even as the 16-row tiles allow (ties: more tiles per
// workgroup, fewer table fills)
static int dec_tn(int N) {
  const int tiles16 = (N + 15) / 16, cus = num_cus();
  int best = 1;
  long best_cost = -1;
  for (int tn = 1; tn <= 4; ++tn) {
    const long wgs = (tiles16 + tn - 1) / tn;
    const long cost = (wgs + cus - 1) / cus * tn;
    if (best_cost < 0 || cost <= best_cost) {
      best = tn;
      best_cost = cost;
    }
  }
  return best;
}

template <bool NIB, bool XRAW, bool MASK>
static int launch_dec_tn(const DecArgs& a, hipStream_t st) {
  switch (dec_tn(a.N)) {
    case 1: return launch_dec_xc<NIB, 1, XRAW, MASK>(a, st);
    case 2: return launch_dec_xc<NIB, 2, XRAW, MASK>(a, st);
    case 3: return launch_dec_xc<NIB, 3, XRAW, MASK>(a, st);
    default: return launch_dec_xc<NIB, 4, XRAW, MASK>(a, st);
  }
}

// K split over workgroups: 12 row tiles per workgroup (one K range per wave),
// gridDim.y groups sized for at most one workgroup per CU. Returns the group
// count, or 0 when the split does not apply (fewer than 2 groups, or one
// group's activations still do not fit). M > 16 (two m-tiles) takes
// more groups, and rounds, until one group's activations fit.
constexpr int kSplitTN = 12;
static int dec_split_groups(bool nibble, int M, int N, int nb, int n_levels) {
  const int wgn = ((N + 15) / 16 + kSplitTN - 1) / kSplitTN;
  // at most one round of workgroups (one per CU: the LDS holds one): a 257th
  // workgroup would run as a second round of its own
  if (wgn > kWsCounters) return 0;  // one completion counter per row group
  int G = num_cus() / wgn;
  // at least four 128-blocks per group: with fewer, every workgroup's fixed
  // costs (prologue, partial stores) outweigh its share of the stream, and
  // the last group reads more slabs (1024 x 4096 at M = 16: G = 32 -> 8,
  // 97 -> 85 us for the seven separate C4 linears)
  if (G > nb / 4) G = nb / 4;
  if (M > 16) {
    if (G < 2) G = nb < 2 ? nb : 2;
    while (G < nb && (dec_xc(M, (nb + G - 1) / G, kDecW) > 8 ||
                      dec_lds(nibble, M, (nb + G - 1) / G, n_levels, kDecW) > 160 * 1024))
      ++G;
  }
  if (G < 2) return 0;
  // the partial sums are addressed through a buffer resource (31-bit offsets)
  if ((int64_t)G * M * N * 4 >= ((int64_t)1 << 31)) return 0;
  const int nbg = (nb + G - 1) / G;
  if (dec_xc(M, nbg, kDecW) > 8 || dec_lds(nibble, M, nbg, n_levels, kDecW) > 160 * 1024) return 0;
  return G;
}

// the split path where the whole activation set does not fit in LDS (each
// workgroup then transforms and holds only its K range of the activations;
// where it fits, one launch without the partial-sum pass measured faster),
// for M >= 2 (M = 1 takes no workspace: it keeps its own paths); M > 16 runs
// only here
static bool dec_use_split(bool nibble, int M, int N, int nb, int n_levels) {
  const bool whole = dec_xc(M, nb, kDecW) <= 8 && dec_lds(nibble, M, nb, n_levels, kDecW) <= 160 * 1024;
  return M >= 2 && (M > 16 || !whole) && dec_split_groups(nibble, M, N, nb, n_levels) > 0;
}

template <bool NIB, bool XRAW, bool MASK>
static int launch_dec_split(const DecArgs& a, hipStream_t st) {
  const int G = dec_split_groups(NIB, a.M, a.N, a.nb, a.n_levels);
  if (!a.ws || !a.cnt || a.ws_bytes < (size_t)G * a.M * a.N * 4) return PE_ERR_WORKSPACE;
  const int xc = dec_xc(a.M, (a.nb + G - 1) / G, kDecW);
  const int mtd = dec_mtd(a.M);
  if (XRAW && xc >= kDecXformMfmaXc) {
    if (mtd > 2) return PE_ERR_DIMS;
    if (mtd == 2)
      return a.ct_host ? launch_dec<NIB, kSplitTN, XRAW, MASK, 1, true, true, 2, XRAW>(a, st, G)
                       : launch_dec<NIB, kSplitTN, XRAW, MASK, 1, false, true, 2, XRAW>(a, st, G);
    return a.ct_host ? launch_dec<NIB, kSplitTN, XRAW, MASK, 1, true, true, 1, XRAW>(a, st, G)
                     : launch_dec<NIB, kSplitTN, XRAW, MASK, 1, false, true, 1, XRAW>(a, st, G);
  }
  if (mtd > 1) {  // two m-tiles (kDecMaxRows = 32): activation registers 4 or 8
    if (mtd != 2) return PE_ERR_DIMS;
    if (a.ct_host)
      return xc <= 4 ? launch_dec<NIB, kSplitTN, XRAW, MASK, 4, true, true, 2>(a, st, G)
                     : launch_dec<NIB, kSplitTN, XRAW, MASK, 8, true, true, 2>(a, st, G);
    return xc <= 4 ? launch_dec<NIB, kSplitTN, XRAW, MASK, 4, false, true, 2>(a, st, G)
                   : launch_dec<NIB, kSplitTN, XRAW, MASK, 8, false, true, 2>(a, st, G);
  }
  if (a.ct_host) {
    if (xc <= 2) return launch_dec<NIB, kSplitTN, XRAW, MASK, 2, true, true>(a, st, G);
    if (xc <= 4) return launch_dec<NIB, kSplitTN, XRAW, MASK, 4, true, true>(a, st, G);
    return launch_dec<NIB, kSplitTN, XRAW, MASK, 8, true, true>(a, st, G);
  }
  if (xc <= 2) return launch_dec<NIB, kSplitTN, XRAW, MASK, 2, false, true>(a, st, G);
  if (xc <= 4) return launch_dec<NIB, kSplitTN, XRAW, MASK, 4, false, true>(a, st, G);
  return launch_dec<NIB, kSplitTN, XRAW, MASK, 8, false, true>(a, st, G);
}

template <bool NIB, bool XRAW>
static int launch_dec_m(const DecArgs& a, hipStream_t st) {
  const bool mask = NIB ? a.n_levels != 16 : a.n_levels != 256;
  if (dec_use_split(NIB, a.M, a.N, a.nb, a.n_levels))
    return mask ? launch_dec_split<NIB, XRAW, true>(a, st) : launch_dec_split<NIB, XRAW, false>(a, st);
  return mask ? launch_dec_tn<NIB, XRAW, true>(a, st) : launch_dec_tn<NIB, XRAW, false>(a, st);
}

size_t gemv_mfma_workspace(bool nibble, int M, int N, int nb, int n_levels) {
  if (M < 1 || M > kDecMaxRows || !dec_use_split(nibble, M, N, nb, n_levels)) return 0;
  return (size_t)dec_split_groups(nibble, M, N, nb, n_levels) * M * N * 4;
}

bool gemv_mfma_fits(bool nibble, int M, int N, int nb, int n_levels) {
  if (M < 1 || M > kDecMaxRows) return false;
  // buffer resources address codes and norms with 31-bit offsets (tiled
  // layouts round N up to 16 rows)
  if ((int64_t)(N + 15) * nb * (nibble ? 64 : kBlock) >= (int64_t)1 << 31) return false;
  if (dec_use_split(nibble, M, N, nb, n_levels)) return true;
  if (M > 16) return false;  // two m-tiles: the split path only
  // the workgroup's 4 * kDecW lane groups hold the activations in <= 8 registers
  return dec_xc(M, nb, kDecW) <= 8 && dec_lds(nibble, M, nb, n_levels, kDecW) <= 160 * 1024;
}

int gemv_mfma(bool nibble, bool xraw, const DecArgs& a, hipStream_t st) {
  if (!gemv_mfma_fits(nibble, a.M, a.N, a.nb, a.n_levels)) return PE_ERR_DIMS;
  if (nibble) return xraw ? launch_dec_m<true, true>(a, st) : launch_dec_m<true, false>(a, st);
  return xraw ? launch_dec_m<false, true>(a, st) : launch_dec_m<false, false>(a, st);
}

}  // namespace pe
