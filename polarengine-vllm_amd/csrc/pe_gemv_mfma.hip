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
//  * one workgroup of NW waves per CU-sized share of rows: TN n-tiles of 16
//    weight rows (TN chosen so the grid covers the CUs once); the NW waves
//    split the 128-blocks of K (contiguous ranges) and combine through LDS;
//  * the prologue never waits behind the weight stream: each wave first
//    issues its activation loads and ONE block of weights, fills its share of
//    the codebook table from scalar loads of ct (SMEM, not the vector memory
//    queue that the weight stream fills), transforms its activations, and
//    only then streams the rest of its blocks with a two-deep prefetch;
//  * fused FWHT: wave w transforms only its own blocks of x (one 16-lane
//    group per block, DPP butterflies) into pair-f16 in LDS;
//  * A = activation pairs (row m = lane % 16, rows >= M zero), B = table
//    lookups half2(ct[lo], ct[hi]); block norms scale the fp32 block partial.

#include "pe_internal.h"

namespace pe {

template <bool NIB, int TN>
struct DecBlk {
  u32x4v lo[TN];
  u32x4v hi[TN];
  uint16_t nb[TN];
};

// Loads of one block of the TN rows; an invalid block (past the wave's range)
// loads 16 bytes of the codebook instead, so the number of loads issued is
// the same on every path (exact vmcnt waits) at no HBM cost.
template <bool NIB, int TN>
__device__ __forceinline__ void dec_load(DecBlk<NIB, TN>& k, const uint8_t* const (&brow)[TN],
                                         const uint16_t* const (&nrow)[TN], int b, bool valid,
                                         const void* dummy) {
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const uint8_t* pc = valid ? brow[j] + (NIB ? b * 64 : b * kBlock)
                              : reinterpret_cast<const uint8_t*>(dummy);
    const uint16_t* pn = valid ? nrow[j] + b : reinterpret_cast<const uint16_t*>(dummy);
    k.lo[j] = ld_nt16v(pc);
    if constexpr (!NIB) k.hi[j] = ld_nt16v(valid ? pc + 64 : pc);
    k.nb[j] = *pn;
  }
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

// Codebook table from wave-uniform (scalar) loads of ct; every lane writes its
// own copy of each entry. Nibble: entry (hi << 4) | lo = half2(ct[lo], ct[hi]),
// wave w takes hi = w, w + NW, ...; int8: entry e = fp16(ct[e]) in the low
// half, wave w takes e = 16 w .. 16 w + 15, then + 16 NW.
template <bool NIB, int NW>
__device__ __forceinline__ void dec_fill_table(const float* __restrict__ ct, int n_levels, int wave,
                                               uint32_t lane4) {
  if constexpr (NIB) {
    float clo[16];
#pragma unroll
    for (int lo = 0; lo < 16; ++lo) clo[lo] = ct[lo < n_levels ? lo : n_levels - 1];
    for (int hi = wave; hi < n_levels; hi += NW) {
      const float chi = ct[hi];
#pragma unroll
      for (int lo = 0; lo < 16; ++lo)
        if (lo < n_levels)
          lds_st32((uint32_t)((hi << 4) | lo) << 8 | lane4, pack_h2(clo[lo], chi));
    }
  } else {
    for (int e0 = wave * 16; e0 < n_levels; e0 += NW * 16) {
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (e0 + k < n_levels)
          lds_st32((uint32_t)(e0 + k) << 8 | lane4, (uint32_t)f2h_bits(ct[e0 + k]));
    }
  }
}

// x: raw fp16 activations [M, K] (XRAW) or pair-f16 x_tf [M][nb][64] (else),
// row stride ldx fp16 elements. XC: activation registers per lane.
template <bool NIB, int TN, int NW, bool XRAW, bool MASK, int XC, int SCHED = 0>
__global__ __launch_bounds__(NW * 64) void gemv_mfma_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ norms,
    const float* __restrict__ ct, int n_levels, uint32_t code_mask,
    const void* __restrict__ x, int64_t ldx, void* __restrict__ y, int64_t ldy,
    const uint16_t* __restrict__ bias, int M, int N, int nb, uint32_t xs_addr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar loads, branches
  const int l16 = lane & 15, g = lane >> 4;
  const uint32_t lane4 = (uint32_t)lane << 2;
  // LDS: [codebook table][activations, 256 B per (row, block) from xs_addr];
  // after the K loop the reduction buffer reuses the start of LDS.

  const int b_begin = (int)((int64_t)nb * wave / NW);
  const int b_end = (int)((int64_t)nb * (wave + 1) / NW);
  const int nbw = b_end - b_begin;  // blocks of this wave (uniform)

  // weight rows of this lane (clamped; clamped rows are never stored)
  const int row_bytes = NIB ? nb * 64 : nb * kBlock;
  const uint8_t* brow[TN];
  const uint16_t* nrow[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    int n = blockIdx.x * TN * 16 + j * 16 + l16;
    n = n < N ? n : N - 1;
    brow[j] = codes + (int64_t)n * row_bytes + 16 * g;
    nrow[j] = norms + (int64_t)n * nb;
  }

  // ---- 0. activations: the workgroup's M x nb (row, block) items are spread
  // over the 16-lane groups of its first PW waves ("prologue waves"): group
  // gi = 4 wave + g takes items gi + 4 PW i (i < XC), lane l16 holding
  // elements 8 l16 .. 8 l16 + 7. Unconditional (clamped) loads.
  constexpr int PW = SCHED == 2 ? NW / 2 : NW;
  const bool pro = wave < PW;  // uniform
  const int nitems = M * nb;
  const int gi = wave * 4 + g;
  int it_m, it_b;
  {
    const int it = gi < nitems ? gi : 0;
    it_m = it / nb;
    it_b = it - it_m * nb;
  }
  u32x4v xr[XC];
  if (pro) {
    const char* xb = reinterpret_cast<const char*>(x);
    int m = it_m, b = it_b;
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      const bool ok = gi + 4 * PW * i < nitems;
      const int64_t off = ok ? ((int64_t)m * ldx + (int64_t)b * kBlock) * 2 + l16 * 16 : 0;
      xr[i] = *reinterpret_cast<const u32x4v*>(xb + off);
      b += 4 * PW;
      while (b >= nb) {
        b -= nb;
        ++m;
      }
    }
  }

  // ---- table + transform of the activations into LDS as pair f16: 256 B per
  // (row, block), pair p = (x_tf[128 b + p], x_tf[128 b + 64 + p]) at byte 4 p.
  // XRAW: FWHT of the item by its 16-lane group first.
  auto prologue = [&]() {
    dec_fill_table<NIB, PW>(ct, n_levels, wave, lane4);
    int m = it_m, b = it_b;
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      if (gi + 4 * PW * i < nitems) {  // uniform inside the group
        const uint32_t blk = xs_addr + (uint32_t)(m * nb + b) * 256u;
        if constexpr (XRAW) {
          const int q = l16;
          float v[8];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            v[2 * k] = h2f((uint16_t)(xr[i][k] & 0xffff));
            v[2 * k + 1] = h2f((uint16_t)(xr[i][k] >> 16));
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
          lds_st128(blk + p0 * 4u, w);
        } else {
          lds_st128(blk + (uint32_t)l16 * 16u, xr[i]);
        }
      }
      b += 4 * PW;
      while (b >= nb) {
        b -= nb;
        ++m;
      }
    }
  };

  DecBlk<NIB, TN> r0, r1;
  if constexpr (SCHED == 1) {
    // prologue first, then the weight stream
    prologue();
    __syncthreads();
    dec_load<NIB, TN>(r0, brow, nrow, b_begin, nbw > 0, ct);
    dec_load<NIB, TN>(r1, brow, nrow, b_begin + 1, nbw > 1, ct);
  } else {
    // every wave has queued its activation loads before any weight load
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (SCHED == 0) {
      dec_load<NIB, TN>(r0, brow, nrow, b_begin, nbw > 0, ct);
      __builtin_amdgcn_sched_barrier(0);
      prologue();
      dec_load<NIB, TN>(r1, brow, nrow, b_begin + 1, nbw > 1, ct);
    } else {
      if (!pro) {
        dec_load<NIB, TN>(r0, brow, nrow, b_begin, nbw > 0, ct);
        dec_load<NIB, TN>(r1, brow, nrow, b_begin + 1, nbw > 1, ct);
      } else {
        prologue();
        dec_load<NIB, TN>(r0, brow, nrow, b_begin, nbw > 0, ct);
        dec_load<NIB, TN>(r1, brow, nrow, b_begin + 1, nbw > 1, ct);
      }
    }
    __syncthreads();
  }

  // ---- 3. K loop, two blocks in flight: A (row m = l16, zero past M) from
  // LDS, B dequantized from the code registers; a block's lookups are issued
  // before its MFMAs.
  float4v acc[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) acc[j] = float4v{0.f, 0.f, 0.f, 0.f};
  const bool arow_ok = l16 < M;
  const uint32_t arow = xs_addr + (uint32_t)(l16 * nb) * 256u + 64u * g;
  auto do_block = [&](const DecBlk<NIB, TN>& k, int b) {
    u32x4v af[4];
    if (arow_ok) {
#pragma unroll
      for (int t = 0; t < 4; ++t) af[t] = lds_ld128(arow + (uint32_t)b * 256u + 16u * t);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) af[t] = u32x4v{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      half8v bf[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint32_t wl = k.lo[j][t], wh = NIB ? 0u : k.hi[j][t];
        if constexpr (MASK) {
          wl &= code_mask;
          wh &= code_mask;
        }
        bf[t] = dec_dequant<NIB>(wl, wh, lane4);
      }
      float4v blk = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t)
        blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, af[t]), bf[t], blk,
                                                     0, 0, 0);
      acc[j] += blk * h2f(k.nb[j]);
    }
  };
  for (int i = 0; i < nbw; i += 2) {
    do_block(r0, b_begin + i);
    dec_load<NIB, TN>(r0, brow, nrow, b_begin + i + 2, i + 2 < nbw, ct);
    __builtin_amdgcn_sched_barrier(0);
    if (i + 1 < nbw) do_block(r1, b_begin + i + 1);
    dec_load<NIB, TN>(r1, brow, nrow, b_begin + i + 3, i + 3 < nbw, ct);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- 4. combine the NW K-slices through LDS: red[w][j][lane][4]
  __syncthreads();
#pragma unroll
  for (int j = 0; j < TN; ++j)
    lds_st128((uint32_t)(((wave * TN + j) * 64 + lane) * 16), __builtin_bit_cast(u32x4v, acc[j]));
  __syncthreads();
  // outputs: rows m < M (D element e of lane l: row 4*(l/16) + e), 16*TN columns
  for (int o = tid; o < TN * 256; o += NW * 64) {
    const int j = o >> 8, le = o & 255, ln = le >> 2, e = le & 3;
    const int m = 4 * (ln >> 4) + e;
    const int n = blockIdx.x * TN * 16 + j * 16 + (ln & 15);
    if (m >= M || n >= N) continue;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w)
      s += __builtin_bit_cast(float, lds_ld32((uint32_t)((((w * TN + j) * 64) * 4 + le) * 4)));
    _Float16 hv = (_Float16)s;
    if (bias) hv = (_Float16)((float)hv + h2f(bias[n]));
    reinterpret_cast<_Float16*>(y)[(int64_t)m * ldy + n] = hv;
  }
}

// ---------------------------------------------------------------------------
// host launch
// ---------------------------------------------------------------------------

constexpr int kDecNW = 16;  // waves per workgroup (one workgroup per CU)

// activation registers per lane: M * nb items of 16 x 16 B over the 4 * NW
// 16-lane groups of the workgroup
static int dec_xc(int M, int nb) { return (M * nb + 4 * kDecNW - 1) / (4 * kDecNW); }

static size_t dec_lds(bool nibble, int M, int nb, int n_levels, int tn) {
  size_t lds = (size_t)table_entries(nibble, n_levels) * 256 + (size_t)M * nb * 256;
  const size_t red = (size_t)kDecNW * tn * 64 * 16;
  return lds < red ? red : lds;
}

template <bool NIB, int TN, bool XRAW, bool MASK, int XC>
static int launch_dec(const DecArgs& a, hipStream_t st) {
  auto kern = gemv_mfma_kernel<NIB, TN, kDecNW, XRAW, MASK, XC>;
  const size_t lds = dec_lds(NIB, a.M, a.nb, a.n_levels, TN);
  if (lds > 160 * 1024 || dec_xc(a.M, a.nb) > XC) return PE_ERR_DIMS;
  static const bool attr_ok = [&] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  }();
  (void)attr_ok;
  const int tiles = (a.N + TN * 16 - 1) / (TN * 16);
  const uint8_t mb = NIB ? (uint8_t)((a.n_levels - 1) * 0x11) : (uint8_t)(a.n_levels - 1);
  const uint32_t xs_addr = (uint32_t)table_entries(NIB, a.n_levels) * 256u;
  kern<<<dim3(tiles), dim3(kDecNW * 64), lds, st>>>(a.codes, a.norms, a.ct, a.n_levels,
                                                   0x01010101u * mb, a.x, a.ldx, a.y, a.ldy,
                                                   a.bias, a.M, a.N, a.nb, xs_addr);
  return launch_status();
}

template <bool NIB, int TN, bool XRAW, bool MASK>
static int launch_dec_xc(const DecArgs& a, hipStream_t st) {
  const int xc = dec_xc(a.M, a.nb);
  if (xc <= 1) return launch_dec<NIB, TN, XRAW, MASK, 1>(a, st);
  if (xc <= 2) return launch_dec<NIB, TN, XRAW, MASK, 2>(a, st);
  if (xc <= 4) return launch_dec<NIB, TN, XRAW, MASK, 4>(a, st);
  return launch_dec<NIB, TN, XRAW, MASK, 8>(a, st);
}

// n-tiles per workgroup: the fewest rounds of one workgroup per CU, each
// CU's share as even as the 16-row tiles allow (ties: more tiles per
// workgroup, fewer table fills)
static int dec_tn(int N) {
  const int tiles16 = (N + 15) / 16, cus = num_cus();
  int best = 1;
  long best_cost = -1;
  for (int tn = 1; tn <= 3; ++tn) {
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
    default: return launch_dec_xc<NIB, 3, XRAW, MASK>(a, st);
  }
}

template <bool NIB, bool XRAW>
static int launch_dec_m(const DecArgs& a, hipStream_t st) {
  const bool mask = NIB ? a.n_levels != 16 : a.n_levels != 256;
  return mask ? launch_dec_tn<NIB, XRAW, true>(a, st) : launch_dec_tn<NIB, XRAW, false>(a, st);
}

bool gemv_mfma_fits(bool nibble, int M, int nb, int n_levels) {
  if (M < 1 || M > 16 || dec_xc(M, nb) > 8) return false;
  return dec_lds(nibble, M, nb, n_levels, 3) <= 160 * 1024;
}

int gemv_mfma(bool nibble, bool xraw, const DecArgs& a, hipStream_t st) {
  if (!gemv_mfma_fits(nibble, a.M, a.nb, a.n_levels)) return PE_ERR_DIMS;
  if (nibble) return xraw ? launch_dec_m<true, true>(a, st) : launch_dec_m<true, false>(a, st);
  return xraw ? launch_dec_m<false, true>(a, st) : launch_dec_m<false, false>(a, st);
}

}  // namespace pe
